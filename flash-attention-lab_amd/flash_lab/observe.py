"""Observability for the benchmarks: GPU clock/power/temperature sampling and roctx ranges.

The counterparts of the reference's bench/clocks.py (an nvidia-smi sampler) and of the NVTX
ranges of bench/decode_trace.py, for MI355X:

* ClockSampler samples the shader (gfx) and memory clocks, socket power and hotspot temperature
  of one GPU through the amdsmi Python bindings, in a background thread or on demand (sample()),
  with host timestamps;
  window(start, end) reports min / median / max over a time window (one benchmark). On gfx950 the
  shader clock under sustained MFMA load settles well below its 2.4 GHz maximum (power limit), so
  a throughput figure is only interpretable next to the clock it ran at.
* roctx_range(name) pushes and pops a roctx range (rocprofiler-sdk roctx), which `rocprofv3 --marker-trace`
  records, so every kernel of a benchmark step can be attributed to that step.

Both degrade to no-ops where the library or the GPU is missing (the CPU test machine), and neither
changes any GPU setting: amdsmi is only read.
"""

from __future__ import annotations

import contextlib
import ctypes
import statistics
import threading
import time

FIELDS = ("gfx_mhz", "mem_mhz", "power_w", "temp_c")


def _amdsmi_reader(device_index: int):
    """A function returning one sample (a tuple of FIELDS, None where unreadable), or None if
    amdsmi cannot see a GPU here."""
    try:
        import amdsmi
    except ImportError:
        return None, None
    try:
        amdsmi.amdsmi_init()
        handles = amdsmi.amdsmi_get_processor_handles()
        handle = handles[device_index]
    except Exception:  # no driver, no device, or no permission: sampling is off
        return None, None

    def clock(kind):
        try:
            return float(amdsmi.amdsmi_get_clock_info(handle, kind)["clk"])
        except Exception:
            return None

    def power():
        try:
            info = amdsmi.amdsmi_get_power_info(handle)
        except Exception:
            return None
        for key in ("current_socket_power", "average_socket_power", "socket_power"):
            value = info.get(key)
            if isinstance(value, (int, float)) and value > 0:
                return float(value)
        return None

    def temperature():
        try:
            return float(
                amdsmi.amdsmi_get_temp_metric(
                    handle,
                    amdsmi.AmdSmiTemperatureType.HOTSPOT,
                    amdsmi.AmdSmiTemperatureMetric.CURRENT,
                )
            )
        except Exception:
            return None

    def sample():
        return (
            clock(amdsmi.AmdSmiClkType.GFX),
            clock(amdsmi.AmdSmiClkType.MEM),
            power(),
            temperature(),
        )

    def shutdown():
        with contextlib.suppress(Exception):
            amdsmi.amdsmi_shut_down()

    return sample, shutdown


class ClockSampler:
    """Samples GPU clocks, power and temperature every interval_ms while the context is open."""

    def __init__(self, device_index: int = 0, interval_ms: int = 50):
        self.device_index = device_index
        self.interval_s = interval_ms / 1e3
        self.samples: list[tuple[float, tuple]] = []
        self.available = False
        self._stop = threading.Event()
        self._thread: threading.Thread | None = None
        self._shutdown = None

    def __enter__(self) -> "ClockSampler":
        sample, self._shutdown = _amdsmi_reader(self.device_index)
        if sample is None:
            return self
        self.available = True
        self._sample = sample
        if self.interval_s <= 0:  # no background thread: the caller samples with sample()
            return self

        def loop():
            while not self._stop.is_set():
                stamp = time.time()
                self.samples.append((stamp, sample()))
                self._stop.wait(self.interval_s)

        self._thread = threading.Thread(target=loop, daemon=True)
        self._thread.start()
        return self

    def sample(self) -> None:
        """Takes one sample now, in the calling thread. A background thread in a Python process
        that is busy launching kernels holds the interpreter lock rarely, so for short regions
        the caller samples explicitly while it waits for the GPU (bench.py does)."""
        if self.available:
            self.samples.append((time.time(), self._sample()))

    def __exit__(self, *exc) -> None:
        self._stop.set()
        if self._thread is not None:
            self._thread.join(timeout=5)
        if self._shutdown is not None:
            self._shutdown()

    def window(self, start: float, end: float) -> dict | None:
        """Min, median and max of each field between two time.time() stamps. A window shorter than
        the sampling interval gets the sample nearest its middle; None without samples."""
        rows = [values for stamp, values in self.samples if start <= stamp <= end]
        if not rows and self.samples:
            middle = (start + end) / 2
            rows = [min(self.samples, key=lambda s: abs(s[0] - middle))[1]]
        if not rows:
            return None
        out: dict = {"samples": len(rows)}
        for i, name in enumerate(FIELDS):
            column = [row[i] for row in rows if row[i] is not None]
            if column:
                out[name] = {
                    "min": min(column),
                    "median": statistics.median(column),
                    "max": max(column),
                }
        return out


def driver_record(device_index: int = 0) -> dict | None:
    """The GPU's driver and firmware identity and its power cap, read once through amdsmi (the
    counterpart of the driver fields of the reference's bench/env.py:39-106); None without amdsmi
    or a visible GPU."""
    try:
        import amdsmi
    except ImportError:
        return None
    try:
        amdsmi.amdsmi_init()
        handle = amdsmi.amdsmi_get_processor_handles()[device_index]
    except Exception:
        return None
    out: dict = {}
    for key, call in (("driver", "amdsmi_get_gpu_driver_info"), ("vbios", "amdsmi_get_gpu_vbios_info"),
                      ("power_cap", "amdsmi_get_power_cap_info"), ("asic", "amdsmi_get_gpu_asic_info")):
        try:
            info = getattr(amdsmi, call)(handle)
        except Exception:
            continue
        if isinstance(info, dict):
            out[key] = {k: v for k, v in info.items() if isinstance(v, (str, int, float))}
    with contextlib.suppress(Exception):
        amdsmi.amdsmi_shut_down()
    return out


_ROCTX = None
_ROCTX_TRIED = False


def _roctx():
    global _ROCTX, _ROCTX_TRIED
    if not _ROCTX_TRIED:
        _ROCTX_TRIED = True
        # rocprofv3 intercepts the rocprofiler-sdk roctx library; the legacy libroctx64 is the
        # fallback for older tools.
        for name in ("librocprofiler-sdk-roctx.so", "/opt/rocm/lib/librocprofiler-sdk-roctx.so",
                     "libroctx64.so", "/opt/rocm/lib/libroctx64.so"):
            try:
                lib = ctypes.CDLL(name)
            except OSError:
                continue
            lib.roctxRangePushA.argtypes = [ctypes.c_char_p]
            lib.roctxRangePushA.restype = ctypes.c_int
            lib.roctxRangePop.argtypes = []
            lib.roctxRangePop.restype = ctypes.c_int
            _ROCTX = lib
            break
    return _ROCTX


@contextlib.contextmanager
def roctx_range(name: str):
    """A roctx range around the block (no-op without a roctx library)."""
    lib = _roctx()
    if lib is not None:
        lib.roctxRangePushA(name.encode())
    try:
        yield
    finally:
        if lib is not None:
            lib.roctxRangePop()
