"""Calibration kernels beside the product library: the matrix-pipe rate probe (mfma_rate.hip),
built into calib/libfl_calib.so, which bench.py --only mfma loads. Nothing in flash_lab uses it.

    python flash-attention-lab_amd/calib/__init__.py     # build it
"""

from __future__ import annotations

import ctypes
import importlib.util
import os
from pathlib import Path

HERE = Path(__file__).resolve().parent
SOURCE = HERE / "mfma_rate.hip"
OUTPUT = HERE / "libfl_calib.so"

# flc_mfma_rate_probe flags (mfma_rate.hip).
PROBE_ZERO_OPERANDS = 1
PROBE_LDS_A = 2


def _csrc_build():
    spec = importlib.util.spec_from_file_location("flash_lab_csrc_build", HERE.parent / "csrc" / "build.py")
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    return module


def build(verbose: bool = False) -> Path:
    """Compiles mfma_rate.hip with the product library's compiler and flags; always rebuilds."""
    csrc = _csrc_build()
    compiler = csrc.hipcc()
    tmp = OUTPUT.with_suffix(".so.tmp")
    csrc._run([compiler, *csrc.FLAGS, f"-I{csrc.CSRC}", "-shared", str(SOURCE), "-o", str(tmp)], verbose)
    os.replace(tmp, OUTPUT)
    return OUTPUT


def load() -> ctypes.CDLL:
    """The calibration library, built first if it is not there."""
    if not OUTPUT.exists():
        build()
    lib = ctypes.CDLL(str(OUTPUT))
    lib.flc_mfma_rate_probe.restype = ctypes.c_int
    lib.flc_mfma_rate_probe.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32,
                                        ctypes.c_int32, ctypes.c_void_p]
    lib.flc_last_error.restype = ctypes.c_char_p
    lib.flc_last_error.argtypes = []
    return lib


if __name__ == "__main__":
    print(f"built {build(verbose=True)}")
