"""Benchmark of the two hot paths on one MI355X; prints ONE JSON line.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--no-e2e]
                    [--only prefill|prefill_causal|decode|<decode name>|e2e_L|copy,...]

Metric: prefill TFLOP/s at (B, H, H_kv, S, D) = (4, 32, 32, 4096, 128) bf16 and
split-KV decode GB/s at 32K keys. A step is one prefill forward over that batch (non-causal), the
configuration the metric is quoted on; `value` is its throughput. The causal prefill, the three
decode configurations (B=1 MHA, B=8 MHA, B=8 GQA, 32K keys; B=8 GQA also as a paged cache of
16-row blocks) and the Llama-3.1-8B-shaped end-to-end run (config L: TTFT and decode ms/step) are
reported under "secondary".

Inputs are synthetic iid N(0, 1) bf16 from torch.Generator(device="cuda").manual_seed(0), drawn in
the reference's order (q, k, v; decode q, k_cache, v_cache: reference bench/run.py:122-141), and
are resident in HBM before timing. Every configuration is checked against the fp64 oracle before
it is timed, with the reference's rule (bench/run.py:102-119): prefill on the reference's 256
sampled query rows of every (batch, head), decode on every sequence in full. A workload that fails
its check is reported "incorrect", is not timed, and makes the exit status non-zero. Prefill FLOPs
are 4 B H S_q S_k D, halved for causal; decode bytes are the K and V bytes read (reference
bench/flops.py:31-57; the reference's variant adding q and o is reported beside them). Decode
timings zero a 1 GiB buffer before each call so the 256 MB Infinity Cache holds no K/V.

roofline: the dominant kernel's algorithmic FLOPs (or bytes) per launch over its mean duration
from HIP events recorded on the stream it is launched on, against MI355X peaks (dense bf16 MFMA
2.5 PFLOP/s, HBM 8 TB/s). cpu_baseline: the reference CPU path (the oracle, a restatement of
flash_lab.reference: PyTorch fp64 on the host cores, core count stated), timed with perf_counter
in the same run on bounded samples of each workload: C1 (B=1, H=4, S=256, D=64 fp32 and fp64,
checked to 1e-5 normwise), the 256-row prefill check causal and non-causal (extrapolated
TFLOP/s), and the full fp64 decode of D1, D8 and G8 (GB/s of bf16 K+V). Each figure is also
attached to its GPU workload under "reference_cpu_path".
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
for _p in (REPO, REPO / "flash-attention-lab_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_HBM_GBPS = 8000.0  # MI355X HBM3E
FLUSH_BYTES = 1 << 30  # larger than the 256 MB Infinity Cache
BASELINE_TFLOPS = 229.2  # reference mma_pipelined, non-causal, H100 SXM5 (reference bench/results/h100-80gb-hbm3/summary-cc64b18.md:154)

PREFILL = dict(batch=4, heads=32, heads_kv=32, seqlen=4096, head_dim=128)
# head_dim 64 at the same tokens and half the FLOP (64 heads of 64): the kernel's D = 64 case.
PREFILL_D64 = dict(batch=4, heads=64, heads_kv=64, seqlen=4096, head_dim=64)
DECODE = {
    "B1-MHA": dict(batch=1, heads=32, heads_kv=32, context=32768, head_dim=128),
    "B8-MHA": dict(batch=8, heads=32, heads_kv=32, context=32768, head_dim=128),
    "B8-GQA": dict(batch=8, heads=32, heads_kv=8, context=32768, head_dim=128),
    # The same cache in 16-row blocks of a pool, in shuffled order (block_tables).
    "B8-GQA-paged16": dict(batch=8, heads=32, heads_kv=8, context=32768, head_dim=128, page_size=16),
    # The same cache with 8 query heads per KV head (a Llama-70B-like group), not a reference
    # configuration: the matrix-core decode kernel's case.
    "B8-GQA8": dict(batch=8, heads=64, heads_kv=8, context=32768, head_dim=128),
}


def attention_flops(batch, heads, seqlen_q, seqlen_k, head_dim, causal) -> float:
    """Matmul FLOPs of one forward: 2 S_q S_k D for Q K^T and again for P V, per head; causal
    counts half (the FlashAttention-2 convention)."""
    flops = 4.0 * batch * heads * seqlen_q * seqlen_k * head_dim
    return flops / 2 if causal else flops


def decode_kv_bytes(batch, heads_kv, context, head_dim, elem) -> float:
    """K and V bytes one decode step reads: every cached row once."""
    return 2.0 * batch * heads_kv * context * head_dim * elem


def decode_bytes_with_qo(batch, heads, heads_kv, context, head_dim, elem) -> float:
    """The reference's decode byte count: K and V plus q read and o written."""
    return decode_kv_bytes(batch, heads_kv, context, head_dim, elem) + 2.0 * batch * heads * head_dim * elem


def summarize(times_ms: list[float]) -> dict:
    ordered = sorted(times_ms)

    def pct(p):
        return ordered[min(len(ordered) - 1, round(p / 100 * (len(ordered) - 1)))]

    return {"median": statistics.median(ordered), "p10": pct(10), "p90": pct(90), "min": ordered[0]}


def cpu_cores() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def env_record() -> dict:
    """What ran, in the spirit of the reference's bench/env.py:39-106: the checkout's git HEAD
    (git is absent where the benchmark runs on a copied tree, so the library's build record, which
    names the HEAD it was built from, stands beside it), the library's own hash and version,
    torch, HIP, ROCm, Python, and the GPU's driver, VBIOS and power cap from amdsmi."""
    import hashlib
    import platform
    import subprocess

    import torch

    from flash_lab import _hip
    from flash_lab.observe import driver_record

    rec: dict = {"python": platform.python_version(), "torch": torch.__version__,
                 "hip": getattr(torch.version, "hip", None)}
    try:
        rec["rocm"] = Path("/opt/rocm/.info/version").read_text().strip()
    except OSError:
        rec["rocm"] = None
    try:
        proc = subprocess.run(["git", "-C", str(REPO), "rev-parse", "HEAD"], capture_output=True,
                              text=True, timeout=10)
        rec["git_head"] = proc.stdout.strip() if proc.returncode == 0 else None
    except (OSError, subprocess.TimeoutExpired):
        rec["git_head"] = None
    lib_path = Path(_hip.LIB._name)
    library = {"path": str(lib_path.relative_to(REPO)) if lib_path.is_relative_to(REPO) else str(lib_path),
               "version": _hip.LIB.fl_version().decode()}
    try:
        library["sha256_16"] = hashlib.sha256(lib_path.read_bytes()).hexdigest()[:16]
    except OSError:
        pass
    try:
        library["build"] = json.loads(lib_path.with_suffix(".build.json").read_text())
        library["build"].pop("flags", None)
    except (OSError, ValueError):
        library["build"] = None
    rec["library"] = library
    rec["gpu_driver"] = driver_record(torch.cuda.current_device())
    return rec


TRAFFIC_PROFILE = REPO / "profiles" / "prefill_pp_kernel_4x32x32x4096x128_bf16.md"


def profiled_traffic(path: Path = TRAFFIC_PROFILE) -> float | None:
    """HBM bytes per launch of the prefill kernel from its committed rocprofv3 summary (FETCH_SIZE
    and WRITE_SIZE runs scaled by a 1 GiB copy's readings); None if there is none. bench.py cannot
    collect counters itself, so the figure comes from the profile of the same command."""
    try:
        for line in path.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch:"):
                return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def sampled_rows(seqlen: int, count: int, seed: int = 0):
    import torch

    if seqlen <= count:
        return torch.arange(seqlen)
    gen = torch.Generator().manual_seed(seed)
    middle = torch.randperm(seqlen - 2, generator=gen)[: count - 2] + 1
    return torch.cat([torch.tensor([0, seqlen - 1]), middle]).sort().values


# ----------------------------------------------------------------------------------------------
# GPU legs


def prefill_inputs(cfg, seed=0):
    import torch

    gen = torch.Generator(device="cuda").manual_seed(seed)
    b, h, hkv, s, d = cfg["batch"], cfg["heads"], cfg["heads_kv"], cfg["seqlen"], cfg["head_dim"]
    q = torch.randn((b, s, h, d), generator=gen, device="cuda", dtype=torch.bfloat16)
    k = torch.randn((b, s, hkv, d), generator=gen, device="cuda", dtype=torch.bfloat16)
    v = torch.randn((b, s, hkv, d), generator=gen, device="cuda", dtype=torch.bfloat16)
    return q, k, v


CHECK_ROWS = 256  # query rows of every (batch, head) the prefill check covers (bench/run.py:36)
FLOOR_BF16 = 1e-3  # the reference's floor for bf16 (bench/run.py:35)


def check_prefill(out, qc, kc, vc, causal, rows) -> dict:
    """The reference's benchmark check (bench/run.py:102-109) on CPU copies of the inputs: error
    on the sampled rows of every (batch, head) against fp64, at most twice SDPA math's error at
    the input dtype plus 1e-3, and every output finite."""
    import torch
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel

    from oracle import c_oracle

    # The oracle's C loops (pinned to its torch attention_rows at 1e-12 in tests/test_oracle.py):
    # the same float64 rows in a fraction of the time.
    ref, _ = c_oracle.attention_rows(qc, kc, vc, rows, causal=causal)
    err = (out.cpu()[:, rows].double() - ref).abs().max().item()
    mask = None
    if causal:
        cols = torch.arange(kc.shape[1])[None, :]
        mask = cols <= rows[:, None] + (kc.shape[1] - qc.shape[1])
    group = qc.shape[2] // kc.shape[2]
    kr, vr = (x.repeat_interleave(group, dim=2) if group > 1 else x for x in (kc, vc))
    with sdpa_kernel(SDPBackend.MATH):
        base = F.scaled_dot_product_attention(
            qc[:, rows].transpose(1, 2).contiguous(),
            kr.transpose(1, 2).contiguous(),
            vr.transpose(1, 2).contiguous(),
            attn_mask=mask,
        ).transpose(1, 2)
    err_torch = (base.double() - ref).nan_to_num(0.0).abs().max().item()
    ok = bool(torch.isfinite(out).all()) and err <= 2 * err_torch + FLOOR_BF16
    return {"max_err_vs_fp64": err, "max_err_torch_vs_fp64": err_torch, "correct": ok,
            "checked": f"{len(rows)} of {qc.shape[1]} query rows of every (batch, head), all outputs finite"}


WARMUP_MIN_S = 0.1  # warm up for at least this long: the clock settles within tens of ms


# --trace: every timed step runs inside a roctx range "<workload>:step" that ends after a device
# synchronize (the reference's bench/decode_trace.py:1-8 with NVTX), so `rocprofv3 --marker-trace
# --kernel-trace` attributes each kernel to its step. The synchronize changes the timing, so a
# traced run is for attribution, not for the JSON figures.
TRACE = False


def time_op(run, steps: int, warmup: int, flush=None, label: str = "step") -> tuple[list[float], float]:
    """Per-step event times (ms) on the current stream, the stream the op launches its kernels
    on, and the wall time of the whole timed region (synchronized on both sides). Warmup is at
    least `warmup` steps and at least WARMUP_MIN_S of work, so the timed steps run at the clock the
    GPU settles at under this load rather than on its way there after an idle spell (the
    correctness check before each workload runs on the CPU)."""
    import torch

    t0 = time.perf_counter()
    done = 0
    while done < warmup or (time.perf_counter() - t0 < WARMUP_MIN_S and done < 1000):
        if flush is not None:
            flush.zero_()
        run()
        done += 1
        if done % 8 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        if flush is not None:
            flush.zero_()
        if TRACE:
            from flash_lab.observe import roctx_range

            with roctx_range(f"{label}:step"):
                starts[i].record()
                run()
                ends[i].record()
                torch.cuda.synchronize()
            continue
        starts[i].record()
        run()
        ends[i].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return [s.elapsed_time(e) for s, e in zip(starts, ends)], wall


CLOCK_WINDOW_S = 1.0  # the GPU clock and power are sampled over this much of the same work
PREROLL_S = 1.0  # after this much of it, unsampled


def gpu_window(run, step_ms: float, flush=None, seconds: float = CLOCK_WINDOW_S) -> dict:
    """Shader and memory clock, socket power and hotspot temperature of the GPU (amdsmi, through
    flash_lab.observe.ClockSampler) while it runs the workload's step again for `seconds` (the
    timed steps themselves are too short for the sampled metrics, which refresh every few
    milliseconds at best), in the reference's form (bench/clocks.py:18-71, the
    gpu_during_timing field of its result files): min / median / max per field. Launches go out
    in batches of about 25 ms of work with at most two batches queued, and one sample is taken
    after each batch, so every sample falls while the GPU is busy with this workload."""
    import torch

    from flash_lab.observe import ClockSampler

    per_batch = max(1, int(25.0 / max(step_ms, 1e-3)))
    queued = []

    def batch():
        for _ in range(per_batch):
            if flush is not None:
                flush.zero_()
            run()
        event = torch.cuda.Event()
        event.record()
        queued.append(event)
        if len(queued) > 2:
            queued.pop(0).synchronize()

    with ClockSampler(interval_ms=0) as sampler:
        if not sampler.available:
            return {"available": False, "reason": "amdsmi cannot read this GPU"}
        # The board's metrics lag the load (readings from an idle spell a fraction of a second
        # earlier, e.g. the host-side check before the timing), so the same work runs PREROLL_S
        # before the sampled window.
        start = time.time()
        while time.time() - start < PREROLL_S:
            batch()
        start = time.time()
        steps = 0
        while time.time() - start < seconds:
            batch()
            steps += per_batch
            sampler.sample()
        torch.cuda.synchronize()
        end = time.time()
        window = sampler.window(start, end)
    return {"available": window is not None, "window_s": end - start, "preroll_s": PREROLL_S,
            "steps": steps, **(window or {})}


# ----------------------------------------------------------------------------------------------
# The reference CPU path: the oracle (PyTorch fp64) on the host cores, timed with perf_counter.

CPU_LEG_BUDGET_S = 6.0  # timed work per CPU leg, beyond its warmup
CPU_MIN_REPS = 3
CPU_MAX_REPS = 10
CPU_DECODE_REPS = 10  # the decode legs always run this many (a median of at least 10 runs)


def time_cpu(fn, budget_s: float = CPU_LEG_BUDGET_S, warmed_up: bool = False,
             min_reps: int = CPU_MIN_REPS) -> dict:
    """perf_counter times (ms) of fn() on the host: 2 warmup runs (1 when a run takes over a
    second, none when the caller has just run the same computation), then runs until budget_s is
    spent, at least min_reps and at most max(min_reps, CPU_MAX_REPS); median, p10, p90 and the
    counts."""
    warmup = 0
    if not warmed_up:
        t0 = time.perf_counter()
        fn()
        warmup = 1
        if time.perf_counter() - t0 < 1.0:
            fn()
            warmup = 2
    times = []
    start = time.perf_counter()
    while len(times) < max(min_reps, CPU_MAX_REPS) and (
        len(times) < min_reps or time.perf_counter() - start < budget_s
    ):
        t0 = time.perf_counter()
        fn()
        times.append((time.perf_counter() - t0) * 1e3)
    return {"ms": summarize(times), "reps": len(times), "warmup": warmup}


def cpu_setup() -> dict:
    """Uses every host core this process may run on; returns the record of what was used."""
    import torch

    cores = cpu_cores()
    torch.set_num_threads(cores)
    return {"cores": cores, "threads": torch.get_num_threads(), "cpu_model": cpu_model(),
            "heading": f"reference CPU path ({cores} cores)"}


def cpu_c1_leg() -> dict:
    """C1: the CPU configuration of BASELINE.json (B=1, H=H_kv=4, S=256, D=64 fp32, iid N(0,1)
    from torch.manual_seed(0), non-causal, scale 1/8): the oracle at fp32 and at fp64, and the
    fp32 output against fp64 at 1e-5 relative (normwise: max |x - ref| / max |ref|)."""
    import torch

    from oracle import reference

    torch.manual_seed(0)
    q, k, v = (torch.randn(1, 256, 4, 64) for _ in range(3))
    out32 = reference.attention(q, k, v, dtype=torch.float32)
    out64 = reference.attention(q, k, v)
    rel = ((out32.double() - out64).abs().max() / out64.abs().max()).item()
    flops = attention_flops(1, 4, 256, 256, 64, causal=False)
    legs = {}
    for name, dtype in (("fp32", torch.float32), ("fp64", torch.float64)):
        t = time_cpu(lambda: reference.attention(q, k, v, dtype=dtype))
        legs[name] = {**t, "gflops": flops / (t["ms"]["median"] / 1e3) / 1e9}
    return {"workload": "C1: (B,H,H_kv,S,D)=(1,4,4,256,64) fp32 inputs, non-causal",
            "fp32": legs["fp32"], "fp64": legs["fp64"], "fp32_vs_fp64_normwise": rel,
            "correct": rel <= 1e-5}


def cpu_prefill_leg(qc, kc, vc, rows, causal) -> dict:
    """The 256-row fp64 check of the prefill workload (oracle attention_rows, as the reference's
    bench/run.py:75-109) timed on the host; TFLOP/s extrapolated as 4 B H rows S_k D / t (half
    of that for causal rows, like the GPU count)."""
    from oracle import reference

    t = time_cpu(lambda: reference.attention_rows(qc, kc, vc, rows, causal=causal), warmed_up=True)
    b, s_k, h = qc.shape[0], kc.shape[1], qc.shape[2]
    flops = attention_flops(b, h, len(rows), s_k, qc.shape[3], causal)
    return {**t, "tflops": flops / (t["ms"]["median"] / 1e3) / 1e12,
            "sample": f"oracle fp64 attention_rows, {len(rows)} of {qc.shape[1]} query rows x all "
                      f"{b * h} (batch, head), {'causal' if causal else 'non-causal'}"}


CPU_DECODE_SEQUENCES = 2  # sequences of a decode batch the CPU leg times (a bounded sample)


def cpu_decode_leg(qc, kc, vc, lens) -> dict:
    """The fp64 decode of the oracle (every key of each sampled sequence) timed on the host, at
    least CPU_DECODE_REPS times, in GB/s of the bf16 K+V bytes of the sequences it covers. Batches
    of more than CPU_DECODE_SEQUENCES sequences are sampled (their first ones): the full B=8
    decode takes about a second per run on the host, and the sample keeps the leg to seconds while
    giving every figure ten or more runs."""
    from oracle import reference

    n = min(CPU_DECODE_SEQUENCES, qc.shape[0])
    qs, ks, vs, ls = qc[:n], kc[:n], vc[:n], lens[:n]
    t = time_cpu(lambda: reference.decode(qs, ks, vs, ls), min_reps=CPU_DECODE_REPS)
    kv_bytes = 2.0 * int(ls.sum()) * kc.shape[2] * kc.shape[3] * kc.element_size()
    return {**t, "gbps": kv_bytes / (t["ms"]["median"] / 1e3) / 1e9,
            "sample": f"oracle fp64 decode of {n} of {qc.shape[0]} sequences x {kc.shape[1]} keys "
                      f"x {qc.shape[2]} heads ({kv_bytes:.4g} B of bf16 K+V)"}


# ----------------------------------------------------------------------------------------------
# GPU legs


def bench_prefill(steps: int, warmup: int, causal: bool, cpu: bool, cfg: dict = PREFILL,
                  label: str | None = None, clocks: bool = True) -> dict:
    import torch

    import flash_lab

    label = label or ("prefill_causal" if causal else "prefill")
    q, k, v = prefill_inputs(cfg)
    qc, kc, vc = q.cpu(), k.cpu(), v.cpu()
    rows = sampled_rows(cfg["seqlen"], CHECK_ROWS)
    check = check_prefill(flash_lab.attention(q, k, v, causal=causal), qc, kc, vc, causal, rows)
    if not check["correct"]:
        return {"status": "incorrect", **check}
    run = lambda: flash_lab.attention(q, k, v, causal=causal)  # noqa: E731
    times, wall = time_op(run, steps, warmup, label=label)
    flops = attention_flops(cfg["batch"], cfg["heads"], cfg["seqlen"], cfg["seqlen"],
                            cfg["head_dim"], causal)
    mean_ms = sum(times) / len(times)
    stats = summarize(times)
    gpu = gpu_window(run, stats["median"]) if clocks else None
    del q, k, v
    torch.cuda.empty_cache()
    result = {
        "status": "ok",
        "config": {**cfg, "causal": causal},
        "causal": causal,
        "flops": flops,
        "ms": stats,
        "mean_ms": mean_ms,
        "wall_ms_per_step": 1e3 * wall / steps,
        "tflops": flops / (stats["median"] / 1e3) / 1e12,
        "tflops_mean": flops / (mean_ms / 1e3) / 1e12,
        "frac_of_peak": flops / (mean_ms / 1e3) / 1e12 / PEAK_BF16_TFLOPS,
        **check,
    }
    if gpu is not None:
        result["gpu_clocks"] = gpu
    if cpu:
        result["reference_cpu_path"] = cpu_prefill_leg(qc, kc, vc, rows, causal)
    return result


def bench_decode(name: str, steps: int, warmup: int, flush, cpu: bool) -> dict:
    import torch

    import flash_lab
    from flash_lab import _hip
    from oracle import reference

    cfg = DECODE[name]
    b, h, hkv, ctx, d = cfg["batch"], cfg["heads"], cfg["heads_kv"], cfg["context"], cfg["head_dim"]
    gen = torch.Generator(device="cuda").manual_seed(0)
    q = torch.randn(b, 1, h, d, generator=gen, device="cuda", dtype=torch.bfloat16)
    k_cache = torch.randn((b, ctx, hkv, d), generator=gen, device="cuda", dtype=torch.bfloat16)
    v_cache = torch.randn((b, ctx, hkv, d), generator=gen, device="cuda", dtype=torch.bfloat16)
    seq_lens = torch.full((b,), ctx, dtype=torch.int32, device="cuda")
    tables = None
    page_size = cfg.get("page_size")
    if page_size:
        # Scatter the cache into shuffled blocks of a pool; the check below reads the contiguous
        # copy, which holds the same rows.
        per_seq = ctx // page_size
        order = torch.randperm(b * per_seq, generator=gen, device="cuda")
        tables = order.view(b, per_seq).to(torch.int32)
        pools = []
        for cache in (k_cache, v_cache):
            pool = torch.empty((b * per_seq, page_size, hkv, d), device="cuda", dtype=torch.bfloat16)
            pool[order] = cache.reshape(b * per_seq, page_size, hkv, d)
            pools.append(pool)
        k_used, v_used = pools
    else:
        k_used, v_used = k_cache, v_cache
    out = flash_lab.decode(q, k_used, v_used, seq_lens, block_tables=tables)
    # The reference's check (bench/run.py:112-119): every sequence in full against fp64, at most
    # twice the error of the same op sequence at bf16 plus 1e-3.
    qc, kc, vc, lc = q.cpu(), k_cache.cpu(), v_cache.cpu(), seq_lens.cpu()
    del k_cache, v_cache
    ref = reference.decode(qc, kc, vc, lc)
    plain = reference.decode(qc, kc, vc, lc, dtype=torch.bfloat16)
    err = (out.cpu().double() - ref).abs().max().item()
    err_torch = (plain.double() - ref).abs().max().item()
    ok = bool(torch.isfinite(out).all()) and err <= 2 * err_torch + FLOOR_BF16
    check = {"max_err_vs_fp64": err, "max_err_torch_vs_fp64": err_torch,
             "checked": f"all {b} sequences x {ctx} keys x {h} heads, all outputs finite"}
    if not ok:
        return {"status": "incorrect", **check}
    run = lambda: flash_lab.decode(q, k_used, v_used, seq_lens, block_tables=tables)  # noqa: E731
    times, _ = time_op(run, steps, warmup, flush, label=name)
    stats = summarize(times)
    mean_ms = sum(times) / len(times)
    # Sampled without the flush between steps (its memset would dominate the window); every
    # benchmark cache here is larger than the 256 MB Infinity Cache, so the steps still stream
    # from HBM.
    gpu = gpu_window(run, stats["median"])
    kv = decode_kv_bytes(b, hkv, ctx, d, 2)
    splits, _ = _hip.decode_plan(b, h, hkv, d, ctx, torch.bfloat16,
                                 cu_count_=_hip.cu_count(torch.cuda.current_device()))
    del q, k_used, v_used, tables
    torch.cuda.empty_cache()
    result = {
        "status": "ok",
        "page_size": page_size,
        "kv_bytes": kv,
        "bytes_with_q_o": decode_bytes_with_qo(b, h, hkv, ctx, d, 2),
        "num_splits": splits,
        "ms": stats,
        "mean_ms": mean_ms,
        "gbps": kv / (stats["median"] / 1e3) / 1e9,
        "gbps_mean": kv / (mean_ms / 1e3) / 1e9,
        "frac_of_peak": kv / (mean_ms / 1e3) / 1e9 / PEAK_HBM_GBPS,
        "gpu_clocks": gpu,
        "roofline": {"bound": "hbm", "achieved": kv / (mean_ms / 1e3) / 1e9, "peak": PEAK_HBM_GBPS,
                     "unit": "GB/s", "frac": kv / (mean_ms / 1e3) / 1e9 / PEAK_HBM_GBPS,
                     "per_launch": f"{kv:.4g} B of K+V (every cached row once), mean {mean_ms:.4f} ms "
                                   "for the split and merge kernels"},
        **check,
    }
    # The reference CPU path for the three decode configurations BASELINE.json names (the paged
    # and 8-head variants are this repo's additions and have the same oracle work as B8-GQA).
    if cpu and name in ("B1-MHA", "B8-MHA", "B8-GQA"):
        result["reference_cpu_path"] = cpu_decode_leg(qc, kc, vc, lc)
    return result


# ----------------------------------------------------------------------------------------------
# --only sweep: the reference's other benchmark suites (bench/suites.py:63-125), each shape checked
# and timed like the headline legs, beside the reference's H100 figure for the kernel this build
# replaces (mma_pipelined for prefill, splitkv for decode). Sources, under the reference's
# bench/results/h100-80gb-hbm3/: summary-cc64b18.md (medians of three runs) where the summary has
# the suite, else the single run file named. The reference's decode GB/s count the q and o bytes
# too (bench/flops.py:51-57); here they are compared against "gbps_with_q_o".
SUMMARY = "summary-cc64b18.md"
SWEEP_PREFILL = [
    # (B, H, H_kv, S, D): (non-causal, causal) H100 TFLOP/s, source
    ((4, 32, 32, 1024, 128), (219.3, 177.4), f"{SUMMARY}:140,147"),
    ((4, 32, 32, 4096, 128), (229.2, 216.7), f"{SUMMARY}:154,161"),
    ((2, 32, 32, 8192, 128), (230.8, 224.2), f"{SUMMARY}:168,175"),
    ((1, 32, 32, 16384, 128), (228.1, 231.6), f"{SUMMARY}:182,189"),
    ((8, 16, 16, 2048, 64), (200.2, 177.2), f"{SUMMARY}:196,203"),
    ((4, 32, 8, 4096, 128), (227.4, 212.5), f"{SUMMARY}:210,217"),
    ((32, 32, 32, 512, 128), (214.6, 170.3), "20261003-074548-ef88a7a-prefill_seqlen.json"),
    ((16, 32, 32, 1024, 128), (207.6, 199.6), "20261003-074548-ef88a7a-prefill_seqlen.json"),
    ((8, 32, 32, 2048, 128), (223.2, 211.5), "20261003-074548-ef88a7a-prefill_seqlen.json"),
]
_DECODE_CTX = {(1, 32, 512): (174.4, 40), (1, 32, 2048): (597.1, 46), (1, 32, 8192): (1679.9, 52),
               (1, 32, 32768): (2171.0, 58), (1, 8, 512): (43.0, 64), (1, 8, 2048): (161.1, 70),
               (1, 8, 8192): (521.9, 76), (1, 8, 32768): (674.2, 82), (8, 32, 512): (1102.4, 88),
               (8, 32, 2048): (2100.0, 94), (8, 32, 8192): (2483.4, 100),
               (8, 32, 32768): (2691.7, 106), (8, 8, 512): (322.2, 112), (8, 8, 2048): (652.5, 118),
               (8, 8, 8192): (948.8, 124), (8, 8, 32768): (1135.0, 130)}
SWEEP_DECODE = [
    # (B, H, H_kv, context, D): H100 GB/s (K+V+q+o), source
    *[((b, 32, hkv, ctx, 128), gbps, f"{SUMMARY}:{line}")
      for (b, hkv, ctx), (gbps, line) in _DECODE_CTX.items()],
    *[((b, 32, 8, 2048, 128), gbps, f"{SUMMARY}:{line}")
      for b, gbps, line in ((4, 566.2, 17), (16, 904.5, 23), (64, 1096.4, 29))],
    *[((b, 32, 8, ctx, 64), gbps, "20261003-074603-ef88a7a-decode_d64.json")
      for (b, ctx), gbps in {(1, 2048): 84.9, (1, 8192): 292.2, (1, 32768): 603.3,
                             (8, 2048): 581.3, (8, 8192): 884.2, (8, 32768): 1048.6}.items()],
    *[((1, 32, hkv, ctx, 128), gbps, "20261003-074642-ef88a7a-decode_long.json")
      for (hkv, ctx), gbps in {(32, 65536): 2421.7, (32, 131072): 2594.3, (8, 65536): 742.2,
                               (8, 131072): 800.1}.items()],
]


def bench_sweep(steps: int, decode_steps: int) -> dict:
    """Every SWEEP_PREFILL shape (non-causal and causal) and SWEEP_DECODE shape: checked against
    fp64 first (prefill: 256 sampled rows of every (batch, head); decode: every sequence in full),
    then timed (median of the event-timed steps; decode after a 1 GiB flush per step), with the
    roofline fraction and the reference's H100 figure beside each."""
    import torch

    import flash_lab
    from oracle import c_oracle, reference

    prefill = []
    for (b, h, hkv, sq, d), ref_tflops, source in SWEEP_PREFILL:
        cfg = dict(batch=b, heads=h, heads_kv=hkv, seqlen=sq, head_dim=d)
        for causal, ref in zip((False, True), ref_tflops):
            print(f"# sweep prefill {cfg} causal={causal}", file=sys.stderr, flush=True)
            r = bench_prefill(steps, 3, causal, False, cfg, label="sweep_prefill", clocks=False)
            row = {"config": {**cfg, "causal": causal}, "status": r["status"],
                   "reference_h100": {"tflops": ref, "source": source}}
            if r["status"] == "ok":
                row.update(tflops=r["tflops"], frac_of_peak=r["frac_of_peak"], ms=r["ms"]["median"],
                           vs_reference=r["tflops"] / ref, max_err_vs_fp64=r["max_err_vs_fp64"],
                           max_err_torch_vs_fp64=r["max_err_torch_vs_fp64"])
            prefill.append(row)
    decode = []
    flush = torch.empty(FLUSH_BYTES // 4, dtype=torch.int32, device="cuda")
    for (b, h, hkv, ctx, d), ref_gbps, source in SWEEP_DECODE:
        print(f"# sweep decode B={b} H={h} H_kv={hkv} ctx={ctx} D={d}", file=sys.stderr, flush=True)
        gen = torch.Generator(device="cuda").manual_seed(0)
        q = torch.randn(b, 1, h, d, generator=gen, device="cuda", dtype=torch.bfloat16)
        k_cache = torch.randn((b, ctx, hkv, d), generator=gen, device="cuda", dtype=torch.bfloat16)
        v_cache = torch.randn((b, ctx, hkv, d), generator=gen, device="cuda", dtype=torch.bfloat16)
        lens = torch.full((b,), ctx, dtype=torch.int32, device="cuda")
        out = flash_lab.decode(q, k_cache, v_cache, lens)
        qc, kc, vc, lc = q.cpu(), k_cache.cpu(), v_cache.cpu(), lens.cpu()
        ref, _ = c_oracle.decode(qc, kc, vc, lc)
        plain = reference.decode(qc, kc, vc, lc, dtype=torch.bfloat16)
        err = (out.cpu().double() - ref).abs().max().item()
        err_torch = (plain.double() - ref).abs().max().item()
        row = {"config": dict(batch=b, heads=h, heads_kv=hkv, context=ctx, head_dim=d),
               "reference_h100": {"gbps_with_q_o": ref_gbps, "source": source},
               "max_err_vs_fp64": err, "max_err_torch_vs_fp64": err_torch}
        if not (bool(torch.isfinite(out).all()) and err <= 2 * err_torch + FLOOR_BF16):
            decode.append({**row, "status": "incorrect"})
            continue
        times, _ = time_op(lambda: flash_lab.decode(q, k_cache, v_cache, lens), decode_steps, 10,
                           flush, label="sweep_decode")
        ms = summarize(times)["median"]
        kv = decode_kv_bytes(b, hkv, ctx, d, 2)
        with_qo = decode_bytes_with_qo(b, h, hkv, ctx, d, 2)
        row.update(status="ok", ms=ms, gbps=kv / ms / 1e6, gbps_with_q_o=with_qo / ms / 1e6,
                   frac_of_peak=kv / ms / 1e6 / PEAK_HBM_GBPS,
                   vs_reference=with_qo / ms / 1e6 / ref_gbps)
        decode.append(row)
        del q, k_cache, v_cache, out
        torch.cuda.empty_cache()
    del flush
    torch.cuda.empty_cache()
    bad = [r for r in prefill + decode if r["status"] != "ok"]
    return {"status": "incorrect" if bad else "ok", "prefill": prefill, "decode": decode}


# Config L, the reference's end-to-end figures (bench/results/h100-80gb-hbm3/summary-cc64b18.md:
# 270-271): Llama-3.1-8B with real weights on one H100, B=1, 8,192-token prompt, 256 new tokens.
E2E_REFERENCE = {"ttft_ms_triton_prefill": 274.8, "ttft_ms_mma_pipelined": 311.7,
                 "decode_step_ms": 9.58, "hardware": "H100 SXM5, real Llama-3.1-8B weights"}
E2E_PROMPT = 8192
E2E_NEW_TOKENS = 256


def tokens_follow_sdpa(tokens, ref_tokens, ref_logits) -> dict:
    """The reference's rule for greedy tokens (tests/test_e2e_llama.py:94-106): equal to SDPA's
    up to the first step where they differ, which must be a near-tie of SDPA's top two logits
    (within two bf16 steps of the larger); nothing after that step is compared."""
    import torch

    n = min(len(tokens), len(ref_tokens))
    differ = (tokens[:n].cpu() != ref_tokens[:n].cpu()).nonzero()
    out = {"tokens_checked": n, "first_difference": None, "tokens_follow_sdpa": True}
    if len(differ):
        step = int(differ[0])
        first, second = ref_logits[step].float().topk(2).values.tolist()
        tie = 2 * torch.finfo(torch.bfloat16).eps * 2 ** math.floor(math.log2(abs(first)))
        out.update(first_difference=step, margin=first - second, near_tie=tie,
                   tokens_follow_sdpa=first - second <= tie)
    return out


def bench_e2e_l(budget_s: float) -> dict:
    """Config L through flash_lab.hf: a Llama-3.1-8B-shaped model (32 layers, random bf16 weights
    seeded on the GPU), B=1, an 8,192-token random prompt, 256 greedy tokens with a static cache
    and the compiled decode step, as the reference's bench/e2e.py:42-177 times it. The logits at
    the last prompt position are checked first against an fp32 copy of the weights (at most twice
    SDPA's bf16 error plus 1e-3). One untimed warmup generation pays for the compilation; the
    median of the timed runs is reported. Runs stop early (status "budget") if `budget_s` of wall
    time is spent before the timed runs start."""
    import torch

    try:
        import transformers  # noqa: F401
    except ImportError as exc:
        return {"status": "skipped", "reason": f"transformers not importable: {exc}"}
    import e2e
    import flash_lab.hf

    t_start = time.perf_counter()
    config = {"model": "Llama-3.1-8B-shaped, 32 layers, random bf16 weights (seed 0)",
              "batch": 1, "prompt_len": E2E_PROMPT, "new_tokens": E2E_NEW_TOKENS,
              "cache": "static", "decode": "generate() compiled step (fullgraph, HIP graphs)"}
    name = flash_lab.hf.register()
    model = e2e.build_model(32, seed=0)
    gen = torch.Generator().manual_seed(0)
    ids = torch.randint(0, 128000, (1, E2E_PROMPT), generator=gen).cuda()
    eos = model.config.eos_token_id
    want = e2e.reference_logits(model, {E2E_PROMPT: ids}, E2E_PROMPT)[E2E_PROMPT]
    model.set_attn_implementation("sdpa")
    err_torch = (e2e.last_logits(model, ids) - want).abs().max().item()
    model.set_attn_implementation(name)
    err = (e2e.last_logits(model, ids, E2E_PROMPT + E2E_NEW_TOKENS) - want).abs().max().item()
    check = {"max_logit_err_vs_fp32": err, "max_logit_err_sdpa_vs_fp32": err_torch}
    if not err <= 2 * err_torch + FLOOR_BF16:
        return {"status": "incorrect", "config": config, **check}
    # The reference's token rule (tests/test_e2e_llama.py:94-135): the 256 greedy tokens of the
    # compiled static-cache run follow SDPA's, up to a step where SDPA's own top two logits are
    # within two bf16 steps of each other.
    print("# e2e_L: sdpa greedy tokens", file=sys.stderr, flush=True)
    model.set_attn_implementation("sdpa")
    with torch.no_grad():
        sdpa_out = model.generate(
            ids, attention_mask=torch.ones_like(ids), max_new_tokens=E2E_NEW_TOKENS,
            min_new_tokens=E2E_NEW_TOKENS, do_sample=False, temperature=None, top_p=None,
            pad_token_id=eos, return_dict_in_generate=True, output_logits=True,
        )
    sdpa_tokens = sdpa_out.sequences[0, ids.shape[1]:]
    sdpa_logits = torch.stack(sdpa_out.logits)[:, 0]
    del sdpa_out
    model.set_attn_implementation(name)
    torch._dynamo.reset()
    print("# e2e_L: warmup generation (compiles the decode step)", file=sys.stderr, flush=True)
    tokens, _ = e2e.generate(model, ids, E2E_NEW_TOKENS, eos, progress_every=64)
    check.update(tokens_follow_sdpa(tokens[0], sdpa_tokens, sdpa_logits))
    del sdpa_logits
    if not check["tokens_follow_sdpa"]:
        return {"status": "incorrect", "config": config, **check}
    warm_s = time.perf_counter() - t_start
    runs = []
    for i in range(2):
        if time.perf_counter() - t_start > budget_s:
            break
        print(f"# e2e_L: timed run {i + 1}", file=sys.stderr, flush=True)
        runs.append(e2e.generate(model, ids, E2E_NEW_TOKENS, eos))
    del model
    torch.cuda.empty_cache()
    if not runs:
        return {"status": "budget", "config": config, "setup_s": warm_s, **check}
    ttft = [gaps[0] for _, gaps in runs]
    steps = [g for _, gaps in runs for g in gaps[1:]]
    step_ms = summarize(steps)
    return {
        "status": "ok",
        "config": config,
        "runs": len(runs),
        "ttft_ms": statistics.median(ttft),
        "ttft_ms_runs": ttft,
        "decode_step_ms": step_ms,
        "decode_tokens_per_s": 1e3 / step_ms["median"],
        "reference_h100": E2E_REFERENCE,
        "setup_s": warm_s,
        "wall_s": time.perf_counter() - t_start,
        **check,
    }


# ----------------------------------------------------------------------------------------------


def parse_args(argv=None):
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument("--decode-steps", type=int, default=100)
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--no-e2e", action="store_true", help="leave out the config L leg")
    parser.add_argument("--e2e-budget-s", type=float, default=300.0,
                        help="wall-time bound of the config L leg before its timed runs")
    parser.add_argument("--trace", action="store_true",
                        help="roctx range per timed step, for rocprofv3 --marker-trace (timings "
                             "then include a synchronize per step)")
    parser.add_argument(
        "--only",
        help="comma list of workloads to run: prefill, prefill_causal, prefill_d64, "
        f"prefill_d64_causal, decode (all of them), {', '.join(DECODE)}, e2e_L, sweep (the "
        "reference's other benchmark shapes, prefill and decode, beside its H100 figures), copy (a "
        "1 GiB device copy, the calibration of the traffic counters), gemm (a dense bf16 hipBLASLt "
        "GEMM), mfma (register-only MFMA chains: the matrix pipes' rate under the power limit); "
        "default: all but sweep, copy, gemm and mfma",
    )
    return parser.parse_args(argv)


def selected_workloads(only: str | None, e2e: bool = True) -> list[str]:
    everything = (["prefill", "prefill_causal", "prefill_d64", "prefill_d64_causal", *DECODE]
                  + (["e2e_L"] if e2e else []))
    if not only:
        return everything
    names = []
    for item in only.split(","):
        item = item.strip()
        if item == "decode":
            names += list(DECODE)
        elif item in everything or item in ("copy", "gemm", "mfma", "e2e_L", "sweep"):
            names.append(item)
        else:
            raise SystemExit(f"unknown workload {item!r}")
    return names


def bench_copy(steps: int) -> dict:
    """A plain 1 GiB device-to-device copy: its FETCH_SIZE / WRITE_SIZE readings per dispatch
    calibrate the traffic counters against a known byte count."""
    import torch

    src = torch.empty(FLUSH_BYTES // 4, dtype=torch.int32, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    times, _ = time_op(lambda: dst.copy_(src), steps, 2)
    mean_ms = sum(times) / len(times)
    return {"status": "ok", "bytes_read": FLUSH_BYTES, "bytes_written": FLUSH_BYTES,
            "mean_ms": mean_ms, "gbps_read_plus_write": 2 * FLUSH_BYTES / (mean_ms / 1e3) / 1e9}


def bench_gemm(steps: int) -> dict:
    """A dense bf16 GEMM through torch.matmul (hipBLASLt), 8192^3 = 2^40 FLOP like the prefill
    launch, on iid N(0,1) operands and again on zeros: the MFMA rate the chip sustains under its
    power limit with a vendor kernel, the context of the prefill kernel's fraction of peak (MFMA
    power depends on the operands' bits, so the two rates differ)."""
    import torch

    n = 8192
    gen = torch.Generator(device="cuda").manual_seed(0)
    a = torch.randn(n, n, device="cuda", dtype=torch.bfloat16, generator=gen)
    b = torch.randn(n, n, device="cuda", dtype=torch.bfloat16, generator=gen)
    c = torch.empty(n, n, device="cuda", dtype=torch.bfloat16)
    flops = 2.0 * n ** 3
    out = {"status": "ok", "shape": [n, n, n], "flops": flops, "via": "torch.matmul (hipBLASLt)"}
    for label in ("randn", "zeros"):
        if label == "zeros":
            a.zero_()
            b.zero_()
        times, _ = time_op(lambda: torch.matmul(a, b, out=c), steps, 5, label=f"gemm_{label}")
        ms = summarize(times)
        out[label] = {"ms": ms, "tflops": flops / ms["median"] / 1e9,
                      "frac_of_peak": flops / ms["median"] / 1e9 / PEAK_BF16_TFLOPS}
    return out


def bench_mfma_rate(steps: int) -> dict:
    """The matrix-pipe rate probe (flc_mfma_rate_probe of the calibration library calib/, built
    here if it is missing; not part of the product library): one workgroup of 8 waves per CU
    running v_mfma_f32_32x32x16_bf16 chains with nothing else beside them, on pseudo-random
    operands shaped like N(0,1) draws, on zeros, and on random operands whose A side is read from
    LDS for every MFMA (the prefill kernel's fragment traffic, 1 KiB per wave per MFMA). The MFMA
    rate the board's power limit leaves on random data, before and with the LDS traffic: the
    ceiling the prefill kernel is held under."""
    import torch

    import calib

    lib = calib.load()
    workgroups, iters = 256, 6000
    out = torch.empty(workgroups * 512, device="cuda")
    flops = float(workgroups) * 8 * iters * 16 * 32768

    def run(flags):
        stream = torch.cuda.current_stream().cuda_stream
        if lib.flc_mfma_rate_probe(out.data_ptr(), workgroups, iters, flags, stream) != 0:
            raise RuntimeError(lib.flc_last_error().decode())

    result = {"status": "ok", "workgroups": workgroups, "waves_per_workgroup": 8, "iters": iters,
              "flops": flops, "instruction": "v_mfma_f32_32x32x16_bf16",
              "library": str(calib.OUTPUT.relative_to(REPO))}
    for label, flags in (("random", 0), ("zeros", calib.PROBE_ZERO_OPERANDS),
                         ("random_lds_a", calib.PROBE_LDS_A)):
        times, _ = time_op(lambda: run(flags), steps, 5, label=f"mfma_{label}")
        ms = summarize(times)
        result[label] = {"ms": ms, "tflops": flops / ms["median"] / 1e9,
                         "frac_of_peak": flops / ms["median"] / 1e9 / PEAK_BF16_TFLOPS,
                         "gpu_clocks": gpu_window(lambda: run(flags), ms["median"])}
    return result


def overall_status(headline: dict | None, secondary: dict) -> int:
    """0 when every workload that ran is ok (a leg skipped for a missing optional dependency or
    its wall-time bound is not a failure), else 1."""
    bad = {"incorrect", "error"}
    if headline is not None and headline.get("status") != "ok":
        return 1
    return 1 if any(r.get("status") in bad for r in secondary.values()) else 0


def main(argv=None) -> int:
    args = parse_args(argv)
    if args.gpus != 1:
        print(
            "bench.py measures one GPU: this build runs on a single MI355X and has no multi-GPU "
            f"path (asked for --gpus {args.gpus}).",
            file=sys.stderr,
        )
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    from flash_lab import ops

    if not ops.HAS_EXTENSION:
        print(f"the HIP library did not load: {ops.EXTENSION_ERROR}", file=sys.stderr)
        return 2

    global TRACE
    TRACE = args.trace
    cpu = not args.no_cpu_baseline
    cpu_record = cpu_setup() if cpu else None
    props = torch.cuda.get_device_properties(0)
    workloads = selected_workloads(args.only, e2e=not args.no_e2e)
    secondary = {}
    headline = None

    def guarded(label, fn):
        try:
            return fn()
        except Exception as exc:  # recorded and reported, never silently dropped
            print(f"# {label} failed: {exc!r}", file=sys.stderr, flush=True)
            return {"status": "error", "error": repr(exc)}

    env = guarded("env", env_record)

    if "prefill" in workloads:
        headline = guarded("prefill", lambda: bench_prefill(args.steps, args.warmup, False, cpu))
        print(f"# prefill non-causal: {json.dumps(headline)}", file=sys.stderr, flush=True)
    if "prefill_causal" in workloads:
        secondary["prefill_causal"] = guarded(
            "prefill_causal", lambda: bench_prefill(args.steps, args.warmup, True, cpu))
        print(f"# prefill causal: {json.dumps(secondary['prefill_causal'])}", file=sys.stderr,
              flush=True)
    for name, causal in (("prefill_d64", False), ("prefill_d64_causal", True)):
        if name in workloads:
            secondary[name] = guarded(name, lambda: bench_prefill(
                args.steps, args.warmup, causal, False, PREFILL_D64, label=name))
            print(f"# {name}: {json.dumps(secondary[name])}", file=sys.stderr, flush=True)
    decodes = [name for name in DECODE if name in workloads]
    if decodes:
        flush = torch.empty(FLUSH_BYTES // 4, dtype=torch.int32, device="cuda")
        for name in decodes:
            secondary[f"decode_{name}"] = guarded(
                name, lambda: bench_decode(name, args.decode_steps, 10, flush, cpu))
            print(f"# decode {name}: {json.dumps(secondary[f'decode_{name}'])}", file=sys.stderr,
                  flush=True)
        del flush
        torch.cuda.empty_cache()
    if "sweep" in workloads:
        secondary["sweep"] = guarded("sweep", lambda: bench_sweep(10, 50))
        print(f"# sweep: {json.dumps(secondary['sweep'])}", file=sys.stderr, flush=True)
    if "copy" in workloads:
        secondary["copy"] = bench_copy(args.steps)
        print(f"# copy: {json.dumps(secondary['copy'])}", file=sys.stderr, flush=True)
    if "mfma" in workloads:
        secondary["mfma"] = guarded("mfma", lambda: bench_mfma_rate(args.steps))
        print(f"# mfma: {json.dumps(secondary['mfma'])}", file=sys.stderr, flush=True)
    if "gemm" in workloads:
        secondary["gemm"] = guarded("gemm", lambda: bench_gemm(args.steps))
        print(f"# gemm: {json.dumps(secondary['gemm'])}", file=sys.stderr, flush=True)
    if "e2e_L" in workloads:
        secondary["e2e_L"] = guarded("e2e_L", lambda: bench_e2e_l(args.e2e_budget_s))
        print(f"# e2e_L: {json.dumps(secondary['e2e_L'])}", file=sys.stderr, flush=True)

    if headline is not None and headline["status"] == "ok":
        value = headline["tflops"]
        ms = headline["ms"]["median"]
        roofline = {
            "bound": "mfma",
            "achieved": headline["tflops_mean"],
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": headline["tflops_mean"] / PEAK_BF16_TFLOPS,
            "traffic": profiled_traffic(),
            "traffic_source": str(TRAFFIC_PROFILE.relative_to(REPO)),
            "kernel": "prefill_pp_kernel<bf16_tag, 128>",
            "gfx_mhz_median": (headline.get("gpu_clocks") or {}).get("gfx_mhz", {}).get("median"),
            "per_launch": f"{headline['flops']:.4g} FLOP (4 B H S^2 D), mean {headline['mean_ms']:.4f} ms",
        }
    else:
        value, ms, roofline = 0.0, None, None

    cpu_baseline = None
    if cpu:
        legs = {"C1": guarded("cpu C1", cpu_c1_leg)}
        if headline is not None and "reference_cpu_path" in headline:
            legs["P_noncausal"] = headline["reference_cpu_path"]
        for key, label in (("prefill_causal", "P_causal"), ("decode_B1-MHA", "D1"),
                           ("decode_B8-MHA", "D8"), ("decode_B8-GQA", "G8")):
            if key in secondary and "reference_cpu_path" in secondary[key]:
                legs[label] = secondary[key]["reference_cpu_path"]
        p = legs.get("P_noncausal")
        cpu_baseline = {
            "value": p["tflops"] if p else None,
            "unit": "TFLOP/s",
            "cores": cpu_record["cores"],
            "kind": "port",
            "sample": (
                f"oracle fp64 attention_rows (restatement of flash_lab.reference), {CHECK_ROWS} of "
                f"4096 query rows x all 128 (batch, head) of (4,32,32,4096,128), non-causal, "
                f"median of {p['reps']} runs ({p['ms']['median']:.0f} ms; p10 {p['ms']['p10']:.0f}, "
                f"p90 {p['ms']['p90']:.0f})" if p else "prefill leg not run"
            ),
            **cpu_record,
            "legs": legs,
        }

    result = {
        "metric": "prefill TFLOP/s @(4,32,32,4096,128) bf16; split-KV decode GB/s @32K KV",
        "value": value,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": value / BASELINE_TFLOPS if value else None,
        "baseline": {"value": BASELINE_TFLOPS, "unit": "TFLOP/s",
                     "what": "reference mma_pipelined, non-causal, H100 SXM5 (reference bench/results/h100-80gb-hbm3/summary-cc64b18.md:154)"},
        "dtype": "bf16",
        "data": "synthetic iid N(0,1), torch.Generator seed 0",
        "config": {
            "workload": "prefill forward (B,H,H_kv,S,D)=(4,32,32,4096,128) bf16 [B,S,H,D], non-causal",
            **PREFILL,
            "causal": False,
            "softmax_scale": 1 / math.sqrt(PREFILL["head_dim"]),
        },
        "roofline": roofline,
        "cpu_baseline": cpu_baseline,
        # The headline leg's own record: its check, step-time distribution and the GPU clock and
        # power sampled over a second of the same work.
        "headline": headline,
        "secondary": secondary,
        "device": {"name": props.name, "cus": props.multi_processor_count,
                   "arch": getattr(props, "gcnArchName", "")},
        "env": env,
    }
    print(json.dumps(result), flush=True)
    return overall_status(headline, secondary)


if __name__ == "__main__":
    raise SystemExit(main())
