"""Benchmark of the two hot paths on one MI355X; prints ONE JSON line.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--only prefill|decode]

Metric: prefill TFLOP/s at (B, H, H_kv, S, D) = (4, 32, 32, 4096, 128) bf16 and
split-KV decode GB/s at 32K keys. A step is one prefill forward over that batch (non-causal), the
configuration the metric is quoted on; `value` is its throughput. The causal prefill and the three
decode configurations (B=1 MHA, B=8 MHA, B=8 GQA, 32K keys; B=8 GQA also as a paged cache of
16-row blocks) are reported under "secondary".

Inputs are synthetic iid N(0, 1) bf16 from torch.Generator(device="cuda").manual_seed(0), drawn in
the reference's order (q, k, v; decode q, k_cache, v_cache: reference bench/run.py:122-141), and
are resident in HBM before timing. Every configuration is checked against the fp64 oracle before
it is timed (prefill on sampled rows, decode on its first sequence). Prefill FLOPs are
4 B H S_q S_k D, halved for causal; decode bytes are the K and V bytes read (reference
bench/flops.py:31-57; the reference's variant adding q and o is reported beside them). Decode
timings zero a 1 GiB buffer before each call so the 256 MB Infinity Cache holds no K/V.

roofline: the dominant kernel's algorithmic FLOPs (or bytes) per launch over its mean duration
from HIP events recorded on the stream it is launched on, against MI355X peaks (dense bf16 MFMA
2.5 PFLOP/s, HBM 8 TB/s). cpu_baseline: the oracle (PyTorch fp64 on the host cores) on a bounded
sample of the prefill workload: 256 query rows of every (batch, head), extrapolated.
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
BASELINE_TFLOPS = 229.2  # reference mma_pipelined, non-causal, H100

PREFILL = dict(batch=4, heads=32, heads_kv=32, seqlen=4096, head_dim=128)
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


def check_prefill(out, q, k, v, causal, rows) -> dict:
    """The reference's benchmark check (bench/run.py:102-109): error on sampled rows against
    fp64, at most twice SDPA math's error at the input dtype plus 1e-3."""
    import torch
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel

    from oracle import reference

    qc, kc, vc = q.cpu(), k.cpu(), v.cpu()
    ref = reference.attention_rows(qc, kc, vc, rows, causal=causal)
    err = (out.cpu()[:, rows].double() - ref).abs().max().item()
    mask = None
    if causal:
        cols = torch.arange(kc.shape[1])[None, :]
        mask = cols <= rows[:, None] + (kc.shape[1] - qc.shape[1])
    with sdpa_kernel(SDPBackend.MATH):
        base = F.scaled_dot_product_attention(
            qc[:, rows].transpose(1, 2).contiguous(),
            kc.transpose(1, 2).contiguous(),
            vc.transpose(1, 2).contiguous(),
            attn_mask=mask,
        ).transpose(1, 2)
    err_torch = (base.double() - ref).nan_to_num(0.0).abs().max().item()
    ok = bool(torch.isfinite(out).all()) and err <= 2 * err_torch + 1e-3
    return {"max_err_vs_fp64": err, "max_err_torch_vs_fp64": err_torch, "correct": ok}


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


def bench_prefill(steps: int, warmup: int, causal: bool) -> dict:
    import torch

    import flash_lab

    cfg = PREFILL
    q, k, v = prefill_inputs(cfg)
    rows = sampled_rows(cfg["seqlen"], 64)
    check = check_prefill(flash_lab.attention(q, k, v, causal=causal), q, k, v, causal, rows)
    if not check["correct"]:
        return {"status": "incorrect", **check}
    times, wall = time_op(lambda: flash_lab.attention(q, k, v, causal=causal), steps, warmup,
                          label="prefill_causal" if causal else "prefill")
    flops = attention_flops(cfg["batch"], cfg["heads"], cfg["seqlen"], cfg["seqlen"],
                            cfg["head_dim"], causal)
    mean_ms = sum(times) / len(times)
    stats = summarize(times)
    del q, k, v
    torch.cuda.empty_cache()
    return {
        "status": "ok",
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


def bench_decode(name: str, steps: int, warmup: int, flush) -> dict:
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
    # Check the first sequence in full against fp64 (the reference checks all of them; one keeps
    # the CPU side short at 32K keys), with the reference's rule.
    args = (q[:1].cpu(), k_cache[:1].cpu(), v_cache[:1].cpu(), seq_lens[:1].cpu())
    ref = reference.decode(*args)
    plain = reference.decode(*args, dtype=torch.bfloat16)
    err = (out[:1].cpu().double() - ref).abs().max().item()
    err_torch = (plain.double() - ref).abs().max().item()
    ok = bool(torch.isfinite(out).all()) and err <= 2 * err_torch + 1e-3
    if not ok:
        return {"status": "incorrect", "max_err_vs_fp64": err, "max_err_torch_vs_fp64": err_torch}
    del k_cache, v_cache
    times, _ = time_op(lambda: flash_lab.decode(q, k_used, v_used, seq_lens, block_tables=tables),
                       steps, warmup, flush, label=name)
    stats = summarize(times)
    mean_ms = sum(times) / len(times)
    kv = decode_kv_bytes(b, hkv, ctx, d, 2)
    splits, _ = _hip.decode_plan(b, h, hkv, d, ctx, torch.bfloat16,
                                 cu_count_=_hip.cu_count(torch.cuda.current_device()))
    del q, k_used, v_used, tables
    torch.cuda.empty_cache()
    return {
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
        "roofline": {"bound": "hbm", "achieved": kv / (mean_ms / 1e3) / 1e9, "peak": PEAK_HBM_GBPS,
                     "unit": "GB/s", "frac": kv / (mean_ms / 1e3) / 1e9 / PEAK_HBM_GBPS,
                     "per_launch": f"{kv:.4g} B of K+V (every cached row once), mean {mean_ms:.4f} ms "
                                   "for the split and merge kernels"},
        "max_err_vs_fp64": err,
        "max_err_torch_vs_fp64": err_torch,
    }


# ----------------------------------------------------------------------------------------------
# CPU baseline: the oracle on the host cores


def cpu_baseline(rows_count: int = 256, reps: int = 3) -> dict:
    """fp64 prefill rows (the oracle's attention_rows) on the host: rows_count query rows of every
    (batch, head) of the headline shape, non-causal; TFLOP/s extrapolated from the sampled rows."""
    import torch

    from oracle import reference

    cores = cpu_cores()
    torch.set_num_threads(cores)
    gen = torch.Generator().manual_seed(0)
    cfg = PREFILL
    b, h, hkv, s, d = cfg["batch"], cfg["heads"], cfg["heads_kv"], cfg["seqlen"], cfg["head_dim"]
    q = torch.randn((b, s, h, d), generator=gen).to(torch.bfloat16)
    k = torch.randn((b, s, hkv, d), generator=gen).to(torch.bfloat16)
    v = torch.randn((b, s, hkv, d), generator=gen).to(torch.bfloat16)
    rows = sampled_rows(s, rows_count)
    reference.attention_rows(q, k, v, rows[:8])  # warm up allocator and threads
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        reference.attention_rows(q, k, v, rows)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    flops = 4.0 * b * h * len(rows) * s * d
    return {
        "value": flops / t / 1e12,
        "unit": "TFLOP/s",
        "cores": cores,
        "kind": "port",
        "sample": (
            f"oracle fp64 attention_rows, {len(rows)} of {s} query rows x all {b * h} (batch, head)"
            f" of (4,32,32,4096,128), non-causal, median of {reps}: {t * 1e3:.0f} ms"
        ),
        "cpu_model": cpu_model(),
    }


# ----------------------------------------------------------------------------------------------


def parse_args(argv=None):
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument("--decode-steps", type=int, default=100)
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--trace", action="store_true",
                        help="roctx range per timed step, for rocprofv3 --marker-trace (timings "
                             "then include a synchronize per step)")
    parser.add_argument(
        "--only",
        help="comma list of workloads to run: prefill, prefill_causal, decode (all three), "
        f"{', '.join(DECODE)}, copy (a 1 GiB device copy, the calibration of the traffic "
        "counters); default: all but copy",
    )
    return parser.parse_args(argv)


def selected_workloads(only: str | None) -> list[str]:
    everything = ["prefill", "prefill_causal", *DECODE]
    if not only:
        return everything
    names = []
    for item in only.split(","):
        item = item.strip()
        if item == "decode":
            names += list(DECODE)
        elif item in everything or item == "copy":
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
    props = torch.cuda.get_device_properties(0)
    workloads = selected_workloads(args.only)
    secondary = {}
    headline = None
    if "prefill" in workloads:
        headline = bench_prefill(args.steps, args.warmup, causal=False)
        print(f"# prefill non-causal: {json.dumps(headline)}", file=sys.stderr, flush=True)
    if "prefill_causal" in workloads:
        secondary["prefill_causal"] = bench_prefill(args.steps, args.warmup, causal=True)
        print(f"# prefill causal: {json.dumps(secondary['prefill_causal'])}", file=sys.stderr,
              flush=True)
    decodes = [name for name in DECODE if name in workloads]
    if decodes:
        flush = torch.empty(FLUSH_BYTES // 4, dtype=torch.int32, device="cuda")
        for name in decodes:
            secondary[f"decode_{name}"] = bench_decode(name, args.decode_steps, 10, flush)
            print(f"# decode {name}: {json.dumps(secondary[f'decode_{name}'])}", file=sys.stderr,
                  flush=True)
        del flush
    if "copy" in workloads:
        secondary["copy"] = bench_copy(args.steps)
        print(f"# copy: {json.dumps(secondary['copy'])}", file=sys.stderr, flush=True)

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
            "per_launch": f"{headline['flops']:.4g} FLOP (4 B H S^2 D), mean {headline['mean_ms']:.4f} ms",
        }
    else:
        value, ms, roofline = 0.0, None, None

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
                     "what": "reference mma_pipelined, non-causal, H100 SXM5 (BASELINE.md)"},
        "dtype": "bf16",
        "data": "synthetic iid N(0,1), torch.Generator seed 0",
        "config": {
            "workload": "prefill forward (B,H,H_kv,S,D)=(4,32,32,4096,128) bf16 [B,S,H,D], non-causal",
            **PREFILL,
            "causal": False,
            "softmax_scale": 1 / math.sqrt(PREFILL["head_dim"]),
        },
        "roofline": roofline,
        "cpu_baseline": None,
        "secondary": secondary,
        "device": {"name": props.name, "cus": props.multi_processor_count,
                   "arch": getattr(props, "gcnArchName", "")},
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline()
    print(json.dumps(result), flush=True)
    return 0 if headline is None or headline["status"] == "ok" else 1


if __name__ == "__main__":
    raise SystemExit(main())
