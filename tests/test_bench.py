"""CPU checks of the benchmark's host logic: work models, statistics, workload selection and the
committed traffic figure (the reference's tests/test_bench.py:1-62 covers the same models)."""

import pytest

import bench


def test_attention_flops_counts_two_matmuls_and_halves_causal():
    full = bench.attention_flops(2, 4, 128, 256, 64, causal=False)
    assert full == 4 * 2 * 4 * 128 * 256 * 64
    assert bench.attention_flops(2, 4, 128, 256, 64, causal=True) == full / 2
    # The headline configuration is 2^40 FLOP non-causal.
    assert bench.attention_flops(4, 32, 4096, 4096, 128, causal=False) == 2.0**40


def test_decode_bytes_read_the_kv_cache_once():
    assert bench.decode_kv_bytes(1, 32, 32768, 128, 2) == 2**29
    assert bench.decode_kv_bytes(8, 32, 32768, 128, 2) == 2**32
    assert bench.decode_kv_bytes(8, 8, 32768, 128, 2) == 2**30
    # The reference's variant adds q read and o written: 536,887,296 B at B=1 MHA.
    assert bench.decode_bytes_with_qo(1, 32, 32, 32768, 128, 2) == 536_887_296


def test_summarize():
    assert bench.summarize([5.0, 1.0, 3.0, 2.0, 4.0]) == {
        "median": 3.0, "p10": 1.0, "p90": 5.0, "min": 1.0
    }


def test_workload_selection():
    prefills = ["prefill", "prefill_causal", "prefill_d64", "prefill_d64_causal"]
    assert bench.selected_workloads(None) == [*prefills, *bench.DECODE, "e2e_L"]
    assert bench.selected_workloads(None, e2e=False) == [*prefills, *bench.DECODE]
    assert bench.selected_workloads("decode,copy") == [*bench.DECODE, "copy"]
    # The sweep of the reference's other suites runs only when asked for.
    assert bench.selected_workloads("sweep") == ["sweep"]
    assert "sweep" not in bench.selected_workloads(None)
    assert bench.selected_workloads("e2e_L", e2e=False) == ["e2e_L"]
    # The calibration legs (hipBLASLt GEMM, MFMA rate probe) run only when asked for.
    assert bench.selected_workloads("mfma,gemm,prefill") == ["mfma", "gemm", "prefill"]
    assert "mfma" not in bench.selected_workloads(None) and "gemm" not in bench.selected_workloads(None)
    with pytest.raises(SystemExit):
        bench.selected_workloads("nope")


def test_sampled_rows_keep_the_ends():
    rows = bench.sampled_rows(4096, 64)
    assert len(rows) == 64 and rows[0] == 0 and rows[-1] == 4095
    assert bool((rows[1:] > rows[:-1]).all())


def test_profiled_traffic_is_parsed(tmp_path):
    path = tmp_path / "p.md"
    path.write_text("# x\n\ntraffic_bytes_per_launch: 123456\n")
    assert bench.profiled_traffic(path) == 123456.0
    assert bench.profiled_traffic(tmp_path / "missing.md") is None
    # The committed prefill profile carries the figure, and it is close to the algorithmic
    # minimum of q + k + v + o + lse = 514 MiB.
    committed = bench.profiled_traffic()
    assert committed is not None and 500 * 2**20 < committed < 600 * 2**20


def test_more_than_one_gpu_is_refused(capsys):
    assert bench.main(["--gpus", "2"]) == 2
    assert "one GPU" in capsys.readouterr().err


def test_trace_option_parses():
    args = bench.parse_args(["--trace", "--only", "decode"])
    assert args.trace and args.only == "decode"
    assert not bench.parse_args([]).trace


def test_exit_status_fails_on_any_incorrect_workload():
    ok = {"status": "ok"}
    assert bench.overall_status(ok, {"a": ok, "e2e_L": {"status": "skipped"}}) == 0
    assert bench.overall_status(ok, {"e2e_L": {"status": "budget"}}) == 0
    assert bench.overall_status(ok, {"decode_B8-GQA": {"status": "incorrect"}}) == 1
    assert bench.overall_status(ok, {"prefill_causal": {"status": "error"}}) == 1
    assert bench.overall_status({"status": "incorrect"}, {}) == 1
    assert bench.overall_status(None, {"a": ok}) == 0


def test_cpu_timer_respects_reps_and_budget():
    calls = []
    t = bench.time_cpu(lambda: calls.append(1), budget_s=0.0)
    # Two warmup runs (a fast function), then the minimum number of timed runs.
    assert t["warmup"] == 2 and t["reps"] == bench.CPU_MIN_REPS
    assert len(calls) == 2 + bench.CPU_MIN_REPS
    t = bench.time_cpu(lambda: None, budget_s=60.0, warmed_up=True)
    assert t["warmup"] == 0 and t["reps"] == bench.CPU_MAX_REPS
    assert set(t["ms"]) == {"median", "p10", "p90", "min"}


def test_cpu_timer_minimum_reps():
    t = bench.time_cpu(lambda: None, budget_s=0.0, warmed_up=True, min_reps=bench.CPU_DECODE_REPS)
    assert t["reps"] == bench.CPU_DECODE_REPS >= 10


def test_cpu_decode_leg_samples_two_sequences():
    import torch

    gen = torch.Generator().manual_seed(0)
    q = torch.randn(4, 1, 8, 64, generator=gen).to(torch.bfloat16)
    k = torch.randn(4, 300, 2, 64, generator=gen).to(torch.bfloat16)
    lens = torch.tensor([300, 100, 200, 300], dtype=torch.int32)
    leg = bench.cpu_decode_leg(q, k, k, lens)
    assert leg["reps"] >= 10 and "2 of 4 sequences" in leg["sample"]
    # GB/s of the bf16 K+V bytes of the two sequences it timed: 2 x (300 + 100) x 2 x 64 x 2 B.
    assert leg["gbps"] == pytest.approx(2 * 400 * 2 * 64 * 2 / (leg["ms"]["median"] / 1e3) / 1e9)


def test_sweep_tables_cover_the_reference_suites():
    # bench/suites.py:63-125 of the reference: 9 prefill shapes (prefill_bf16 and prefill_seqlen),
    # 16 decode_ctx + 3 decode_batch + 6 decode_d64 + 4 decode_long shapes.
    assert len(bench.SWEEP_PREFILL) == 9 and len(bench.SWEEP_DECODE) == 29
    assert len({shape for shape, _, _ in bench.SWEEP_DECODE}) == 29
    assert all(v > 0 for _, pair, _ in bench.SWEEP_PREFILL for v in pair)


def test_tokens_follow_sdpa_rule():
    import torch

    ref = torch.tensor([5, 6, 7, 8])
    logits = torch.zeros(4, 10)
    logits[2, 7], logits[2, 3] = 10.0, 10.0 - 1e-3  # a near-tie at step 2
    same = bench.tokens_follow_sdpa(ref.clone(), ref, logits)
    assert same["tokens_follow_sdpa"] and same["tokens_checked"] == 4 and same["first_difference"] is None
    tie = bench.tokens_follow_sdpa(torch.tensor([5, 6, 3, 1]), ref, logits)
    assert tie["tokens_follow_sdpa"] and tie["first_difference"] == 2
    logits[1, 6], logits[1, 2] = 10.0, 9.0  # a clear winner at step 1
    assert not bench.tokens_follow_sdpa(torch.tensor([5, 2, 7, 8]), ref, logits)["tokens_follow_sdpa"]


def test_cpu_c1_leg_meets_the_fp32_rule():
    # BASELINE.json configs[0], the reference's CPU-runnable case: fp32 within 1e-5 normwise of fp64.
    leg = bench.cpu_c1_leg()
    assert leg["correct"] and leg["fp32_vs_fp64_normwise"] <= 1e-5
    assert leg["fp32"]["reps"] >= bench.CPU_MIN_REPS and leg["fp64"]["gflops"] > 0
