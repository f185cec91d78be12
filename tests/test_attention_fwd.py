"""Prefill kernel parity against the fp64 oracle, under the reference's tolerance rule.

Shape list, edge cases and rule follow the reference's tests/test_attention_fwd.py:18-177: ragged
lengths, S_q != S_k both ways (causal rows without keys), GQA, packed strided inputs, scores of
order 100, bitwise determinism, rejection of unsupported inputs, and the full output of the two
long shapes in bf16 and fp16. Every shape runs on both kernels of this build (the 8-wave ping-pong
kernel and the 4-wave one). Added here: the headline shape (4, 32, 32, 4096, 128) checked on the
reference benchmark's 256 sampled rows, and the two tensor-core impl names serving the same kernel.
"""

import pytest
import torch

import flash_lab
from parity import PrefillOracle, check_prefill

pytestmark = pytest.mark.gpu

IMPLS = [
    ("mma_pipelined", torch.bfloat16),
    ("mma_pipelined", torch.float16),
]

SHAPES = [
    # batch, seqlen_q, seqlen_k, heads, heads_kv, head_dim
    (1, 1, 1, 1, 1, 64),
    (3, 7, 7, 8, 8, 64),
    (1, 16, 16, 1, 1, 128),
    (3, 63, 63, 8, 2, 128),
    (1, 128, 128, 8, 1, 64),
    (3, 257, 257, 8, 8, 128),
    (1, 1024, 1024, 8, 2, 64),
    (2, 1024, 1024, 4, 4, 128),
    (2, 37, 101, 4, 2, 64),  # S_q < S_k
    (1, 101, 37, 4, 4, 128),  # S_q > S_k: causal rows without keys
    (1, 700, 300, 2, 1, 128),  # S_q > S_k over three blocks: a block, and waves, with no keys
    (2, 1, 300, 8, 2, 128),
    # Causal pairs of 256-row blocks whose waves switch from the light to the heavy block with 1,
    # 2 or 3 idle periods, or none, or have no heavy keys (the one-stream schedule's cases).
    (2, 900, 1000, 8, 2, 128),
    (1, 481, 482, 4, 4, 64),
    (2, 355, 131, 4, 2, 128),
    # Head_dim 64 (384-row blocks of three 4-wave groups): S_q > S_k over three blocks (causal rows
    # without keys, groups without rows), and a last block whose 32 rows are one wave's.
    (1, 900, 400, 4, 2, 64),
    (2, 800, 1200, 8, 2, 64),
]
SLOW_SHAPES = [(1, 4096, 4096, 4, 4, 128), (1, 8192, 8192, 2, 1, 64)]


def make_inputs(shape, dtype, scale=1.0):
    batch, seqlen_q, seqlen_k, heads, heads_kv, head_dim = shape
    q = torch.randn(batch, seqlen_q, heads, head_dim, device="cuda", dtype=dtype) * scale
    k = torch.randn(batch, seqlen_k, heads_kv, head_dim, device="cuda", dtype=dtype) * scale
    v = torch.randn(batch, seqlen_k, heads_kv, head_dim, device="cuda", dtype=dtype)
    return q, k, v


def sampled_rows(seqlen, count, seed=0):
    """First, last and a seeded sample of the rows in between (the reference's bench/run.py)."""
    if seqlen <= count:
        return torch.arange(seqlen)
    gen = torch.Generator().manual_seed(seed)
    middle = torch.randperm(seqlen - 2, generator=gen)[: count - 2] + 1
    return torch.cat([torch.tensor([0, seqlen - 1]), middle]).sort().values


# The library runs the 8-wave ping-pong kernel when it fills at least 256 workgroups and the
# 4-wave kernel below that (head_dim 64 and 128 alike); the prefill_pp_min_wg knob routes a shape
# to either one, so both are checked on every shape. The ping-pong kernel runs a causal pair of
# query blocks as two blocks (prefill_pp.hip, the default) or as one stream of key tiles
# (prefill_causal.hip, the prefill_causal_stream knob at 1): "pp_stream" checks the second.
ROUTES = {
    "auto": {},
    "pingpong": {"prefill_pp_min_wg": 0},
    "pp_stream": {"prefill_pp_min_wg": 0, "prefill_causal_stream": 1},
    "wg128": {"prefill_pp_min_wg": 1 << 30},
}


def set_route(knobs, name):
    for knob, value in ROUTES[name].items():
        knobs(knob, value)


@pytest.fixture(params=list(ROUTES), ids=str)
def route(request, knobs):
    set_route(knobs, request.param)
    return request.param


@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("shape", SHAPES, ids=str)
@pytest.mark.parametrize("impl,dtype", IMPLS, ids=lambda x: str(x).replace("torch.", ""))
def test_matches_reference(impl, dtype, shape, causal, route):
    print(f"prefill {impl} {dtype} {shape} causal={causal} route={route}", flush=True)
    q, k, v = make_inputs(shape, dtype)
    out, lse = flash_lab.attention(q, k, v, causal=causal, impl=impl, return_lse=True)
    check_prefill(out, lse, q, k, v, causal)


# Oracle side of the slow shapes, computed once per (shape, dtype, causal) and shared by the two
# kernels (the fp64 reference of a 4K or 8K sequence takes seconds on the host).
_LONG_CASES = {}


def _long_case(shape, dtype, causal):
    key = (shape, dtype, causal)
    if key not in _LONG_CASES:
        gen = torch.Generator(device="cuda").manual_seed(sum(shape))
        batch, seqlen_q, seqlen_k, heads, heads_kv, head_dim = shape
        q = torch.randn(batch, seqlen_q, heads, head_dim, device="cuda", dtype=dtype, generator=gen)
        k = torch.randn(batch, seqlen_k, heads_kv, head_dim, device="cuda", dtype=dtype, generator=gen)
        v = torch.randn(batch, seqlen_k, heads_kv, head_dim, device="cuda", dtype=dtype, generator=gen)
        _LONG_CASES[key] = ((q, k, v), PrefillOracle(q, k, v, causal))
    return _LONG_CASES[key]


@pytest.mark.slow
@pytest.mark.parametrize("kernel", ["pingpong", "pp_stream", "wg128"])
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("shape", SLOW_SHAPES, ids=str)
def test_long_sequences_full_output(shape, dtype, causal, kernel, knobs):
    # The reference checks the whole output of its long shapes for every dtype
    # (tests/test_attention_fwd.py:110-118); so does this test, on both kernels.
    if kernel == "pp_stream" and not causal:
        pytest.skip("the causal schedule knob does not change a non-causal call")
    print(f"prefill long {shape} {dtype} causal={causal} kernel={kernel}", flush=True)
    set_route(knobs, kernel)
    (q, k, v), oracle = _long_case(shape, dtype, causal)
    out, lse = flash_lab.attention(q, k, v, causal=causal, return_lse=True)
    oracle.check(out, lse)


@pytest.mark.parametrize("schedule", ["stream", "blocks"])
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
def test_headline_shape_sampled_rows(causal, schedule, knobs):
    if schedule == "stream":
        if not causal:
            pytest.skip("the causal schedule knob does not change a non-causal call")
        knobs("prefill_causal_stream", 1)
    # (B, H, H_kv, S, D) = (4, 32, 32, 4096, 128) bf16, seeded like the benchmark (q, k, v order),
    # on the 256 sampled rows of the reference's benchmark check (bench/run.py:36, 75-79).
    gen = torch.Generator(device="cuda").manual_seed(0)
    shape = (4, 4096, 32, 128)
    q, k, v = (torch.randn(shape, device="cuda", dtype=torch.bfloat16, generator=gen) for _ in range(3))
    out, lse = flash_lab.attention(q, k, v, causal=causal, return_lse=True)
    check_prefill(out, lse, q, k, v, causal, rows=sampled_rows(4096, 256), c_ref=True)


# The other shapes of the reference's bf16 prefill benchmarks (bench/suites.py:63-94): prefill_bf16
# (1K to 16K keys, head_dim 64, GQA with 8 KV heads) and prefill_seqlen (16K tokens per call,
# S = 512 to 16384; its 4K, 8K and 16K rows are the ones above). (B, H, H_kv, S, D), bf16, seeded
# like the benchmark, 256 sampled query rows of every (batch, head), causal and not.
PREFILL_SUITE = [
    (4, 32, 32, 1024, 128),
    (2, 32, 32, 8192, 128),
    (1, 32, 32, 16384, 128),
    (8, 16, 16, 2048, 64),
    (4, 32, 8, 4096, 128),
    (32, 32, 32, 512, 128),
    (16, 32, 32, 1024, 128),
    (8, 32, 32, 2048, 128),
]


@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("shape", PREFILL_SUITE, ids=lambda s: f"B{s[0]}-H{s[1]}-Hkv{s[2]}-S{s[3]}-D{s[4]}")
def test_reference_suite_shapes_sampled_rows(shape, causal):
    batch, heads, heads_kv, seqlen, head_dim = shape
    print(f"prefill suite shape {shape} causal={causal}", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(0)
    q = torch.randn(batch, seqlen, heads, head_dim, device="cuda", dtype=torch.bfloat16, generator=gen)
    k = torch.randn(batch, seqlen, heads_kv, head_dim, device="cuda", dtype=torch.bfloat16, generator=gen)
    v = torch.randn(batch, seqlen, heads_kv, head_dim, device="cuda", dtype=torch.bfloat16, generator=gen)
    out, lse = flash_lab.attention(q, k, v, causal=causal, return_lse=True)
    check_prefill(out, lse, q, k, v, causal, rows=sampled_rows(seqlen, 256), c_ref=True)


def test_ragged_long_sequence_sampled_rows():
    # 4,196 rows: 16 full 256-row blocks and a ragged 17th per (batch, head), on a grid large
    # enough for the ping-pong kernel. 256 sampled rows of every (batch, head), plus rows of the
    # ragged block.
    gen = torch.Generator(device="cuda").manual_seed(5)
    shape = (2, 4196, 32, 128)
    q, k, v = (torch.randn(shape, device="cuda", dtype=torch.bfloat16, generator=gen) for _ in range(3))
    out, lse = flash_lab.attention(q, k, v, causal=False, return_lse=True)
    rows = torch.unique(torch.cat([sampled_rows(4196, 256), torch.arange(4096, 4196, 7)]))
    check_prefill(out, lse, q, k, v, False, rows=rows)


@pytest.mark.parametrize("impl,dtype", IMPLS, ids=lambda x: str(x).replace("torch.", ""))
def test_large_scores(impl, dtype, route):
    # Scores of order 100 overflow exp() unless the running max is subtracted (on each kernel: the
    # two move their reference points under different rules).
    q, k, v = make_inputs((2, 129, 129, 4, 2, 64), dtype, scale=10.0)
    out, lse = flash_lab.attention(q, k, v, causal=True, impl=impl, return_lse=True)
    check_prefill(out, lse, q, k, v, causal=True)


@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_dominant_key_after_the_first_tiles(dtype, head_dim, causal, route):
    # Rows whose largest key arrives after their first 64-key tile and holds 15-75% of the row
    # (its score 5 to 8 above the row's typical one): the kernels move their reference points to
    # such keys (a point left below one keeps its probability far above 1 and rounded to the input
    # type, an error that scales with the key's share). In a CPU emulation of the kernels'
    # arithmetic on these inputs the moved point gives 0.3 of this rule's bound, a point that
    # never moves after the first tile 0.5. Non-causal: row r < S - 64 gets key
    # 64 + (37 r mod (S - 64)) (a bijection, so every planted key is its row's own); causal: row
    # r >= 64 gets its own diagonal key, in its last tile, a masked one.
    print(f"prefill dominant key {dtype} D={head_dim} causal={causal} route={route}", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(7)
    batch, seqlen, heads = 2, 700, 4
    q, k, v = (torch.randn(batch, seqlen, heads, head_dim, device="cuda", generator=gen)
               for _ in range(3))
    if causal:
        rows = torch.arange(64, seqlen, device="cuda")
        keys = rows
    else:
        rows = torch.arange(seqlen - 64, device="cuda")
        keys = 64 + (rows * 37) % (seqlen - 64)
    share = torch.linspace(5.0, 8.0, len(rows), device="cuda")[None, :, None, None]
    k[:, keys] = q[:, rows] / q[:, rows].norm(dim=-1, keepdim=True) * share
    q, k, v = q.to(dtype), k.to(dtype), v.to(dtype)
    out, lse = flash_lab.attention(q, k, v, causal=causal, return_lse=True)
    check_prefill(out, lse, q, k, v, causal)


@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("impl,dtype", IMPLS, ids=lambda x: str(x).replace("torch.", ""))
def test_strided_inputs(impl, dtype, head_dim, route):
    # q, k, v sliced out of one packed [B, S, 3, H, D] projection: no copies, unusual strides.
    qkv = torch.randn(2, 77, 3, 4, head_dim, device="cuda", dtype=dtype)
    q, k, v = qkv.unbind(dim=2)
    assert not q.is_contiguous()
    out, lse = flash_lab.attention(q, k, v, causal=True, impl=impl, return_lse=True)
    check_prefill(out, lse, q, k, v, causal=True)


@pytest.mark.parametrize("scale", [0.05, 0.5])
def test_explicit_softmax_scale(scale, route):
    q, k, v = make_inputs((2, 70, 90, 4, 2, 128), torch.bfloat16)
    out, lse = flash_lab.attention(q, k, v, causal=True, softmax_scale=scale, return_lse=True)
    check_prefill(out, lse, q, k, v, causal=True, scale=scale)


@pytest.mark.parametrize("impl,dtype", IMPLS, ids=lambda x: str(x).replace("torch.", ""))
def test_deterministic(impl, dtype):
    q, k, v = make_inputs((2, 300, 300, 8, 2, 128), dtype)
    first = flash_lab.attention(q, k, v, causal=True, impl=impl)
    second = flash_lab.attention(q, k, v, causal=True, impl=impl)
    assert torch.equal(first, second)


@pytest.mark.parametrize("impl,dtype", IMPLS, ids=lambda x: str(x).replace("torch.", ""))
def test_rejects_unsupported_inputs(impl, dtype):
    q, k, v = make_inputs((1, 8, 8, 2, 2, 96), dtype)
    with pytest.raises(ValueError, match="head_dim"):
        flash_lab.attention(q, k, v, impl=impl)
    q, k, v = make_inputs((1, 8, 8, 2, 2, 64), torch.float64)
    with pytest.raises(ValueError, match="dtype"):
        flash_lab.attention(q, k, v, impl=impl)


def test_both_tensor_core_names_run_the_same_kernel():
    q, k, v = make_inputs((2, 100, 100, 4, 2, 128), torch.bfloat16)
    a = flash_lab.attention(q, k, v, causal=True, impl="mma_pipelined")
    b = flash_lab.attention(q, k, v, causal=True, impl="mma")
    assert torch.equal(a, b)


def test_auto_picks_the_hip_kernel():
    q, k, v = make_inputs((1, 64, 64, 2, 2, 64), torch.bfloat16)
    torch.testing.assert_close(
        flash_lab.attention(q, k, v), flash_lab.attention(q, k, v, impl="mma_pipelined"),
        rtol=0, atol=0,
    )


def test_reference_kernels_this_build_does_not_ship():
    q, k, v = make_inputs((1, 32, 32, 2, 2, 64), torch.bfloat16)
    with pytest.raises(RuntimeError, match="not available in this build"):
        flash_lab.attention(q, k, v, impl="triton")
    q32, k32, v32 = (x.float() for x in (q, k, v))
    with pytest.raises(ValueError, match="no available implementation"):
        flash_lab.attention(q32, k32, v32)
