"""Decode kernel parity against the fp64 oracle, under the reference's tolerance rule.

Cases follow the reference's tests/test_decode.py:11-119: three dtypes, GQA groups 1 to 8 (and a
group of 3), ragged and random lengths, split counts with empty splits, a strided cache carved out
of a larger allocation, rank-3 queries, bitwise determinism, rejections. Added: the three
benchmark shapes at 32K keys, split-count invariance within tolerance, lengths outside the cache
(clamped on the device instead of read out of bounds), paged caches, and both split kernels (the
vector one and the matrix-core one for GQA groups) on every shape, with groups up to 32.
"""

import pytest
import torch

import flash_lab
from parity import check_decode, normwise_rel
from oracle import reference

pytestmark = pytest.mark.gpu

IMPLS = ["decode_inplace", "splitkv"]
DTYPES = [torch.bfloat16, torch.float16, torch.float32]

CASES = [
    # batch, heads, heads_kv, max_seqlen, head_dim, seq_lens
    (1, 8, 8, 64, 64, [64]),
    (4, 8, 1, 1100, 128, [1, 5, 1023, 1100]),
    (3, 32, 4, 4097, 128, [4097, 64, 1024]),
    (2, 6, 2, 300, 64, [300, 17]),
    (2, 32, 8, 700, 128, [700, 333]),
    (16, 8, 2, 512, 64, "random"),
]


def make_case(case, dtype, gen):
    batch, heads, heads_kv, max_seqlen, head_dim, lens = case
    q = torch.randn(batch, 1, heads, head_dim, device="cuda", dtype=dtype, generator=gen)
    shape = (batch, max_seqlen, heads_kv, head_dim)
    k_cache = torch.randn(shape, device="cuda", dtype=dtype, generator=gen)
    v_cache = torch.randn(shape, device="cuda", dtype=dtype, generator=gen)
    if lens == "random":
        seq_lens = torch.randint(1, max_seqlen + 1, (batch,), device="cuda", generator=gen)
    else:
        seq_lens = torch.tensor(lens, device="cuda")
    return q, k_cache, v_cache, seq_lens.to(torch.int32)


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"B{c[0]}-H{c[1]}-Hkv{c[2]}-S{c[3]}-D{c[4]}")
@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).removeprefix("torch."))
@pytest.mark.parametrize("impl", IMPLS)
def test_matches_reference(impl, dtype, case):
    print(f"decode {impl} {dtype} {case}", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(0)
    q, k_cache, v_cache, seq_lens = make_case(case, dtype, gen)
    out, lse = flash_lab.decode(q, k_cache, v_cache, seq_lens, impl=impl, return_lse=True)
    check_decode(out, lse, q, k_cache, v_cache, seq_lens)


# The matrix-core split kernel (bf16/fp16, up to 32 query heads per KV head) serves groups of 4 and
# more by default. With the decode_mfma_min_group knob at 1 it takes every group, MHA included, so
# the shapes above and some larger groups run through it against the oracle.
MFMA_CASES = CASES + [
    (2, 64, 8, 3000, 128, [3000, 77]),  # group 8
    (2, 64, 4, 1500, 128, [1500, 999]),  # group 16
    (1, 32, 1, 2100, 64, [2100]),  # group 32 (one KV head)
    (2, 24, 2, 900, 128, [900, 31]),  # group 12
    (2, 64, 1, 700, 128, [700, 250]),  # group 64: more than the kernel's 32 columns (vector kernel)
]


@pytest.fixture
def mfma_everywhere(knobs):
    knobs("decode_mfma_min_group", 1)


@pytest.fixture
def vector_only(knobs):
    knobs("decode_mfma_min_group", 1000)


@pytest.mark.parametrize("case", MFMA_CASES, ids=lambda c: f"B{c[0]}-H{c[1]}-Hkv{c[2]}-S{c[3]}-D{c[4]}")
@pytest.mark.parametrize("dtype", DTYPES[:2], ids=lambda d: str(d).removeprefix("torch."))
@pytest.mark.parametrize("impl", IMPLS)
def test_mfma_kernel_matches_reference(impl, dtype, case, mfma_everywhere):
    print(f"decode (matrix cores) {impl} {dtype} {case}", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(0)
    q, k_cache, v_cache, seq_lens = make_case(case, dtype, gen)
    out, lse = flash_lab.decode(q, k_cache, v_cache, seq_lens, impl=impl, return_lse=True)
    check_decode(out, lse, q, k_cache, v_cache, seq_lens)


@pytest.mark.parametrize("num_splits", [1, 2, 8, 64, None])
def test_mfma_kernel_split_counts(num_splits, mfma_everywhere):
    gen = torch.Generator(device="cuda").manual_seed(1)
    q, k_cache, v_cache, seq_lens = make_case(
        (3, 16, 2, 2000, 128, [2000, 40, 777]), torch.bfloat16, gen
    )
    out, lse = flash_lab.decode(
        q, k_cache, v_cache, seq_lens, impl="splitkv", num_splits=num_splits, return_lse=True
    )
    check_decode(out, lse, q, k_cache, v_cache, seq_lens)


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"B{c[0]}-H{c[1]}-Hkv{c[2]}-S{c[3]}-D{c[4]}")
@pytest.mark.parametrize("dtype", DTYPES[:2], ids=lambda d: str(d).removeprefix("torch."))
@pytest.mark.parametrize("impl", IMPLS)
def test_vector_kernel_matches_reference(impl, dtype, case, vector_only):
    # The groups the matrix-core kernel takes by default, on the vector kernel.
    print(f"decode (vector kernel) {impl} {dtype} {case}", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(0)
    q, k_cache, v_cache, seq_lens = make_case(case, dtype, gen)
    out, lse = flash_lab.decode(q, k_cache, v_cache, seq_lens, impl=impl, return_lse=True)
    check_decode(out, lse, q, k_cache, v_cache, seq_lens)


def test_gqa_benchmark_shape_on_the_vector_kernel(vector_only):
    # B8-GQA at 32K keys on the vector kernel (the matrix-core kernel serves it by default).
    gen = torch.Generator(device="cuda").manual_seed(0)
    q = torch.randn(8, 1, 32, 128, device="cuda", dtype=torch.bfloat16, generator=gen)
    k_cache = torch.randn(8, 32768, 8, 128, device="cuda", dtype=torch.bfloat16, generator=gen)
    v_cache = torch.randn(8, 32768, 8, 128, device="cuda", dtype=torch.bfloat16, generator=gen)
    seq_lens = torch.full((8,), 32768, device="cuda", dtype=torch.int32)
    out, lse = flash_lab.decode(q, k_cache, v_cache, seq_lens, return_lse=True)
    check_decode(out, lse, q, k_cache, v_cache, seq_lens)


@pytest.mark.parametrize("num_splits", [1, 2, 8, 64, None])
def test_splitkv_split_counts(num_splits):
    # More splits than keys leaves some splits empty; they must not disturb the merge.
    gen = torch.Generator(device="cuda").manual_seed(1)
    q, k_cache, v_cache, seq_lens = make_case(
        (3, 16, 4, 2000, 128, [2000, 40, 777]), torch.bfloat16, gen
    )
    out, lse = flash_lab.decode(
        q, k_cache, v_cache, seq_lens, impl="splitkv", num_splits=num_splits, return_lse=True
    )
    check_decode(out, lse, q, k_cache, v_cache, seq_lens)


@pytest.mark.parametrize("impl", IMPLS)
def test_strided_cache_and_rank3_query(impl):
    # Caches carved out of a larger allocation (every other KV head), q given as [B, H, D].
    gen = torch.Generator(device="cuda").manual_seed(2)
    big = torch.randn(2, 600, 8, 128, device="cuda", dtype=torch.bfloat16, generator=gen)
    k_cache, v_cache = big[:, :, 0::2], big[:, :, 1::2]
    q = torch.randn(2, 16, 128, device="cuda", dtype=torch.bfloat16, generator=gen)
    seq_lens = torch.tensor([600, 123], device="cuda", dtype=torch.int32)
    out, lse = flash_lab.decode(q, k_cache, v_cache, seq_lens, impl=impl, return_lse=True)
    assert out.shape == q.shape
    check_decode(out, lse, q, k_cache, v_cache, seq_lens)


@pytest.mark.parametrize("impl", IMPLS)
def test_deterministic(impl):
    gen = torch.Generator(device="cuda").manual_seed(3)
    q, k_cache, v_cache, seq_lens = make_case(
        (4, 32, 8, 3000, 128, [3000, 1, 2048, 999]), torch.bfloat16, gen
    )
    first = flash_lab.decode(q, k_cache, v_cache, seq_lens, impl=impl)
    second = flash_lab.decode(q, k_cache, v_cache, seq_lens, impl=impl)
    assert torch.equal(first, second)


def test_auto_is_splitkv():
    gen = torch.Generator(device="cuda").manual_seed(4)
    q, k_cache, v_cache, seq_lens = make_case((2, 8, 8, 64, 64, [64, 3]), torch.bfloat16, gen)
    auto = flash_lab.decode(q, k_cache, v_cache, seq_lens)
    torch.testing.assert_close(
        auto, flash_lab.decode(q, k_cache, v_cache, seq_lens, impl="splitkv"), rtol=0, atol=0
    )


@pytest.mark.parametrize("impl", IMPLS)
def test_rejects_unsupported(impl):
    q = torch.randn(1, 1, 4, 96, device="cuda", dtype=torch.bfloat16)
    cache = torch.randn(1, 8, 4, 96, device="cuda", dtype=torch.bfloat16)
    seq_lens = torch.tensor([8], device="cuda", dtype=torch.int32)
    with pytest.raises(ValueError, match="head_dim"):
        flash_lab.decode(q, cache, cache, seq_lens, impl=impl)


@pytest.mark.parametrize(
    "batch,heads_kv",
    [(1, 32), pytest.param(8, 32, marks=pytest.mark.slow), (8, 8)],
    ids=["B1-MHA", "B8-MHA", "B8-GQA"],
)
def test_benchmark_shapes_at_32k(batch, heads_kv):
    # The three decode configurations of the benchmark: 32K valid keys in a [B, 32768, H_kv, 128]
    # bf16 cache, seeded like the benchmark (q, k_cache, v_cache order).
    gen = torch.Generator(device="cuda").manual_seed(0)
    q = torch.randn(batch, 1, 32, 128, device="cuda", dtype=torch.bfloat16, generator=gen)
    shape = (batch, 32768, heads_kv, 128)
    k_cache = torch.randn(shape, device="cuda", dtype=torch.bfloat16, generator=gen)
    v_cache = torch.randn(shape, device="cuda", dtype=torch.bfloat16, generator=gen)
    seq_lens = torch.full((batch,), 32768, device="cuda", dtype=torch.int32)
    out, lse = flash_lab.decode(q, k_cache, v_cache, seq_lens, return_lse=True)
    check_decode(out, lse, q, k_cache, v_cache, seq_lens)


def test_split_count_changes_results_only_within_tolerance():
    gen = torch.Generator(device="cuda").manual_seed(5)
    q, k_cache, v_cache, seq_lens = make_case(
        (2, 8, 2, 5000, 128, [5000, 2500]), torch.float32, gen
    )
    ref = reference.decode(q.cpu(), k_cache.cpu(), v_cache.cpu(), seq_lens.cpu())
    for n in (1, 3, 16, 128):
        out = flash_lab.decode(q, k_cache, v_cache, seq_lens, num_splits=n)
        # fp32 path: within 1e-5 relative (normwise) of fp64 for every split count.
        assert normwise_rel(out.cpu(), ref) <= 1e-5, n


@pytest.mark.parametrize(
    "case,dtype",
    [((2, 4, 4, 100, 64, [100, 100]), torch.float32), ((2, 32, 4, 100, 128, [100, 100]), torch.bfloat16)],
    ids=["vector-fp32", "matrix-core-bf16"],
)
def test_lengths_outside_the_cache_are_clamped(case, dtype):
    # seq_lens is not checked on the host; the kernel clamps it to [0, S_max] so that a bad value
    # cannot read outside the cache. A length above S_max behaves as S_max.
    gen = torch.Generator(device="cuda").manual_seed(6)
    q, k_cache, v_cache, _ = make_case(case, dtype, gen)
    too_long = torch.tensor([100000, 100], device="cuda", dtype=torch.int32)
    full = torch.tensor([100, 100], device="cuda", dtype=torch.int32)
    torch.testing.assert_close(
        flash_lab.decode(q, k_cache, v_cache, too_long),
        flash_lab.decode(q, k_cache, v_cache, full),
        rtol=0, atol=0,
    )
    empty = torch.tensor([0, 100], device="cuda", dtype=torch.int32)
    out, lse = flash_lab.decode(q, k_cache, v_cache, empty, return_lse=True)
    assert torch.all(out[0] == 0) and torch.isneginf(lse[0]).all()


# Paged caches: [num_blocks, page_size, H_kv, D] pools with per-sequence block tables. The
# reference defines the layout and its oracle (flash_lab/layouts.py:145-158, reference.py:155-164)
# but every reference kernel rejects it; here both decode impls run it.


def to_paged(cache, page_size, gen, spare=5):
    """Scatters a contiguous [B, S_max, H_kv, D] cache into shuffled blocks of a larger pool."""
    batch, max_seqlen = cache.shape[:2]
    per_seq = -(-max_seqlen // page_size)
    padded = torch.zeros(batch, per_seq * page_size, *cache.shape[2:], dtype=cache.dtype,
                         device=cache.device)
    padded[:, :max_seqlen] = cache
    num_blocks = batch * per_seq + spare
    order = torch.randperm(num_blocks, generator=gen)[: batch * per_seq].to(cache.device)
    pool = torch.randn(num_blocks, page_size, *cache.shape[2:], dtype=cache.dtype,
                       device=cache.device)  # unused blocks hold noise
    pool[order] = padded.reshape(batch * per_seq, page_size, *cache.shape[2:])
    return pool, order.view(batch, per_seq).to(torch.int32)


PAGED_CASES = [
    # batch, heads, heads_kv, max_seqlen, head_dim, seq_lens, page_size
    (3, 8, 2, 300, 128, [300, 1, 157], 16),
    (2, 32, 8, 2000, 128, [2000, 1333], 64),
    (4, 8, 8, 129, 64, [129, 64, 65, 3], 1),
    (2, 6, 2, 500, 64, [500, 250], 7),  # a page size that is not a power of two
    (1, 32, 32, 4096, 128, [4096], 256),
]


@pytest.mark.parametrize("case", PAGED_CASES, ids=lambda c: f"B{c[0]}-H{c[1]}-Hkv{c[2]}-S{c[3]}-D{c[4]}-P{c[6]}")
@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).removeprefix("torch."))
@pytest.mark.parametrize("impl", IMPLS)
def test_paged_matches_reference(impl, dtype, case):
    print(f"paged decode {impl} {dtype} {case}", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(3)
    *contig, page_size = case
    q, k_cache, v_cache, seq_lens = make_case(tuple(contig), dtype, gen)
    cpu_gen = torch.Generator().manual_seed(4)
    k_pool, tables = to_paged(k_cache, page_size, cpu_gen)
    cpu_gen = torch.Generator().manual_seed(4)
    v_pool, _ = to_paged(v_cache, page_size, cpu_gen)
    out, lse = flash_lab.decode(q, k_pool, v_pool, seq_lens, block_tables=tables, impl=impl,
                                return_lse=True)
    # The oracle reads the pool through the same tables (reference.py:155-164).
    ref, ref_lse = reference.decode(q.cpu(), k_pool.cpu(), v_pool.cpu(), seq_lens.cpu(),
                                    block_tables=tables.cpu(), return_lse=True)
    plain_ref = reference.decode(q.cpu(), k_cache.cpu(), v_cache.cpu(), seq_lens.cpu())
    torch.testing.assert_close(ref, plain_ref, rtol=0, atol=0)  # the pool holds the same rows
    check_decode(out, lse, q, k_cache, v_cache, seq_lens)


@pytest.mark.parametrize("case", PAGED_CASES, ids=lambda c: f"B{c[0]}-H{c[1]}-Hkv{c[2]}-S{c[3]}-D{c[4]}-P{c[6]}")
@pytest.mark.parametrize("dtype", DTYPES[:2], ids=lambda d: str(d).removeprefix("torch."))
@pytest.mark.parametrize("impl", IMPLS)
def test_paged_mfma_kernel_matches_reference(impl, dtype, case, mfma_everywhere):
    # Every paged case (page sizes 1, 7, 16, 64, 256; head_dim 64 and 128) on the matrix-core kernel.
    print(f"paged decode (matrix cores) {impl} {dtype} {case}", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(3)
    *contig, page_size = case
    q, k_cache, v_cache, seq_lens = make_case(tuple(contig), dtype, gen)
    cpu_gen = torch.Generator().manual_seed(4)
    k_pool, tables = to_paged(k_cache, page_size, cpu_gen)
    cpu_gen = torch.Generator().manual_seed(4)
    v_pool, _ = to_paged(v_cache, page_size, cpu_gen)
    out, lse = flash_lab.decode(q, k_pool, v_pool, seq_lens, block_tables=tables, impl=impl,
                                return_lse=True)
    check_decode(out, lse, q, k_cache, v_cache, seq_lens)


@pytest.mark.parametrize("route", ["auto", "vector"])
@pytest.mark.parametrize("num_splits", [1, 4, 32])
def test_paged_equals_contiguous_bitwise(num_splits, route, knobs):
    # Same keys in the same order per split: a paged cache must give the contiguous cache's bits,
    # on the matrix-core kernel (this group of 4 by default) and on the vector kernel.
    if route == "vector":
        knobs("decode_mfma_min_group", 1000)
    gen = torch.Generator(device="cuda").manual_seed(8)
    q, k_cache, v_cache, seq_lens = make_case((3, 32, 8, 3000, 128, [3000, 17, 2048]),
                                              torch.bfloat16, gen)
    cpu_gen = torch.Generator().manual_seed(9)
    k_pool, tables = to_paged(k_cache, 32, cpu_gen)
    cpu_gen = torch.Generator().manual_seed(9)
    v_pool, _ = to_paged(v_cache, 32, cpu_gen)
    want = flash_lab.decode(q, k_cache, v_cache, seq_lens, num_splits=num_splits, return_lse=True)
    got = flash_lab.decode(q, k_pool, v_pool, seq_lens, block_tables=tables,
                           num_splits=num_splits, return_lse=True)
    assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1])


def test_paged_block_numbers_outside_the_pool_are_clamped():
    # Table entries are device data the host never reads; out-of-range ones are clamped to the
    # pool instead of read out of bounds.
    gen = torch.Generator(device="cuda").manual_seed(10)
    q, k_cache, v_cache, seq_lens = make_case((2, 4, 4, 64, 64, [64, 40]), torch.float32, gen)
    pool = torch.randn(6, 16, 4, 64, device="cuda", generator=gen)
    bad = torch.tensor([[0, 99, -5, 2], [5, 1000000, 3, 4]], device="cuda", dtype=torch.int32)
    clamped = bad.clamp(0, 5)
    out = flash_lab.decode(q, pool, pool, seq_lens, block_tables=bad)
    want = flash_lab.decode(q, pool, pool, seq_lens, block_tables=clamped)
    assert torch.isfinite(out).all() and torch.equal(out, want)


def test_paged_decode_in_a_graph():
    # The paged step captures in a HIP graph like the contiguous one (no host reads).
    gen = torch.Generator(device="cuda").manual_seed(11)
    q, k_cache, v_cache, seq_lens = make_case((2, 16, 4, 1024, 128, [1024, 500]), torch.bfloat16, gen)
    cpu_gen = torch.Generator().manual_seed(12)
    k_pool, tables = to_paged(k_cache, 16, cpu_gen)
    cpu_gen = torch.Generator().manual_seed(12)
    v_pool, _ = to_paged(v_cache, 16, cpu_gen)
    eager = flash_lab.decode(q, k_pool, v_pool, seq_lens, block_tables=tables)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        flash_lab.decode(q, k_pool, v_pool, seq_lens, block_tables=tables)  # warm up off-graph
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = flash_lab.decode(q, k_pool, v_pool, seq_lens, block_tables=tables)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(captured, eager)
        eager_again = flash_lab.decode(q, k_pool, v_pool, seq_lens, block_tables=tables)
        torch.cuda.synchronize()
        assert torch.equal(eager_again, eager)


@pytest.mark.parametrize("impl", IMPLS)
def test_paged_splits_longer_than_the_staged_table(impl):
    # A split touching more than 1024 blocks (decode_inplace: one split; pages of one row) reads
    # the block numbers from the table in global memory instead of LDS (with one KV head per
    # workgroup, so the sums run in another order than the contiguous cache's): the reference
    # rule against the fp64 oracle.
    gen = torch.Generator(device="cuda").manual_seed(13)
    q, k_cache, v_cache, seq_lens = make_case((2, 8, 2, 3000, 64, [3000, 2100]), torch.bfloat16, gen)
    cpu_gen = torch.Generator().manual_seed(14)
    k_pool, tables = to_paged(k_cache, 1, cpu_gen)
    cpu_gen = torch.Generator().manual_seed(14)
    v_pool, _ = to_paged(v_cache, 1, cpu_gen)
    splits = 1 if impl == "decode_inplace" else 2
    out, lse = flash_lab.decode(q, k_pool, v_pool, seq_lens, block_tables=tables, impl=impl,
                                num_splits=splits, return_lse=True)
    check_decode(out, lse, q, k_cache, v_cache, seq_lens)


# The decode shapes of the reference's other benchmark suites (bench/suites.py:76-125): contexts
# of 512 to 8K keys for B in {1, 8} and H_kv in {32, 8} (decode_ctx; its 32K rows are above, plus
# B=1 GQA at 32K, the reference's weakest row, bench/results/h100-80gb-hbm3/summary-cc64b18.md:82),
# head_dim 64 with 8 KV heads (decode_d64), one sequence at 64K and 128K keys (decode_long) and
# batches up to 64 at 2K keys (decode_batch). bf16 caches fully valid, seeded like the benchmark;
# every sequence and head is checked in full against float64 (the oracle's C loops read the
# bf16 cache in place).
SUITE_SHAPES = sorted({
    *[(b, 32, hkv, ctx, 128) for b in (1, 8) for hkv in (32, 8) for ctx in (512, 2048, 8192)],
    (1, 32, 8, 32768, 128),
    *[(b, 32, 8, ctx, 64) for b in (1, 8) for ctx in (2048, 8192, 32768)],
    *[(1, 32, hkv, ctx, 128) for hkv in (32, 8) for ctx in (65536, 131072)],
    *[(b, 32, 8, 2048, 128) for b in (4, 16, 64)],
})


@pytest.mark.parametrize("shape", SUITE_SHAPES, ids=lambda s: f"B{s[0]}-H{s[1]}-Hkv{s[2]}-S{s[3]}-D{s[4]}")
def test_reference_suite_shapes(shape):
    batch, heads, heads_kv, context, head_dim = shape
    print(f"decode suite shape {shape}", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(0)
    q = torch.randn(batch, 1, heads, head_dim, device="cuda", dtype=torch.bfloat16, generator=gen)
    cache_shape = (batch, context, heads_kv, head_dim)
    k_cache = torch.randn(cache_shape, device="cuda", dtype=torch.bfloat16, generator=gen)
    v_cache = torch.randn(cache_shape, device="cuda", dtype=torch.bfloat16, generator=gen)
    seq_lens = torch.full((batch,), context, device="cuda", dtype=torch.int32)
    # The planned split count, and at 64K keys and more also the largest (128 splits of 512 or
    # 1024 keys), so the split arithmetic runs at the cap.
    counts = [None, 128] if context >= 65536 else [None]
    for num_splits in counts:
        out, lse = flash_lab.decode(q, k_cache, v_cache, seq_lens, num_splits=num_splits,
                                    return_lse=True)
        check_decode(out, lse, q, k_cache, v_cache, seq_lens, c_ref=True)


# The matrix-core kernel's four-KV-heads-per-workgroup layout (wave w takes KV head 4 q + w) is
# chosen on the host only for calls large enough to fill the CUs with long splits; the
# decode_mfma_span knob pins it on small shapes, so ragged and short lengths (a partial last tile,
# sequences shorter than a split, empty splits), fp16, head_dim 64, one split and paged caches run
# through it against the oracle.
SPAN4_CASES = [
    # batch, heads, heads_kv, max_seqlen, head_dim, seq_lens (heads_kv a multiple of 4)
    (8, 32, 8, 3000, 128, [3000, 1, 500, 1777, 2048, 31, 999, 2999]),
    (2, 64, 8, 2000, 64, [2000, 77]),  # head_dim 64, 8 query heads per KV head
    (3, 16, 4, 1500, 128, [1500, 700, 3]),
    (2, 128, 4, 600, 128, [600, 129]),  # 32 query heads per KV head
]


@pytest.fixture
def span4(knobs):
    knobs("decode_mfma_span", 4)


@pytest.mark.parametrize("num_splits", [None, 1, 2, 8, 64])
@pytest.mark.parametrize("dtype", DTYPES[:2], ids=lambda d: str(d).removeprefix("torch."))
@pytest.mark.parametrize("case", SPAN4_CASES, ids=lambda c: f"B{c[0]}-H{c[1]}-Hkv{c[2]}-S{c[3]}-D{c[4]}")
def test_four_kv_heads_per_workgroup(case, dtype, num_splits, span4):
    print(f"decode (four KV heads per workgroup) {dtype} {case} splits={num_splits}", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(20)
    q, k_cache, v_cache, seq_lens = make_case(case, dtype, gen)
    out, lse = flash_lab.decode(q, k_cache, v_cache, seq_lens, num_splits=num_splits,
                                return_lse=True)
    check_decode(out, lse, q, k_cache, v_cache, seq_lens)


def test_four_kv_heads_per_workgroup_empty_sequence(span4):
    # A sequence of length 0 gives zeros and -inf on every split; the others are unaffected.
    gen = torch.Generator(device="cuda").manual_seed(21)
    q, k_cache, v_cache, _ = make_case((3, 32, 8, 900, 128, [900, 900, 900]), torch.bfloat16, gen)
    lens = torch.tensor([900, 0, 450], device="cuda", dtype=torch.int32)
    for num_splits in (1, 4):
        out, lse = flash_lab.decode(q, k_cache, v_cache, lens, num_splits=num_splits,
                                    return_lse=True)
        assert torch.all(out[1] == 0) and torch.isneginf(lse[1]).all()
        keep = torch.tensor([0, 2], device="cuda")
        check_decode(out[keep], lse[keep], q[keep], k_cache[keep], v_cache[keep], lens[keep])


@pytest.mark.parametrize("num_splits", [1, 4, 32])
def test_four_kv_heads_per_workgroup_paged_equals_contiguous_bitwise(num_splits, span4):
    gen = torch.Generator(device="cuda").manual_seed(22)
    q, k_cache, v_cache, seq_lens = make_case((3, 32, 8, 3000, 128, [3000, 17, 2048]),
                                              torch.bfloat16, gen)
    cpu_gen = torch.Generator().manual_seed(23)
    k_pool, tables = to_paged(k_cache, 16, cpu_gen)
    cpu_gen = torch.Generator().manual_seed(23)
    v_pool, _ = to_paged(v_cache, 16, cpu_gen)
    want = flash_lab.decode(q, k_cache, v_cache, seq_lens, num_splits=num_splits, return_lse=True)
    got = flash_lab.decode(q, k_pool, v_pool, seq_lens, block_tables=tables,
                           num_splits=num_splits, return_lse=True)
    assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1])
    check_decode(want[0], want[1], q, k_cache, v_cache, seq_lens)


def test_inplace_large_batch_takes_four_kv_heads_per_workgroup():
    # decode_inplace (one split) with batch * H_kv = 2048: the default rule picks four KV heads
    # per workgroup (512 workgroups) here, with no knob.
    gen = torch.Generator(device="cuda").manual_seed(24)
    q, k_cache, v_cache, seq_lens = make_case((256, 32, 8, 300, 128, "random"), torch.bfloat16, gen)
    out, lse = flash_lab.decode(q, k_cache, v_cache, seq_lens, impl="decode_inplace",
                                return_lse=True)
    check_decode(out, lse, q, k_cache, v_cache, seq_lens)
