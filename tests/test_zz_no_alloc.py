"""fl_decode_noalloc, the decode entry point that allocates nothing (its split partials go to the
library's scratch array), against fl_decode with a torch-allocated workspace: bitwise equal
outputs for the same split count, on consecutive calls where the second is smaller than the first
(so stale partials of the first call would show), on both split kernels and a paged cache."""

import pytest
import torch

from flash_lab import _hip
import flash_lab

pytestmark = pytest.mark.gpu


def make(batch, heads, heads_kv, max_seqlen, head_dim, lens, seed):
    gen = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randn(batch, heads, head_dim, device="cuda", dtype=torch.bfloat16, generator=gen)
    shape = (batch, max_seqlen, heads_kv, head_dim)
    k = torch.randn(shape, device="cuda", dtype=torch.bfloat16, generator=gen)
    v = torch.randn(shape, device="cuda", dtype=torch.bfloat16, generator=gen)
    return q, k, v, torch.tensor(lens, device="cuda", dtype=torch.int32)


def noalloc(q, k, v, lens, num_splits, block_tables=None):
    o = torch.empty_like(q)
    lse = torch.empty(q.shape[:2], device="cuda", dtype=torch.float32)
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated()
    splits = _hip.decode_noalloc(q, k, v, lens, o, lse, q.shape[-1] ** -0.5, num_splits,
                                 block_tables)
    torch.cuda.synchronize()
    assert torch.cuda.memory_allocated() == before  # nothing from torch's allocator either
    return o, lse, splits


CASES = [
    # (batch, heads, heads_kv, max_seqlen, head_dim, lens, num_splits): a larger call, then a smaller
    ((4, 32, 8, 4096, 128, [4096, 100, 3000, 1], 16), (2, 8, 2, 1000, 128, [1000, 7], 4)),  # GQA 4
    ((2, 32, 32, 8192, 128, [8192, 5000], 0), (1, 4, 4, 700, 64, [700], 8)),  # MHA, planned count
]


@pytest.mark.parametrize("first,second", CASES, ids=["gqa", "mha"])
def test_noalloc_matches_fl_decode_on_consecutive_calls(first, second):
    for seed, (*shape, lens, num_splits) in enumerate((first, second)):
        print(f"noalloc decode {shape} lens={lens} splits={num_splits}", flush=True)
        q, k, v, seq_lens = make(*shape, lens, seed)
        o, lse, splits = noalloc(q, k, v, seq_lens, num_splits)
        want_o, want_lse = flash_lab.decode(q, k, v, seq_lens, num_splits=splits, return_lse=True)
        assert splits > 1
        assert torch.equal(o, want_o) and torch.equal(lse, want_lse)


def test_noalloc_paged_cache_and_one_split():
    q, k, v, seq_lens = make(3, 16, 4, 2048, 128, [2048, 33, 1500], 7)
    # The same cache as shuffled 16-row pages of a pool.
    gen = torch.Generator().manual_seed(3)
    per_seq = 2048 // 16
    order = torch.randperm(3 * per_seq, generator=gen).cuda()
    tables = order.view(3, per_seq).to(torch.int32)
    pools = []
    for cache in (k, v):
        pool = torch.empty((3 * per_seq, 16, 4, 128), device="cuda", dtype=torch.bfloat16)
        pool[order] = cache.reshape(3 * per_seq, 16, 4, 128)
        pools.append(pool)
    for num_splits in (8, 1):
        o, lse, splits = noalloc(q, *pools, seq_lens, num_splits, block_tables=tables)
        want_o, want_lse = flash_lab.decode(q, *pools, seq_lens, block_tables=tables,
                                            num_splits=splits, return_lse=True)
        assert splits == num_splits
        assert torch.equal(o, want_o) and torch.equal(lse, want_lse)


def test_noalloc_replays_in_a_graph():
    # The entry point for code under graph capture: a first call outside the capture (it looks
    # up the scratch array's address on this device), then a captured call, replayed after q and
    # seq_lens change in place; each replay must give fl_decode's bits at the same split count.
    q, k, v, seq_lens = make(2, 32, 8, 4096, 128, [4096, 1000], 30)
    o = torch.empty_like(q)
    lse = torch.empty(q.shape[:2], device="cuda", dtype=torch.float32)
    splits = _hip.decode_noalloc(q, k, v, seq_lens, o, lse, 128 ** -0.5, 16)
    assert splits == 16
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        _hip.decode_noalloc(q, k, v, seq_lens, o, lse, 128 ** -0.5, 16)
    gen = torch.Generator(device="cuda").manual_seed(31)
    for lens in ([4096, 1000], [17, 4096], [2048, 1]):
        q.copy_(torch.randn(q.shape, device="cuda", dtype=q.dtype, generator=gen))
        seq_lens.copy_(torch.tensor(lens, device="cuda", dtype=torch.int32))
        graph.replay()
        torch.cuda.synchronize()
        want_o, want_lse = flash_lab.decode(q, k, v, seq_lens, num_splits=16, return_lse=True)
        torch.cuda.synchronize()
        assert torch.equal(o, want_o) and torch.equal(lse, want_lse), lens
