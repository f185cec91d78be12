"""The ops trace under torch.compile with fullgraph=True, i.e. without graph breaks (the
reference's tests/test_torch_compile.py:1-52), and the decode step replays inside a HIP graph."""

import pytest
import torch

import flash_lab

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("impl", ["mma_pipelined", "mma"])
def test_attention_compiles_without_graph_breaks(impl):
    torch._dynamo.reset()

    def block(q, k, v):
        out, lse = flash_lab.attention(q, k, v, causal=True, impl=impl, return_lse=True)
        return out * 2 + 1, lse.exp()

    q = torch.randn(2, 96, 4, 64, device="cuda", dtype=torch.bfloat16)
    k = torch.randn(2, 96, 2, 64, device="cuda", dtype=torch.bfloat16)
    v = torch.randn(2, 96, 2, 64, device="cuda", dtype=torch.bfloat16)
    compiled = torch.compile(block, fullgraph=True)
    for got, want in zip(compiled(q, k, v), block(q, k, v), strict=True):
        torch.testing.assert_close(got, want)


@pytest.mark.parametrize("impl", ["decode_inplace", "splitkv"])
def test_decode_compiles_without_graph_breaks(impl):
    torch._dynamo.reset()

    def step(q, k_cache, v_cache, seq_lens):
        return flash_lab.decode(q, k_cache, v_cache, seq_lens, impl=impl) * 2

    q = torch.randn(3, 1, 8, 128, device="cuda", dtype=torch.bfloat16)
    k_cache = torch.randn(3, 500, 2, 128, device="cuda", dtype=torch.bfloat16)
    v_cache = torch.randn(3, 500, 2, 128, device="cuda", dtype=torch.bfloat16)
    seq_lens = torch.tensor([500, 7, 260], device="cuda", dtype=torch.int32)
    compiled = torch.compile(step, fullgraph=True)
    torch.testing.assert_close(
        compiled(q, k_cache, v_cache, seq_lens), step(q, k_cache, v_cache, seq_lens)
    )


def test_paged_decode_compiles_without_graph_breaks():
    torch._dynamo.reset()

    def step(q, k_pool, v_pool, seq_lens, tables):
        return flash_lab.decode(q, k_pool, v_pool, seq_lens, block_tables=tables) * 2

    q = torch.randn(2, 1, 8, 128, device="cuda", dtype=torch.bfloat16)
    k_pool = torch.randn(40, 16, 2, 128, device="cuda", dtype=torch.bfloat16)
    v_pool = torch.randn(40, 16, 2, 128, device="cuda", dtype=torch.bfloat16)
    tables = torch.randperm(40, device="cuda")[:32].view(2, 16).to(torch.int32)
    seq_lens = torch.tensor([256, 77], device="cuda", dtype=torch.int32)
    compiled = torch.compile(step, fullgraph=True)
    torch.testing.assert_close(
        compiled(q, k_pool, v_pool, seq_lens, tables), step(q, k_pool, v_pool, seq_lens, tables)
    )


def test_decode_replays_in_a_hip_graph():
    # generate() captures the decode step; the op allocates its outputs and workspace from the
    # caching allocator and launches on the current stream, so it can be captured. Each replay is
    # checked against the eager result, with eager work and syncs in between.
    q = torch.randn(2, 1, 8, 128, device="cuda", dtype=torch.bfloat16)
    k_cache = torch.randn(2, 3000, 2, 128, device="cuda", dtype=torch.bfloat16)
    v_cache = torch.randn(2, 3000, 2, 128, device="cuda", dtype=torch.bfloat16)
    seq_lens = torch.tensor([3000, 1200], device="cuda", dtype=torch.int32)
    eager = flash_lab.decode(q, k_cache, v_cache, seq_lens, num_splits=8)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        flash_lab.decode(q, k_cache, v_cache, seq_lens, num_splits=8)  # warm the allocator
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = flash_lab.decode(q, k_cache, v_cache, seq_lens, num_splits=8)
    for _ in range(3):
        captured.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(captured, eager)
        _ = (q.float() * 2).sum().item()  # eager work between replays
