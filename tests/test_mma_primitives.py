"""MFMA fragment handling on one tile, before it is buried in the kernel (the role of the
reference's tests/test_mma_primitives.py:1-32). The tile op runs the prefill kernel's own
fragment code: the K-operand LDS read, the V-operand transpose read with its key permutation, the
P-operand packing, and the 32 x 32 accumulator layout."""

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("k", [16, 32, 64])
def test_tile_times_transposed_tile(flash_ops, k):
    # B given as [16, K] rows, like K in Q K^T.
    a = torch.randn(16, k, device="cuda", dtype=torch.bfloat16)
    b = torch.randn(16, k, device="cuda", dtype=torch.bfloat16)
    c = flash_ops.mma_tile_test(a, b, False)
    torch.testing.assert_close(c, a.float() @ b.float().T, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("k", [16, 32, 64])
def test_tile_times_tile_through_the_transpose_read(flash_ops, k):
    # B given as [K, 16] rows, like V in P V.
    a = torch.randn(16, k, device="cuda", dtype=torch.bfloat16)
    b = torch.randn(k, 16, device="cuda", dtype=torch.bfloat16)
    c = flash_ops.mma_tile_test(a, b, True)
    torch.testing.assert_close(c, a.float() @ b.float(), rtol=1e-5, atol=1e-5)


def test_fragment_positions_with_an_identity(flash_ops):
    # A = I picks rows of B, so any lane, register or key-order mix-up shows as a permutation.
    a = torch.eye(16, device="cuda", dtype=torch.bfloat16)
    b = torch.arange(256, device="cuda", dtype=torch.float32).view(16, 16).to(torch.bfloat16)
    torch.testing.assert_close(flash_ops.mma_tile_test(a, b, True), b.float())
    torch.testing.assert_close(flash_ops.mma_tile_test(a, b, False), b.float().T)


def test_key_order_over_64_keys(flash_ops):
    # One-hot rows of A select single keys among 64, covering both 32-key blocks of the
    # accumulator and all four 16-key MFMA steps of the transpose-read path.
    keys = torch.tensor([0, 3, 4, 7, 8, 12, 15, 16, 21, 31, 32, 37, 44, 48, 58, 63])
    a = torch.zeros(16, 64, device="cuda", dtype=torch.bfloat16)
    a[torch.arange(16), keys] = 1
    b = (torch.arange(64 * 16, dtype=torch.float32) % 251).view(64, 16).to(torch.bfloat16).cuda()
    torch.testing.assert_close(flash_ops.mma_tile_test(a, b, True), b.float()[keys])


@pytest.mark.parametrize("lds_a", [False, True], ids=["registers", "lds"])
def test_rate_probe_runs(lds_a):
    # The calibration kernel behind bench.py's `mfma` leg, from its own library (not the product
    # one): zero operands give exact zeros, random ones finite sums, the same on every call.
    import calib

    lib = calib.load()
    flags = calib.PROBE_LDS_A if lds_a else 0
    out = torch.full((8 * 512,), float("nan"), device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    assert lib.flc_mfma_rate_probe(out.data_ptr(), 8, 3, flags | calib.PROBE_ZERO_OPERANDS, stream) == 0
    torch.cuda.synchronize()
    assert (out == 0).all()
    assert lib.flc_mfma_rate_probe(out.data_ptr(), 8, 3, flags, stream) == 0
    first = out.clone()
    assert lib.flc_mfma_rate_probe(out.data_ptr(), 8, 3, flags, stream) == 0
    torch.cuda.synchronize()
    assert torch.isfinite(first).all() and (first != 0).any()
    assert torch.equal(first, out)
