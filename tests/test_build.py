"""The library built for this GPU loads, and op registration works (the reference's
tests/test_build.py:1-17)."""

from pathlib import Path

import pytest
import torch

pytestmark = pytest.mark.gpu


def test_extension_registers_ops(flash_ops):
    for op in ("smoke_axpy", "mma_tile_test", "attention_mma_pipelined", "decode_splitkv"):
        assert hasattr(flash_ops, op)


@pytest.mark.parametrize("n", [1, 1000, 1 << 20])
def test_smoke_kernel(flash_ops, n):
    x = torch.randn(n, device="cuda")
    y = torch.randn(n, device="cuda")
    torch.testing.assert_close(flash_ops.smoke_axpy(x, y, 2.5), 2.5 * x + y)


def test_native_library_is_the_one_loaded(flash_ops):
    # The HIP kernels come from the in-tree library, mapped into this process.
    from flash_lab import _hip

    maps = Path("/proc/self/maps").read_text()
    assert str(_hip.LIB_PATH.resolve()) in maps
