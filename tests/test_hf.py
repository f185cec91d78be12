"""flash_lab.hf.attention_forward, the transformers attention function, on synthetic tensors in
transformers' [B, H, S, D] layout (the reference's tests/test_hf.py:1-81). Unused cache rows hold
large values, so a kernel that read past the valid rows would show it in the output."""

import pytest
import torch

from flash_lab.hf import attention_forward
from oracle import reference


class Module(torch.nn.Module):
    is_causal = True


def hf_inputs(batch, seqlen_q, cache_len, heads, heads_kv, head_dim, device="cpu"):
    q = torch.randn(batch, heads, seqlen_q, head_dim, device=device, dtype=torch.bfloat16)
    k = 50 * torch.ones(batch, heads_kv, cache_len, head_dim, device=device, dtype=torch.bfloat16)
    v = 50 * torch.ones(batch, heads_kv, cache_len, head_dim, device=device, dtype=torch.bfloat16)
    return q, k, v


def test_rejects_what_it_cannot_run():
    q, k, v = hf_inputs(2, 4, 8, 4, 2, 64)
    positions = torch.arange(4).expand(2, 4)
    with pytest.raises(ValueError, match="dropout"):
        attention_forward(Module(), q, k, v, None, dropout=0.1, position_ids=positions)
    with pytest.raises(ValueError, match="position_ids"):
        attention_forward(Module(), q, k, v, None)
    with pytest.raises(NotImplementedError, match="sliding"):
        attention_forward(Module(), q, k, v, None, position_ids=positions, sliding_window=4)
    padded = torch.stack([torch.arange(4), torch.tensor([1, 1, 0, 1])])
    with pytest.raises(ValueError, match="unpadded"):
        attention_forward(Module(), q, k, v, None, position_ids=padded)
    with pytest.raises(ValueError, match="does not fit"):
        attention_forward(Module(), q, k, v, None, position_ids=positions + 5)


def test_register_with_transformers():
    transformers = pytest.importorskip("transformers")
    import flash_lab.hf

    name = flash_lab.hf.register()
    mapping = transformers.AttentionInterface._global_mapping
    assert "flash_lab" in mapping and name in mapping
    # transformers 5 reads any name containing "flash" as a flash-attention kernel to import, so
    # the function is reachable under "fl_lab" there; older versions take "flash_lab" itself.
    assert name == ("fl_lab" if flash_lab.hf.reserved_by_transformers("flash_lab") else "flash_lab")
    assert not flash_lab.hf.reserved_by_transformers(name)


@pytest.mark.gpu
@pytest.mark.parametrize("kernel", [None, 0, 1 << 30], ids=["auto", "pingpong", "wg128"])
@pytest.mark.parametrize("prefill_impl", ["auto", "mma_pipelined"])
def test_prefill_reads_only_the_valid_cache_rows(prefill_impl, kernel, knobs):
    # transformers' [B, H, S, D] cache arrives as transposed views, read in place by either kernel.
    knobs("prefill_pp_min_wg", kernel)
    q, k, v = hf_inputs(2, 77, 200, 8, 2, 128, device="cuda")
    k[:, :, :77].normal_()
    v[:, :, :77].normal_()
    positions = torch.arange(77, device="cuda").expand(2, 77)
    out, weights = attention_forward(
        Module(), q, k, v, None, scaling=0.1, position_ids=positions, prefill_impl=prefill_impl
    )
    assert weights is None
    ref = reference.attention(
        q.transpose(1, 2).cpu(),
        k[:, :, :77].transpose(1, 2).cpu(),
        v[:, :, :77].transpose(1, 2).cpu(),
        causal=True,
        softmax_scale=0.1,
    )
    assert out.shape == (2, 77, 8, 128)
    torch.testing.assert_close(out.cpu().double(), ref, atol=2e-2, rtol=0)


@pytest.mark.gpu
@pytest.mark.parametrize("decode_impl", ["splitkv", "decode_inplace"])
def test_decode_step_uses_position_ids_as_lengths(decode_impl):
    q, k, v = hf_inputs(3, 1, 300, 8, 2, 128, device="cuda")
    k[:, :, :251].normal_()
    v[:, :, :251].normal_()
    # One position per sequence (generate's layout), or one shared row (a plain forward call).
    for positions in (torch.full((3, 1), 250, device="cuda"), torch.tensor([[250]], device="cuda")):
        out, _ = attention_forward(
            Module(), q, k, v, None, scaling=0.1, position_ids=positions, decode_impl=decode_impl
        )
        ref = reference.attention(
            q.transpose(1, 2).cpu(),
            k[:, :, :251].transpose(1, 2).cpu(),
            v[:, :, :251].transpose(1, 2).cpu(),
            causal=True,
            softmax_scale=0.1,
        )
        assert out.shape == (3, 1, 8, 128)
        torch.testing.assert_close(out.cpu().double(), ref, atol=2e-2, rtol=0)


def test_sequence_ends_are_read_once_per_position_tensor():
    from flash_lab import hf

    positions = torch.arange(10).expand(2, 10).clone()
    assert hf._sequence_ends(positions) == {9}
    cached = hf._last_ends
    assert hf._sequence_ends(positions) == {9} and hf._last_ends is cached  # no second read
    positions[1, -1] = 12  # an in-place change is seen through the version counter
    assert hf._sequence_ends(positions) == {9, 12}
    other = torch.arange(5).expand(1, 5)  # another tensor is read afresh
    assert hf._sequence_ends(other) == {4}
