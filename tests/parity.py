"""The parity rule of the reference (docs/numerics.md:33-71; tests/test_attention_fwd.py:18-99;
tests/test_decode.py:11-50), with every oracle-side computation on the CPU.

    err     = max |o - o_ref64|          err_torch     = max |o_torch - o_ref64|
    lse_err = max |lse - lse_ref64|      lse_err_torch = max |lse_torch - lse_ref64|  (finite rows)
    pass if err <= 2 * err_torch + FLOOR[dtype] and every output is finite,
            err <= GUARD[dtype] * (1 + max|v|)                      (prefill)
            lse_err <= 2 * lse_err_torch + LSE_FLOOR[dtype],
            lse is -inf exactly where lse_ref64 is                  (prefill)

o_torch is PyTorch's own computation at the input dtype: SDPA's math backend for prefill outputs,
the oracle's op sequence at the input dtype for LSEs and decode. It runs on CPU copies of the
inputs.
"""

import torch
import torch.nn.functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel

from oracle import reference

FLOOR = {torch.float32: 1e-6, torch.bfloat16: 1e-3, torch.float16: 1e-3}
GUARD = {torch.float32: 2e-5, torch.bfloat16: 2e-2, torch.float16: 1e-2}
LSE_FLOOR = {torch.float32: 1e-5, torch.bfloat16: 1e-3, torch.float16: 1e-3}


def sdpa_math(q, k, v, causal, rows=None, scale=None):
    """SDPA's math backend at the input dtype with the bottom-right causal mask and repeated KV
    heads, on the CPU; optionally for a subset of query rows."""
    q, k, v = q.cpu(), k.cpu(), v.cpu()
    group = q.shape[2] // k.shape[2]
    k = k.repeat_interleave(group, dim=2)
    v = v.repeat_interleave(group, dim=2)
    seqlen_q, seqlen_k = q.shape[1], k.shape[1]
    row_idx = torch.arange(seqlen_q) if rows is None else rows.cpu()
    mask = None
    if causal:
        cols = torch.arange(seqlen_k)[None, :]
        mask = cols <= row_idx[:, None] + (seqlen_k - seqlen_q)
    qs = q if rows is None else q[:, row_idx]
    with sdpa_kernel(SDPBackend.MATH):
        out = F.scaled_dot_product_attention(
            qs.transpose(1, 2).contiguous(),
            k.transpose(1, 2).contiguous(),
            v.transpose(1, 2).contiguous(),
            attn_mask=mask,
            scale=scale,
        )
    return out.transpose(1, 2)


def check_prefill(out, lse, q, k, v, causal, scale=None, rows=None):
    """Asserts the prefill rule; with `rows`, on those query rows only (long sequences)."""
    dtype = q.dtype
    qc, kc, vc = q.cpu(), k.cpu(), v.cpu()
    assert out.shape == q.shape and out.dtype == dtype
    assert lse.shape == (q.shape[0], q.shape[2], q.shape[1]) and lse.dtype == torch.float32
    out_c, lse_c = out.cpu(), lse.cpu()
    if rows is None:
        ref, ref_lse = reference.attention(qc, kc, vc, causal, scale, return_lse=True)
        got, got_lse = out_c, lse_c
    else:
        ref, ref_lse = reference.attention_rows(qc, kc, vc, rows, causal, scale, return_lse=True)
        got, got_lse = out_c[:, rows], lse_c[:, :, rows]
    assert torch.isfinite(got).all()

    err = (got.double() - ref).abs().max().item()
    # The math backend returns nan for rows without visible keys; those rows are defined as 0.
    err_torch = (
        (sdpa_math(qc, kc, vc, causal, rows, scale).double() - ref).nan_to_num(0.0).abs().max().item()
    )
    assert err <= 2 * err_torch + FLOOR[dtype], f"max error {err:.3g}, torch math {err_torch:.3g}"
    assert err <= GUARD[dtype] * (1 + vc.abs().max().item()), f"max error {err:.3g} above guard"

    visible = torch.isfinite(ref_lse)
    assert torch.equal(torch.isfinite(got_lse), visible)
    assert torch.isneginf(got_lse[~visible]).all()
    if visible.any():
        if rows is None:
            _, torch_lse = reference.attention(qc, kc, vc, causal, scale, return_lse=True, dtype=dtype)
        else:
            _, torch_lse = reference.attention_rows(
                qc, kc, vc, rows, causal, scale, dtype=dtype, return_lse=True
            )
        lse_err = (got_lse.double() - ref_lse)[visible].abs().max().item()
        lse_err_torch = (torch_lse.double() - ref_lse)[visible].abs().max().item()
        assert lse_err <= 2 * lse_err_torch + LSE_FLOOR[dtype], (
            f"lse error {lse_err:.3g}, torch {lse_err_torch:.3g}"
        )
    return err, err_torch


def check_decode(out, lse, q, k_cache, v_cache, seq_lens, scale=None):
    """Asserts the decode rule against the oracle's per-sequence decode on the CPU."""
    dtype = q.dtype
    args = (q.cpu(), k_cache.cpu(), v_cache.cpu(), seq_lens.cpu())
    ref, ref_lse = reference.decode(*args, softmax_scale=scale, return_lse=True)
    plain, plain_lse = reference.decode(*args, softmax_scale=scale, return_lse=True, dtype=dtype)
    out_c, lse_c = out.cpu(), lse.cpu()
    assert out.shape == q.shape and out.dtype == dtype and torch.isfinite(out_c).all()
    err = (out_c.double() - ref).abs().max().item()
    err_torch = (plain.double() - ref).abs().max().item()
    assert err <= 2 * err_torch + FLOOR[dtype], f"max error {err:.3g}, plain torch {err_torch:.3g}"
    lse_err = (lse_c.double() - ref_lse).abs().max().item()
    lse_err_torch = (plain_lse.double() - ref_lse).abs().max().item()
    assert lse_err <= 2 * lse_err_torch + LSE_FLOOR[dtype], f"lse error {lse_err:.3g}"
    return err, err_torch


def normwise_rel(x, ref) -> float:
    """max |x - ref| / max |ref|: the fp32 rule (1e-5) of the north star, immune to near-zero
    entries."""
    return ((x.double() - ref).abs().max() / ref.abs().max()).item()
