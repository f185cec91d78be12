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

from oracle import c_oracle, reference

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


class PrefillOracle:
    """The oracle side of the prefill rule for one input: the fp64 output and LSE, PyTorch's own
    errors at the input dtype, and max |v|. Computed once, it can check several kernels' outputs
    for the same input. With `rows`, only those query rows (long sequences)."""

    def __init__(self, q, k, v, causal, scale=None, rows=None, c_ref=False):
        self.dtype = q.dtype
        self.shape = q.shape
        self.rows = rows
        qc, kc, vc = q.cpu(), k.cpu(), v.cpu()
        if rows is None:
            self.ref, self.ref_lse = reference.attention(qc, kc, vc, causal, scale, return_lse=True)
        elif c_ref:
            # The oracle's C loops (oracle_attention_rows_f64, pinned to attention_rows at 1e-12):
            # the same float64 rows without float64 copies of the long inputs.
            self.ref, self.ref_lse = c_oracle.attention_rows(qc, kc, vc, rows, causal, scale)
        else:
            self.ref, self.ref_lse = reference.attention_rows(
                qc, kc, vc, rows, causal, scale, return_lse=True
            )
        # The math backend returns nan for rows without visible keys; those rows are defined as 0.
        self.err_torch = (
            (sdpa_math(qc, kc, vc, causal, rows, scale).double() - self.ref)
            .nan_to_num(0.0).abs().max().item()
        )
        self.vmax = vc.abs().max().item()
        self.visible = torch.isfinite(self.ref_lse)
        self.lse_err_torch = None
        if self.visible.any():
            if rows is None:
                _, torch_lse = reference.attention(
                    qc, kc, vc, causal, scale, return_lse=True, dtype=self.dtype
                )
            else:
                _, torch_lse = reference.attention_rows(
                    qc, kc, vc, rows, causal, scale, dtype=self.dtype, return_lse=True
                )
            self.lse_err_torch = (torch_lse.double() - self.ref_lse)[self.visible].abs().max().item()

    def check(self, out, lse):
        """Asserts the prefill rule on a kernel's (out, lse); returns (err, err_torch)."""
        dtype = self.dtype
        assert out.shape == self.shape and out.dtype == dtype
        assert lse.shape == (self.shape[0], self.shape[2], self.shape[1]) and lse.dtype == torch.float32
        out_c, lse_c = out.cpu(), lse.cpu()
        if self.rows is None:
            got, got_lse = out_c, lse_c
        else:
            got, got_lse = out_c[:, self.rows], lse_c[:, :, self.rows]
        assert torch.isfinite(got).all()
        err = (got.double() - self.ref).abs().max().item()
        err_torch = self.err_torch
        assert err <= 2 * err_torch + FLOOR[dtype], f"max error {err:.3g}, torch math {err_torch:.3g}"
        assert err <= GUARD[dtype] * (1 + self.vmax), f"max error {err:.3g} above guard"

        visible = self.visible
        assert torch.equal(torch.isfinite(got_lse), visible)
        assert torch.isneginf(got_lse[~visible]).all()
        if visible.any():
            lse_err = (got_lse.double() - self.ref_lse)[visible].abs().max().item()
            assert lse_err <= 2 * self.lse_err_torch + LSE_FLOOR[dtype], (
                f"lse error {lse_err:.3g}, torch {self.lse_err_torch:.3g}"
            )
        return err, err_torch


def check_prefill(out, lse, q, k, v, causal, scale=None, rows=None, c_ref=False):
    """Asserts the prefill rule; with `rows`, on those query rows only (long sequences), the
    float64 side from the oracle's C loops when c_ref is set."""
    return PrefillOracle(q, k, v, causal, scale, rows, c_ref).check(out, lse)


def check_decode(out, lse, q, k_cache, v_cache, seq_lens, scale=None, c_ref=False):
    """Asserts the decode rule against the oracle's per-sequence decode on the CPU. With c_ref the
    float64 side comes from the oracle's C loops (oracle_decode_f64, pinned to the torch oracle
    at 1e-12), which read a long bf16 cache without float64 copies."""
    dtype = q.dtype
    args = (q.cpu(), k_cache.cpu(), v_cache.cpu(), seq_lens.cpu())
    if c_ref:
        ref, ref_lse = c_oracle.decode(*args, softmax_scale=scale)
    else:
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
