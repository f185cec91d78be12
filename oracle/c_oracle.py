"""ctypes access to the C restatement of the oracle (oracle/attn_ref.c). Test infrastructure only."""

from __future__ import annotations

import ctypes
import math

import numpy as np
import torch

from oracle.build import OUTPUT, build

_LIB = None


def _lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not OUTPUT.exists():
            build()
        lib = ctypes.CDLL(str(OUTPUT))
        lib.oracle_attention_f64.restype = ctypes.c_int
        lib.oracle_attention_f64.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_int] * 7 + [
            ctypes.c_double
        ]
        lib.oracle_decode_f64.restype = ctypes.c_int
        lib.oracle_attention_rows_f64.restype = ctypes.c_int
        lib.oracle_attention_rows_f64.argtypes = [ctypes.c_void_p] * 6 + [ctypes.c_int] * 9 + [
            ctypes.c_double
        ]
        lib.oracle_decode_f64.argtypes = [ctypes.c_void_p] * 6 + [ctypes.c_int] * 6 + [
            ctypes.c_double
        ]
        _LIB = lib
    return _LIB


def attention(q, k, v, causal=False, softmax_scale=None):
    """(o [B, S_q, H, D], lse [B, H, S_q]) in float64 from the C loops."""
    qn = np.ascontiguousarray(q.detach().cpu().double().numpy())
    kn = np.ascontiguousarray(k.detach().cpu().double().numpy())
    vn = np.ascontiguousarray(v.detach().cpu().double().numpy())
    batch, seqlen_q, heads, head_dim = qn.shape
    seqlen_k, heads_kv = kn.shape[1], kn.shape[2]
    scale = 1.0 / math.sqrt(head_dim) if softmax_scale is None else softmax_scale
    o = np.zeros_like(qn)
    lse = np.zeros((batch, heads, seqlen_q), dtype=np.float64)
    rc = _lib().oracle_attention_f64(
        qn.ctypes.data, kn.ctypes.data, vn.ctypes.data, o.ctypes.data, lse.ctypes.data,
        batch, seqlen_q, seqlen_k, heads, heads_kv, head_dim, int(bool(causal)), float(scale),
    )
    if rc != 0:
        raise ValueError(f"oracle_attention_f64 rejected the shape (code {rc})")
    return torch.from_numpy(o), torch.from_numpy(lse)


def decode(q, k_cache, v_cache, seq_lens, softmax_scale=None):
    """(o, lse) in float64 of a decode step from the C loops: q [B, 1, H, D] or [B, H, D]
    (o has q's rank), contiguous caches [B, S_max, H_kv, D] in bf16 or fp32, int32 seq_lens [B].
    Reads the caches in their own dtype (no float64 copies), so it fits long caches."""
    if k_cache.dtype not in (torch.bfloat16, torch.float32) or v_cache.dtype != k_cache.dtype:
        raise TypeError("the C decode oracle reads bf16 or fp32 caches")
    elem = 0 if k_cache.dtype == torch.bfloat16 else 2
    q3 = q.reshape(q.shape[0], q.shape[-2], q.shape[-1]) if q.dim() == 4 else q
    qc = q3.detach().cpu().to(k_cache.dtype).contiguous()
    kc = k_cache.detach().cpu().contiguous()
    vc = v_cache.detach().cpu().contiguous()
    lens = seq_lens.detach().cpu().to(torch.int32).contiguous()
    batch, heads, head_dim = qc.shape
    max_seqlen, heads_kv = kc.shape[1], kc.shape[2]
    scale = 1.0 / math.sqrt(head_dim) if softmax_scale is None else softmax_scale
    o = torch.zeros(batch, heads, head_dim, dtype=torch.float64)
    lse = torch.zeros(batch, heads, dtype=torch.float64)
    rc = _lib().oracle_decode_f64(
        qc.data_ptr(), kc.data_ptr(), vc.data_ptr(), lens.data_ptr(), o.data_ptr(), lse.data_ptr(),
        batch, heads, heads_kv, max_seqlen, head_dim, elem, float(scale),
    )
    if rc != 0:
        raise ValueError(f"oracle_decode_f64 rejected the input (code {rc})")
    return (o.unsqueeze(1) if q.dim() == 4 else o), lse


def attention_rows(q, k, v, rows, causal=False, softmax_scale=None):
    """(o [B, len(rows), H, D], lse [B, H, len(rows)]) in float64 from the C loops, for the listed
    query rows (each keeps its position in the full sequence for the causal mask). Reads bf16 or
    fp32 inputs in place."""
    if q.dtype not in (torch.bfloat16, torch.float32) or k.dtype != q.dtype or v.dtype != q.dtype:
        raise TypeError("the C rows oracle reads bf16 or fp32 inputs")
    elem = 0 if q.dtype == torch.bfloat16 else 2
    qc, kc, vc = (x.detach().cpu().contiguous() for x in (q, k, v))
    rows_c = torch.as_tensor(rows).detach().cpu().to(torch.int64).contiguous()
    batch, seqlen_q, heads, head_dim = qc.shape
    seqlen_k, heads_kv = kc.shape[1], kc.shape[2]
    n = rows_c.numel()
    scale = 1.0 / math.sqrt(head_dim) if softmax_scale is None else softmax_scale
    o = torch.zeros(batch, n, heads, head_dim, dtype=torch.float64)
    lse = torch.zeros(batch, heads, n, dtype=torch.float64)
    rc = _lib().oracle_attention_rows_f64(
        qc.data_ptr(), kc.data_ptr(), vc.data_ptr(), rows_c.data_ptr(), o.data_ptr(),
        lse.data_ptr(), batch, seqlen_q, seqlen_k, heads, heads_kv, head_dim, n, int(bool(causal)),
        elem, float(scale),
    )
    if rc != 0:
        raise ValueError(f"oracle_attention_rows_f64 rejected the input (code {rc})")
    return o, lse
