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
