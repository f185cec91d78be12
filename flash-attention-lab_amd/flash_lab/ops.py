"""Public entry points: flash_lab.attention, flash_lab.decode, flash_lab.available_impls.

Same API, selection rules and errors as the reference's flash_lab/ops.py:1-226. Each call
validates its inputs, picks an implementation from the tables below (impl="auto" takes the first
built entry that supports the input), and calls torch.ops.flash_lab.<op>. The ops are the gfx950
HIP kernels registered by flash_lab._hip; impl names the reference also ships as other kernels
(Triton, the fp32 CUDA-core progression, the copy-based decode baseline) are kept in the tables so
that code naming them gets a clear "not available in this build" error instead of "unknown impl".
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from flash_lab.layouts import AttnShape, DecodeShape, check_attention_inputs, check_decode_inputs

try:
    from flash_lab import _hip  # noqa: F401  (loading the library registers the ops)
except ImportError as exc:
    HAS_EXTENSION = False
    EXTENSION_ERROR = str(exc)
else:
    HAS_EXTENSION = True
    EXTENSION_ERROR = ""


@dataclass(frozen=True)
class PrefillImpl:
    """One prefill kernel and what it supports (reference flash_lab/ops.py:33-50)."""

    op: str
    dtypes: tuple[torch.dtype, ...]
    head_dims: tuple[int, ...]
    gqa: bool = True
    causal_unequal_lengths: bool = True  # causal with S_q != S_k, bottom-right aligned

    def unsupported_reason(self, shape: AttnShape, dtype: torch.dtype, causal: bool) -> str | None:
        if dtype not in self.dtypes:
            return f"dtype {dtype} is not one of {self.dtypes}"
        if shape.head_dim not in self.head_dims:
            return f"head_dim {shape.head_dim} is not one of {self.head_dims}"
        if shape.group > 1 and not self.gqa:
            return "grouped-query attention (H_kv < H) is not supported"
        if causal and shape.seqlen_q != shape.seqlen_k and not self.causal_unequal_lengths:
            return "causal attention requires S_q == S_k"
        return None


@dataclass(frozen=True)
class DecodeImpl:
    """One decode kernel and what it supports (reference flash_lab/ops.py:53-68)."""

    op: str
    dtypes: tuple[torch.dtype, ...]
    head_dims: tuple[int, ...]
    paged_op: str | None = None  # the op serving paged caches (None: paged caches unsupported)
    in_auto: bool = True  # False for baselines kept for comparison only

    @property
    def paged(self) -> bool:
        return self.paged_op is not None

    def unsupported_reason(self, shape: DecodeShape, dtype: torch.dtype) -> str | None:
        if dtype not in self.dtypes:
            return f"dtype {dtype} is not one of {self.dtypes}"
        if shape.head_dim not in self.head_dims:
            return f"head_dim {shape.head_dim} is not one of {self.head_dims}"
        if shape.paged and not self.paged:
            return "paged KV caches are not supported"
        return None


_HALF = (torch.bfloat16, torch.float16)
_FP32 = (torch.float32,)
_DIMS = (64, 128)

# In order of preference. The gfx950 MFMA kernel serves both tensor-core names of the reference.
PREFILL_IMPLS: dict[str, PrefillImpl] = {
    "mma_pipelined": PrefillImpl(op="attention_mma_pipelined", dtypes=_HALF, head_dims=_DIMS),
    "mma": PrefillImpl(op="attention_mma", dtypes=_HALF, head_dims=_DIMS),
    # Reference kernels that this build does not ship (Triton, fp32 CUDA-core progression).
    "triton": PrefillImpl(op="attention_triton", dtypes=_HALF, head_dims=_DIMS),
    "fp32_regtile": PrefillImpl(op="attention_fp32_regtile", dtypes=_FP32, head_dims=_DIMS),
    "fp32_fused": PrefillImpl(op="attention_fp32_fused", dtypes=_FP32, head_dims=_DIMS),
    "naive": PrefillImpl(op="attention_naive", dtypes=_FP32, head_dims=_DIMS),
}
_DECODE_DTYPES = (torch.bfloat16, torch.float16, torch.float32)
DECODE_IMPLS: dict[str, DecodeImpl] = {
    "splitkv": DecodeImpl(
        op="decode_splitkv", dtypes=_DECODE_DTYPES, head_dims=_DIMS, paged_op="decode_splitkv_paged"
    ),
    "decode_inplace": DecodeImpl(
        op="decode_inplace", dtypes=_DECODE_DTYPES, head_dims=_DIMS, paged_op="decode_inplace_paged"
    ),
    # The reference's copy-based baseline; not shipped by this build.
    "decode_copy": DecodeImpl(
        op="decode_copy", dtypes=_DECODE_DTYPES, head_dims=_DIMS, in_auto=False
    ),
}


def _op_exists(op: str) -> bool:
    return hasattr(torch.ops.flash_lab, op)


def _register_fakes() -> None:
    """Shape-only versions of the ops, so torch.compile can trace through them
    (reference flash_lab/ops.py:100-118)."""

    def prefill_fake(q, k, v, causal, softmax_scale):
        batch, seqlen_q, heads, _ = q.shape
        return q.new_empty(q.shape), q.new_empty((batch, heads, seqlen_q), dtype=torch.float32)

    def decode_fake(q, k_cache, v_cache, seq_lens, softmax_scale, num_splits):
        return q.new_empty(q.shape), q.new_empty(q.shape[:2], dtype=torch.float32)

    def paged_decode_fake(q, k_cache, v_cache, seq_lens, block_tables, softmax_scale, num_splits):
        return q.new_empty(q.shape), q.new_empty(q.shape[:2], dtype=torch.float32)

    for spec in PREFILL_IMPLS.values():
        if _op_exists(spec.op):
            torch.library.register_fake(f"flash_lab::{spec.op}")(prefill_fake)
    for spec in DECODE_IMPLS.values():
        if _op_exists(spec.op):
            torch.library.register_fake(f"flash_lab::{spec.op}")(decode_fake)
        if spec.paged_op and _op_exists(spec.paged_op):
            torch.library.register_fake(f"flash_lab::{spec.paged_op}")(paged_decode_fake)


if HAS_EXTENSION:
    _register_fakes()

# All ops are registered by the import above, so availability is looked up once.
_BUILT_OPS = frozenset(
    op
    for spec in (*PREFILL_IMPLS.values(), *DECODE_IMPLS.values())
    for op in (spec.op, getattr(spec, "paged_op", None))
    if op and HAS_EXTENSION and _op_exists(op)
)


def available_impls() -> dict[str, list[str]]:
    """Implementations compiled into this build, by entry point."""
    return {
        "attention": [name for name, spec in PREFILL_IMPLS.items() if spec.op in _BUILT_OPS],
        "decode": [name for name, spec in DECODE_IMPLS.items() if spec.op in _BUILT_OPS],
    }


def _select(table: dict, impl: str, device: torch.device, describe, reason_of):
    """The implementation to run (reference flash_lab/ops.py:139-159). describe() names the
    problem in error messages and is only called on failure."""
    if impl != "auto" and impl not in table:
        raise ValueError(f"unknown impl {impl!r}; choose from {['auto', *table]}")
    if device.type != "cuda":
        raise ValueError(f"flash_lab kernels take CUDA tensors, got device {device}")
    missing = "" if HAS_EXTENSION else f" (the HIP extension did not load: {EXTENSION_ERROR})"
    if impl != "auto":
        spec = table[impl]
        reason = reason_of(spec)
        if reason is not None:
            raise ValueError(f"impl {impl!r} cannot run {describe()}: {reason}")
        if spec.op not in _BUILT_OPS:
            raise RuntimeError(f"impl {impl!r} is not available in this build{missing}")
        return spec
    candidates = [s for s in table.values() if getattr(s, "in_auto", True) and s.op in _BUILT_OPS]
    for spec in candidates:
        if reason_of(spec) is None:
            return spec
    raise ValueError(f"no available implementation supports {describe()}{missing}")


def attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    causal: bool = False,
    softmax_scale: float | None = None,
    impl: str = "auto",
    return_lse: bool = False,
):
    """Attention forward. q is [B, S_q, H, D]; k and v are [B, S_k, H_kv, D] with H % H_kv == 0.

    Returns o [B, S_q, H, D] in the input dtype and, with return_lse=True, the natural-log
    log-sum-exp of each score row as fp32 [B, H, S_q]. Causal masking with S_q != S_k is aligned
    to the bottom-right corner: query i sees key j iff j <= i + (S_k - S_q).
    """
    shape = check_attention_inputs(q, k, v)
    scale = 1.0 / math.sqrt(shape.head_dim) if softmax_scale is None else softmax_scale
    if not scale > 0:
        raise ValueError(f"softmax_scale must be positive, got {scale}")
    spec = _select(
        PREFILL_IMPLS,
        impl,
        q.device,
        lambda: (
            f"dtype={q.dtype}, head_dim={shape.head_dim}, heads={shape.heads}/{shape.heads_kv}, "
            f"S_q={shape.seqlen_q}, S_k={shape.seqlen_k}, causal={causal}"
        ),
        lambda s: s.unsupported_reason(shape, q.dtype, causal),
    )
    out, lse = getattr(torch.ops.flash_lab, spec.op)(q, k, v, causal, scale)
    return (out, lse) if return_lse else out


def decode(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    seq_lens: torch.Tensor,
    block_tables: torch.Tensor | None = None,
    softmax_scale: float | None = None,
    impl: str = "auto",
    num_splits: int | None = None,
    return_lse: bool = False,
):
    """One decode step: each sequence's single query token attends to its first seq_lens[b] keys.

    The cache is [B, S_max, H_kv, D], or [num_blocks, page_size, H_kv, D] with block_tables.
    seq_lens values are not checked on the host (that would force a device sync).
    num_splits=None lets the library choose how many workgroups share one sequence's keys.
    """
    q3, shape = check_decode_inputs(q, k_cache, v_cache, seq_lens, block_tables)
    scale = 1.0 / math.sqrt(shape.head_dim) if softmax_scale is None else softmax_scale
    if num_splits is not None and num_splits < 1:
        raise ValueError(f"num_splits must be positive, got {num_splits}")
    spec = _select(
        DECODE_IMPLS,
        impl,
        q.device,
        lambda: (
            f"dtype={q.dtype}, head_dim={shape.head_dim}, heads={shape.heads}/{shape.heads_kv}, "
            f"paged={shape.paged}"
        ),
        lambda s: s.unsupported_reason(shape, q.dtype),
    )
    if block_tables is not None:
        out, lse = getattr(torch.ops.flash_lab, spec.paged_op)(
            q3, k_cache, v_cache, seq_lens, block_tables, scale, num_splits or 0
        )
    else:
        out, lse = getattr(torch.ops.flash_lab, spec.op)(
            q3, k_cache, v_cache, seq_lens, scale, num_splits or 0
        )
    if q.dim() == 4:
        out = out.unsqueeze(1)
    return (out, lse) if return_lse else out
