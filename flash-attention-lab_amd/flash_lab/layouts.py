"""Input validation shared by the public API (flash_lab.ops) and the test oracle.

Same contract as the reference's flash_lab/layouts.py:1-167 (its tests match these messages):
prefill tensors are [B, S, H, D] (batch, sequence, heads, head_dim); K and V may have fewer heads
than Q, query head h reading KV head h // (H // H_kv). Decode takes q [B, 1, H, D] or [B, H, D]
and a [B, S_max, H_kv, D] cache, or a paged [num_blocks, page_size, H_kv, D] pool with
block_tables [B, max_blocks]. Errors are raised before any kernel runs.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class AttnShape:
    """Problem size of one prefill call (reference flash_lab/layouts.py:12-23)."""

    batch: int
    seqlen_q: int
    seqlen_k: int
    heads: int
    heads_kv: int
    head_dim: int

    @property
    def group(self) -> int:
        return self.heads // self.heads_kv


@dataclass(frozen=True)
class DecodeShape:
    """Problem size of one decode call (reference flash_lab/layouts.py:26-41). max_seqlen is S_max
    of a contiguous cache, or max_blocks * page_size of a paged one; page_size is 0 when the cache
    is contiguous."""

    batch: int
    heads: int
    heads_kv: int
    head_dim: int
    max_seqlen: int
    page_size: int

    @property
    def group(self) -> int:
        return self.heads // self.heads_kv

    @property
    def paged(self) -> bool:
        return self.page_size > 0


def _shape(x: torch.Tensor) -> tuple:
    return tuple(x.shape)


def _tensor_or_raise(name: str, x: object) -> None:
    if not isinstance(x, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor, got {type(x).__name__}")


def _heads_divide(heads: int, heads_kv: int) -> None:
    if heads_kv <= 0 or heads % heads_kv:
        raise ValueError(
            f"the number of query heads ({heads}) must be a multiple of KV heads ({heads_kv})"
        )


def _unit_stride_in_d(tensors: dict[str, torch.Tensor]) -> None:
    for name, x in tensors.items():
        if x.stride(-1) != 1:
            raise ValueError(
                f"{name} must be contiguous in its last dimension, got strides {tuple(x.stride())}"
            )


def check_attention_inputs(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, require_unit_stride: bool = True
) -> AttnShape:
    """Validates prefill inputs (reference flash_lab/layouts.py:64-92) and returns their shape."""
    tensors = {"q": q, "k": k, "v": v}
    for name, x in tensors.items():
        _tensor_or_raise(name, x)
        if x.dim() != 4:
            raise ValueError(f"{name} must be 4-D [B, S, H, D], got shape {_shape(x)}")
    if q.dtype != k.dtype or q.dtype != v.dtype:
        raise TypeError(f"q, k, v must share a dtype, got {q.dtype}, {k.dtype}, {v.dtype}")
    if q.device != k.device or q.device != v.device:
        raise ValueError(f"q, k, v must be on one device, got {q.device}, {k.device}, {v.device}")
    if k.shape != v.shape:
        raise ValueError(f"k and v must have the same shape, got {_shape(k)} and {_shape(v)}")

    batch, seqlen_q, heads, head_dim = q.shape
    kv_batch, seqlen_k, heads_kv, kv_head_dim = k.shape
    if kv_batch != batch:
        raise ValueError(f"batch size mismatch: q has {batch}, k and v have {kv_batch}")
    if kv_head_dim != head_dim:
        raise ValueError(f"head_dim mismatch: q has {head_dim}, k and v have {kv_head_dim}")
    if 0 in (batch, seqlen_q, seqlen_k, heads, head_dim):
        raise ValueError(f"empty input: q {_shape(q)}, k {_shape(k)}")
    _heads_divide(heads, heads_kv)
    if require_unit_stride:
        _unit_stride_in_d(tensors)
    return AttnShape(batch, seqlen_q, seqlen_k, heads, heads_kv, head_dim)


def check_decode_inputs(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    seq_lens: torch.Tensor,
    block_tables: torch.Tensor | None = None,
    *,
    require_unit_stride: bool = True,
) -> tuple[torch.Tensor, DecodeShape]:
    """Validates decode inputs (reference flash_lab/layouts.py:95-167). Returns q as a [B, H, D]
    view and the problem shape. seq_lens [B] int32 counts each sequence's valid keys, the token
    being decoded included; its values stay on the device and are not checked here."""
    tensors = {"q": q, "k_cache": k_cache, "v_cache": v_cache, "seq_lens": seq_lens}
    if block_tables is not None:
        tensors["block_tables"] = block_tables
    for name, x in tensors.items():
        _tensor_or_raise(name, x)
    devices = {str(x.device) for x in tensors.values()}
    if len(devices) != 1:
        where = {name: str(x.device) for name, x in tensors.items()}
        raise ValueError(f"decode inputs must be on one device, got {where}")

    if q.dim() == 4:
        if q.shape[1] != 1:
            raise ValueError(f"decode takes one query token per sequence, got q {_shape(q)}")
        q = q.select(1, 0)
    elif q.dim() != 3:
        raise ValueError(f"q must be [B, 1, H, D] or [B, H, D], got shape {_shape(q)}")
    if k_cache.dim() != 4:
        raise ValueError(f"k_cache must be 4-D, got shape {_shape(k_cache)}")
    if k_cache.shape != v_cache.shape:
        raise ValueError(
            "k_cache and v_cache must have the same shape, "
            f"got {_shape(k_cache)} and {_shape(v_cache)}"
        )
    if q.dtype != k_cache.dtype or q.dtype != v_cache.dtype:
        raise TypeError(
            f"q and the caches must share a dtype, got {q.dtype}, {k_cache.dtype}, {v_cache.dtype}"
        )

    batch, heads, head_dim = q.shape
    if seq_lens.dtype != torch.int32:
        raise TypeError(f"seq_lens must be int32, got {seq_lens.dtype}")
    if _shape(seq_lens) != (batch,):
        raise ValueError(f"seq_lens must have shape ({batch},), got {_shape(seq_lens)}")
    if not seq_lens.is_contiguous():
        raise ValueError(f"seq_lens must be contiguous, got stride {seq_lens.stride()}")

    if block_tables is None:
        cache_batch, max_seqlen, heads_kv, cache_head_dim = k_cache.shape
        page_size = 0
        if cache_batch != batch:
            raise ValueError(f"batch size mismatch: q has {batch}, the cache has {cache_batch}")
    else:
        if block_tables.dtype != torch.int32:
            raise TypeError(f"block_tables must be int32, got {block_tables.dtype}")
        if block_tables.dim() != 2 or block_tables.shape[0] != batch:
            raise ValueError(
                f"block_tables must be [{batch}, max_blocks], got {_shape(block_tables)}"
            )
        _, page_size, heads_kv, cache_head_dim = k_cache.shape
        max_seqlen = block_tables.shape[1] * page_size

    if cache_head_dim != head_dim:
        raise ValueError(f"head_dim mismatch: q has {head_dim}, the cache has {cache_head_dim}")
    if 0 in (batch, heads, head_dim, max_seqlen):
        raise ValueError(f"empty input: q {_shape(q)}, k_cache {_shape(k_cache)}")
    _heads_divide(heads, heads_kv)
    if require_unit_stride:
        _unit_stride_in_d({"q": q, "k_cache": k_cache, "v_cache": v_cache})
    return q, DecodeShape(batch, heads, heads_kv, head_dim, max_seqlen, page_size)
