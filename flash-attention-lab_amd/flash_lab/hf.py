"""Hugging Face transformers integration: attn_implementation="flash_lab".

    import flash_lab.hf
    name = flash_lab.hf.register()   # "flash_lab", or "fl_lab" under transformers 5
    model = AutoModelForCausalLM.from_config(config, attn_implementation=name)

Same behaviour as the reference's flash_lab/hf.py:1-88. A forward with several query tokens (the
prompt) runs flash_lab.attention with causal masking on the valid rows of the cache; a forward
with one query token runs flash_lab.decode directly on the cache tensors. With
cache_implementation="static" each layer's cache is a fixed [B, H_kv, max_len, D] buffer that the
decode kernel reads in place through strides, and generate() may compile and graph-capture the
decode step: that path does no host synchronization.

transformers passes no attention mask to an implementation it does not know, so the number of
valid cache rows is taken from position_ids, and batches must be unpadded (every sequence starts
at position 0 and all have the same length); the prompt path checks this.
"""

from __future__ import annotations

import weakref
from functools import partial

import torch

from flash_lab.ops import attention, decode

NAME = "flash_lab"

# The last position_ids tensor the prompt path read on the host, its version counter and the set
# of sequence ends it held. Every layer of one forward receives the same position_ids tensor, so
# only the first layer pays the device-to-host read (a stream sync); the reference's hook reads it
# in every layer. The weak reference makes the identity test exact: a new tensor, even at the same
# address, is never taken for the old one, and an in-place change bumps the version counter.
_last_ends: tuple | None = None


def _sequence_ends(position_ids: torch.Tensor) -> set:
    global _last_ends
    if _last_ends is not None:
        ref, version, ends = _last_ends
        if ref() is position_ids and position_ids._version == version:
            return ends
    ends = set(position_ids[:, -1].tolist())
    _last_ends = (weakref.ref(position_ids), position_ids._version, ends)
    return ends


def attention_forward(
    module: torch.nn.Module,
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    attention_mask: torch.Tensor | None,
    scaling: float | None = None,
    dropout: float = 0.0,
    *,
    prefill_impl: str = "auto",
    decode_impl: str = "auto",
    **kwargs,
) -> tuple[torch.Tensor, None]:
    """transformers' attention-function signature (reference flash_lab/hf.py:27-77): query is
    [B, H, S_q, D], key and value [B, H_kv, S_k, D] (a static cache's whole buffer); the output
    is [B, S_q, H, D]."""
    if dropout:
        raise ValueError("flash_lab attention has no dropout; call model.eval() first")
    if kwargs.get("sliding_window") is not None:
        raise NotImplementedError("flash_lab attention has no sliding-window masking")
    position_ids = kwargs.get("position_ids")
    if position_ids is None:
        raise ValueError("flash_lab attention needs position_ids to find the valid cache rows")

    batch, _, seqlen_q, _ = query.shape
    # [B, S, H, D] views of transformers' [B, H, S, D] tensors; the kernels read the strides.
    q, k, v = (t.transpose(1, 2) for t in (query, key, value))
    last_position = position_ids[:, -1]

    if seqlen_q == 1:
        # The step generate() compiles and replays: stays on the device, no host sync.
        seq_lens = (last_position + 1).to(torch.int32).expand(batch).contiguous()
        return decode(q, k, v, seq_lens, softmax_scale=scaling, impl=decode_impl), None

    ends = set(_sequence_ends(position_ids))
    if len(ends) != 1:
        raise ValueError("flash_lab attention supports unpadded batches only")
    seqlen_k = ends.pop() + 1
    if not seqlen_q <= seqlen_k <= k.shape[1]:
        raise ValueError(
            f"position_ids end at {seqlen_k - 1}, which does not fit {seqlen_q} new tokens "
            f"and a cache of {k.shape[1]} rows"
        )
    out = attention(
        q,
        k[:, :seqlen_k],
        v[:, :seqlen_k],
        causal=getattr(module, "is_causal", True),
        softmax_scale=scaling,
        impl=prefill_impl,
    )
    return out, None


def reserved_by_transformers(name: str) -> bool:
    """Whether transformers would take `name` for a flash-attention kernel to import rather than a
    registered function: transformers 5 does so for every implementation name containing "flash"
    (transformers/utils/generic.py, is_flash_attention_requested), which includes "flash_lab". The
    reference pinned transformers 4.57, which had no such rule."""
    try:
        from transformers.utils.generic import is_flash_attention_requested
    except ImportError:
        return False
    return bool(is_flash_attention_requested(requested_attention_implementation=name))


def register(name: str = NAME, prefill_impl: str = "auto", decode_impl: str = "auto") -> str:
    """Registers (or re-registers) attention_forward with transformers under `name`, with the
    given kernel choices, and returns the name to pass as attn_implementation (reference
    flash_lab/hf.py:80-88). Where transformers reserves `name` for its flash-attention kernels
    (see reserved_by_transformers), the function is also registered under the name with "flash"
    shortened to "fl" ("flash_lab" -> "fl_lab"), and that is the name returned."""
    from transformers import AttentionInterface

    function = partial(attention_forward, prefill_impl=prefill_impl, decode_impl=decode_impl)
    AttentionInterface.register(name, function)
    if reserved_by_transformers(name):
        name = name.replace("flash", "fl")
        AttentionInterface.register(name, function)
    return name
