"""Test oracle: plain PyTorch attention used as ground truth. TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg may import this module, and
only as the checker; the flash_lab package never does. It restates the reference's oracle,
flash_lab/reference.py:1-205 (the reference exports it as flash_lab.reference).

Definitions (reference flash_lab/reference.py:1-7, docs/numerics.md:9-22): everything is computed
in float64 unless another dtype is asked for. The causal mask is aligned to the bottom-right
corner: query i sees key j iff j <= i + (S_k - S_q). A row that sees no key returns zeros and an
LSE of -inf. LSE values are the natural-log log-sum-exp of the scaled scores, [B, H, S_q].

The op sequence of attention() (einsum, scale, mask, logsumexp, shift, exp, einsum) is the
reference's own, kept on purpose: with dtype=bf16/fp16 this function is the "plain torch at the
input dtype" baseline whose error sets the 2x tolerance of the parity tests, so it must round the
way the reference's does.

Pinning (tests/test_oracle.py): torch SDPA in fp64 at atol 1e-12, closed forms (one key, identical
keys, empty rows), GQA == repeated KV heads, bottom-right rows == prefixes, attention_tiled ==
attention, decode == prefill rows, paged == contiguous, an independent C restatement
(oracle/attn_ref.c), and planted mistakes that must fail those checks.
"""

from __future__ import annotations

import math

import torch

from flash_lab.layouts import check_attention_inputs, check_decode_inputs

NEG_INF = float("-inf")


def causal_mask(seqlen_q: int, seqlen_k: int, device: torch.device | None = None) -> torch.Tensor:
    """[S_q, S_k] bool, True where the key is hidden (reference flash_lab/reference.py:16-20)."""
    offset = seqlen_k - seqlen_q
    row = torch.arange(seqlen_q, device=device).unsqueeze(1)
    col = torch.arange(seqlen_k, device=device).unsqueeze(0)
    return col > row + offset


def _repeat_kv(x: torch.Tensor, group: int) -> torch.Tensor:
    """[B, S, H_kv, D] -> [B, S, H, D]: query head h lines up with KV head h // group."""
    if group == 1:
        return x
    return x.repeat_interleave(group, dim=2)


def _scale_of(head_dim: int, softmax_scale: float | None) -> float:
    return 1.0 / math.sqrt(head_dim) if softmax_scale is None else softmax_scale


def _softmax_rows(scores: torch.Tensor, v_: torch.Tensor):
    """LSE and output from masked, scaled scores [B, H, q, k]; rows without keys give 0 / -inf.
    Op order of reference flash_lab/reference.py:50-56."""
    lse = torch.logsumexp(scores, dim=-1)
    shift = lse.masked_fill(torch.isneginf(lse), 0.0)
    probs = torch.exp(scores - shift.unsqueeze(-1))
    out = torch.einsum("bhqk,bkhd->bqhd", probs, v_)
    return out, lse


def attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    causal: bool = False,
    softmax_scale: float | None = None,
    return_lse: bool = False,
    dtype: torch.dtype = torch.float64,
):
    """Dense attention with the full score matrix (reference flash_lab/reference.py:32-57).
    Returns o [B, S_q, H, D] in `dtype` (and lse [B, H, S_q])."""
    shape = check_attention_inputs(q, k, v, require_unit_stride=False)
    scale = _scale_of(shape.head_dim, softmax_scale)
    q_ = q.to(dtype)
    k_ = _repeat_kv(k.to(dtype), shape.group)
    v_ = _repeat_kv(v.to(dtype), shape.group)
    scores = torch.einsum("bqhd,bkhd->bhqk", q_, k_) * scale
    if causal:
        scores = scores.masked_fill(causal_mask(shape.seqlen_q, shape.seqlen_k, q.device), NEG_INF)
    out, lse = _softmax_rows(scores, v_)
    return (out, lse) if return_lse else out


def attention_rows(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    rows: torch.Tensor,
    causal: bool = False,
    softmax_scale: float | None = None,
    dtype: torch.dtype = torch.float64,
    return_lse: bool = False,
):
    """attention() for the listed query rows only, [B, len(rows), H, D]; the causal mask uses
    each row's position in the full sequence (reference flash_lab/reference.py:60-87). For
    checking long sequences whose full score matrix would not fit in memory."""
    shape = check_attention_inputs(q, k, v, require_unit_stride=False)
    scale = _scale_of(shape.head_dim, softmax_scale)
    rows = rows.to(q.device)
    q_ = q[:, rows].to(dtype)
    k_ = _repeat_kv(k.to(dtype), shape.group)
    v_ = _repeat_kv(v.to(dtype), shape.group)
    scores = torch.einsum("bqhd,bkhd->bhqk", q_, k_) * scale
    if causal:
        col = torch.arange(shape.seqlen_k, device=q.device).unsqueeze(0)
        hidden = col > rows.unsqueeze(1) + (shape.seqlen_k - shape.seqlen_q)
        scores = scores.masked_fill(hidden, NEG_INF)
    out, lse = _softmax_rows(scores, v_)
    return (out, lse) if return_lse else out


def attention_tiled(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    causal: bool = False,
    softmax_scale: float | None = None,
    return_lse: bool = False,
    block_q: int = 64,
    block_k: int = 64,
    dtype: torch.dtype = torch.float64,
):
    """FlashAttention-2 forward in tensor ops (reference flash_lab/reference.py:90-152): query
    blocks, key tiles, online softmax with the -inf-safe reference point, causal tiles past the
    diagonal skipped. It never forms the [S_q, S_k] matrix, so agreement with attention() checks
    the algorithm the kernels implement, independently of any kernel."""
    shape = check_attention_inputs(q, k, v, require_unit_stride=False)
    scale = _scale_of(shape.head_dim, softmax_scale)
    sq, sk = shape.seqlen_q, shape.seqlen_k
    offset = sk - sq
    qt = q.to(dtype).transpose(1, 2)  # [B, H, S_q, D]
    kt = _repeat_kv(k.to(dtype), shape.group).transpose(1, 2)
    vt = _repeat_kv(v.to(dtype), shape.group).transpose(1, 2)
    out = torch.zeros_like(qt)
    lse = torch.full(qt.shape[:-1], NEG_INF, dtype=dtype, device=q.device)

    for q0 in range(0, sq, block_q):
        q1 = min(q0 + block_q, sq)
        stats = (shape.batch, shape.heads, q1 - q0)
        run_max = torch.full(stats, NEG_INF, dtype=dtype, device=q.device)
        run_sum = torch.zeros(stats, dtype=dtype, device=q.device)
        acc = torch.zeros((*stats, shape.head_dim), dtype=dtype, device=q.device)
        # The block's last row sees keys up to q1 - 1 + offset; later tiles are skipped.
        k_stop = min(sk, q1 + offset) if causal else sk
        for k0 in range(0, max(k_stop, 0), block_k):
            k1 = min(k0 + block_k, sk)
            s = qt[:, :, q0:q1] @ kt[:, :, k0:k1].transpose(-1, -2) * scale
            if causal and k1 - 1 > q0 + offset:  # the tile crosses the diagonal
                r = torch.arange(q0, q1, device=q.device).unsqueeze(1)
                c = torch.arange(k0, k1, device=q.device).unsqueeze(0)
                s = s.masked_fill(c > r + offset, NEG_INF)
            new_max = torch.maximum(run_max, s.amax(dim=-1))
            ref = new_max.masked_fill(torch.isneginf(new_max), 0.0)
            alpha = torch.exp(run_max - ref)
            p = torch.exp(s - ref.unsqueeze(-1))
            run_sum = alpha * run_sum + p.sum(dim=-1)
            acc = alpha.unsqueeze(-1) * acc + p @ vt[:, :, k0:k1]
            run_max = new_max
        seen = run_sum > 0
        denom = run_sum.masked_fill(~seen, 1.0)
        out[:, :, q0:q1] = acc / denom.unsqueeze(-1)
        lse[:, :, q0:q1] = torch.where(seen, run_max + torch.log(denom), NEG_INF)

    out = out.transpose(1, 2)
    return (out, lse) if return_lse else out


def gather_cache(
    cache: torch.Tensor, block_tables: torch.Tensor | None, batch_idx: int, length: int
) -> torch.Tensor:
    """Rows 0..length-1 of one sequence as [length, H_kv, D] from a contiguous or paged cache
    (reference flash_lab/reference.py:155-164)."""
    if block_tables is None:
        return cache[batch_idx, :length]
    page = cache.shape[1]
    pages = block_tables[batch_idx, : (length + page - 1) // page].long()
    return cache[pages].flatten(0, 1)[:length]


def decode(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    seq_lens: torch.Tensor,
    block_tables: torch.Tensor | None = None,
    softmax_scale: float | None = None,
    return_lse: bool = False,
    dtype: torch.dtype = torch.float64,
):
    """One query token per sequence against its first seq_lens[b] cached keys, one sequence at a
    time through attention() (reference flash_lab/reference.py:167-205). Returns o with q's rank
    ([B, 1, H, D] or [B, H, D]) and lse [B, H]."""
    q3, shape = check_decode_inputs(
        q, k_cache, v_cache, seq_lens, block_tables, require_unit_stride=False
    )
    scale = _scale_of(shape.head_dim, softmax_scale)
    outs, lses = [], []
    for b, length in enumerate(seq_lens.tolist()):
        if not 1 <= length <= shape.max_seqlen:
            raise ValueError(f"seq_lens[{b}] = {length} is outside [1, {shape.max_seqlen}]")
        keys = gather_cache(k_cache, block_tables, b, length)
        values = gather_cache(v_cache, block_tables, b, length)
        o_b, lse_b = attention(
            q3[b][None, None], keys[None], values[None], softmax_scale=scale, return_lse=True,
            dtype=dtype,
        )
        outs.append(o_b[0, 0])
        lses.append(lse_b[0, :, 0])
    out = torch.stack(outs)
    if q.dim() == 4:
        out = out.unsqueeze(1)
    lse = torch.stack(lses)
    return (out, lse) if return_lse else out
