"""Pins the oracle (oracle/reference.py) before anything is checked against it. CPU only.

Each check follows one the reference runs on its own oracle (reference tests/test_reference.py),
or fixes the result from mathematics: torch SDPA in fp64, closed forms (one key, identical keys,
rows without keys), GQA == repeated KV heads, bottom-right rows == prefix attention, the tiled
FlashAttention-2 form == the dense form, decode == prefill rows, paged == contiguous. On top: an
independent C restatement (oracle/attn_ref.c) must agree to 1e-12, and planted mistakes (a dropped
scale, a top-left mask, a wrong GQA head map, a log2 LSE, nan for empty rows, a transposed
operand) must each fail at least one of these checks.
"""

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import c_oracle
from oracle import reference

EXACT = {"rtol": 0.0, "atol": 1e-12}


def make_qkv(batch, seqlen_q, seqlen_k, heads, heads_kv, head_dim, scale=1.0):
    q = torch.randn(batch, seqlen_q, heads, head_dim, dtype=torch.float64) * scale
    k = torch.randn(batch, seqlen_k, heads_kv, head_dim, dtype=torch.float64) * scale
    v = torch.randn(batch, seqlen_k, heads_kv, head_dim, dtype=torch.float64)
    return q, k, v


def sdpa_fp64(q, k, v, causal):
    """torch SDPA on [B, S, H, D] inputs (top-left causal: only comparable when S_q == S_k)."""
    group = q.shape[2] // k.shape[2]
    k = k.repeat_interleave(group, dim=2)
    v = v.repeat_interleave(group, dim=2)
    out = F.scaled_dot_product_attention(
        q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), is_causal=causal
    )
    return out.transpose(1, 2)


def close(a, b, atol=1e-12):
    return a.shape == b.shape and bool(
        torch.allclose(a, b, rtol=0.0, atol=atol, equal_nan=False)
    )


# ---------------------------------------------------------------------------------------------
# Checks, each a function of an attention implementation so planted mistakes can be fed through.


def check_sdpa(attn) -> bool:
    ok = True
    for causal in (False, True):
        for shape in [(2, 7, 4, 4, 16), (1, 33, 8, 2, 32), (3, 1, 2, 1, 8)]:
            batch, seqlen, heads, heads_kv, head_dim = shape
            q, k, v = make_qkv(batch, seqlen, seqlen, heads, heads_kv, head_dim)
            ok &= close(attn(q, k, v, causal=causal), sdpa_fp64(q, k, v, causal))
    return ok


def check_single_key(attn) -> bool:
    q, k, v = make_qkv(2, 5, 1, 4, 2, 8)
    out, lse = attn(q, k, v, return_lse=True)
    expected = v.repeat_interleave(2, dim=2).expand_as(out)
    scores = torch.einsum("bqhd,bkhd->bhqk", q, k.repeat_interleave(2, dim=2)) / math.sqrt(8)
    return close(out, expected) and close(lse, scores[..., 0])


def check_identical_keys(attn) -> bool:
    q, k, v = make_qkv(1, 4, 6, 2, 2, 8)
    k = k[:, :1].expand_as(k)
    out = attn(q, k, v)
    return close(out, v.mean(dim=1, keepdim=True).expand_as(out))


def check_gqa(attn) -> bool:
    q, k, v = make_qkv(2, 9, 11, 8, 2, 16)
    grouped = attn(q, k, v, causal=True)
    repeated = attn(q, k.repeat_interleave(4, dim=2), v.repeat_interleave(4, dim=2), causal=True)
    return close(grouped, repeated)


def check_bottom_right(attn) -> bool:
    seqlen_q, seqlen_k = 3, 7
    q, k, v = make_qkv(1, seqlen_q, seqlen_k, 2, 2, 8)
    out = attn(q, k, v, causal=True)
    ok = True
    for i in range(seqlen_q):
        visible = seqlen_k - seqlen_q + i + 1
        row = attn(q[:, i : i + 1], k[:, :visible], v[:, :visible])
        ok &= close(out[:, i : i + 1], row)
    return ok


def check_empty_rows(attn) -> bool:
    # S_q > S_k with bottom-right alignment: the first S_q - S_k rows see no keys.
    q, k, v = make_qkv(2, 5, 2, 2, 1, 8)
    out, lse = attn(q, k, v, causal=True, return_lse=True)
    return bool(
        torch.all(out[:, :3] == 0)
        and torch.all(torch.isneginf(lse[:, :, :3]))
        and torch.isfinite(out).all()
        and torch.isfinite(lse[:, :, 3:]).all()
    )


def check_c_restatement(attn) -> bool:
    ok = True
    for shape, causal in [
        ((2, 13, 13, 4, 2, 16), False),
        ((2, 13, 13, 4, 2, 16), True),
        ((1, 5, 17, 2, 1, 8), True),
        ((1, 17, 5, 4, 4, 8), True),
        ((2, 9, 9, 3, 3, 32), False),
    ]:
        q, k, v = make_qkv(*shape)
        o_c, lse_c = c_oracle.attention(q, k, v, causal=causal, softmax_scale=0.3)
        o_t, lse_t = attn(q, k, v, causal=causal, softmax_scale=0.3, return_lse=True)
        finite = torch.isfinite(lse_c)
        ok &= close(o_t, o_c) and bool(torch.equal(torch.isfinite(lse_t), finite))
        ok &= close(lse_t[finite], lse_c[finite])
    return ok


CHECKS = [
    check_sdpa,
    check_single_key,
    check_identical_keys,
    check_gqa,
    check_bottom_right,
    check_empty_rows,
    check_c_restatement,
]


@pytest.mark.parametrize("check", CHECKS, ids=lambda c: c.__name__)
def test_oracle_passes(check):
    assert check(reference.attention)


# ---------------------------------------------------------------------------------------------
# Planted mistakes: variants of the oracle with one plausible error each.


def _mutant(*, scale_on=True, top_left=False, gqa_tile=False, log2_lse=False, nan_rows=False,
            transpose_qk=False):
    def attn(q, k, v, causal=False, softmax_scale=None, return_lse=False):
        head_dim = q.shape[-1]
        scale = 1.0 / math.sqrt(head_dim) if softmax_scale is None else softmax_scale
        group = q.shape[2] // k.shape[2]
        if gqa_tile:
            k_, v_ = k.repeat(1, 1, group, 1), v.repeat(1, 1, group, 1)
        else:
            k_, v_ = k.repeat_interleave(group, dim=2), v.repeat_interleave(group, dim=2)
        if transpose_qk and q.shape[1] == k.shape[1]:
            scores = torch.einsum("bkhd,bqhd->bhqk", q, k_)
        else:
            scores = torch.einsum("bqhd,bkhd->bhqk", q, k_)
        if scale_on:
            scores = scores * scale
        if causal:
            sq, sk = q.shape[1], k.shape[1]
            offset = 0 if top_left else sk - sq
            hidden = torch.arange(sk)[None, :] > torch.arange(sq)[:, None] + offset
            scores = scores.masked_fill(hidden, float("-inf"))
        lse = torch.logsumexp(scores, dim=-1)
        if nan_rows:
            probs = torch.exp(scores - lse.unsqueeze(-1))
        else:
            probs = torch.exp(scores - lse.masked_fill(torch.isneginf(lse), 0.0).unsqueeze(-1))
        out = torch.einsum("bhqk,bkhd->bqhd", probs, v_)
        if log2_lse:
            lse = lse / math.log(2)
        return (out, lse) if return_lse else out

    return attn


MUTANTS = {
    "dropped_scale": _mutant(scale_on=False),
    "top_left_mask": _mutant(top_left=True),
    "gqa_tiled_heads": _mutant(gqa_tile=True),
    "log2_lse": _mutant(log2_lse=True),
    "nan_for_empty_rows": _mutant(nan_rows=True),
    "transposed_qk": _mutant(transpose_qk=True),
}


@pytest.mark.parametrize("name", sorted(MUTANTS))
def test_planted_mistakes_are_caught(name):
    mutant = MUTANTS[name]
    failed = [c.__name__ for c in CHECKS if not c(mutant)]
    assert failed, f"no check catches the planted mistake {name}"


def test_unmutated_restatement_passes_every_check():
    # The mutant factory with no mistake planted is a correct oracle: the checks do not reject
    # correct code, so a failure above is the planted mistake.
    clean = _mutant()
    assert all(c(clean) for c in CHECKS)


# ---------------------------------------------------------------------------------------------
# The rest of the oracle: rows, tiled form, decode, paged caches.


def test_large_scores_stay_finite_in_fp32():
    # Scores around +-100 overflow exp() in fp32 unless the row max is subtracted first.
    q, k, v = make_qkv(1, 64, 64, 2, 2, 64, scale=10.0)
    out32 = reference.attention(q.float(), k.float(), v.float(), causal=True, dtype=torch.float32)
    out64 = reference.attention(q, k, v, causal=True)
    assert torch.isfinite(out32).all()
    torch.testing.assert_close(out32.double(), out64, rtol=0.0, atol=1e-2)


TILED_CASES = [
    # batch, seqlen_q, seqlen_k, heads, heads_kv, head_dim, block_q, block_k
    (2, 16, 16, 2, 2, 8, 16, 16),
    (1, 37, 37, 4, 2, 16, 16, 8),
    (2, 1, 29, 3, 1, 8, 16, 8),
    (1, 29, 13, 2, 2, 8, 8, 8),
    (1, 13, 50, 2, 1, 8, 4, 16),
    (1, 64, 64, 1, 1, 32, 64, 64),
]


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("case", TILED_CASES)
def test_tiled_matches_dense(case, causal):
    batch, seqlen_q, seqlen_k, heads, heads_kv, head_dim, block_q, block_k = case
    q, k, v = make_qkv(batch, seqlen_q, seqlen_k, heads, heads_kv, head_dim)
    out, lse = reference.attention(q, k, v, causal=causal, return_lse=True)
    out_t, lse_t = reference.attention_tiled(
        q, k, v, causal=causal, return_lse=True, block_q=block_q, block_k=block_k
    )
    torch.testing.assert_close(out_t, out, **EXACT)
    torch.testing.assert_close(lse_t, lse, **EXACT)


@pytest.mark.parametrize("seqlen_q,seqlen_k", [(50, 70), (70, 50)])
@pytest.mark.parametrize("causal", [False, True])
def test_attention_rows_matches_full_rows(seqlen_q, seqlen_k, causal):
    q, k, v = make_qkv(2, seqlen_q, seqlen_k, 4, 2, 16)
    rows = torch.tensor([0, 7, 31, seqlen_q - 1])
    full, full_lse = reference.attention(q, k, v, causal=causal, return_lse=True)
    part, part_lse = reference.attention_rows(q, k, v, rows, causal=causal, return_lse=True)
    torch.testing.assert_close(part, full[:, rows], **EXACT)
    torch.testing.assert_close(part_lse, full_lse[:, :, rows], **EXACT)


def make_cache(batch, max_seqlen, heads_kv, head_dim):
    k = torch.randn(batch, max_seqlen, heads_kv, head_dim, dtype=torch.float64)
    v = torch.randn(batch, max_seqlen, heads_kv, head_dim, dtype=torch.float64)
    return k, v


def to_paged(cache, page_size, generator):
    """Scatters a contiguous [B, S_max, H_kv, D] cache into shuffled pages of a larger pool."""
    batch, max_seqlen = cache.shape[:2]
    pages_per_seq = max_seqlen // page_size
    num_blocks = batch * pages_per_seq + 3
    order = torch.randperm(num_blocks, generator=generator)[: batch * pages_per_seq]
    block_tables = order.view(batch, pages_per_seq).to(torch.int32)
    pool = torch.zeros(num_blocks, page_size, *cache.shape[2:], dtype=cache.dtype)
    pool[order.long()] = cache.reshape(batch * pages_per_seq, page_size, *cache.shape[2:])
    return pool, block_tables


def test_decode_matches_prefill_rows():
    batch, max_seqlen, heads, heads_kv, head_dim = 3, 20, 4, 2, 16
    k_cache, v_cache = make_cache(batch, max_seqlen, heads_kv, head_dim)
    q = torch.randn(batch, 1, heads, head_dim, dtype=torch.float64)
    seq_lens = torch.tensor([1, 7, 20], dtype=torch.int32)
    out, lse = reference.decode(q, k_cache, v_cache, seq_lens, return_lse=True)
    assert out.shape == q.shape and lse.shape == (batch, heads)
    for b, n in enumerate(seq_lens.tolist()):
        row, row_lse = reference.attention(
            q[b : b + 1], k_cache[b : b + 1, :n], v_cache[b : b + 1, :n], return_lse=True
        )
        torch.testing.assert_close(out[b : b + 1], row, **EXACT)
        torch.testing.assert_close(lse[b], row_lse[0, :, 0], **EXACT)


def test_decode_matches_c_restatement():
    batch, max_seqlen, heads, heads_kv, head_dim = 2, 40, 6, 2, 16
    k_cache, v_cache = make_cache(batch, max_seqlen, heads_kv, head_dim)
    q = torch.randn(batch, heads, head_dim, dtype=torch.float64)
    seq_lens = torch.tensor([40, 9], dtype=torch.int32)
    out, lse = reference.decode(q, k_cache, v_cache, seq_lens, return_lse=True)
    for b, n in enumerate(seq_lens.tolist()):
        o_c, lse_c = c_oracle.attention(q[b : b + 1, None], k_cache[b : b + 1, :n],
                                        v_cache[b : b + 1, :n])
        torch.testing.assert_close(out[b], o_c[0, 0], **EXACT)
        torch.testing.assert_close(lse[b], lse_c[0, :, 0], **EXACT)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
def test_c_decode_reads_the_cache_dtype_and_matches_the_oracle(dtype):
    # oracle_decode_f64 (the C loops the long-cache GPU checks use) reads bf16 / fp32 caches in
    # place and must give the float64 decode of the same values: GQA, ragged lengths (1 and the
    # full cache), rank-3 and rank-4 queries, an explicit scale.
    gen = torch.Generator().manual_seed(7)
    batch, max_seqlen, heads, heads_kv, head_dim = 3, 50, 8, 2, 32
    k_cache = torch.randn(batch, max_seqlen, heads_kv, head_dim, generator=gen).to(dtype)
    v_cache = torch.randn(batch, max_seqlen, heads_kv, head_dim, generator=gen).to(dtype)
    q = torch.randn(batch, 1, heads, head_dim, generator=gen).to(dtype)
    seq_lens = torch.tensor([50, 1, 17], dtype=torch.int32)
    for query, scale in ((q, None), (q[:, 0], 0.37)):
        want, want_lse = reference.decode(query, k_cache, v_cache, seq_lens, softmax_scale=scale,
                                          return_lse=True)
        got, got_lse = c_oracle.decode(query, k_cache, v_cache, seq_lens, softmax_scale=scale)
        assert got.shape == want.shape and got.dtype == torch.float64
        torch.testing.assert_close(got, want, **EXACT)
        torch.testing.assert_close(got_lse, want_lse, **EXACT)
    with pytest.raises(ValueError, match="rejected"):
        c_oracle.decode(q, k_cache, v_cache, torch.tensor([50, 0, 3], dtype=torch.int32))


@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
@pytest.mark.parametrize("seqlen_q,seqlen_k", [(70, 50), (40, 90)], ids=["sq>sk", "sq<sk"])
def test_c_rows_match_attention_rows(seqlen_q, seqlen_k, dtype, causal):
    # oracle_attention_rows_f64 (the C loops the long prefill checks use) against attention_rows:
    # GQA, both S_q != S_k directions (with causal rows that see no key), first and last rows.
    gen = torch.Generator().manual_seed(8)
    q = torch.randn(2, seqlen_q, 6, 32, generator=gen).to(dtype)
    k = torch.randn(2, seqlen_k, 3, 32, generator=gen).to(dtype)
    v = torch.randn(2, seqlen_k, 3, 32, generator=gen).to(dtype)
    rows = torch.tensor([0, 5, 19, 20, 21, seqlen_q - 1])
    want, want_lse = reference.attention_rows(q, k, v, rows, causal, 0.3, return_lse=True)
    got, got_lse = c_oracle.attention_rows(q, k, v, rows, causal, 0.3)
    assert got.shape == want.shape and got_lse.shape == want_lse.shape
    torch.testing.assert_close(got, want, **EXACT)
    assert torch.equal(torch.isneginf(got_lse), torch.isneginf(want_lse))
    finite = torch.isfinite(want_lse)
    torch.testing.assert_close(got_lse[finite], want_lse[finite], **EXACT)
    with pytest.raises(ValueError, match="rejected"):
        c_oracle.attention_rows(q, k, v, torch.tensor([0, seqlen_q]), causal)


def test_paged_decode_matches_contiguous():
    batch, max_seqlen, heads, heads_kv, head_dim, page_size = 3, 16, 4, 1, 8, 4
    k_cache, v_cache = make_cache(batch, max_seqlen, heads_kv, head_dim)
    k_pool, block_tables = to_paged(k_cache, page_size, torch.Generator().manual_seed(1))
    v_pool, _ = to_paged(v_cache, page_size, torch.Generator().manual_seed(1))
    q = torch.randn(batch, heads, head_dim, dtype=torch.float64)
    seq_lens = torch.tensor([5, 16, 9], dtype=torch.int32)
    contiguous = reference.decode(q, k_cache, v_cache, seq_lens)
    paged = reference.decode(q, k_pool, v_pool, seq_lens, block_tables=block_tables)
    assert paged.shape == q.shape
    torch.testing.assert_close(paged, contiguous, **EXACT)


def test_decode_rejects_lengths_outside_the_cache():
    k_cache, v_cache = make_cache(2, 8, 1, 8)
    q = torch.randn(2, 1, 1, 8, dtype=torch.float64)
    with pytest.raises(ValueError, match="outside"):
        reference.decode(q, k_cache, v_cache, torch.tensor([3, 9], dtype=torch.int32))
    with pytest.raises(ValueError, match="outside"):
        reference.decode(q, k_cache, v_cache, torch.tensor([0, 1], dtype=torch.int32))


def test_causal_mask_closed_form():
    mask = reference.causal_mask(3, 5)
    expected = torch.tensor(
        [[False, False, False, True, True],
         [False, False, False, False, True],
         [False, False, False, False, False]]
    )
    assert torch.equal(mask, expected)


def test_cpu_reference_path_fp32_within_1e5_of_fp64():
    # B=1, H=H_kv=4, S=256, D=64 fp32, iid N(0,1) from seed 0, non-causal,
    # scale 1/sqrt(D); the fp32 path within 1e-5 relative (normwise) of fp64.
    torch.manual_seed(0)
    q = torch.randn(1, 256, 4, 64)
    k = torch.randn(1, 256, 4, 64)
    v = torch.randn(1, 256, 4, 64)
    out32 = reference.attention(q, k, v, dtype=torch.float32)
    out64 = reference.attention(q, k, v)
    assert out32.shape == (1, 256, 4, 64)
    rel = (out32.double() - out64).abs().max() / out64.abs().max()
    assert rel <= 1e-5, f"normwise relative error {rel:.3g}"
