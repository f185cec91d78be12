"""The C ABI boundary on the CPU: the library loads, exports every function the header declares,
plans decode splits on the host, and rejects bad arguments before any launch. No compute call
reaches a device here."""

import ctypes
import re
from pathlib import Path

import pytest
import torch

from flash_lab import _hip

HEADER = Path(__file__).resolve().parent.parent / "include" / "flash_lab_hip.h"


def declared_functions() -> set[str]:
    text = HEADER.read_text()
    return set(re.findall(r"^\s*(?:int|int64_t|const char\*)\s+(fl_\w+)\s*\(", text, flags=re.M))


def test_header_declares_the_abi():
    assert declared_functions() >= {
        "fl_attention_fwd",
        "fl_decode_plan",
        "fl_decode",
        "fl_smoke_axpy",
        "fl_mfma_tile_test",
        "fl_set_knob",
        "fl_get_knob",
        "fl_last_error",
        "fl_version",
    }


def test_library_exports_every_declared_function():
    lib = ctypes.CDLL(str(_hip.LIB_PATH))
    for name in sorted(declared_functions()):
        assert hasattr(lib, name), name
    assert set(_hip.SIGNATURES) == declared_functions()


def test_struct_layouts_match_the_header():
    # Natural C alignment: 5 pointers + 12 int64 + 8 int32 + double = 176 bytes;
    # 6 pointers + 10 int64 + 7 int32 (+4 pad) + double + pointer + size_t
    # + pointer + int64 + 2 int32 (paged cache) = 208 bytes.
    assert ctypes.sizeof(_hip.AttnParams) == 176
    assert ctypes.sizeof(_hip.DecodeParams) == 208
    assert _hip.AttnParams.softmax_scale.offset == 168
    assert _hip.DecodeParams.softmax_scale.offset == 160


def test_knobs_are_validated_and_restored(knobs):
    # Routing overrides: known knobs within range only; None (-1) restores the built-in rule.
    assert _hip.get_knob("prefill_pp_min_wg") is None
    knobs("prefill_pp_min_wg", 0)
    assert _hip.get_knob("prefill_pp_min_wg") == 0
    knobs("decode_wg_per_cu", 64)
    assert _hip.get_knob("decode_wg_per_cu") == 64
    for name, bad in (("decode_wg_per_cu", 0), ("decode_wg_per_cu", 65),
                      ("decode_mfma_min_group", 0), ("prefill_pp_min_wg", -5),
                      ("prefill_pp_min_wg", (1 << 30) + 1), ("decode_mfma_span", 0),
                      ("decode_mfma_span", 5)):
        with pytest.raises(RuntimeError, match="out of range"):
            _hip.set_knob(name, bad)
    assert _hip.LIB.fl_set_knob(7, 1) == 1 and b"unknown knob" in _hip.LIB.fl_last_error()
    assert _hip.LIB.fl_get_knob(-1) == -2
    with _hip.knob("decode_mfma_min_group", 1000):
        assert _hip.get_knob("decode_mfma_min_group") == 1000
    assert _hip.get_knob("decode_mfma_min_group") is None
    knobs("decode_wg_per_cu", None)
    assert _hip.get_knob("decode_wg_per_cu") is None


def test_version():
    assert b"gfx950" in _hip.LIB.fl_version()


@pytest.mark.parametrize(
    "batch,heads,heads_kv,expected_splits",
    # The largest power of two whose workgroups fill the planned slots at once, with >= 512 keys
    # per split. MHA (vector kernel, contiguous cache): 4 KV heads per workgroup, one planned per
    # CU (256 slots): 64 x 4 workgroups at B=8, 32 x 8 at B=4; at B=1 that rule gives 8 x 32, and
    # 16 splits of 2048 keys with 2 KV heads per workgroup (256 workgroups) win there. GQA with 4
    # query heads per KV head (matrix-core kernel): four KV heads per workgroup (one per wave),
    # one per CU, splits of >= 1024 keys: 16 x 16 at B=8; at B=1 that cannot fill the CUs, so one
    # KV head per workgroup: 8 x 32.
    [(1, 32, 32, 16), (4, 32, 32, 8), (8, 32, 32, 4), (8, 32, 8, 16), (1, 32, 8, 32)],
    ids=["B1-MHA", "B4-MHA", "B8-MHA", "B8-GQA", "B1-GQA"],
)
def test_decode_plan_on_256_cus(batch, heads, heads_kv, expected_splits):
    splits, ws = _hip.decode_plan(batch, heads, heads_kv, 128, 32768, torch.bfloat16)
    assert splits == expected_splits
    assert ws == batch * heads * splits * (128 + 2) * 4


def test_decode_plan_routes_by_group(knobs):
    # Groups of 4 to 32 query heads per KV head (bf16/fp16, head_dim 128) go to the matrix-core
    # kernel, four KV heads per workgroup and one workgroup per CU: B=8 with 8 KV heads takes 16
    # splits (256 workgroups) whatever the group. Smaller groups and fp32 stay on the vector
    # kernel, and the decode_mfma_min_group knob moves the threshold.
    plan = lambda heads, dtype=torch.bfloat16: _hip.decode_plan(8, heads, 8, 128, 32768, dtype)[0]
    assert plan(32) == plan(64) == plan(256) == 16  # groups 4, 8, 32
    assert plan(16) == 32  # group 2: vector kernel, 4 KV heads per workgroup, 3 per CU
    assert plan(32, torch.float16) == 16
    assert plan(32, torch.float32) == 16  # 2 KV heads per workgroup, 3 per CU
    # head_dim 64 (128-byte rows): from 4 query heads per KV head as well.
    assert _hip.decode_plan(8, 32, 8, 64, 32768, torch.bfloat16)[0] == 16
    assert _hip.decode_plan(8, 64, 8, 64, 32768, torch.bfloat16)[0] == 16
    # Short caches: as many splits as fill the CUs with >= 128 keys each.
    assert _hip.decode_plan(1, 32, 8, 128, 8448, torch.bfloat16)[0] == 32
    assert _hip.decode_plan(1, 32, 8, 128, 2048, torch.bfloat16)[0] == 16
    assert _hip.decode_plan(1, 32, 8, 128, 100, torch.bfloat16)[0] == 1
    knobs("decode_mfma_min_group", 1000)
    assert plan(32) == 32
    knobs("decode_mfma_min_group", 1)
    assert plan(8) == 16
    # One KV head per workgroup where four cannot fill the CUs with splits of >= 1024 keys.
    assert _hip.decode_plan(2, 32, 8, 128, 32768, torch.bfloat16)[0] == 16


def test_decode_mfma_span_knob(knobs):
    # The decode_mfma_span knob pins the matrix-core kernel's layout whatever the call's size:
    # at 4 the plan takes the four-KV-heads split count (one workgroup per CU, splits of >= 1024
    # keys where the cache allows), at 1 the one-KV-head plan.
    plan = lambda b, s: _hip.decode_plan(b, 32, 8, 128, s, torch.bfloat16)[0]
    assert plan(2, 32768) == 16 and plan(8, 32768) == 16
    knobs("decode_mfma_span", 4)
    assert plan(2, 32768) == 32  # 2 x 2 groups of four KV heads x 32 splits of 1024 keys
    assert plan(1, 2048) == 2
    knobs("decode_mfma_span", 1)
    assert plan(8, 32768) == 4  # one KV head per workgroup: 64 x 4 fills 256 CUs
    knobs("decode_mfma_span", None)
    assert plan(8, 32768) == 16


def test_decode_plan_requested_and_inplace():
    assert _hip.decode_plan(2, 8, 8, 64, 1000, torch.float16, num_splits=7) == (7, 2 * 8 * 7 * 66 * 4)
    # decode_inplace: one split and no workspace whatever is asked.
    assert _hip.decode_plan(2, 8, 8, 64, 1000, torch.float16, num_splits=7, allow_splits=False) == (
        1,
        0,
    )
    # Splits keep >= 512 keys while that leaves enough workgroups; with few workgroups (one
    # sequence, 8 KV heads) they go down to 64 keys, and a cache under 128 keys is not split.
    # B=8 MHA at 4K keys: 64 workgroups of 4 KV heads per split, one per CU: 4 splits.
    assert _hip.decode_plan(8, 32, 32, 128, 4096, torch.bfloat16)[0] == 4  # 1024 keys each
    assert _hip.decode_plan(1, 8, 8, 128, 1000, torch.bfloat16)[0] == 8  # 125 keys each
    assert _hip.decode_plan(1, 8, 8, 128, 100, torch.bfloat16)[0] == 1
    assert _hip.decode_plan(1, 8, 8, 128, 128, torch.bfloat16)[0] == 2


def test_decode_plan_rejections():
    with pytest.raises(RuntimeError, match=r"num_splits must be in \[0, 128\]"):
        _hip.decode_plan(1, 8, 8, 128, 100, torch.bfloat16, num_splits=129)
    with pytest.raises(RuntimeError, match="unsupported head_dim 96"):
        _hip.decode_plan(1, 8, 8, 96, 100, torch.bfloat16)
    with pytest.raises(RuntimeError, match="multiple of KV heads"):
        _hip.decode_plan(1, 6, 4, 128, 100, torch.bfloat16)


def _attn_params(**over):
    p = _hip.AttnParams()
    p.q = p.k = p.v = p.o = p.lse = 256
    p.batch, p.seqlen_q, p.seqlen_k, p.heads, p.heads_kv, p.head_dim = 1, 8, 8, 2, 2, 128
    p.q_batch_stride = p.k_batch_stride = p.v_batch_stride = p.o_batch_stride = 8 * 2 * 128
    p.q_seq_stride = p.k_seq_stride = p.v_seq_stride = p.o_seq_stride = 2 * 128
    p.q_head_stride = p.k_head_stride = p.v_head_stride = p.o_head_stride = 128
    p.dtype = 0
    p.softmax_scale = 0.125
    for key, value in over.items():
        setattr(p, key, value)
    return p


@pytest.mark.parametrize(
    "over,message",
    [
        ({"dtype": 2}, "takes bf16 or fp16"),
        ({"head_dim": 96}, "unsupported head_dim 96"),
        ({"heads_kv": 3}, "multiple of KV heads"),
        ({"seqlen_k": 0}, "empty input"),
        ({"softmax_scale": -1.0}, "softmax_scale must be positive"),
        ({"q": 258}, "q must have 16-byte aligned rows"),
        ({"k_seq_stride": 2 * 128 + 4}, "k must have 16-byte aligned rows"),
        ({"q": 0}, "null tensor pointer"),
    ],
)
def test_attention_rejects_before_launch(over, message):
    rc = _hip.LIB.fl_attention_fwd(ctypes.byref(_attn_params(**over)), None)
    assert rc != 0
    assert message in _hip.LIB.fl_last_error().decode()


def test_decode_rejects_missing_workspace():
    p = _hip.DecodeParams()
    p.q = p.k_cache = p.v_cache = p.o = p.lse = p.seq_lens = 256
    p.batch, p.heads, p.heads_kv, p.head_dim, p.max_seqlen = 1, 8, 8, 128, 1000
    p.q_batch_stride, p.q_head_stride = 8 * 128, 128
    p.k_batch_stride = p.v_batch_stride = 1000 * 8 * 128
    p.k_seq_stride = p.v_seq_stride = 8 * 128
    p.k_head_stride = p.v_head_stride = 128
    p.o_batch_stride, p.o_head_stride = 8 * 128, 128
    p.dtype, p.softmax_scale, p.num_splits = 0, 0.1, 4
    assert _hip.LIB.fl_decode(ctypes.byref(p), None) != 0
    assert "workspace" in _hip.LIB.fl_last_error().decode()
    p.num_splits = 0
    assert _hip.LIB.fl_decode(ctypes.byref(p), None) != 0
    assert "num_splits must be in [1, 128]" in _hip.LIB.fl_last_error().decode()


def _paged_params(page_size, max_blocks, num_blocks=64):
    p = _hip.DecodeParams()
    p.q = p.k_cache = p.v_cache = p.o = p.lse = p.seq_lens = p.workspace = 256
    p.batch, p.heads, p.heads_kv, p.head_dim = 1, 8, 8, 128
    p.max_seqlen = max_blocks * page_size
    p.q_batch_stride, p.q_head_stride = 8 * 128, 128
    p.k_batch_stride = p.v_batch_stride = page_size * 8 * 128
    p.k_seq_stride = p.v_seq_stride = 8 * 128
    p.k_head_stride = p.v_head_stride = 128
    p.o_batch_stride, p.o_head_stride = 8 * 128, 128
    p.dtype, p.softmax_scale = 0, 0.1
    p.block_tables, p.block_tables_stride = 256, max_blocks
    p.page_size, p.num_blocks = page_size, num_blocks
    return p


def test_paged_plan_bounds_the_blocks_per_split():
    # A paged split stages its block numbers in LDS when they fit (at most 1024): the plan takes
    # more splits when one would touch more blocks. Requested counts are honoured (a longer split
    # reads the table from global memory), and so are caches too long even for 128 splits.
    splits, ws = ctypes.c_int32(), ctypes.c_size_t()
    p = _paged_params(page_size=1, max_blocks=100000)
    p.batch = 64  # the occupancy rule alone would pick 8 splits: 12,629 blocks each
    assert _hip.LIB.fl_decode_plan(ctypes.byref(p), 0, 1, 256, ctypes.byref(splits),
                                   ctypes.byref(ws)) == 0
    assert splits.value == 128  # 782 keys, at most 911 blocks per split
    assert _hip.LIB.fl_decode_plan(ctypes.byref(p), 4, 1, 256, ctypes.byref(splits),
                                   ctypes.byref(ws)) == 0
    assert splits.value == 4
    p = _paged_params(page_size=1, max_blocks=200000)
    assert _hip.LIB.fl_decode_plan(ctypes.byref(p), 0, 1, 256, ctypes.byref(splits),
                                   ctypes.byref(ws)) == 0
    assert splits.value == 128
    p = _paged_params(page_size=16, max_blocks=64)
    assert _hip.LIB.fl_decode_plan(ctypes.byref(p), 0, 0, 256, ctypes.byref(splits),
                                   ctypes.byref(ws)) == 0
    assert splits.value == 1  # decode_inplace


def test_paged_decode_rejects_bad_geometry():
    p = _paged_params(page_size=0, max_blocks=4)
    assert _hip.LIB.fl_decode(ctypes.byref(p), None) != 0
    assert "page_size" in _hip.LIB.fl_last_error().decode()
    p = _paged_params(page_size=16, max_blocks=4, num_blocks=0)
    assert _hip.LIB.fl_decode(ctypes.byref(p), None) != 0
    assert "num_blocks" in _hip.LIB.fl_last_error().decode()
    p = _paged_params(page_size=16, max_blocks=4)
    p.block_tables = 258  # not 4-byte aligned
    p.num_splits = 1
    assert _hip.LIB.fl_decode(ctypes.byref(p), None) != 0
    assert "block_tables" in _hip.LIB.fl_last_error().decode()


def test_tile_test_rejects_bad_k():
    assert _hip.LIB.fl_mfma_tile_test(256, 256, 256, 48, 0, None) != 0
    assert "K in {16, 32, 64}" in _hip.LIB.fl_last_error().decode()


def test_rate_probe_lives_outside_the_product_library():
    # The calibration probe is built into calib/libfl_calib.so, which the product library does
    # not contain; its argument checks run on the host.
    import calib

    assert not hasattr(_hip.LIB, "fl_mfma_rate_probe")
    lib = calib.load()
    assert lib.flc_mfma_rate_probe(256, 0, 10, 0, None) != 0
    assert "workgroups" in lib.flc_last_error().decode()
    assert lib.flc_mfma_rate_probe(256, 8, 0, 0, None) != 0
    assert "iters" in lib.flc_last_error().decode()
    assert lib.flc_mfma_rate_probe(256, 8, 10, 4, None) != 0
    assert "flags" in lib.flc_last_error().decode()
    assert lib.flc_mfma_rate_probe(None, 8, 10, 0, None) != 0
    assert "null" in lib.flc_last_error().decode()


def test_noalloc_decode_rejects_workspaces_beyond_its_scratch_array():
    # fl_decode_noalloc keeps the split partials in a 16 MiB array of its own; a call that would
    # need more is refused on the host, before any device call (so this runs without a GPU).
    p = _hip.DecodeParams()
    p.batch, p.heads, p.heads_kv, p.head_dim, p.max_seqlen = 64, 64, 8, 128, 32768
    p.num_splits, p.dtype, p.softmax_scale = 128, 0, 0.088
    assert _hip.LIB.fl_decode_noalloc(ctypes.byref(p), None) == 1
    assert b"exceeds the library's 16 MiB scratch array" in _hip.LIB.fl_last_error()
    p.heads_kv = 7  # shape errors come first, as in fl_decode
    assert _hip.LIB.fl_decode_noalloc(ctypes.byref(p), None) == 1
    assert b"multiple of KV heads" in _hip.LIB.fl_last_error()
