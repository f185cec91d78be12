"""The gfx950 kernels as torch ops: ctypes over the C ABI of libflash_lab_hip.so.

This module replaces the reference's compiled op registry (csrc/bindings.cpp:7-42) and its C++
host wrappers (csrc/common/attn_host.h, csrc/decode/decode.cu:282-347). Importing it loads the
library and registers, under torch.ops.flash_lab, ops with the reference's names and schemas:

    attention_mma_pipelined / attention_mma
        (Tensor q, Tensor k, Tensor v, bool causal, float softmax_scale) -> (Tensor, Tensor)
    decode_splitkv / decode_inplace
        (Tensor q, Tensor k_cache, Tensor v_cache, Tensor seq_lens, float softmax_scale,
         int num_splits) -> (Tensor, Tensor)
    smoke_axpy(Tensor x, Tensor y, float alpha) -> Tensor
    mma_tile_test(Tensor a, Tensor b, bool trans_b) -> Tensor

Each op allocates its outputs (and the decode workspace) with torch on the input's device, passes
the current stream, and raises RuntimeError with the library's message when a call fails. Nothing
here synchronizes, reads seq_lens on the host or allocates outside torch's caching allocator, so
the ops can be captured in a HIP graph. If the library cannot be loaded, importing this module
raises ImportError; there is no other code path.
"""

from __future__ import annotations

import contextlib
import ctypes
import functools
import math
import os
from pathlib import Path

import torch

LIB_NAME = "libflash_lab_hip.so"
LIB_PATH = Path(os.environ.get("FLASH_LAB_HIP_LIB", Path(__file__).with_name(LIB_NAME)))

DTYPE_CODES = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}


class AttnParams(ctypes.Structure):
    """fl_attn_params of include/flash_lab_hip.h."""

    _fields_ = [
        ("q", ctypes.c_void_p),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("o", ctypes.c_void_p),
        ("lse", ctypes.c_void_p),
        *[
            (f"{t}_{s}_stride", ctypes.c_int64)
            for t in ("q", "k", "v", "o")
            for s in ("batch", "seq", "head")
        ],
        ("batch", ctypes.c_int32),
        ("seqlen_q", ctypes.c_int32),
        ("seqlen_k", ctypes.c_int32),
        ("heads", ctypes.c_int32),
        ("heads_kv", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("causal", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("softmax_scale", ctypes.c_double),
    ]


class DecodeParams(ctypes.Structure):
    """fl_decode_params of include/flash_lab_hip.h."""

    _fields_ = [
        ("q", ctypes.c_void_p),
        ("k_cache", ctypes.c_void_p),
        ("v_cache", ctypes.c_void_p),
        ("o", ctypes.c_void_p),
        ("lse", ctypes.c_void_p),
        ("seq_lens", ctypes.c_void_p),
        ("q_batch_stride", ctypes.c_int64),
        ("q_head_stride", ctypes.c_int64),
        ("k_batch_stride", ctypes.c_int64),
        ("k_seq_stride", ctypes.c_int64),
        ("k_head_stride", ctypes.c_int64),
        ("v_batch_stride", ctypes.c_int64),
        ("v_seq_stride", ctypes.c_int64),
        ("v_head_stride", ctypes.c_int64),
        ("o_batch_stride", ctypes.c_int64),
        ("o_head_stride", ctypes.c_int64),
        ("batch", ctypes.c_int32),
        ("heads", ctypes.c_int32),
        ("heads_kv", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("max_seqlen", ctypes.c_int32),
        ("num_splits", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("softmax_scale", ctypes.c_double),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
        ("block_tables", ctypes.c_void_p),
        ("block_tables_stride", ctypes.c_int64),
        ("page_size", ctypes.c_int32),
        ("num_blocks", ctypes.c_int32),
    ]


# Every symbol include/flash_lab_hip.h declares, with its ctypes signature.
SIGNATURES = {
    "fl_attention_fwd": (ctypes.c_int, [ctypes.POINTER(AttnParams), ctypes.c_void_p]),
    "fl_decode_plan": (
        ctypes.c_int,
        [
            ctypes.POINTER(DecodeParams),
            ctypes.c_int32,
            ctypes.c_int32,
            ctypes.c_int32,
            ctypes.POINTER(ctypes.c_int32),
            ctypes.POINTER(ctypes.c_size_t),
        ],
    ),
    "fl_decode": (ctypes.c_int, [ctypes.POINTER(DecodeParams), ctypes.c_void_p]),
    "fl_decode_noalloc": (ctypes.c_int, [ctypes.POINTER(DecodeParams), ctypes.c_void_p]),
    "fl_smoke_axpy": (
        ctypes.c_int,
        [
            ctypes.c_void_p,
            ctypes.c_void_p,
            ctypes.c_float,
            ctypes.c_void_p,
            ctypes.c_int64,
            ctypes.c_void_p,
        ],
    ),
    "fl_mfma_tile_test": (
        ctypes.c_int,
        [
            ctypes.c_void_p,
            ctypes.c_void_p,
            ctypes.c_void_p,
            ctypes.c_int32,
            ctypes.c_int32,
            ctypes.c_void_p,
        ],
    ),
    "fl_set_knob": (ctypes.c_int, [ctypes.c_int32, ctypes.c_int64]),
    "fl_get_knob": (ctypes.c_int64, [ctypes.c_int32]),
    "fl_last_error": (ctypes.c_char_p, []),
    "fl_version": (ctypes.c_char_p, []),
}


def load_library(path: Path = LIB_PATH) -> ctypes.CDLL:
    """Loads the library and attaches the C signatures. torch is imported first, so the HIP
    runtime the library links against is the one torch already loaded."""
    if not path.exists():
        raise ImportError(
            f"{path} is missing; build it with `python flash-attention-lab_amd/csrc/build.py`"
        )
    try:
        lib = ctypes.CDLL(str(path))
    except OSError as exc:
        raise ImportError(f"could not load {path}: {exc}") from exc
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    return lib


LIB = load_library()


def _check(rc: int) -> None:
    if rc != 0:
        raise RuntimeError(LIB.fl_last_error().decode())


# Routing overrides of the library (enum fl_knob): test and experiment hooks that pin a call to
# one of the kernels. None restores the built-in rule.
KNOBS = {"prefill_pp_min_wg": 0, "decode_mfma_min_group": 1, "decode_wg_per_cu": 2,
         "decode_mfma_span": 3, "prefill_causal_stream": 4}


def set_knob(name: str, value: int | None) -> None:
    _check(LIB.fl_set_knob(KNOBS[name], -1 if value is None else int(value)))


def get_knob(name: str) -> int | None:
    value = LIB.fl_get_knob(KNOBS[name])
    return None if value == -1 else value


@contextlib.contextmanager
def knob(name: str, value: int | None):
    """Sets a routing knob for the duration of the block, then restores its previous value."""
    previous = get_knob(name)
    set_knob(name, value)
    try:
        yield
    finally:
        set_knob(name, previous)


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


class _on_device:
    """Makes `device` current for the call when it is not already (the role of the reference's
    OptionalCUDAGuard)."""

    def __init__(self, device: torch.device):
        self.device = device
        self.ctx = None

    def __enter__(self):
        if self.device.index is not None and self.device.index != torch.cuda.current_device():
            self.ctx = torch.cuda.device(self.device)
            self.ctx.__enter__()

    def __exit__(self, *exc):
        if self.ctx is not None:
            self.ctx.__exit__(*exc)


@functools.lru_cache(maxsize=None)
def cu_count(index: int) -> int:
    return torch.cuda.get_device_properties(index).multi_processor_count


def _require(cond: bool, message: str, *args) -> None:
    """Raises RuntimeError(message % args) unless cond; the message is only formatted on failure
    (these checks run on every op call)."""
    if not cond:
        raise RuntimeError(message % args if args else message)


def _check_cuda(**tensors: torch.Tensor) -> None:
    for name, x in tensors.items():
        _require(x.is_cuda, "%s must be a CUDA tensor", name)


# ----------------------------------------------------------------------------------------------
# Prefill


def prefill(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool, softmax_scale: float):
    """Op-boundary checks of the reference (csrc/common/attn_host.h:18-57), output allocation,
    and the fl_attention_fwd call."""
    _check_cuda(q=q, k=k, v=v)
    _require(q.dtype in (torch.bfloat16, torch.float16), "attention_mma_pipelined takes bf16 or fp16")
    _require(k.dtype == q.dtype and v.dtype == q.dtype, "k and v must have dtype %s", q.dtype)
    _require(q.dim() == 4 and k.dim() == 4 and v.dim() == 4, "q, k, v must be [B, S, H, D]")
    _require(k.shape == v.shape, "k and v must have the same shape")
    _require(
        q.shape[0] == k.shape[0] and q.shape[3] == k.shape[3],
        "q and k must agree on batch size and head_dim",
    )
    _require(q.device == k.device and q.device == v.device, "q, k, v on different devices")
    for name, x in (("q", q), ("k", k), ("v", v)):
        _require(x.stride(-1) == 1, "%s must be contiguous in its last dimension", name)
    batch, seqlen_q, heads, head_dim = q.shape
    # The kernel needs non-overlapping K and V rows (sequence stride >= head_dim); broadcast or
    # overlapping views, which the reference also accepts, are passed as contiguous copies.
    if k.shape[1] > 1 and k.stride(1) < head_dim:
        k = k.contiguous()
    if v.shape[1] > 1 and v.stride(1) < head_dim:
        v = v.contiguous()
    o = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    lse = torch.empty((batch, heads, seqlen_q), dtype=torch.float32, device=q.device)
    p = AttnParams(
        q.data_ptr(),
        k.data_ptr(),
        v.data_ptr(),
        o.data_ptr(),
        lse.data_ptr(),
        *q.stride()[:3],
        *k.stride()[:3],
        *v.stride()[:3],
        *o.stride()[:3],
        batch,
        seqlen_q,
        k.shape[1],
        heads,
        k.shape[2],
        head_dim,
        int(bool(causal)),
        DTYPE_CODES[q.dtype],
        float(softmax_scale),
    )
    with _on_device(q.device):
        _check(LIB.fl_attention_fwd(ctypes.byref(p), _stream(q.device)))
    return o, lse


# ----------------------------------------------------------------------------------------------
# Decode


def _decode_params(q, k_cache, v_cache, seq_lens, o, lse, softmax_scale,
                   block_tables=None) -> DecodeParams:
    batch, heads, head_dim = q.shape
    if block_tables is not None:
        # [num_blocks, page_size, H_kv, D] caches: the batch strides are block strides.
        p = _decode_params(q, k_cache, v_cache, seq_lens, o, lse, softmax_scale)
        p.max_seqlen = block_tables.shape[1] * k_cache.shape[1]
        p.block_tables = block_tables.data_ptr()
        p.block_tables_stride = block_tables.stride(0)
        p.page_size = k_cache.shape[1]
        p.num_blocks = k_cache.shape[0]
        return p
    return DecodeParams(
        q.data_ptr(),
        k_cache.data_ptr(),
        v_cache.data_ptr(),
        o.data_ptr(),
        lse.data_ptr(),
        seq_lens.data_ptr(),
        q.stride(0),
        q.stride(1),
        *k_cache.stride()[:3],
        *v_cache.stride()[:3],
        o.stride(0),
        o.stride(1),
        batch,
        heads,
        k_cache.shape[2],
        head_dim,
        k_cache.shape[1],
        1,
        DTYPE_CODES[q.dtype],
        float(softmax_scale),
        None,
        0,
    )


def decode(q, k_cache, v_cache, seq_lens, softmax_scale: float, num_splits: int, allow_splits: bool,
           block_tables=None):
    """Op-boundary checks of the reference (csrc/decode/decode_host.h:18-53,
    csrc/decode/decode.cu:286-311), output and workspace allocation, fl_decode_plan + fl_decode.
    With block_tables the caches are paged, [num_blocks, page_size, H_kv, D] (a layout the
    reference defines but none of its kernels runs)."""
    _check_cuda(q=q, k_cache=k_cache, v_cache=v_cache, seq_lens=seq_lens)
    _require(q.dtype in DTYPE_CODES, "decode takes bf16, fp16, or fp32")
    _require(
        k_cache.dtype == q.dtype and v_cache.dtype == q.dtype,
        "k_cache and v_cache must have dtype %s",
        q.dtype,
    )
    _require(seq_lens.dtype == torch.int32, "seq_lens must have dtype int32")
    _require(q.dim() == 3 and k_cache.dim() == 4, "q must be [B, H, D], caches [B, S_max, H_kv, D]")
    _require(k_cache.shape == v_cache.shape, "k_cache and v_cache must have the same shape")
    if block_tables is None:
        _require(
            k_cache.shape[0] == q.shape[0] and k_cache.shape[3] == q.shape[2],
            "q and the caches must agree on batch size and head_dim",
        )
    else:
        _check_cuda(block_tables=block_tables)
        _require(block_tables.dtype == torch.int32, "block_tables must have dtype int32")
        _require(
            block_tables.dim() == 2 and block_tables.shape[0] == q.shape[0]
            and block_tables.shape[1] >= 1 and block_tables.stride(1) == 1,
            "block_tables must be [B, max_blocks] with unit stride in its last dimension",
        )
        _require(k_cache.shape[3] == q.shape[2], "q and the caches must agree on head_dim")
        _require(
            block_tables.shape[1] * k_cache.shape[1] < 2**31,
            "paged cache too long (max_blocks * page_size must fit in int32)",
        )
    _require(seq_lens.dim() == 1 and seq_lens.shape[0] == q.shape[0], "seq_lens must be [B]")
    _require(seq_lens.is_contiguous(), "seq_lens must be contiguous")
    for name, x in (("q", q), ("k_cache", k_cache), ("v_cache", v_cache)):
        _require(x.stride(-1) == 1, "%s must be contiguous in its last dimension", name)
    _require(0 <= num_splits <= 128, "num_splits must be in [0, 128]")

    o = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    lse = torch.empty(q.shape[:2], dtype=torch.float32, device=q.device)
    p = _decode_params(q, k_cache, v_cache, seq_lens, o, lse, softmax_scale, block_tables)
    index = q.device.index if q.device.index is not None else torch.cuda.current_device()
    splits, ws_bytes = ctypes.c_int32(), ctypes.c_size_t()
    _check(LIB.fl_decode_plan(ctypes.byref(p), int(num_splits), int(bool(allow_splits)),
                              cu_count(index), ctypes.byref(splits), ctypes.byref(ws_bytes)))
    splits, ws_bytes = splits.value, ws_bytes.value
    p.num_splits = splits
    workspace = None
    if ws_bytes:
        workspace = torch.empty(ws_bytes // 4, dtype=torch.float32, device=q.device)
        p.workspace = workspace.data_ptr()
        p.workspace_bytes = ws_bytes
    with _on_device(q.device):
        _check(LIB.fl_decode(ctypes.byref(p), _stream(q.device)))
    return o, lse


def decode_noalloc(q, k_cache, v_cache, seq_lens, o, lse, softmax_scale: float, num_splits: int,
                   block_tables=None) -> int:
    """fl_decode_noalloc on caller-provided outputs o [B, H, D] and lse [B, H]: the split workspace
    is the library's own scratch array, so nothing is allocated. num_splits 0 takes the planned
    count. Returns the split count used. The arguments are taken as valid (the public ops check
    them); this is the allocation-free path for callers that manage their own buffers."""
    p = _decode_params(q, k_cache, v_cache, seq_lens, o, lse, softmax_scale, block_tables)
    index = q.device.index if q.device.index is not None else torch.cuda.current_device()
    splits, ws_bytes = ctypes.c_int32(), ctypes.c_size_t()
    _check(LIB.fl_decode_plan(ctypes.byref(p), int(num_splits), 1, cu_count(index),
                              ctypes.byref(splits), ctypes.byref(ws_bytes)))
    p.num_splits = splits.value
    with _on_device(q.device):
        _check(LIB.fl_decode_noalloc(ctypes.byref(p), _stream(q.device)))
    return splits.value


def decode_plan(batch, heads, heads_kv, head_dim, max_seqlen, dtype, num_splits=0,
                allow_splits=True, cu_count_=256) -> tuple[int, int]:
    """(num_splits, workspace bytes) the library picks for a decode shape; host-only."""
    p = DecodeParams()
    p.batch, p.heads, p.heads_kv, p.head_dim, p.max_seqlen = batch, heads, heads_kv, head_dim, max_seqlen
    p.dtype = DTYPE_CODES[dtype]
    splits = ctypes.c_int32()
    ws = ctypes.c_size_t()
    _check(LIB.fl_decode_plan(ctypes.byref(p), num_splits, int(allow_splits), cu_count_,
                              ctypes.byref(splits), ctypes.byref(ws)))
    return splits.value, ws.value


# ----------------------------------------------------------------------------------------------
# Op registration


# The reference's schemas, verbatim (csrc/bindings.cpp:9-41).
PREFILL_SCHEMA = "(Tensor q, Tensor k, Tensor v, bool causal, float softmax_scale) -> (Tensor, Tensor)"
DECODE_SCHEMA = (
    "(Tensor q, Tensor k_cache, Tensor v_cache, Tensor seq_lens, float softmax_scale,"
    " int num_splits) -> (Tensor, Tensor)"
)
# Paged-cache decode has no op in the reference (its kernels reject paged caches): the same
# schema with the block tables after seq_lens.
PAGED_DECODE_SCHEMA = (
    "(Tensor q, Tensor k_cache, Tensor v_cache, Tensor seq_lens, Tensor block_tables,"
    " float softmax_scale, int num_splits) -> (Tensor, Tensor)"
)


def _register() -> None:
    lib = "flash_lab"

    def prefill_op(name):
        @torch.library.custom_op(
            f"{lib}::{name}", mutates_args=(), device_types="cuda", schema=PREFILL_SCHEMA
        )
        def op(
            q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool, softmax_scale: float
        ) -> tuple[torch.Tensor, torch.Tensor]:
            return prefill(q, k, v, causal, softmax_scale)

        return op

    def decode_op(name, allow_splits):
        @torch.library.custom_op(
            f"{lib}::{name}", mutates_args=(), device_types="cuda", schema=DECODE_SCHEMA
        )
        def op(
            q: torch.Tensor,
            k_cache: torch.Tensor,
            v_cache: torch.Tensor,
            seq_lens: torch.Tensor,
            softmax_scale: float,
            num_splits: int,
        ) -> tuple[torch.Tensor, torch.Tensor]:
            return decode(q, k_cache, v_cache, seq_lens, softmax_scale, num_splits, allow_splits)

        return op

    prefill_op("attention_mma_pipelined")
    prefill_op("attention_mma")
    def paged_decode_op(name, allow_splits):
        @torch.library.custom_op(
            f"{lib}::{name}", mutates_args=(), device_types="cuda", schema=PAGED_DECODE_SCHEMA
        )
        def op(
            q: torch.Tensor,
            k_cache: torch.Tensor,
            v_cache: torch.Tensor,
            seq_lens: torch.Tensor,
            block_tables: torch.Tensor,
            softmax_scale: float,
            num_splits: int,
        ) -> tuple[torch.Tensor, torch.Tensor]:
            return decode(q, k_cache, v_cache, seq_lens, softmax_scale, num_splits, allow_splits,
                          block_tables)

        return op

    decode_op("decode_splitkv", True)
    decode_op("decode_inplace", False)
    paged_decode_op("decode_splitkv_paged", True)
    paged_decode_op("decode_inplace_paged", False)

    @torch.library.custom_op(
        f"{lib}::smoke_axpy", mutates_args=(), device_types="cuda",
        schema="(Tensor x, Tensor y, float alpha) -> Tensor",
    )
    def smoke_axpy(x: torch.Tensor, y: torch.Tensor, alpha: float) -> torch.Tensor:
        _check_cuda(x=x, y=y)
        _require(x.dtype == torch.float32 and y.dtype == torch.float32, "x and y must be fp32")
        _require(x.shape == y.shape, "x and y must have the same shape")
        xc, yc = x.contiguous(), y.contiguous()
        out = torch.empty_like(xc)
        with _on_device(x.device):
            _check(
                LIB.fl_smoke_axpy(
                    xc.data_ptr(), yc.data_ptr(), float(alpha), out.data_ptr(), xc.numel(),
                    _stream(x.device),
                )
            )
        return out

    @smoke_axpy.register_fake
    def _(x, y, alpha):
        return torch.empty_like(x, memory_format=torch.contiguous_format)

    @torch.library.custom_op(
        f"{lib}::mma_tile_test", mutates_args=(), device_types="cuda",
        schema="(Tensor a, Tensor b, bool trans_b) -> Tensor",
    )
    def mma_tile_test(a: torch.Tensor, b: torch.Tensor, trans_b: bool) -> torch.Tensor:
        _check_cuda(a=a, b=b)
        _require(a.dtype == torch.bfloat16 and b.dtype == torch.bfloat16, "a and b must be bf16")
        _require(a.dim() == 2 and a.shape[0] == 16 and a.shape[1] in (16, 32, 64),
                 "a must be [16, K]")
        k = a.shape[1]
        want = (k, 16) if trans_b else (16, k)
        _require(tuple(b.shape) == want, "b must be [K, 16] with trans_b, else [16, K]")
        ac, bc = a.contiguous(), b.contiguous()
        c = torch.empty((16, 16), dtype=torch.float32, device=a.device)
        with _on_device(a.device):
            _check(
                LIB.fl_mfma_tile_test(
                    ac.data_ptr(), bc.data_ptr(), c.data_ptr(), k, int(bool(trans_b)),
                    _stream(a.device),
                )
            )
        return c

    @mma_tile_test.register_fake
    def _(a, b, trans_b):
        return a.new_empty((16, 16), dtype=torch.float32)


_register()

OPS = (
    "attention_mma_pipelined",
    "attention_mma",
    "decode_splitkv",
    "decode_inplace",
    "decode_splitkv_paged",
    "decode_inplace_paged",
    "smoke_axpy",
    "mma_tile_test",
)


def default_scale(head_dim: int) -> float:
    return 1.0 / math.sqrt(head_dim)
