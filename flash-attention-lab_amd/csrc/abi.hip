// The C ABI declared in include/flash_lab_hip.h: argument checks, parameter derivation and
// kernel launch. Host code only (the kernels live in prefill_fwd.hip, prefill_pp.hip, decode.hip,
// decode_mfma.hip and smoke.hip).
//
// The checks restate the reference's op-boundary checks (csrc/common/attn_host.h:18-50,
// csrc/decode/decode_host.h:18-53, csrc/decode/decode.cu:286-293) on plain pointers and strides;
// messages keep the reference's wording where its tests match on it.
#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <mutex>
#include <string>

#include "flash_lab_hip.h"
#include "launch.hpp"

namespace {

// Routing overrides (fl_set_knob); -1 = the built-in rule.
std::atomic<int> g_knobs[FL_KNOB_COUNT] = {-1, -1, -1, -1, -1};
constexpr int64_t kKnobMin[FL_KNOB_COUNT] = {0, 1, 1, 1, 0};
constexpr int64_t kKnobMax[FL_KNOB_COUNT] = {int64_t{1} << 30, int64_t{1} << 20, 64, 4, 1};

thread_local std::string g_last_error;

int fail(int code, const std::string& message) {
  g_last_error = message;
  return code;
}

std::string fmt(const char* f, long long a) {
  char buf[256];
  std::snprintf(buf, sizeof(buf), f, a);
  return buf;
}

bool aligned(const void* p, uintptr_t bytes) { return (reinterpret_cast<uintptr_t>(p) % bytes) == 0; }

// A kernel that moves 16 bytes at a time needs every row to start on a 16-byte boundary: the data
// pointer is 16-byte aligned and every outer stride (of a dimension longer than 1) is a multiple
// of 16 bytes.
bool rows_16_byte(const void* p, int elem_bytes, int64_t size0, int64_t stride0, int64_t size1,
                  int64_t stride1, int64_t size2, int64_t stride2) {
  const int64_t elems = 16 / elem_bytes;
  return aligned(p, 16) && (size0 == 1 || stride0 % elems == 0) &&
         (size1 == 1 || stride1 % elems == 0) && (size2 == 1 || stride2 % elems == 0);
}

int elem_bytes(int32_t dtype) { return dtype == FL_DTYPE_F32 ? 4 : 2; }

bool valid_scale(double s) { return std::isfinite(s) && s > 0.0; }

fl::DType decode_dtype(int32_t dtype) {
  return dtype == FL_DTYPE_BF16 ? fl::DType::bf16 : dtype == FL_DTYPE_F16 ? fl::DType::f16 : fl::DType::f32;
}

// Cache blocks one split may touch at most: its keys (rounded up to the kernel's largest batch of
// 128 keys) over page_size, plus a partial block at each end.
int64_t pages_per_split(int max_seqlen, int num_splits, int page_size) {
  const int64_t keys = (static_cast<int64_t>(max_seqlen) + num_splits - 1) / num_splits + 127;
  return keys / page_size + 2;
}

// Largest power of two (at most 128) whose workgroups fit `capacity` and whose splits keep at
// least min_keys keys.
int largest_splits(int64_t workgroups, int max_seqlen, int64_t capacity, int min_keys) {
  int n = 1;
  while (n < 128 && workgroups * 2 * n <= capacity && max_seqlen / (2 * n) >= min_keys) n *= 2;
  return n;
}

int64_t resident_capacity(int cu_count, int resident_per_cu) {
  const int v = fl::knob(FL_KNOB_DECODE_WG_PER_CU);
  if (v >= 1) resident_per_cu = v;
  return static_cast<int64_t>(resident_per_cu) * (cu_count > 0 ? cu_count : 256);
}

// Largest power of two (at most 128) whose split workgroups all fit the planned slots at once
// (resident_per_cu per CU, the caller's planned_per_cu figure) while each split of the longest
// possible sequence keeps at least 512 keys. One wave of workgroups that fills the GPU streams
// the cache with no tail; measured on MI355X at 32K keys, this beat aiming for two or more
// workgroups per slot. When that leaves fewer workgroups than a quarter of the slots (a short
// cache or few sequences and heads, e.g. one 8K-key sequence with 8 KV heads: 32 workgroups),
// splits go down to 64 keys: many short splits beat a few long ones that leave most CUs idle.
// The matrix-core kernel (one resident workgroup per CU, four 32-key tiles per pass) takes the
// largest count that fills the CUs with at least 128 keys per split: on one 8,448-key sequence
// with 8 KV heads, 32 splits of 264 keys took 14.8 us against 17.4 us for 16 of 528, and at 32K
// keys 32 splits were the fastest too (29.3 us).
int choose_num_splits(int64_t workgroups, int max_seqlen, int cu_count, int resident_per_cu,
                      bool mfma) {
  const int64_t capacity = resident_capacity(cu_count, resident_per_cu);
  auto largest = [&](int min_keys) { return largest_splits(workgroups, max_seqlen, capacity, min_keys); };
  if (mfma) return largest(128);
  const int n = largest(512);
  return workgroups * n * 4 < capacity ? largest(64) : n;
}

// Fewest split workgroups for which a workgroup spans several KV heads: below it, one KV head per
// workgroup gives the GPU more workgroups for the same splits.
constexpr int64_t kMinSpanWorkgroups = 256;
// Keys per split the vector kernel prefers when a cache is long enough to fill the GPU with them.
constexpr int kLongSplitKeys = 2048;

// Split workgroups per CU the plan aims for (the FL_KNOB_DECODE_WG_PER_CU knob overrides it). The
// vector kernel with one query head per workgroup (MHA), two batches of rows in flight per lane,
// streams fastest with one workgroup per CU on a contiguous cache: bf16 at 32K keys, B=8 MHA 609
// us with 4 splits against 639 with 16 (five per CU), B=4 309 against 333, B=16 1,196 against
// 1,296; B=8 at 8K keys 160 against 174, at 4K keys (B=32) 317 against 339; fp16, fp32 and D = 64
// alike. On a paged cache each row address waits for a block-table lookup in LDS, and a second
// workgroup per CU hides it: B=8 MHA with 16-row pages 638 us at two per CU, 670 at five, 740 at
// one. Workgroups of several query heads keep the residency figure (three per CU): at B=8 with a
// group of 2, 167 us against 176 at one per CU; with a group of 4, 174 at either. The matrix-core
// kernel fits one per CU.
int planned_per_cu(const fl_decode_params* p, const fl::DecodeLayout& layout) {
  if (layout.mfma || layout.heads_per_wg > 1) return layout.resident_per_cu;
  return p->block_tables != nullptr ? (layout.resident_per_cu < 2 ? layout.resident_per_cu : 2) : 1;
}

// KV heads per workgroup for a decode with num_splits splits: the widest span the layout allows
// that still yields kMinSpanWorkgroups workgroups, else 1. fl_decode_plan and fl_decode both
// derive it from the same parameters.
int decode_span(const fl_decode_params* p, const fl::DecodeLayout& layout, int num_splits) {
  const int group = p->heads / p->heads_kv;
  for (int s = layout.kv_span; s > 1; s /= 2) {
    const int64_t wg = static_cast<int64_t>(p->batch) * (p->heads_kv / s) * (group / layout.wg_heads);
    if (wg * num_splits >= kMinSpanWorkgroups) return s;
  }
  return 1;
}

// Matrix-core kernel with four KV heads per workgroup, one per wave: the workgroup's loads for a
// key then cover the four heads' rows, one contiguous 1 KiB segment at D = 128 (one KV head per
// workgroup reads 256-byte rows at the cache's row stride). It needs enough work for one
// workgroup per CU with long splits: bf16, 32K keys, B=8 with 8 KV heads 169.4 us (16 splits)
// against 174.2 (one KV head per workgroup, 4 splits); B=4 92.2 against 95.0; B=16 at 8K keys
// 91.0 against 94.5; D = 64 with 8 query heads per KV head 91.4 against 99.5; at B=1 and 2 (too
// few workgroups unless the splits get short) it loses or ties. fl_decode_plan and fl_decode both
// derive it from the same parameters.
constexpr int kMfmaSpan = 4;
constexpr int kMfmaSpanSplitKeys = 1024;
int mfma_span(const fl_decode_params* p, const fl::DecodeLayout& layout, int num_splits) {
  if (!layout.mfma || p->heads_kv % kMfmaSpan != 0) return 1;
  const int forced = fl::knob(FL_KNOB_DECODE_MFMA_SPAN);
  if (forced >= 1) return forced == kMfmaSpan ? kMfmaSpan : 1;
  const int64_t wg = static_cast<int64_t>(p->batch) * (p->heads_kv / kMfmaSpan) * num_splits;
  const bool long_splits = num_splits == 1 || p->max_seqlen / num_splits >= kMfmaSpanSplitKeys;
  return wg >= kMinSpanWorkgroups && long_splits ? kMfmaSpan : 1;
}

// Split count for the four-heads-per-workgroup layout: the largest power of two that keeps one
// workgroup per CU and splits of at least kMfmaSpanSplitKeys keys; 0 if that does not fill the
// CUs (the one-head layout's plan applies then).
int mfma_span_splits(const fl_decode_params* p, const fl::DecodeLayout& layout, int cu_count) {
  if (!layout.mfma || p->heads_kv % kMfmaSpan != 0) return 0;
  const int64_t cus = cu_count > 0 ? cu_count : 256;
  const int64_t groups = static_cast<int64_t>(p->batch) * (p->heads_kv / kMfmaSpan);
  int n = 1;
  while (n < fl::kMaxSplits && groups * 2 * n <= cus && p->max_seqlen / (2 * n) >= kMfmaSpanSplitKeys)
    n *= 2;
  return mfma_span(p, layout, n) == kMfmaSpan ? n : 0;
}

int check_decode_shape(const fl_decode_params* p) {
  if (p == nullptr) return fail(FL_ERR_INVALID, "null decode parameters");
  if (p->block_tables != nullptr && (p->page_size <= 0 || p->num_blocks <= 0))
    return fail(FL_ERR_INVALID, "a paged cache needs page_size > 0 and num_blocks > 0");
  if (p->dtype != FL_DTYPE_BF16 && p->dtype != FL_DTYPE_F16 && p->dtype != FL_DTYPE_F32)
    return fail(FL_ERR_UNSUPPORTED, "decode takes bf16, fp16, or fp32");
  if (p->head_dim != 64 && p->head_dim != 128)
    return fail(FL_ERR_UNSUPPORTED, fmt("unsupported head_dim %lld", p->head_dim));
  if (p->batch <= 0 || p->heads <= 0 || p->heads_kv <= 0 || p->max_seqlen <= 0)
    return fail(FL_ERR_INVALID, "empty input");
  if (p->heads % p->heads_kv != 0)
    return fail(FL_ERR_INVALID, "query heads must be a multiple of KV heads");
  return FL_OK;
}

}  // namespace

int fl::knob(int which) {
  return which >= 0 && which < FL_KNOB_COUNT ? g_knobs[which].load(std::memory_order_relaxed) : -1;
}

namespace {

// Checks, parameter derivation and launch of a decode call whose split workspace (used when
// num_splits > 1) is `workspace`, `workspace_bytes` long: the caller's (fl_decode) or the
// library's scratch array (fl_decode_noalloc).
int decode_call(const fl_decode_params* p, float* workspace, size_t workspace_bytes,
                fl_stream_t stream) {
  if (int rc = check_decode_shape(p)) return rc;
  if (!p->q || !p->k_cache || !p->v_cache || !p->o || !p->lse || !p->seq_lens)
    return fail(FL_ERR_INVALID, "null tensor pointer");
  if (!valid_scale(p->softmax_scale)) return fail(FL_ERR_INVALID, "softmax_scale must be positive");
  if (p->num_splits < 1 || p->num_splits > fl::kMaxSplits)
    return fail(FL_ERR_INVALID, "num_splits must be in [1, 128]");
  const int eb = elem_bytes(p->dtype);
  if (!rows_16_byte(p->q, eb, p->batch, p->q_batch_stride, p->heads, p->q_head_stride, 1, 0))
    return fail(FL_ERR_INVALID, "q must have 16-byte aligned rows");
  // Cache dimensions: [B, S_max] rows, or [num_blocks, page_size] for a paged cache.
  const int64_t outer = p->block_tables != nullptr ? p->num_blocks : p->batch;
  const int64_t rows = p->block_tables != nullptr ? p->page_size : p->max_seqlen;
  if (!rows_16_byte(p->k_cache, eb, outer, p->k_batch_stride, rows, p->k_seq_stride, p->heads_kv,
                    p->k_head_stride))
    return fail(FL_ERR_INVALID, "k_cache must have 16-byte aligned rows (data pointer and strides)");
  if (!rows_16_byte(p->v_cache, eb, outer, p->v_batch_stride, rows, p->v_seq_stride, p->heads_kv,
                    p->v_head_stride))
    return fail(FL_ERR_INVALID, "v_cache must have 16-byte aligned rows (data pointer and strides)");
  if (!aligned(p->o, eb) || !aligned(p->lse, 4) || !aligned(p->seq_lens, 4))
    return fail(FL_ERR_INVALID, "o, lse and seq_lens must be aligned to their element size");
  if (p->block_tables != nullptr && !aligned(p->block_tables, 4))
    return fail(FL_ERR_INVALID, "block_tables must be 4-byte aligned");

  const int group = p->heads / p->heads_kv;
  const fl::DType dt = decode_dtype(p->dtype);
  const fl::DecodeLayout layout = fl::decode_layout(dt, p->head_dim, p->heads_kv, group);
  const int head_chunks = group / layout.heads_per_wg;
  const int64_t blocks = static_cast<int64_t>(p->batch) * p->heads_kv * head_chunks * p->num_splits;
  if (blocks > (int64_t{1} << 24) || static_cast<int64_t>(p->batch) * p->heads > (int64_t{1} << 24))
    return fail(FL_ERR_INVALID, "batch * heads too large");

  fl::DecodeArgs a{};
  a.q = p->q;
  a.k = p->k_cache;
  a.v = p->v_cache;
  a.o = p->o;
  a.lse = p->lse;
  a.seq_lens = p->seq_lens;
  a.q_bs = p->q_batch_stride;
  a.q_hs = p->q_head_stride;
  a.k_bs = p->k_batch_stride;
  a.k_ss = p->k_seq_stride;
  a.k_hs = p->k_head_stride;
  a.v_bs = p->v_batch_stride;
  a.v_ss = p->v_seq_stride;
  a.v_hs = p->v_head_stride;
  a.o_bs = p->o_batch_stride;
  a.o_hs = p->o_head_stride;
  a.batch = p->batch;
  a.heads = p->heads;
  a.heads_kv = p->heads_kv;
  a.group = group;
  a.max_seqlen = p->max_seqlen;
  a.num_splits = p->num_splits;
  a.head_chunks = head_chunks;
  a.kv_span = decode_span(p, layout, p->num_splits);
  a.mfma = layout.mfma;
  a.mfma_span = mfma_span(p, layout, p->num_splits);
  a.block_tables = p->block_tables;
  a.block_tables_stride = p->block_tables_stride;
  a.page_size = p->page_size;
  a.num_blocks = p->num_blocks;
  a.page_table_global =
      p->block_tables != nullptr &&
      pages_per_split(p->max_seqlen, p->num_splits, p->page_size) > fl::kMaxSplitPages;
  if (a.page_table_global) a.kv_span = 1;
  a.page_shift = -1;
  for (int s = 0; s < 31; ++s)
    if (p->page_size == (1 << s)) a.page_shift = s;
  a.scale_log2 = static_cast<float>(p->softmax_scale * 1.4426950408889634);
  if (p->num_splits > 1) {
    const size_t need =
        static_cast<size_t>(p->batch) * p->heads * p->num_splits * (p->head_dim + 2) * sizeof(float);
    if (workspace == nullptr || workspace_bytes < need)
      return fail(FL_ERR_INVALID, "decode workspace is missing or smaller than fl_decode_plan reports");
    if (!aligned(workspace, 16)) return fail(FL_ERR_INVALID, "decode workspace must be 16-byte aligned");
    a.partial_o = workspace;
    a.partial_ml = workspace + static_cast<size_t>(p->batch) * p->heads * p->num_splits * p->head_dim;
  }
  const hipError_t err = fl::launch_decode(a, dt, p->head_dim, static_cast<hipStream_t>(stream));
  if (err != hipSuccess) return fail(FL_ERR_LAUNCH, std::string("decode launch: ") + hipGetErrorString(err));
  return FL_OK;
}

// The split workspace of fl_decode_noalloc: a file-scope device array, one copy per GPU (each GPU
// the library runs on holds it until the process ends). In host code `scratch` is a host-side
// stand-in for the array, not its device address: the address comes from hipGetSymbolAddress,
// looked up once per device with that device current, and only that address is passed on.
constexpr size_t kScratchBytes = size_t{16} << 20;
static __device__ __attribute__((aligned(256))) float scratch[kScratchBytes / sizeof(float)];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
float* g_scratch_ptr[kMaxDevices] = {};

// Device address of the current device's scratch array.
int scratch_for_current_device(float** out) {
  int device = -1;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) return fail(FL_ERR_LAUNCH, std::string("hipGetDevice: ") + hipGetErrorString(err));
  if (device < 0 || device >= kMaxDevices)
    return fail(FL_ERR_INVALID, fmt("device %lld is beyond the scratch table", device));
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[device] == nullptr) {
    void* ptr = nullptr;
    err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || ptr == nullptr)
      return fail(FL_ERR_LAUNCH, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(err));
    g_scratch_ptr[device] = static_cast<float*>(ptr);
  }
  *out = g_scratch_ptr[device];
  return FL_OK;
}

}  // namespace

extern "C" {

int fl_set_knob(int32_t knob, int64_t value) {
  if (knob < 0 || knob >= FL_KNOB_COUNT) return fail(FL_ERR_INVALID, fmt("unknown knob %lld", knob));
  if (value != -1 && (value < kKnobMin[knob] || value > kKnobMax[knob]))
    return fail(FL_ERR_INVALID, fmt("knob value %lld out of range", value));
  g_knobs[knob].store(static_cast<int>(value), std::memory_order_relaxed);
  return FL_OK;
}

int64_t fl_get_knob(int32_t knob) {
  if (knob < 0 || knob >= FL_KNOB_COUNT) return -2;
  return g_knobs[knob].load(std::memory_order_relaxed);
}

const char* fl_last_error(void) { return g_last_error.c_str(); }

const char* fl_version(void) { return "flash_lab_hip 0.1.0 gfx950"; }

int fl_attention_fwd(const fl_attn_params* p, fl_stream_t stream) {
  if (p == nullptr) return fail(FL_ERR_INVALID, "null attention parameters");
  if (p->dtype != FL_DTYPE_BF16 && p->dtype != FL_DTYPE_F16)
    return fail(FL_ERR_UNSUPPORTED, "attention_mma_pipelined takes bf16 or fp16");
  if (p->head_dim != 64 && p->head_dim != 128)
    return fail(FL_ERR_UNSUPPORTED, fmt("unsupported head_dim %lld", p->head_dim));
  if (p->batch <= 0 || p->seqlen_q <= 0 || p->seqlen_k <= 0 || p->heads <= 0 || p->heads_kv <= 0)
    return fail(FL_ERR_INVALID, "empty input");
  if (p->heads % p->heads_kv != 0)
    return fail(FL_ERR_INVALID, "query heads must be a multiple of KV heads");
  if (!valid_scale(p->softmax_scale)) return fail(FL_ERR_INVALID, "softmax_scale must be positive");
  if (!p->q || !p->k || !p->v || !p->o || !p->lse)
    return fail(FL_ERR_INVALID, "null tensor pointer");
  const int eb = elem_bytes(p->dtype);
  if (!rows_16_byte(p->q, eb, p->batch, p->q_batch_stride, p->seqlen_q, p->q_seq_stride, p->heads,
                    p->q_head_stride))
    return fail(FL_ERR_INVALID, "q must have 16-byte aligned rows (data pointer and strides)");
  if (!rows_16_byte(p->k, eb, p->batch, p->k_batch_stride, p->seqlen_k, p->k_seq_stride,
                    p->heads_kv, p->k_head_stride))
    return fail(FL_ERR_INVALID, "k must have 16-byte aligned rows (data pointer and strides)");
  if (!rows_16_byte(p->v, eb, p->batch, p->v_batch_stride, p->seqlen_k, p->v_seq_stride,
                    p->heads_kv, p->v_head_stride))
    return fail(FL_ERR_INVALID, "v must have 16-byte aligned rows (data pointer and strides)");
  if (!rows_16_byte(p->o, eb, p->batch, p->o_batch_stride, p->seqlen_q, p->o_seq_stride, p->heads,
                    p->o_head_stride))
    return fail(FL_ERR_INVALID, "o must have 16-byte aligned rows (data pointer and strides)");
  if (!aligned(p->lse, 4)) return fail(FL_ERR_INVALID, "lse must be 4-byte aligned");
  // Tile loads address K and V rows through 32-bit byte offsets from a per-tile base, and rely on
  // rows not overlapping (sequence stride >= head_dim) to zero-fill past the end.
  const int64_t max_seq_stride = ((int64_t{1} << 31) / 2 - p->head_dim) / fl::kPrefillBlockN;
  if (p->seqlen_k > 1 && (p->k_seq_stride < p->head_dim || p->v_seq_stride < p->head_dim))
    return fail(FL_ERR_INVALID, "k and v rows must not overlap (sequence stride >= head_dim)");
  if (p->k_seq_stride > max_seq_stride || p->v_seq_stride > max_seq_stride)
    return fail(FL_ERR_INVALID, "k or v sequence stride too large");

  const int64_t q_blocks = (static_cast<int64_t>(p->seqlen_q) + fl::kPrefillBlockM - 1) /
                           fl::kPrefillBlockM;
  const int64_t blocks = q_blocks * p->batch * p->heads;
  if (blocks > (int64_t{1} << 24))
    return fail(FL_ERR_INVALID, "batch * heads * query blocks exceeds the grid limit");

  fl::PrefillArgs a{};
  a.q = static_cast<const uint16_t*>(p->q);
  a.k = static_cast<const uint16_t*>(p->k);
  a.v = static_cast<const uint16_t*>(p->v);
  a.o = static_cast<uint16_t*>(p->o);
  a.lse = p->lse;
  a.q_bs = p->q_batch_stride;
  a.q_ss = p->q_seq_stride;
  a.q_hs = p->q_head_stride;
  a.k_bs = p->k_batch_stride;
  a.k_ss = p->k_seq_stride;
  a.k_hs = p->k_head_stride;
  a.v_bs = p->v_batch_stride;
  a.v_ss = p->v_seq_stride;
  a.v_hs = p->v_head_stride;
  a.o_bs = p->o_batch_stride;
  a.o_ss = p->o_seq_stride;
  a.o_hs = p->o_head_stride;
  a.batch = p->batch;
  a.seqlen_q = p->seqlen_q;
  a.seqlen_k = p->seqlen_k;
  a.heads = p->heads;
  a.heads_kv = p->heads_kv;
  a.group = p->heads / p->heads_kv;
  a.causal_offset = p->seqlen_k - p->seqlen_q;
  a.causal = p->causal != 0;
  a.scale = static_cast<float>(p->softmax_scale);
  a.scale_log2 = static_cast<float>(p->softmax_scale * 1.4426950408889634);
  a.q_blocks = static_cast<int>(q_blocks);

  const fl::DType dt = p->dtype == FL_DTYPE_BF16 ? fl::DType::bf16 : fl::DType::f16;
  const hipError_t err = fl::launch_prefill(a, dt, p->head_dim, static_cast<hipStream_t>(stream));
  if (err != hipSuccess) return fail(FL_ERR_LAUNCH, std::string("prefill launch: ") + hipGetErrorString(err));
  return FL_OK;
}

int fl_decode_plan(const fl_decode_params* p, int32_t requested_splits, int32_t allow_splits,
                   int32_t cu_count, int32_t* num_splits, size_t* workspace_bytes) {
  if (int rc = check_decode_shape(p)) return rc;
  if (requested_splits < 0 || requested_splits > 128)
    return fail(FL_ERR_INVALID, "num_splits must be in [0, 128]");
  if (num_splits == nullptr || workspace_bytes == nullptr)
    return fail(FL_ERR_INVALID, "null output pointer");
  const int group = p->heads / p->heads_kv;
  const fl::DecodeLayout layout =
      fl::decode_layout(decode_dtype(p->dtype), p->head_dim, p->heads_kv, group);
  int n = 1;
  if (allow_splits && requested_splits > 0) {
    n = requested_splits;
  } else if (allow_splits) {
    // The widest span whose workgroups (with the split count it leads to) reach
    // kMinSpanWorkgroups; else one KV head per workgroup.
    int64_t planned_wg = 0;
    for (int s = layout.kv_span; s >= 1; s /= 2) {
      const int64_t wg = static_cast<int64_t>(p->batch) * (p->heads_kv / s) * (group / layout.wg_heads);
      n = choose_num_splits(wg, p->max_seqlen, cu_count, planned_per_cu(p, layout), layout.mfma != 0);
      planned_wg = wg * n;
      if (s == 1 || planned_wg >= kMinSpanWorkgroups) break;
    }
    if (const int n4 = mfma_span_splits(p, layout, cu_count)) n = n4;
    // MHA at head_dim 128, 16-bit (the measured case), with at most two workgroups per CU that
    // way (few sequences, a long cache): at least 16 splits of at least kLongSplitKeys keys
    // instead, if some span then still gives every CU a workgroup. B=1, 32 KV heads, 32K keys: 16
    // splits of 2 KV heads 83.2-83.7 us against 84.7-85.3 for 32 splits of 4.
    const int cus = cu_count > 0 ? cu_count : 256;
    if (!layout.mfma && group == 1 && p->head_dim == 128 && p->dtype != FL_DTYPE_F32 &&
        planned_wg <= 2 * cus) {
      const int64_t capacity = resident_capacity(cu_count, planned_per_cu(p, layout));
      for (int s = layout.kv_span; s >= 1; s /= 2) {
        const int64_t wg = static_cast<int64_t>(p->batch) * (p->heads_kv / s) * (group / layout.wg_heads);
        const int m = largest_splits(wg, p->max_seqlen, capacity, kLongSplitKeys);
        if (m >= 16 && wg * m >= kMinSpanWorkgroups && p->max_seqlen / m >= kLongSplitKeys) {
          n = m;
          break;
        }
      }
    }
  }
  if (p->block_tables != nullptr && allow_splits && requested_splits == 0) {
    // A paged split stages its block numbers in LDS when they fit: take more splits if one would
    // touch too many (a longer split still works, reading the table from global memory).
    while (n < fl::kMaxSplits && pages_per_split(p->max_seqlen, n, p->page_size) > fl::kMaxSplitPages)
      n *= 2;
  }
  *num_splits = n;
  *workspace_bytes =
      n > 1 ? static_cast<size_t>(p->batch) * p->heads * n * (p->head_dim + 2) * sizeof(float) : 0;
  return FL_OK;
}

int fl_decode(const fl_decode_params* p, fl_stream_t stream) {
  if (p == nullptr) return fail(FL_ERR_INVALID, "null decode parameters");
  return decode_call(p, p->workspace, p->workspace_bytes, stream);
}

int fl_decode_noalloc(const fl_decode_params* p, fl_stream_t stream) {
  if (int rc = check_decode_shape(p)) return rc;
  float* ws = nullptr;
  if (p->num_splits > 1) {
    // Compared in floating point so that no product of the sizes can overflow before the check.
    const double need = static_cast<double>(p->batch) * p->heads * p->num_splits *
                        (p->head_dim + 2) * sizeof(float);
    if (need > static_cast<double>(kScratchBytes))
      return fail(FL_ERR_INVALID,
                  fmt("fl_decode_noalloc: the split workspace (%lld bytes) exceeds the library's "
                      "16 MiB scratch array; use fewer splits or fl_decode",
                      static_cast<long long>(need)));
    if (int rc = scratch_for_current_device(&ws)) return rc;
  }
  return decode_call(p, ws, kScratchBytes, stream);
}

int fl_smoke_axpy(const float* x, const float* y, float alpha, float* out, int64_t n,
                  fl_stream_t stream) {
  if (n < 0) return fail(FL_ERR_INVALID, "n must be non-negative");
  if (n > 0 && (!x || !y || !out)) return fail(FL_ERR_INVALID, "null tensor pointer");
  if (n > (int64_t{1} << 40)) return fail(FL_ERR_INVALID, "n too large");
  const hipError_t err = fl::launch_axpy(x, y, alpha, out, n, static_cast<hipStream_t>(stream));
  if (err != hipSuccess) return fail(FL_ERR_LAUNCH, std::string("axpy launch: ") + hipGetErrorString(err));
  return FL_OK;
}

int fl_mfma_tile_test(const void* a, const void* b, float* c, int32_t k, int32_t trans_b,
                      fl_stream_t stream) {
  if (k != 16 && k != 32 && k != 64) return fail(FL_ERR_INVALID, "a must be [16, K] with K in {16, 32, 64}");
  if (!a || !b || !c) return fail(FL_ERR_INVALID, "null tensor pointer");
  const hipError_t err =
      fl::launch_mfma_tile_test(static_cast<const uint16_t*>(a), static_cast<const uint16_t*>(b), c,
                                k, trans_b != 0, static_cast<hipStream_t>(stream));
  if (err != hipSuccess) return fail(FL_ERR_LAUNCH, std::string("tile test launch: ") + hipGetErrorString(err));
  return FL_OK;
}

}  // extern "C"
