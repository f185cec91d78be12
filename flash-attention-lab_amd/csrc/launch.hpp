// Internal interface between the C ABI (abi.cpp) and the kernel files. Device-side argument
// structs are passed to the kernels by value; everything in them is already validated.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "flash_lab_hip.h"

namespace fl {

// Prefill problem as the kernels see it. Tensors are [B, S, H, D] with unit stride in D; strides
// are in elements. Query head h reads KV head h / group; query row i sees key j iff
// j <= i + causal_offset (bottom-right aligned causal mask).
struct PrefillArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  float* lse;  // [B, H, S_q]
  int64_t q_bs, q_ss, q_hs;
  int64_t k_bs, k_ss, k_hs;
  int64_t v_bs, v_ss, v_hs;
  int64_t o_bs, o_ss, o_hs;
  int batch, seqlen_q, seqlen_k, heads, heads_kv, group, causal_offset, causal;
  float scale;       // softmax scale, natural-log domain (used for the LSE)
  float scale_log2;  // scale * log2(e): probabilities are 2^(s * scale_log2 - ref)
  int q_blocks;      // ceil(S_q / rows per workgroup)
};

// Decode problem. q [B, H, D], caches [B, S_max, H_kv, D], o [B, H, D], lse [B, H].
struct DecodeArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  float* lse;
  const int32_t* seq_lens;
  int64_t q_bs, q_hs;
  int64_t k_bs, k_ss, k_hs;
  int64_t v_bs, v_ss, v_hs;
  int64_t o_bs, o_hs;
  int batch, heads, heads_kv, group, max_seqlen;
  int num_splits;
  int head_chunks;   // group / query heads served per workgroup (of each KV head)
  int kv_span;       // adjacent KV heads per workgroup (1, 2 or 4; divides heads_kv)
  float scale_log2;  // q is multiplied by this, so scores are in the log2 domain
  float* partial_o;  // [B, H, num_splits, D] unnormalized fp32 partial outputs
  float* partial_ml; // [B, H, num_splits, 2] (max in log2 units, sum) per split
  // Paged cache (block_tables non-null): k/v are [num_blocks, page_size, H_kv, D], k_bs/v_bs the
  // block strides, block_tables [B, *] int32 with row stride block_tables_stride.
  const int32_t* block_tables;
  int64_t block_tables_stride;
  int page_size, num_blocks;
  int page_shift;  // log2(page_size) when it is a power of two, else -1
  // Some split touches more than kMaxSplitPages blocks: block numbers are read from global memory
  // (and kv_span is 1).
  int page_table_global;
  // The matrix-core split kernel (decode_mfma.hip) serves the call: one workgroup per KV head and
  // split, with all `group` query heads (kv_span and head_chunks then only shape the merge pass).
  int mfma;
  // Matrix-core kernel: KV heads per workgroup, 1 (the four waves share one KV head's tiles) or 4
  // (wave w takes KV head 4 q + w over all of the split's tiles).
  int mfma_span;
};

// How the decode kernels find cache rows: contiguous cache, paged cache with the split's block
// numbers staged in LDS, or paged cache with the block numbers read from the table in global memory
// (splits that touch more than kMaxSplitPages blocks).
enum PageMode { kContiguous = 0, kPagedLds = 1, kPagedGlobal = 2 };

// Largest split count a decode call may use.
constexpr int kMaxSplits = 128;
// Most cache blocks one split of a paged decode may touch (its block numbers are staged in LDS).
constexpr int kMaxSplitPages = 1024;
// Most query heads per KV head the matrix-core decode kernel serves (its MFMA tile's columns).
constexpr int kMaxDecodeMfmaHeads = 32;

enum class DType : int { bf16 = 0, f16 = 1, f32 = 2 };

// Routing overrides set through fl_set_knob (tests and experiments); -1 means "use the built-in
// rule". Indexed by enum fl_knob of include/flash_lab_hip.h.
int knob(int which);

// Rows of queries per prefill workgroup (the kernel's tile height) and keys per tile.
constexpr int kPrefillBlockM = 128;
constexpr int kPrefillBlockN = 64;

hipError_t launch_prefill(const PrefillArgs& args, DType dtype, int head_dim, hipStream_t stream);
// Ping-pong variant (head_dim 128 and 64): 8 waves, 256 query rows per workgroup.
hipError_t launch_prefill_pingpong(const PrefillArgs& args, DType dtype, int head_dim,
                                   hipStream_t stream);
// The same kernel for causal calls with a pair of query blocks per workgroup run as one stream of
// key tiles (prefill_causal.hip); launch_prefill_pingpong routes causal calls to it when the
// FL_KNOB_PREFILL_CAUSAL_STREAM knob is 1.
// Query rows per workgroup of the ping-pong kernel at this head_dim.
int prefill_pp_block_rows(int head_dim);
hipError_t launch_prefill_causal_stream(const PrefillArgs& args, DType dtype, int head_dim,
                                        hipStream_t stream);

// How decode work is laid out. The vector kernel (decode.hip): each workgroup serves heads_per_wg
// query heads (a power of two dividing the GQA group) of each of kv_span adjacent KV heads. The
// matrix-core kernel (mfma = 1): one KV head and its whole group per workgroup (kv_span 1,
// wg_heads = group). heads_per_wg is also the merge pass's chunk of heads either way. A CU holds
// resident_per_cu split workgroups at once (registers or LDS).
struct DecodeLayout {
  int heads_per_wg;
  int kv_span;
  int resident_per_cu;
  int mfma;
  int wg_heads;  // query heads per KV head in one split workgroup
};
DecodeLayout decode_layout(DType dtype, int head_dim, int heads_kv, int group);
hipError_t launch_decode(const DecodeArgs& args, DType dtype, int head_dim, hipStream_t stream);
// The matrix-core split kernel alone (launch_decode runs it and the merge pass when args.mfma).
hipError_t launch_decode_mfma_split(const DecodeArgs& args, DType dtype, int head_dim,
                                    hipStream_t stream);

hipError_t launch_axpy(const float* x, const float* y, float alpha, float* out, int64_t n,
                       hipStream_t stream);
hipError_t launch_mfma_tile_test(const uint16_t* a, const uint16_t* b, float* c, int k,
                                 int trans_b, hipStream_t stream);
}  // namespace fl
