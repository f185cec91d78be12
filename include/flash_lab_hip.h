/*
 * flash_lab_hip.h — C ABI of the gfx950 (MI355X) attention kernels.
 *
 * This library replaces the reference's op registry and host wrappers
 * (reference csrc/bindings.cpp:7-42 plus the TORCH_LIBRARY_IMPL blocks of
 * csrc/prefill/mma_pipelined.cu:162-189, csrc/decode/decode.cu:282-347,
 * csrc/common/smoke.cu:29-45 and csrc/prefill/mma_tile_test.cu:62-88).
 * The functions take plain pointers, element strides and sizes; no torch
 * types cross this boundary. The caller owns every buffer: inputs are
 * borrowed, outputs and the decode workspace are allocated by the caller
 * (the Python layer allocates them through the torch caching allocator, so
 * the calls are safe under stream capture). Nothing here allocates device
 * memory or synchronizes; every kernel is launched on the given stream.
 *
 * Return value: 0 on success, otherwise an FL_ERR_* code; fl_last_error()
 * then returns a message for the calling thread.
 */
#ifndef FLASH_LAB_HIP_H
#define FLASH_LAB_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* A hipStream_t. NULL is the null stream of the current device. */
typedef void* fl_stream_t;

enum fl_dtype { FL_DTYPE_BF16 = 0, FL_DTYPE_F16 = 1, FL_DTYPE_F32 = 2 };

enum fl_status {
  FL_OK = 0,
  FL_ERR_INVALID = 1,     /* bad argument: shape, stride, alignment, dtype */
  FL_ERR_UNSUPPORTED = 2, /* valid, but no kernel is built for it (head_dim, dtype) */
  FL_ERR_LAUNCH = 3       /* the HIP runtime reported an error at launch */
};

/*
 * Prefill (attention forward). Replaces AttnParams (reference
 * csrc/common/params.h:9-27) as filled by make_attn_params
 * (csrc/common/attn_host.h:59-93). q is [B, S_q, H, D]; k and v are
 * [B, S_k, H_kv, D]; o is [B, S_q, H, D] in the input dtype; lse is
 * [B, H, S_q] fp32, contiguous. Strides are in elements; D has unit stride.
 * The library derives group = H / H_kv, causal_offset = S_k - S_q and
 * scale * log2(e) (computed in double, as the reference does).
 */
typedef struct fl_attn_params {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  float* lse;
  int64_t q_batch_stride, q_seq_stride, q_head_stride;
  int64_t k_batch_stride, k_seq_stride, k_head_stride;
  int64_t v_batch_stride, v_seq_stride, v_head_stride;
  int64_t o_batch_stride, o_seq_stride, o_head_stride;
  int32_t batch, seqlen_q, seqlen_k, heads, heads_kv, head_dim;
  int32_t causal; /* nonzero: bottom-right aligned causal mask */
  int32_t dtype;  /* enum fl_dtype: BF16 or F16 */
  double softmax_scale;
} fl_attn_params;

/*
 * FlashAttention-2 forward on MFMA. Serves the attention_mma_pipelined and
 * attention_mma ops (reference csrc/prefill/mma_pipelined.cu:162-183,
 * csrc/prefill/mma.cu), head_dim 64 or 128, bf16 or fp16.
 */
int fl_attention_fwd(const fl_attn_params* p, fl_stream_t stream);

/*
 * Decode. Replaces DecodeParams (reference csrc/common/params.h:31-53) as
 * filled by make_decode_params (csrc/decode/decode_host.h:55-85). q is
 * [B, H, D]; caches are [B, S_max, H_kv, D] read in place through strides;
 * seq_lens [B] int32 on the device (never read by the host); o [B, H, D] in
 * the input dtype; lse [B, H] fp32 contiguous. num_splits must be resolved
 * by fl_decode_plan first. workspace is 16-byte aligned fp32 device memory of
 * at least the size fl_decode_plan reports (unused, may be NULL, when
 * num_splits == 1).
 *
 * Paged caches (block_tables != NULL; the reference defines the layout,
 * flash_lab/layouts.py:145-158, and its oracle, reference.py:155-164, but
 * every reference kernel rejects it, ops.py:61-62): k_cache and v_cache are
 * [num_blocks, page_size, H_kv, D] and the *_batch_stride fields are the
 * block strides; block_tables is [B, max_blocks] int32 on the device with
 * row stride block_tables_stride, and max_seqlen = max_blocks * page_size.
 * Key j of sequence b is row j % page_size of block
 * block_tables[b][j / page_size]; entries outside [0, num_blocks) are
 * clamped on the device rather than read out of bounds.
 */
typedef struct fl_decode_params {
  const void* q;
  const void* k_cache;
  const void* v_cache;
  void* o;
  float* lse;
  const int32_t* seq_lens;
  int64_t q_batch_stride, q_head_stride;
  int64_t k_batch_stride, k_seq_stride, k_head_stride;
  int64_t v_batch_stride, v_seq_stride, v_head_stride;
  int64_t o_batch_stride, o_head_stride;
  int32_t batch, heads, heads_kv, head_dim, max_seqlen;
  int32_t num_splits; /* >= 1 */
  int32_t dtype;      /* enum fl_dtype: BF16, F16 or F32 */
  double softmax_scale;
  float* workspace;
  size_t workspace_bytes;
  const int32_t* block_tables; /* NULL: contiguous [B, S_max, H_kv, D] caches */
  int64_t block_tables_stride;
  int32_t page_size, num_blocks;
} fl_decode_params;

/*
 * Split count and workspace size for a decode call; host-only, touches no
 * device. Replaces choose_num_splits and the workspace sizing of run_decode
 * (reference csrc/decode/decode.cu:272-311). requested_splits 0 lets the
 * library choose from cu_count (allow_splits != 0) or forces 1
 * (allow_splits == 0, the decode_inplace op). Requested counts must be in
 * [0, 128].
 */
int fl_decode_plan(const fl_decode_params* p, int32_t requested_splits, int32_t allow_splits,
                   int32_t cu_count, int32_t* num_splits, size_t* workspace_bytes);

/*
 * Split-KV decode: partial passes over contiguous key ranges with fp32
 * partials, then a fixed-order log-sum-exp merge (reference
 * csrc/decode/decode.cu:40-235). With num_splits == 1 the single pass
 * writes o and lse directly (the decode_inplace op).
 */
int fl_decode(const fl_decode_params* p, fl_stream_t stream);

/*
 * fl_decode without a caller workspace: the split partials go to a scratch
 * array the library holds in device memory (a file-scope __device__ array of
 * 16 MiB; each GPU the library runs on holds its own copy until the process
 * ends). No counterpart in the reference: this entry point is for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc). It allocates nothing
 * itself: no hipMalloc, no hipFree, no allocating library call.
 *
 * Parameters are fl_decode's; workspace and workspace_bytes are ignored. The
 * kernels run on `stream`, which must belong to the current device. A call
 * whose workspace (B * H * num_splits * (head_dim + 2) * 4 bytes, 0 for one
 * split) exceeds 16 MiB is rejected with FL_ERR_INVALID before any launch.
 * Every call on a GPU shares that GPU's array: calls on one stream are
 * ordered and safe, calls that overlap on one GPU (several streams or
 * threads at once) race. The kernels write every partial they read, so the
 * array's previous contents never reach an output.
 */
int fl_decode_noalloc(const fl_decode_params* p, fl_stream_t stream);

/* out = alpha * x + y over n fp32 elements (reference csrc/common/smoke.cu:12-45). */
int fl_smoke_axpy(const float* x, const float* y, float alpha, float* out, int64_t n,
                  fl_stream_t stream);

/*
 * One wave computes a 16 x 16 fp32 tile through the same fragment code as
 * the prefill kernel (reference csrc/prefill/mma_tile_test.cu:20-84).
 * a is [16, k] bf16 row-major, k in {16, 32, 64}. trans_b == 0: b is
 * [16, k] and c = a b^T (b read like K in Q K^T). trans_b != 0: b is [k, 16]
 * and c = a b (b read like V in P V, through the LDS transpose read).
 * c is [16, 16] fp32 row-major.
 */
int fl_mfma_tile_test(const void* a, const void* b, float* c, int32_t k, int32_t trans_b,
                      fl_stream_t stream);

/*
 * Routing overrides. No counterpart in the reference (its kernel choice is
 * fixed at build time): a test and experiment hook that pins a call to one
 * of this library's kernels, so the parity tests can run every shape on
 * each of them. Process-wide; set it from one thread while no other call is
 * in flight. value -1 restores the built-in rule; fl_set_knob rejects an
 * unknown knob or a value outside the knob's range with FL_ERR_INVALID.
 *   FL_KNOB_PREFILL_PP_MIN_WG      [0, 2^30]: fewest ping-pong workgroups
 *                                  for which prefill runs the ping-pong
 *                                  kernel (default 256 non-causal, 128
 *                                  causal; 0 = always, 2^30 = never).
 *   FL_KNOB_DECODE_MFMA_MIN_GROUP  [1, 2^20]: smallest GQA group the
 *                                  matrix-core decode kernel takes (default
 *                                  4 at head_dim 128 and 64; above 32 =
 *                                  never).
 *   FL_KNOB_DECODE_WG_PER_CU       [1, 64]: resident split workgroups per CU
 *                                  that fl_decode_plan assumes.
 *   FL_KNOB_DECODE_MFMA_SPAN       [1, 4]: KV heads per workgroup of the
 *                                  matrix-core decode kernel, 1 or 4 (4 only
 *                                  where H_kv is a multiple of 4; other
 *                                  values act as 1), whatever the size of
 *                                  the call.
 *   FL_KNOB_PREFILL_CAUSAL_STREAM  [0, 1]: how the 8-wave kernel runs a
 *                                  causal pair of query blocks: 0 = two
 *                                  blocks one after the other (the default),
 *                                  1 = one stream of key tiles (measured
 *                                  slower; kept for comparison).
 */
enum fl_knob {
  FL_KNOB_PREFILL_PP_MIN_WG = 0,
  FL_KNOB_DECODE_MFMA_MIN_GROUP = 1,
  FL_KNOB_DECODE_WG_PER_CU = 2,
  FL_KNOB_DECODE_MFMA_SPAN = 3,
  FL_KNOB_PREFILL_CAUSAL_STREAM = 4,
  FL_KNOB_COUNT = 5
};
int fl_set_knob(int32_t knob, int64_t value);
/* Current value of a knob (-1: the built-in rule), or -2 for an unknown knob. */
int64_t fl_get_knob(int32_t knob);

/* Message of the last failed call on this thread ("" if none). */
const char* fl_last_error(void);

/* Library version string, for environment records. */
const char* fl_version(void);

#ifdef __cplusplus
}
#endif

#endif /* FLASH_LAB_HIP_H */
