// Split-KV decode for gfx950: one query token per sequence against its first seq_lens[b] cached
// keys, read in place through strides from a [B, S_max, H_kv, D] cache or a paged
// [num_blocks, page_size, H_kv, D] pool with per-sequence block tables.
//
// Serves the decode_splitkv and decode_inplace ops of the reference (csrc/decode/decode.cu:40-347)
// and their paged forms (a layout the reference defines, flash_lab/layouts.py:145-158, but does not
// run). The arithmetic follows the reference's definitions (scores in the log2 domain, exp2 online
// softmax, fixed-order log-sum-exp merge of the splits, decode.cu:67-75, 116-133, 204-228); the
// decomposition is this file's own:
//
//  * A workgroup (4 waves) serves kSpan adjacent KV heads (4 where they divide H_kv, so one key's
//    rows of the span are one contiguous 1 KiB segment at D = 128 bf16) and, for each, the kHeads
//    query heads of its group it is given, over one contiguous key range (its split). Every K and
//    V row it reads serves all kHeads heads of its KV head.
//  * A cache row (D elements) is read as 16-byte pieces by a group of D * elem / 16 lanes, so
//    every load instruction moves whole rows. Each lane keeps, per head, the running max and sum of
//    its group's keys and the output columns of its own piece; no lane ever needs another lane's
//    V data, and the only cross-lane step in the loop is the dot-product reduction of the group.
//  * Each lane has kUnroll rows of K and of V in flight in each of two register buffers
//    (non-temporal loads: the cache is read once). The rows stay packed: q.k goes through v_dot2
//    (bf16, fp16) and V elements are unpacked one at a time where they are used, which keeps the
//    kernel at 63 registers for one query head and 161 for four.
//  * At the end the row groups are merged by a fixed butterfly inside each wave, then the four
//    waves in order through LDS. With one split the workgroup writes o and lse; otherwise it
//    writes its unnormalized partial output and (max, sum), and decode_merge_kernel combines the
//    splits in a fixed order. No atomics: results are bitwise reproducible for a given split count.
//    (Merging in the split kernel's last workgroup per head group was measured slower: every
//    workgroup then has to wait for its partials to reach device scope and for an atomic before it
//    frees its slot, which costs more than the second launch.)

#include "gfx950.hpp"
#include "launch.hpp"

namespace fl {
namespace decode {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
// Cache rows of K and of V per lane in each of the two register buffers, for workgroups serving
// fewer than four query heads (FL_DECODE_UNROLL) and four or more (FL_DECODE_UNROLL_GQA, whose
// per-head state takes more registers). With the prefetch kept in flight (the scheduling barrier
// in the key loop), two rows stream fastest for one query head: B1-MHA 87.7 -> 83.2-83.7 us,
// B8-MHA 645 -> 641-643 us against four rows; one row 110 us, three 89.7 us. Four query heads
// and more keep four rows (two: B8 with 8 per KV head 232 -> 258 us).
#ifndef FL_DECODE_UNROLL
#define FL_DECODE_UNROLL 2
#endif
#ifndef FL_DECODE_UNROLL_GQA
#define FL_DECODE_UNROLL_GQA 4
#endif
template <int kHeads>
constexpr int kUnrollFor = kHeads >= 4 ? FL_DECODE_UNROLL_GQA : FL_DECODE_UNROLL;
constexpr float kLn2 = 0.693147180559945309f;

// One lane's 16-byte piece of a cache row, per storage type: the dot product with the lane's piece
// of q (q kept in its storage form and unscaled; bf16 and fp16 pairs go through v_dot2, which
// multiplies exactly and accumulates in fp32, so K is never unpacked) and element e of a V piece
// as a float (unpacked right where it is used, so no unpacked copy of the rows in flight is held).
// Vector elements are copied to scalars before __builtin_bit_cast: bit-casting the element lvalue
// q[w] directly made the compiler read element 0 for every w.
template <typename Tag>
struct Piece;

template <>
struct Piece<bf16_tag> {
  using QPiece = u32x4;
  static __device__ __forceinline__ QPiece load_q(const void* p) { return load16(p); }
  static __device__ __forceinline__ float dot(const QPiece& q, const u32x4& k) {
    float d = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const uint32_t qw = q[w];
      const uint32_t kw = k[w];
      d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, qw), __builtin_bit_cast(bf16x2, kw), d,
                                          false);
    }
    return d;
  }
  static __device__ __forceinline__ float elem(const u32x4& v, int e) {
    const uint32_t w = v[e / 2];
    return __uint_as_float(e % 2 ? (w & 0xffff0000u) : (w << 16));
  }
};

template <>
struct Piece<f16_tag> {
  using QPiece = u32x4;
  static __device__ __forceinline__ QPiece load_q(const void* p) { return load16(p); }
  static __device__ __forceinline__ float dot(const QPiece& q, const u32x4& k) {
    float d = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const uint32_t qw = q[w];
      const uint32_t kw = k[w];
      d = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, qw), __builtin_bit_cast(f16x2, kw), d, false);
    }
    return d;
  }
  static __device__ __forceinline__ float elem(const u32x4& v, int e) {
    const uint32_t w = v[e / 2];
    return Elem<f16_tag>::to_float(static_cast<uint16_t>(e % 2 ? (w >> 16) : (w & 0xffffu)));
  }
};

template <>
struct Piece<f32_tag> {
  using QPiece = f32x4;
  static __device__ __forceinline__ QPiece load_q(const void* p) {
    return __builtin_bit_cast(f32x4, load16(p));
  }
  static __device__ __forceinline__ float dot(const QPiece& q, const u32x4& k) {
    float d = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) d = fmaf(q[e], __uint_as_float(k[e]), d);
    return d;
  }
  static __device__ __forceinline__ float elem(const u32x4& v, int e) { return __uint_as_float(v[e]); }
};

// LDS layout of merge_splits: the splits' (max, sum) per head, then per-part partial sums.
template <int kHeads, int D>
struct MergeShape {
  static constexpr int kVecs = kHeads * D / 4;       // 4-column output vectors
  static constexpr int kParts = kThreads / kVecs;    // threads per output vector
  static constexpr int kFloats = 2 * kHeads * kMaxSplits + (kParts > 1 ? kThreads * 5 : 0);
  static_assert(kVecs <= kThreads && kThreads % kVecs == 0, "one thread per vector and part");
};

// Combines the splits of the kHeads consecutive query heads h0 .. h0 + kHeads - 1 of sequence b:
// m = max_s m_s, l = sum_s l_s 2^(m_s - m), o = sum_s o_s 2^(m_s - m) / l, lse = m ln 2 + ln l;
// empty splits (m_s = -inf) contribute nothing. All threads of the workgroup take part. Thread t
// owns one 4-column output vector (t % kVecs) and the splits p, p + kParts, ... (p = t / kVecs), so
// its loads are independent and in flight together; the kParts partial sums are then added in part
// order. Every sum has a fixed order, so the result is the same on every run. The pass is short and
// latency-bound: the first kFirst partial-output loads of each thread do not depend on the maxima
// and are issued before the (max, sum) pairs are read, so the two loads overlap.
// `lds` must hold MergeShape::kFloats floats, 16-byte aligned.
template <typename Tag, int D, int kHeads>
__device__ __forceinline__ void merge_splits(const DecodeArgs& a, int b, int h0, float* lds) {
  using S = typename Elem<Tag>::storage;
  using Shape = MergeShape<kHeads, D>;
  constexpr int kVecs = Shape::kVecs;
  constexpr int kParts = Shape::kParts;
  constexpr int kVecsPerRow = D / 4;
  constexpr int kFirst = 8;
  const int tid = threadIdx.x;
  const int n = a.num_splits;
  const int n4 = (n + 3) & ~3;
  float* ms = lds;                        // [kHeads][kMaxSplits], -inf past n up to n4
  float* ls = lds + kHeads * kMaxSplits;  // [kHeads][kMaxSplits]
  const int vec = tid % kVecs;
  const int part = tid / kVecs;
  const int g = vec / kVecsPerRow;
  // Slots of the heads are consecutive: slot(g, s) = (b H + h0) n + g n + s.
  const int64_t slot0 = (static_cast<int64_t>(b) * a.heads + h0) * n;
  const f32x4* po =
      reinterpret_cast<const f32x4*>(a.partial_o + (slot0 + g * n) * D) + vec % kVecsPerRow;
  f32x4 first[kFirst];
#pragma unroll
  for (int j = 0; j < kFirst; ++j) {
    const int s = part + j * kParts;
    first[j] = s < n ? po[s * kVecsPerRow] : f32x4{0.f, 0.f, 0.f, 0.f};
  }
  for (int i = tid; i < kHeads * n4; i += kThreads) {
    const int gi = i / n4;
    const int s = i - gi * n4;
    f32x2 ml = {-INFINITY, 0.f};
    if (s < n) ml = *reinterpret_cast<const f32x2*>(a.partial_ml + 2 * (slot0 + gi * n + s));
    ms[gi * kMaxSplits + s] = ml[0];
    ls[gi * kMaxSplits + s] = ml[1];
  }
  __syncthreads();
  float mm = -INFINITY;
  const f32x4* ms4 = reinterpret_cast<const f32x4*>(ms + g * kMaxSplits);
  for (int s4 = 0; s4 < n4 / 4; ++s4) {
    const f32x4 v = ms4[s4];
    mm = fmaxf(mm, fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3])));
  }
  f32x4 num = {0.f, 0.f, 0.f, 0.f};
  float den = 0.f;
  auto add = [&](int s, const f32x4& o_s) {
    const float m_s = ms[g * kMaxSplits + s];
    const float f = m_s == -INFINITY ? 0.f : exp2_fast(m_s - mm);
    den += ls[g * kMaxSplits + s] * f;
    num += o_s * f;
  };
#pragma unroll
  for (int j = 0; j < kFirst; ++j) {
    const int s = part + j * kParts;
    if (s < n) add(s, first[j]);
  }
#pragma unroll 8
  for (int s = part + kFirst * kParts; s < n; s += kParts) add(s, po[s * kVecsPerRow]);
  if constexpr (kParts > 1) {
    f32x4* part_o = reinterpret_cast<f32x4*>(lds + 2 * kHeads * kMaxSplits);  // [kParts][kVecs]
    float* part_l = reinterpret_cast<float*>(part_o + kThreads);              // [kParts][kVecs]
    part_o[tid] = num;
    part_l[tid] = den;
    __syncthreads();
    if (part == 0) {
#pragma unroll
      for (int p = 1; p < kParts; ++p) {
        num += part_o[p * kVecs + vec];
        den += part_l[p * kVecs + vec];
      }
    }
  }
  if (part == 0) {
    const int h = h0 + g;
    const int d0 = (vec % kVecsPerRow) * 4;
    S* orow = static_cast<S*>(a.o) + b * a.o_bs + h * a.o_hs + d0;
#pragma unroll
    for (int e = 0; e < 4; ++e) orow[e] = Elem<Tag>::from_float(den > 0.f ? num[e] / den : 0.f);
    if (d0 == 0) a.lse[b * a.heads + h] = den > 0.f ? mm * kLn2 + logf(den) : -INFINITY;
  }
}

// Waves per SIMD the register budget must allow: 5 for one head (96 VGPRs), 3 up to four heads
// (168), 2 for eight. Without the hint the four-head kernel takes 170 VGPRs, which leaves room for
// only two waves per SIMD.
template <int kHeads>
constexpr int kWavesPerSimd = kHeads == 1 ? 5 : kHeads <= 4 ? 3 : 2;

template <typename Tag, int D, int kHeads, int kSpan, int kPageMode>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(kWavesPerSimd<kHeads>)))
decode_split_kernel(const DecodeArgs a) {
  constexpr bool kPaged = kPageMode != kContiguous;
  using S = typename Elem<Tag>::storage;
  constexpr int kEPL = 16 / static_cast<int>(sizeof(S));  // elements per 16-byte piece
  constexpr int kLPR = D / kEPL;                           // lanes per cache row
  constexpr int kLPK = kLPR * kSpan;                       // lanes per key (kSpan adjacent heads)
  constexpr int kGPW = 64 / kLPK;                          // row groups per wave
  constexpr int kGroups = kWaves * kGPW;                   // row groups per workgroup
  constexpr int kUnroll = kUnrollFor<kHeads>;
  constexpr int kKeysPerIter = kGroups * kUnroll;
  static_assert(kLPK >= 1 && kLPK <= 64 && 64 % kLPK == 0, "row pieces must tile a wave");

  __shared__ float red_o[kWaves][kSpan * kHeads][D];
  __shared__ float red_m[kWaves][kSpan * kHeads];
  __shared__ float red_l[kWaves][kSpan * kHeads];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int piece = lane % kLPR;                   // which 16-byte piece of a row
  const int sp = (lane / kLPR) % kSpan;            // which KV head of the workgroup's span
  const int group = wave * kGPW + lane / kLPK;     // row group within the workgroup

  int w = blockIdx.x;
  const int split = w % a.num_splits;
  w /= a.num_splits;
  const int hchunk = w % a.head_chunks;
  w /= a.head_chunks;
  const int hblocks = a.heads_kv / kSpan;
  const int hblk = w % hblocks;
  const int b = w / hblocks;
  const int hkv = hblk * kSpan + sp;
  const int h0 = hkv * a.group + hchunk * kHeads;

  // Lengths are not checked on the host (that would need a sync); clamp them to the cache so an
  // out-of-range value cannot read outside it.
  const int len = min(max(a.seq_lens[b], 0), a.max_seqlen);
  const int per_split =
      ((len + a.num_splits - 1) / a.num_splits + kKeysPerIter - 1) / kKeysPerIter * kKeysPerIter;
  const int k_begin = split * per_split;
  const int k_end = min(len, k_begin + per_split);

  using P = Piece<Tag>;
  typename P::QPiece q[kHeads];
#pragma unroll
  for (int g = 0; g < kHeads; ++g) {
    const S* qrow = static_cast<const S*>(a.q) + b * a.q_bs + (h0 + g) * a.q_hs;
    q[g] = P::load_q(qrow + piece * kEPL);
  }
  const float sl2 = a.scale_log2;  // scores are q.k * scale_log2 (log2 domain)

  float o[kHeads][kEPL];
  float m[kHeads];  // running max, log2 units (same on every lane of a row group)
  float l[kHeads];  // running sum (same on every lane of a row group)
#pragma unroll
  for (int g = 0; g < kHeads; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < kEPL; ++e) o[g][e] = 0.f;
  }

  // Contiguous cache: rows of sequence b at b * bs + key * ss. Paged cache
  // ([num_blocks, page_size, H_kv, D]): key lives in block block_tables[b][key / page_size], row
  // key % page_size, block numbers clamped to the pool so a bad table entry cannot read outside
  // it. kPagedLds stages the split's block numbers in LDS once (the host picks it when every split
  // touches at most kMaxSplitPages blocks): LDS reads do not wait behind the rows in flight.
  // kPagedGlobal reads each block number from the table in global memory.
  __shared__ int page_table[kPageMode == kPagedLds ? kMaxSplitPages : 1];
  int page0 = 0;
  const int32_t* table_row = nullptr;
  if constexpr (kPaged) table_row = a.block_tables + static_cast<int64_t>(b) * a.block_tables_stride;
  if constexpr (kPageMode == kPagedLds) {
    if (k_begin < k_end) {
      page0 = k_begin / a.page_size;
      const int pages = (k_end - 1) / a.page_size - page0 + 1;
      for (int i = tid; i < pages; i += kThreads)
        page_table[i] = min(max(table_row[page0 + i], 0), a.num_blocks - 1);
    }
    __syncthreads();
  }
  const S* kbase = static_cast<const S*>(a.k) + (kPaged ? 0 : b * a.k_bs) + hkv * a.k_hs + piece * kEPL;
  const S* vbase = static_cast<const S*>(a.v) + (kPaged ? 0 : b * a.v_bs) + hkv * a.v_hs + piece * kEPL;
  // (block, row) of a key; page sizes that are powers of two (the usual ones) take a shift.
  auto locate = [&](int key, int& block, int& row) {
    const int page = a.page_shift >= 0 ? key >> a.page_shift : key / a.page_size;
    if constexpr (kPageMode == kPagedLds) {
      block = page_table[page - page0];
    } else {
      block = min(max(table_row[page], 0), a.num_blocks - 1);
    }
    row = key - page * a.page_size;
  };
  auto k_row = [&](int key) -> const S* {
    if constexpr (kPaged) {
      int block, row;
      locate(key, block, row);
      return kbase + static_cast<int64_t>(block) * a.k_bs + static_cast<int64_t>(row) * a.k_ss;
    } else {
      return kbase + static_cast<int64_t>(key) * a.k_ss;
    }
  };
  auto v_row = [&](int key) -> const S* {
    if constexpr (kPaged) {
      int block, row;
      locate(key, block, row);
      return vbase + static_cast<int64_t>(block) * a.v_bs + static_cast<int64_t>(row) * a.v_ss;
    } else {
      return vbase + static_cast<int64_t>(key) * a.v_ss;
    }
  };

  // Batches of kKeysPerIter keys, double-buffered in registers: the next batch's loads are issued
  // before the current batch is used, so each wave keeps rows in flight while it computes. Keys past
  // the split's end are clamped to its last row (always a valid, finite row) and masked out of the
  // softmax, so every load is issued unconditionally.
  auto load_batch = [&](int base, u32x4 (&kr)[kUnroll], u32x4 (&vr)[kUnroll]) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int key = min(base + u * kGroups + group, k_end - 1);
      kr[u] = load16_stream(k_row(key));
      vr[u] = load16_stream(v_row(key));
    }
  };
  auto use_batch = [&](int base, const u32x4 (&kr)[kUnroll], const u32x4 (&vr)[kUnroll]) {
#pragma unroll
    for (int g = 0; g < kHeads; ++g) {
      float s[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const float dot = group_sum<kLPR>(P::dot(q[g], kr[u])) * sl2;
        s[u] = base + u * kGroups + group < k_end ? dot : -INFINITY;
      }
      float mx = s[0];
#pragma unroll
      for (int u = 1; u < kUnroll; ++u) mx = fmaxf(mx, s[u]);
      const float m_new = fmaxf(m[g], mx);
      const float ref = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = exp2_fast(m[g] - ref);
      m[g] = m_new;
      float lsum = l[g] * alpha;
#pragma unroll
      for (int e = 0; e < kEPL; ++e) o[g][e] *= alpha;
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const float p = exp2_fast(s[u] - ref);
        lsum += p;
#pragma unroll
        for (int e = 0; e < kEPL; ++e) o[g][e] = fmaf(p, P::elem(vr[u], e), o[g][e]);
      }
      l[g] = lsum;
    }
  };
  // The prefetches are unconditional (past the end they re-read the split's last row, which the
  // cache serves), and a scheduling barrier keeps them ahead of the current batch's use. Without
  // either, the compiler waits for every load in flight, the prefetch included, before it uses the
  // current batch, or moves the K loads down to their dot products: one batch in flight instead of
  // two (B1-MHA 89.2 -> 88.5 us, B=1 with 8 KV heads on this kernel 41.8 -> 38.3 us).
  u32x4 ka[kUnroll], va[kUnroll], kb[kUnroll], vb[kUnroll];
  if (k_begin < k_end) load_batch(k_begin, ka, va);
  for (int base = k_begin; base < k_end; base += 2 * kKeysPerIter) {
    load_batch(base + kKeysPerIter, kb, vb);
    __builtin_amdgcn_sched_barrier(0);
    use_batch(base, ka, va);
    if (base + kKeysPerIter >= k_end) break;
    load_batch(base + 2 * kKeysPerIter, ka, va);
    __builtin_amdgcn_sched_barrier(0);
    use_batch(base + kKeysPerIter, kb, vb);
  }

  // Merge the row groups of this wave: butterfly over lanes with the same piece.
#pragma unroll
  for (int mask = kLPK; mask < 64; mask <<= 1) {
#pragma unroll
    for (int g = 0; g < kHeads; ++g) {
      const float m_o = __shfl_xor(m[g], mask);
      const float l_o = __shfl_xor(l[g], mask);
      const float m_new = fmaxf(m[g], m_o);
      // Groups without keys (m = -inf) contribute nothing; two empty groups stay empty.
      const float f = m[g] == -INFINITY ? 0.f : exp2_fast(m[g] - m_new);
      const float f_o = m_o == -INFINITY ? 0.f : exp2_fast(m_o - m_new);
      l[g] = l[g] * f + l_o * f_o;
#pragma unroll
      for (int e = 0; e < kEPL; ++e) {
        const float o_o = __shfl_xor(o[g][e], mask);
        o[g][e] = o[g][e] * f + o_o * f_o;
      }
      m[g] = m_new;
    }
  }
  if (lane < kLPK) {  // row group 0 of the wave: one lane per (head of the span, piece)
#pragma unroll
    for (int g = 0; g < kHeads; ++g) {
#pragma unroll
      for (int e = 0; e < kEPL; ++e) red_o[wave][sp * kHeads + g][piece * kEPL + e] = o[g][e];
      if (piece == 0) {
        red_m[wave][sp * kHeads + g] = m[g];
        red_l[wave][sp * kHeads + g] = l[g];
      }
    }
  }
  __syncthreads();

  // Merge the four waves in order and write o/lse (one split) or the partials.
  for (int idx = tid; idx < kSpan * kHeads * D; idx += kThreads) {
    const int g = idx / D;  // (head of the span) * kHeads + query head
    const int d = idx - g * D;
    float mm = -INFINITY;
#pragma unroll
    for (int wv = 0; wv < kWaves; ++wv) mm = fmaxf(mm, red_m[wv][g]);
    float num = 0.f;
    float den = 0.f;
#pragma unroll
    for (int wv = 0; wv < kWaves; ++wv) {
      const float mw = red_m[wv][g];
      if (mw != -INFINITY) {
        const float f = exp2_fast(mw - mm);
        num += red_o[wv][g][d] * f;
        den += red_l[wv][g] * f;
      }
    }
    const int h = (hblk * kSpan + g / kHeads) * a.group + hchunk * kHeads + g % kHeads;
    if (a.num_splits == 1) {
      S* orow = static_cast<S*>(a.o) + b * a.o_bs + h * a.o_hs;
      orow[d] = Elem<Tag>::from_float(den > 0.f ? num / den : 0.f);
      if (d == 0) a.lse[b * a.heads + h] = den > 0.f ? mm * kLn2 + logf(den) : -INFINITY;
    } else {
      const int64_t slot = (static_cast<int64_t>(b) * a.heads + h) * a.num_splits + split;
      a.partial_o[slot * D + d] = num;
      if (d == 0) {
        a.partial_ml[2 * slot] = mm;
        a.partial_ml[2 * slot + 1] = den;
      }
    }
  }
}

// Merge pass: one workgroup per head group (kHeads query heads of one KV head).
template <typename Tag, int D, int kHeads>
__global__ void __launch_bounds__(kThreads) decode_merge_kernel(const DecodeArgs a) {
  __shared__ __attribute__((aligned(16))) float lds[MergeShape<kHeads, D>::kFloats];
  int w = blockIdx.x;
  const int hchunk = w % a.head_chunks;
  w /= a.head_chunks;
  const int hkv = w % a.heads_kv;
  const int b = w / a.heads_kv;
  merge_splits<Tag, D, kHeads>(a, b, hkv * a.group + hchunk * kHeads, lds);
}

// Launches the vector split kernel; a (span, page mode) pair with no instantiation (a span whose
// rows do not fit a wave, or a span above 1 with block numbers read from global memory, which the
// host never plans) is reported instead of leaving the outputs unwritten.
template <typename Tag, int D, int kHeads, int kSpan>
hipError_t launch_split(const DecodeArgs& args, int groups, hipStream_t stream) {
  constexpr int kLPR = D * static_cast<int>(sizeof(typename Elem<Tag>::storage)) / 16;
  if constexpr (kSpan * kLPR <= 64) {
    const dim3 grid(groups / kSpan * args.num_splits);
    if (args.block_tables == nullptr) {
      hipLaunchKernelGGL((decode_split_kernel<Tag, D, kHeads, kSpan, kContiguous>), grid,
                         dim3(kThreads), 0, stream, args);
      return hipGetLastError();
    }
    if (!args.page_table_global) {
      hipLaunchKernelGGL((decode_split_kernel<Tag, D, kHeads, kSpan, kPagedLds>), grid,
                         dim3(kThreads), 0, stream, args);
      return hipGetLastError();
    }
    if constexpr (kSpan == 1) {  // the rare long-split case: one instantiation per type
      hipLaunchKernelGGL((decode_split_kernel<Tag, D, kHeads, 1, kPagedGlobal>), grid,
                         dim3(kThreads), 0, stream, args);
      return hipGetLastError();
    }
  }
  return hipErrorInvalidValue;
}

template <typename Tag, int D, int kHeads>
hipError_t launch_heads(const DecodeArgs& args, DType dtype, hipStream_t stream) {
  const int groups = args.batch * args.heads_kv * args.head_chunks;
  hipError_t err = hipSuccess;
  if (args.mfma) {
    err = launch_decode_mfma_split(args, dtype, D, stream);
  } else {
    switch (args.kv_span) {
      case 4: err = launch_split<Tag, D, kHeads, 4>(args, groups, stream); break;
      case 2: err = launch_split<Tag, D, kHeads, 2>(args, groups, stream); break;
      case 1: err = launch_split<Tag, D, kHeads, 1>(args, groups, stream); break;
      default: err = hipErrorInvalidValue; break;
    }
  }
  if (err != hipSuccess || args.num_splits == 1) return err;
  hipLaunchKernelGGL((decode_merge_kernel<Tag, D, kHeads>), dim3(groups), dim3(kThreads), 0, stream,
                     args);
  return hipGetLastError();
}

template <typename Tag, int D>
hipError_t launch_dim(const DecodeArgs& args, DType dtype, int k_heads, hipStream_t stream) {
  switch (k_heads) {
    case 1: return launch_heads<Tag, D, 1>(args, dtype, stream);
    case 2: return launch_heads<Tag, D, 2>(args, dtype, stream);
    case 4: return launch_heads<Tag, D, 4>(args, dtype, stream);
    default: return launch_heads<Tag, D, 8>(args, dtype, stream);
  }
}

template <typename Tag>
hipError_t launch_type(const DecodeArgs& args, DType dtype, int head_dim, int k_heads,
                       hipStream_t stream) {
  return head_dim == 64 ? launch_dim<Tag, 64>(args, dtype, k_heads, stream)
                        : launch_dim<Tag, 128>(args, dtype, k_heads, stream);
}

}  // namespace
}  // namespace decode

// Smallest GQA group the matrix-core kernel serves (the FL_KNOB_DECODE_MFMA_MIN_GROUP knob
// overrides it; a value above kMaxDecodeMfmaHeads turns the kernel off): 4 query heads per KV head
// at D = 128 and 64. With 4, bf16 at 32K keys: D = 128, B=8 169 vs 172-175 us, B=1 33.7 vs 38.2;
// D = 64, B=8 86.4 vs 93.8, B=4 50.7 vs 56.2, B=1 23.4 vs 24.4, one 8.4K-key sequence 14.9 vs
// 18.0. With 2 it is mixed (D = 128: B=2 54.3 vs 49.3, B=4 89.3 vs 90.6; D = 64: B=2 33.7 vs
// 30.4, B=8 85.7 vs 89.5), so groups of 2 stay on the vector kernel.
int decode_mfma_min_group(int head_dim) {
  (void)head_dim;
  const int v = knob(FL_KNOB_DECODE_MFMA_MIN_GROUP);
  if (v >= 1) return v;
  return 4;
}

DecodeLayout decode_layout(DType dtype, int head_dim, int heads_kv, int group) {
  DecodeLayout layout{};
  int k = 1;
  while (k < 8 && group % (2 * k) == 0) k *= 2;
  layout.heads_per_wg = k;
  if (dtype != DType::f32 && group >= decode_mfma_min_group(head_dim) &&
      group <= kMaxDecodeMfmaHeads) {
    // One KV head per workgroup. Two fit a CU (256 registers per lane, 64 KiB of LDS at D = 128),
    // but one per CU streamed faster (B=8, 8 KV heads, 32K keys: 6.03-6.09 TB/s against
    // 5.86-5.95 with two; B=1: 3.75-4.0 against 3.3-3.7).
    layout.mfma = 1;
    layout.wg_heads = group;
    layout.kv_span = 1;
    layout.resident_per_cu = 1;
    return layout;
  }
  layout.wg_heads = k;
  // Lanes per cache row: 16-byte pieces of head_dim elements. A span of s KV heads puts s * lanes
  // per row on one key, which must fit a wave.
  const int lanes_per_row = head_dim * (dtype == DType::f32 ? 4 : 2) / 16;
  layout.kv_span = 1;
  for (int s = 4; s > 1; s /= 2) {
    if (heads_kv % s == 0 && s * lanes_per_row <= 64) {
      layout.kv_span = s;
      break;
    }
  }
  layout.resident_per_cu = k == 1 ? decode::kWavesPerSimd<1>
                           : k <= 4 ? decode::kWavesPerSimd<4>
                                    : decode::kWavesPerSimd<8>;
  return layout;
}

hipError_t launch_decode(const DecodeArgs& args, DType dtype, int head_dim, hipStream_t stream) {
  const int k_heads = args.group / args.head_chunks;
  switch (dtype) {
    case DType::bf16: return decode::launch_type<bf16_tag>(args, dtype, head_dim, k_heads, stream);
    case DType::f16: return decode::launch_type<f16_tag>(args, dtype, head_dim, k_heads, stream);
    default: return decode::launch_type<f32_tag>(args, dtype, head_dim, k_heads, stream);
  }
}

}  // namespace fl
