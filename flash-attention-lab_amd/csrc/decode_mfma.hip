// Split-KV decode on the matrix cores, for grouped-query attention (several query heads per KV
// head). Same problem, workspace format and merge pass as decode.hip; this kernel takes the place
// of that file's split kernel when the group is large enough that per-head vector arithmetic (one
// dot product and one D-wide multiply-add per query head per cached row) would bound it.
//
// Serves the decode_splitkv and decode_inplace ops of the reference (csrc/decode/decode.cu:40-347);
// the arithmetic follows its definitions (scores in the log2 domain, exp2 online softmax, partials
// merged by a fixed-order log-sum-exp, decode.cu:67-75, 116-133, 204-228). The decomposition is
// this file's own: for one KV head, a decode step is a small prefill whose rows are the query
// heads of the group, so it runs on the prefill kernels' MFMA tiles (prefill_tile.hpp).
//
//  * Scores are computed transposed, S^T = K Q^T on v_mfma_f32_32x32x16 (K the A operand from LDS,
//    Q^T the B operand in registers: one query head per column, columns past the group zero), and
//    the output as O^T = V^T P^T (V^T read with ds_read_b64_tr_b16). Lane l holds query head
//    l % 32 and 16 of a tile's 32 keys, so softmax state and output rescaling are per lane.
//    The online softmax keeps the running max of each head's scores as its reference point (as
//    the reference and prefill_pp.hip do); O and l are rescaled only on tiles where some head's
//    max grows, so most tiles of a long sequence skip the rescale of O.
//  * Workgroup: 4 waves and one split, in one of two layouts (mfma_span, chosen on the host): one
//    KV head with all of its query heads (up to 32), wave w taking the split's 32-key tiles w,
//    w + 4, w + 8, ... (the four waves read neighbouring rows); or four adjacent KV heads, wave w
//    taking KV head 4 q + w over all of the split's tiles, so that for each key the workgroup
//    reads the four heads' rows, one contiguous 1 KiB segment at D = 128. The second needs more
//    work to fill the GPU and is used when there is enough of it.
//  * Each wave loads its tiles into registers with 16-byte non-temporal loads (every load
//    instruction moves whole rows: four 256-byte rows at D = 128), one tile ahead, and writes each
//    tile into its own LDS buffer (K 8 KiB + V 8 KiB at D = 128) in the XOR-swizzled layout the
//    fragment reads expect, then reads the fragments back. No wave touches another's buffer, so the
//    loop has no barriers. (Loading straight into LDS with global_load_lds_dwordx4 streamed at
//    about 4.1 TB/s in a probe of this access pattern, plain loads at 6.5-6.7 TB/s.)
//  * Rows past the split's end are clamped to its last row (always valid memory) and masked out of
//    the softmax.
//  * Paged caches ([num_blocks, page_size, H_kv, D] pools with block tables) as in decode.hip: the
//    split's block numbers are staged in LDS (or, for splits touching more than kMaxSplitPages
//    blocks, read from the table in global memory), clamped to the pool, and every lane computes
//    the address of the row it loads. The keys and their order are the contiguous cache's, so the
//    results are bitwise the same.
//  * At the end the four waves are merged in order through LDS (one KV head; with four, each wave's
//    state is its own head's and is written as it is), and the workgroup writes o and lse
//    (one split) or its unnormalized partial output and (reference point, sum), which decode.hip's
//    merge pass combines as it would (max, sum). No atomics: results are bitwise reproducible for a
//    given split count.
#include "gfx950.hpp"
#include "launch.hpp"
#include "prefill_tile.hpp"

namespace fl {
namespace decode_mfma {
namespace {

using prefill::acc_key;
using prefill::k_frag;
using prefill::p_frag;
using prefill::v_frag;

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kTileKeys = 32;  // one MFMA key block
// One tile in flight beyond the one in use: B8-GQA 182.3 -> 180.1 us, one sequence with 8 KV
// heads at 32K keys 36.8 -> 35.1 us against two.
#ifndef FL_DMFMA_AHEAD
#define FL_DMFMA_AHEAD 1
#endif
constexpr int kAhead = FL_DMFMA_AHEAD;  // tiles in flight in registers per wave
constexpr float kLn2 = 0.693147180559945309f;
// Running max before the first tile: finite, so the first tile's max passes it and masked scores
// (-inf) still give 0.
constexpr float kNoRef = -1e30f;

template <int D>
constexpr int kTileBytes = kTileKeys * D * 2;  // one tensor's tile
template <int D>
constexpr int kLoads = kTileBytes<D> / 1024;  // 16-byte loads per lane per tensor tile
template <int D>
constexpr int kWaveBytes = 2 * kTileBytes<D>;  // a wave's LDS tile: K, then V
template <int D>
constexpr int kLdsBytes = kWaves * kWaveBytes<D>;
// Final merge through LDS (reusing the tile buffers): (reference point, sum) per wave and column,
// then each wave's output rows with one float of padding (conflict-free stores from the 32
// columns).
template <int D>
constexpr int kRedPitch = D + 1;
template <int D>
constexpr int kRedBytes = 4 * (2 * kWaves * kMaxDecodeMfmaHeads + kWaves * kMaxDecodeMfmaHeads * kRedPitch<D>);
template <int D>
constexpr int kSmemBytes = kLdsBytes<D> > kRedBytes<D> ? kLdsBytes<D> : kRedBytes<D>;

template <typename Tag, int D, int kPageMode>
__global__ void __launch_bounds__(kThreads) decode_mfma_kernel(const DecodeArgs a) {
  using E = Elem<Tag>;
  constexpr bool kPaged = kPageMode != kContiguous;
  constexpr int kChunksPerRow = D / 8;              // 16-byte chunks per cache row
  constexpr int kRowsPerLoad = 64 / kChunksPerRow;  // rows per wave-wide load instruction
  constexpr int kCols = kMaxDecodeMfmaHeads;
  __shared__ __attribute__((aligned(16))) uint16_t smem[kSmemBytes<D> / 2];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5;
  const int col = lane & 31;  // the query head (within the group) of this lane's column

  int w = blockIdx.x;
  const int split = w % a.num_splits;
  w /= a.num_splits;
  const int span = a.mfma_span;  // 1, or 4: wave w takes KV head 4 q + w over all the split's tiles
  const int hq = w % (a.heads_kv / span);
  const int b = w / (a.heads_kv / span);
  const int hkv = span == 1 ? hq : hq * span + wave;
  const int group = a.group;  // <= kCols (checked on the host)
  const int h0 = hkv * group;

  // Lengths are not checked on the host (that would need a sync); clamp them to the cache so an
  // out-of-range value cannot read outside it.
  const int len = min(max(a.seq_lens[b], 0), a.max_seqlen);
  const int per_split =
      ((len + a.num_splits - 1) / a.num_splits + kTileKeys - 1) / kTileKeys * kTileKeys;
  const int k_begin = split * per_split;
  const int k_end = min(len, k_begin + per_split);
  const int tiles = k_begin < k_end ? (k_end - k_begin + kTileKeys - 1) / kTileKeys : 0;
  const int my_tiles = span == 1 ? (tiles > wave ? (tiles - wave + kWaves - 1) / kWaves : 0) : tiles;

  // Q^T, the B operand: lane (col, half) holds q[h0 + col][16 ks + 8 half .. + 7], zero past the
  // group.
  u32x4 qf[D / 16];
  {
    const bool ok = col < group;
    const uint16_t* qrow =
        static_cast<const uint16_t*>(a.q) + b * a.q_bs + (h0 + (ok ? col : 0)) * a.q_hs + 8 * half;
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) qf[ks] = ok ? load16(qrow + 16 * ks) : u32x4{0, 0, 0, 0};
  }

  // Paged cache: the split's block numbers, clamped to the pool (kPagedLds), or the table row.
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

  // Tile loads: load j of a tensor tile gives lane l row kRowsPerLoad j + l / kChunksPerRow, chunk
  // l % kChunksPerRow (whole rows per instruction), which it stores at that row's swizzled chunk.
  const int lane_row = lane / kChunksPerRow;
  const int lane_col = 8 * (lane % kChunksPerRow);
  const uint16_t* kbase =
      static_cast<const uint16_t*>(a.k) + (kPaged ? 0 : b * a.k_bs) + hkv * a.k_hs + lane_col;
  const uint16_t* vbase =
      static_cast<const uint16_t*>(a.v) + (kPaged ? 0 : b * a.v_bs) + hkv * a.v_hs + lane_col;
  // Offsets (elements) of a key's K and V rows from kbase / vbase.
  auto row_offsets = [&](int key, int64_t& ko, int64_t& vo) __attribute__((always_inline)) {
    if constexpr (kPaged) {
      const int page = a.page_shift >= 0 ? key >> a.page_shift : key / a.page_size;
      int block;
      if constexpr (kPageMode == kPagedLds) {
        block = page_table[page - page0];
      } else {
        block = min(max(table_row[page], 0), a.num_blocks - 1);
      }
      const int row = key - page * a.page_size;
      ko = static_cast<int64_t>(block) * a.k_bs + static_cast<int64_t>(row) * a.k_ss;
      vo = static_cast<int64_t>(block) * a.v_bs + static_cast<int64_t>(row) * a.v_ss;
    } else {
      ko = static_cast<int64_t>(key) * a.k_ss;
      vo = static_cast<int64_t>(key) * a.v_ss;
    }
  };
  char* wave_lds = reinterpret_cast<char*>(smem) + wave * kWaveBytes<D>;
  auto tile_start = [&](int i) __attribute__((always_inline)) {
    return k_begin + (span == 1 ? wave + kWaves * i : i) * kTileKeys;
  };
  using Regs = u32x4[2 * kLoads<D>];  // K loads, then V loads
  auto load_tile = [&](int i, Regs& r) __attribute__((always_inline)) {
    const int t0 = tile_start(i);
#pragma unroll
    for (int j = 0; j < kLoads<D>; ++j) {
      const int key = min(t0 + kRowsPerLoad * j + lane_row, k_end - 1);
      int64_t ko, vo;
      row_offsets(key, ko, vo);
      r[j] = load16_stream(kbase + ko);
      r[kLoads<D> + j] = load16_stream(vbase + vo);
    }
  };
  auto store_tile = [&](const Regs& r) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < kLoads<D>; ++j) {
      const int off = 2 * prefill::tile_offset<D>(kRowsPerLoad * j + lane_row, lane_col);
      *reinterpret_cast<u32x4*>(wave_lds + off) = r[j];
      *reinterpret_cast<u32x4*>(wave_lds + kTileBytes<D> + off) = r[kLoads<D> + j];
    }
  };

  f32x16 o[D / 32];
#pragma unroll
  for (int nb = 0; nb < D / 32; ++nb) o[nb] = f32x16{};
  // Reference point of o and l for the lane's head (log2 units, the same in both halves of a
  // column; kNoRef until the first tile): the running max of its scores, as in the reference's
  // online softmax. Probabilities are 2^(s scale_log2 - ref) <= 1, and the largest key seen so far
  // has p = 1 exactly, which the rounding of P to the input type keeps exact.
  float ref = kNoRef;
  float l = 0.f;  // the lane's part of the running sum (its 16 keys of each tile)
  const float sl2 = a.scale_log2;

  // Tile i from register set r: into LDS, fragments back, the set refilled with tile i + kAhead,
  // then S^T, the softmax and O^T. LDS operations of a wave complete in order, so the fragment
  // reads see the stores before them and the next tile's stores come after these reads.
  auto step = [&](int i, Regs& r) __attribute__((always_inline)) {
    store_tile(r);
    const uint16_t* kt = reinterpret_cast<const uint16_t*>(wave_lds);
    const uint16_t* vt = reinterpret_cast<const uint16_t*>(wave_lds + kTileBytes<D>);
    u32x4 kf[D / 16];
    u32x4 vf[2][D / 32];
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) kf[ks] = k_frag<D>(kt, 0, ks, lane);
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
      for (int nb = 0; nb < D / 32; ++nb) vf[kk][nb] = v_frag<D>(vt, nb, kk, lane);
    }
    // Unconditional (past the split the keys clamp to its last row): a load skipped on some path
    // leaves the compiler unsure how many are in flight, and it then waits for all of them.
    load_tile(i + kAhead, r);
    __builtin_amdgcn_sched_barrier(0);

    f32x16 s = f32x16{};
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) s = E::mfma32(kf[ks], qf[ks], s);
    const int t0 = tile_start(i);
    if (t0 + kTileKeys > k_end) {  // the split's last, partial tile (wave-uniform)
      const int lim = k_end - 1 - t0 - 4 * half;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        if (acc_key(j, 0) > lim) s[j] = -INFINITY;
      }
    }
    // The running max moves (and O and l are rescaled, a wave-uniform branch) only on tiles where
    // some head's max grows, so O, which the compiler keeps in accumulator registers, is left
    // alone on most tiles of a long sequence.
    float mx = s[0];
#pragma unroll
    for (int j = 1; j < 16; ++j) mx = fmaxf(mx, s[j]);
    // scale_log2 > 0, so the max commutes with it; every column sees a valid key of the tile.
    mx = max_halves(mx) * sl2;
    if (wave_any(mx > ref)) {
      const float moved = fmaxf(ref, mx);
      const float alpha = exp2_fast(ref - moved);  // 0 on the first tile
      ref = moved;
#pragma unroll
      for (int nb = 0; nb < D / 32; ++nb) o[nb] *= alpha;
      l *= alpha;
    }
    f32x16 p;
    float rs = 0.f;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      p[j] = exp2_fast(fmaf(s[j], sl2, -ref));
      rs += p[j];
    }
    l += rs;
    const u32x4 p0 = p_frag<Tag, 0>(p);
    const u32x4 p1 = p_frag<Tag, 1>(p);
#pragma unroll
    for (int nb = 0; nb < D / 32; ++nb) {
      o[nb] = E::mfma32(vf[0][nb], p0, o[nb]);
      o[nb] = E::mfma32(vf[1][nb], p1, o[nb]);
    }
  };

  // Guarded as a whole so the first loads are unconditional too (a split with no tile for this
  // wave has no valid row to clamp to).
  if (my_tiles > 0) {
    Regs r[kAhead];
    static_for<0, kAhead>([&](auto t) __attribute__((always_inline)) {
      load_tile(decltype(t)::value, r[decltype(t)::value]);
    });
    int i = 0;
    for (; i + kAhead <= my_tiles; i += kAhead) {
      static_for<0, kAhead>([&](auto t) __attribute__((always_inline)) {
        step(i + decltype(t)::value, r[decltype(t)::value]);
      });
    }
    static_for<0, kAhead>([&](auto t) __attribute__((always_inline)) {
      if (i + decltype(t)::value < my_tiles) step(i + decltype(t)::value, r[decltype(t)::value]);
    });
  }

  // Merge the four waves in order; the tile buffers are free after the barrier.
  __syncthreads();
  float* red_m = reinterpret_cast<float*>(smem);  // [kWaves][kCols]
  float* red_l = red_m + kWaves * kCols;          // [kWaves][kCols]
  float* red_o = red_l + kWaves * kCols;          // [kWaves][kCols][kRedPitch]
  const float lt = sum_halves(l);
  if (half == 0) {
    // A wave that saw no key (l = 0, ref still kNoRef) records -inf, as the merges expect.
    red_m[wave * kCols + col] = lt > 0.f ? ref : -INFINITY;
    red_l[wave * kCols + col] = lt;
  }
  if (col < group) {
    float* row = red_o + (wave * kCols + col) * kRedPitch<D>;
#pragma unroll
    for (int nb = 0; nb < D / 32; ++nb) {
#pragma unroll
      for (int j = 0; j < 16; ++j) row[32 * nb + acc_key(j, half)] = o[nb][j];
    }
  }
  __syncthreads();
  // Span 1: the four waves' states of one KV head are merged in wave order. Span 4: each wave's
  // state is its own KV head's and is written as it is.
  const int outs = span == 1 ? group * D : kWaves * group * D;
  for (int idx = tid; idx < outs; idx += kThreads) {
    const int wv0 = span == 1 ? 0 : idx / (group * D);
    const int r = idx - wv0 * group * D;
    const int g = r / D;
    const int d = r - g * D;
    float mm = -INFINITY;
    float num = 0.f;
    float den = 0.f;
    if (span == 1) {
#pragma unroll
      for (int wv = 0; wv < kWaves; ++wv) mm = fmaxf(mm, red_m[wv * kCols + g]);
#pragma unroll
      for (int wv = 0; wv < kWaves; ++wv) {
        const float mw = red_m[wv * kCols + g];
        if (mw != -INFINITY) {
          const float f = exp2_fast(mw - mm);
          num += red_o[(wv * kCols + g) * kRedPitch<D> + d] * f;
          den += red_l[wv * kCols + g] * f;
        }
      }
    } else {
      mm = red_m[wv0 * kCols + g];
      if (mm != -INFINITY) {
        num = red_o[(wv0 * kCols + g) * kRedPitch<D> + d];
        den = red_l[wv0 * kCols + g];
      }
    }
    const int h = (span == 1 ? h0 : (hq * span + wv0) * group) + g;
    if (a.num_splits == 1) {
      uint16_t* orow = static_cast<uint16_t*>(a.o) + b * a.o_bs + h * a.o_hs;
      orow[d] = E::from_float(den > 0.f ? num / den : 0.f);
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

template <typename Tag, int D>
hipError_t launch_typed(const DecodeArgs& args, hipStream_t stream) {
  const dim3 grid(args.batch * (args.heads_kv / args.mfma_span) * args.num_splits);
  if (args.block_tables == nullptr) {
    hipLaunchKernelGGL((decode_mfma_kernel<Tag, D, kContiguous>), grid, dim3(kThreads), 0, stream, args);
  } else if (!args.page_table_global) {
    hipLaunchKernelGGL((decode_mfma_kernel<Tag, D, kPagedLds>), grid, dim3(kThreads), 0, stream, args);
  } else {
    hipLaunchKernelGGL((decode_mfma_kernel<Tag, D, kPagedGlobal>), grid, dim3(kThreads), 0, stream, args);
  }
  return hipGetLastError();
}

}  // namespace
}  // namespace decode_mfma

hipError_t launch_decode_mfma_split(const DecodeArgs& args, DType dtype, int head_dim,
                                    hipStream_t stream) {
  using namespace decode_mfma;
  if (args.group > kMaxDecodeMfmaHeads) return hipErrorInvalidValue;
  if (dtype == DType::bf16) {
    return head_dim == 64 ? launch_typed<bf16_tag, 64>(args, stream)
                          : launch_typed<bf16_tag, 128>(args, stream);
  }
  if (dtype == DType::f16) {
    return head_dim == 64 ? launch_typed<f16_tag, 64>(args, stream)
                          : launch_typed<f16_tag, 128>(args, stream);
  }
  return hipErrorInvalidValue;
}

}  // namespace fl
