// FlashAttention-2 forward (prefill) for gfx950: bf16/fp16 inputs, fp32 accumulation on
// v_mfma_f32_32x32x16, exp2-domain online softmax, natural-log LSE.
//
// Serves the attention_mma_pipelined and attention_mma ops of the reference
// (csrc/prefill/mma_pipelined.cu:54-183); the algorithm (tiling, online softmax with the
// -inf-safe reference point, bottom-right causal mask, 1/l epilogue) follows the reference's
// definitions (csrc/prefill/mma_tile.cuh:60-174, flash_lab/reference.py:90-152), the mapping onto
// the machine is this file's own:
//
//  * Workgroup: 4 waves x 32 query rows = 128 rows of one (batch, head). Lane layouts are in
//    prefill_tile.hpp: scores and outputs are held transposed so a lane owns one query row.
//  * K and V tiles of 64 keys go global -> registers -> LDS through a two-slot LDS ring: the next
//    tile's global loads are issued before the current tile's math and written to the other slot
//    at the top of the next iteration, one barrier per tile.
//  * Work order: the 1-D grid is remapped so each XCD (workgroups are dealt round-robin over the
//    8 XCDs) runs a contiguous range of (batch, head) pairs and their K/V stay in that XCD's L2.
//    Within a (batch, head) the causal query blocks run heaviest first.
#include <type_traits>

#include "launch.hpp"
#include "prefill_tile.hpp"

namespace fl {
namespace prefill {
namespace {

constexpr int kXcds = 8;
constexpr float kLn2 = 0.693147180559945309f;
// log2 of the largest probability the lazily moved reference point allows.
constexpr float kRescaleSlack = 8.f;

// Max of the 32 scores a lane holds, as a tree of three-input maxes.
__device__ __forceinline__ float max_of(const f32x16& x, const f32x16& y) {
  float t[11];
#pragma unroll
  for (int i = 0; i < 5; ++i) t[i] = fmaxf(fmaxf(x[3 * i], x[3 * i + 1]), x[3 * i + 2]);
#pragma unroll
  for (int i = 0; i < 5; ++i) t[5 + i] = fmaxf(fmaxf(y[3 * i], y[3 * i + 1]), y[3 * i + 2]);
  t[10] = fmaxf(x[15], y[15]);
  const float u0 = fmaxf(fmaxf(t[0], t[1]), t[2]);
  const float u1 = fmaxf(fmaxf(t[3], t[4]), t[5]);
  const float u2 = fmaxf(fmaxf(t[6], t[7]), t[8]);
  const float u3 = fmaxf(t[9], t[10]);
  return fmaxf(fmaxf(u0, u1), fmaxf(u2, u3));
}

// Bijection on [0, n): ids dealt to XCD x (id % 8 == x) get the contiguous range
// [x * n / 8, (x + 1) * n / 8) of work items. A ragged tail keeps its own ids.
__device__ __forceinline__ int xcd_remap(int id, int n) {
  const int per = n / kXcds;
  if (id >= per * kXcds) return id;
  return (id % kXcds) * per + id / kXcds;
}

// Waves per SIMD the register allocation is held to (two: one workgroup's softmax can overlap
// another's MFMA work on the same SIMD).
#ifndef FL_PREFILL_WAVES_PER_EU
#define FL_PREFILL_WAVES_PER_EU 2
#endif
// Scheduling hints that interleave the next tile's score MFMAs with the softmax VALU work, and
// the VALU instructions placed after each MFMA.
#ifndef FL_PREFILL_SCHED
#define FL_PREFILL_SCHED 0
#endif
// Software pipelining: the scores of tile t + 1 computed next to the softmax of tile t (costs a
// second score buffer of 32 registers).
#ifndef FL_PREFILL_PIPELINE
#define FL_PREFILL_PIPELINE 0
#endif
// Scheduling groups that keep the K fragment reads ahead of the score MFMAs.
#ifndef FL_PREFILL_QK_SCHED
#define FL_PREFILL_QK_SCHED 1
#endif
// K fragment reads issued ahead of their MFMAs.
#ifndef FL_PREFILL_K_AHEAD
#define FL_PREFILL_K_AHEAD 2
#endif
#ifndef FL_PREFILL_VALU_PER_MFMA
#define FL_PREFILL_VALU_PER_MFMA 8
#endif
// Instruction classes of __builtin_amdgcn_sched_group_barrier.
constexpr int kSchedValu = 0x002;
constexpr int kSchedMfma = 0x008;
constexpr int kSchedDsRead = 0x100;

template <typename Tag, int D>
__global__ void __launch_bounds__(kThreads)
    __attribute__((amdgpu_waves_per_eu(FL_PREFILL_WAVES_PER_EU, FL_PREFILL_WAVES_PER_EU)))
    prefill_fwd_kernel(const PrefillArgs a) {
  using E = Elem<Tag>;
  constexpr int kTile = kTileElems<D>;
  // Four tile slots: K tiles in slots 0 and 1, V tiles in slots 2 and 3.
  __shared__ __attribute__((aligned(16))) uint16_t smem[4 * kTile];
  auto k_slot = [&](int i) { return smem + i * kTile; };
  auto v_slot = [&](int i) { return smem + (2 + i) * kTile; };

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int half = lane >> 5;

  const int work = xcd_remap(blockIdx.x, gridDim.x);
  const int bh = work / a.q_blocks;
  int qb = work - bh * a.q_blocks;
  if (a.causal) qb = a.q_blocks - 1 - qb;
  const int b = bh / a.heads;
  const int h = bh - b * a.heads;
  const int hkv = h / a.group;
  const int q0 = qb * kBlockM;
  const int row0 = q0 + wave * kRowsPerWave;  // first query row of this wave
  const int my_row = row0 + (lane & 31);      // the query row this lane owns

  const uint16_t* qp = a.q + b * a.q_bs + h * a.q_hs;
  const uint16_t* kp = a.k + b * a.k_bs + hkv * a.k_hs;
  const uint16_t* vp = a.v + b * a.v_bs + hkv * a.v_hs;

  int kv_end = a.seqlen_k;
  if (a.causal) kv_end = min(kv_end, min(q0 + kBlockM, a.seqlen_q) + a.causal_offset);
  const int num_tiles = kv_end > 0 ? (kv_end + kBlockN - 1) / kBlockN : 0;

  // Q^T fragments, the B operand of every S^T step: row my_row, dims 16 ks + 8 half .. + 7.
  u32x4 qf[D / 16];
  {
    const bool ok = my_row < a.seqlen_q;
    const uint16_t* src = qp + static_cast<int64_t>(ok ? my_row : 0) * a.q_ss + 8 * half;
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) qf[ks] = ok ? load16(src + 16 * ks) : u32x4{0, 0, 0, 0};
  }

  // Tiles go from HBM straight into LDS (buffer_load ... lds): each wave moves kDmaPerWave
  // 1 KiB blocks of a tile; lane l's 16 bytes land at block + 16 l, so lane l fetches the
  // logical chunk that the swizzle stores at that position. The buffer resource is rebased on
  // each tile and sized to its valid rows: rows past the end of the sequence (the sequence stride
  // being at least D) fall outside it and arrive as zeros, so 0 * V stays finite.
  constexpr int kChunksPerRow = D / 8;
  constexpr int kRowsPerBlock = 64 / kChunksPerRow;
  constexpr int kDmaPerWave = kBlockN / kRowsPerBlock / kWaves;
  int k_off[kDmaPerWave];
  int v_off[kDmaPerWave];
#pragma unroll
  for (int j = 0; j < kDmaPerWave; ++j) {
    const int row = (wave * kDmaPerWave + j) * kRowsPerBlock + lane / kChunksPerRow;
    const int chunk = (lane % kChunksPerRow) ^ swz<D>(row);
    k_off[j] = static_cast<int>((row * a.k_ss + 8 * chunk) * 2);
    v_off[j] = static_cast<int>((row * a.v_ss + 8 * chunk) * 2);
  }
  auto dma = [&](uint16_t* slot, const uint16_t* base, int64_t seq_stride, const int(&off)[kDmaPerWave],
                 int tile) {
    const int k0 = tile * kBlockN;
    const int rows = min(kBlockN, a.seqlen_k - k0);
    const auto rsrc = buffer_rsrc(base + k0 * seq_stride, static_cast<int>(((rows - 1) * seq_stride + D) * 2));
#pragma unroll
    for (int j = 0; j < kDmaPerWave; ++j)
      buffer_load16_to_lds(rsrc, slot + (wave * kDmaPerWave + j) * 512, off[j]);
  };

  f32x16 o[D / 32];
#pragma unroll
  for (int nb = 0; nb < D / 32; ++nb) o[nb] = f32x16{};
  float ref = -INFINITY;  // reference point of o and l, log2 units; -inf until a key is seen
  float l = 0.f;          // this lane's share of the running sum
  const float sl2 = a.scale_log2;
  // Last key my_row may see in the whole problem.
  const int last_key = a.causal ? min(a.seqlen_k - 1, my_row + a.causal_offset) : a.seqlen_k - 1;

  // S^T of the tile in k_tile for this wave's 32 rows. K fragments are read kKAhead steps ahead
  // of the MFMAs that consume them, so the LDS latency overlaps the MFMA chain.
  auto scores = [&](const uint16_t* k_tile, f32x16 (&s)[2]) {
    constexpr int kSteps = D / 16;
    constexpr int kAhead = FL_PREFILL_K_AHEAD < kSteps ? FL_PREFILL_K_AHEAD : kSteps;
    u32x4 a0[kSteps];
    u32x4 a1[kSteps];
#pragma unroll
    for (int ks = 0; ks < kAhead; ++ks) {
      a0[ks] = k_frag<D>(k_tile, 0, ks, lane);
      a1[ks] = k_frag<D>(k_tile, 1, ks, lane);
    }
    s[0] = f32x16{};
    s[1] = f32x16{};
#pragma unroll
    for (int ks = 0; ks < kSteps; ++ks) {
      if (ks + kAhead < kSteps) {
        a0[ks + kAhead] = k_frag<D>(k_tile, 0, ks + kAhead, lane);
        a1[ks + kAhead] = k_frag<D>(k_tile, 1, ks + kAhead, lane);
      }
      s[0] = E::mfma32(a0[ks], qf[ks], s[0]);
      s[1] = E::mfma32(a1[ks], qf[ks], s[1]);
    }
#if FL_PREFILL_QK_SCHED
    // Keep the reads kAhead steps ahead: the scheduler otherwise pulls each read down to its
    // MFMA and the LDS latency is exposed on every step.
    __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2 * kAhead, 1);
#pragma unroll
    for (int ks = 0; ks < kSteps - kAhead; ++ks) {
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, 2, 1);
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 1);
    }
    __builtin_amdgcn_sched_group_barrier(kSchedMfma, 2 * kAhead, 1);
#endif
  };

  // Prologue: K and V of tile 0 and K of tile 1 in flight (then, pipelined, the scores of tile 0).
  f32x16 s_cur[2];
  if (num_tiles > 0) {
    dma(k_slot(0), kp, a.k_ss, k_off, 0);
    dma(v_slot(0), vp, a.v_ss, v_off, 0);
#if FL_PREFILL_PIPELINE
    if (num_tiles > 1) dma(k_slot(1), kp, a.k_ss, k_off, 1);
#endif
    __syncthreads();
#if FL_PREFILL_PIPELINE
    scores(k_slot(0), s_cur);
#endif
  }

  // Iteration t: scores, softmax and P V of tile t while the next tile's loads are in flight; each
  // load goes to the slot of tile t - 1, which every wave finished with before the last barrier.
  // Pipelined, the scores of tile t + 1 (MFMA) are computed in the same straight-line block as the
  // softmax of tile t (VALU) so the two interleave; K then runs two tiles ahead: K(t + 2) goes to
  // K(t)'s slot, whose scores were computed in the previous iteration.
  for (int t = 0; t < num_tiles; ++t) {
#if FL_PREFILL_PIPELINE
    if (t + 2 < num_tiles) dma(k_slot(t & 1), kp, a.k_ss, k_off, t + 2);
#else
    if (t + 1 < num_tiles) dma(k_slot((t + 1) & 1), kp, a.k_ss, k_off, t + 1);
#endif
    if (t + 1 < num_tiles) dma(v_slot((t + 1) & 1), vp, a.v_ss, v_off, t + 1);

    const int k0 = t * kBlockN;
    // A wave that sees no key of this tile sees none of the later ones either (causal).
    const bool active = !(a.causal && k0 > row0 + kRowsPerWave - 1 + a.causal_offset);
    if (active) {
#if FL_PREFILL_PIPELINE
      f32x16 s_next[2];
#endif
      u32x4 pf[4];
      bool move;
      float alpha;
      auto step = [&](auto masked) {
#if FL_PREFILL_PIPELINE
        // Scores of tile t + 1. On the last tile the slot holds stale data; the result is unused.
        scores(k_slot((t + 1) & 1), s_next);
#else
        scores(k_slot(t & 1), s_cur);
#endif
        if constexpr (decltype(masked)::value) {
          const int lim = last_key - k0;
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            const int kj = acc_key(j, half);
            if (kj > lim) s_cur[0][j] = -INFINITY;
            if (kj + 32 > lim) s_cur[1][j] = -INFINITY;
          }
        }
        // Online softmax in the exp2 domain on raw scores: with scale > 0,
        // max(scale * s) = scale * max(s), and p = 2^(s * scale_log2 - ref). The reference point
        // `ref` of o and l only moves when the row max has grown by more than kRescaleSlack over
        // it, so probabilities stay at most 2^kRescaleSlack (no overflow; a bf16/fp16 P keeps its
        // relative precision) and most tiles skip the rescale of o.
        float mx = max_of(s_cur[0], s_cur[1]);
        mx = fmaxf(mx, xor_lane(mx, 32));
        const float cand = mx * sl2;  // -inf while the row has seen only hidden keys
        move = cand > ref + kRescaleSlack;
        alpha = move ? exp2_fast(ref - cand) : 1.f;  // ref = -inf gives 0
        ref = move ? cand : ref;
        // Rows without a visible key so far have only -inf scores: any finite shift gives p = 0.
        const float shift = ref == -INFINITY ? 0.f : ref;
        float rs0 = 0.f;
        float rs1 = 0.f;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          s_cur[0][j] = exp2_fast(fmaf(s_cur[0][j], sl2, -shift));
          s_cur[1][j] = exp2_fast(fmaf(s_cur[1][j], sl2, -shift));
          rs0 += s_cur[0][j];
          rs1 += s_cur[1][j];
        }
        l = fmaf(l, alpha, rs0 + rs1);
        pf[0] = p_frag<Tag, 0>(s_cur[0]);
        pf[1] = p_frag<Tag, 1>(s_cur[0]);
        pf[2] = p_frag<Tag, 0>(s_cur[1]);
        pf[3] = p_frag<Tag, 1>(s_cur[1]);
#if FL_PREFILL_SCHED
        // Interleave: K reads ahead, then one MFMA per group of VALU instructions.
        __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 4, 0);
#pragma unroll
        for (int i = 0; i < D / 8 - 4; ++i) {
          __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
          __builtin_amdgcn_sched_group_barrier(kSchedValu, FL_PREFILL_VALU_PER_MFMA, 0);
          __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
          __builtin_amdgcn_sched_group_barrier(kSchedValu, FL_PREFILL_VALU_PER_MFMA, 0);
        }
#endif
      };
      const bool need_mask = (k0 + kBlockN > a.seqlen_k) ||
                             (a.causal && k0 + kBlockN - 1 > row0 + a.causal_offset);
      if (need_mask) {
        step(std::true_type{});
      } else {
        step(std::false_type{});
      }
      if (wave_any(move)) {
#pragma unroll
        for (int nb = 0; nb < D / 32; ++nb) o[nb] *= alpha;
      }
      const uint16_t* vt = v_slot(t & 1);
#pragma unroll
      for (int nb = 0; nb < D / 32; ++nb) {
        o[nb] = E::mfma32(v_frag<D>(vt, nb, 0, lane), pf[0], o[nb]);
        o[nb] = E::mfma32(v_frag<D>(vt, nb, 1, lane), pf[1], o[nb]);
        o[nb] = E::mfma32(v_frag<D>(vt, nb, 2, lane), pf[2], o[nb]);
        o[nb] = E::mfma32(v_frag<D>(vt, nb, 3, lane), pf[3], o[nb]);
      }
#if FL_PREFILL_PIPELINE
      s_cur[0] = s_next[0];
      s_cur[1] = s_next[1];
#endif
    }
    // The loads issued above have landed (the barrier waits for them) and every wave is done
    // with the slots they overwrite next.
    __syncthreads();
  }

  // Epilogue: l over both halves, 1/l (0 for rows that saw no key, which then store zeros).
  const float lt = l + xor_lane(l, 32);
  const float inv = lt > 0.f ? 1.f / lt : 0.f;
  if (my_row < a.seqlen_q) {
    uint16_t* orow = a.o + b * a.o_bs + static_cast<int64_t>(my_row) * a.o_ss + h * a.o_hs;
#pragma unroll
    for (int nb = 0; nb < D / 32; ++nb) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = 32 * nb + 8 * g + 4 * half;
        const u32x2 packed{E::pack2(o[nb][4 * g] * inv, o[nb][4 * g + 1] * inv),
                           E::pack2(o[nb][4 * g + 2] * inv, o[nb][4 * g + 3] * inv)};
        *reinterpret_cast<u32x2*>(orow + d) = packed;
      }
    }
    if (half == 0) {
      // l = sum 2^(s scale_log2 - ref), so ln(sum e^(s scale)) = ref ln 2 + ln l.
      a.lse[(static_cast<int64_t>(b) * a.heads + h) * a.seqlen_q + my_row] =
          lt > 0.f ? ref * kLn2 + logf(lt) : -INFINITY;
    }
  }
}

// One wave: a 16 x 16 tile through k_frag / v_frag / p_frag and the accumulator layout of the
// prefill kernel (D = 64 LDS pitch). Inputs are zero-padded to the 32 x 32 MFMA tile.
__global__ void __launch_bounds__(64) mfma_tile_test_kernel(const uint16_t* a, const uint16_t* b,
                                                             float* c, int k, int trans_b) {
  constexpr int D = 64;
  __shared__ __attribute__((aligned(16))) uint16_t tile[kTileElems<D>];
  const int lane = threadIdx.x;
  const int half = lane >> 5;
  const int row = lane & 31;
  for (int i = lane; i < kTileElems<D>; i += 64) tile[i] = 0;
  __syncthreads();
  if (!trans_b) {
    // b [16, k] is K (16 keys), a [16, k] is Q (16 query rows): S^T[key][row] = (a b^T)[row][key].
    for (int i = lane; i < 16 * k; i += 64) tile[tile_offset<D>(i / k, i % k)] = b[i];
    __syncthreads();
    f32x16 s = f32x16{};
    for (int ks = 0; ks < k / 16; ++ks) {
      uint32_t w[4];
      for (int e = 0; e < 4; ++e) {
        const int d = 16 * ks + 8 * half + 2 * e;
        w[e] = row < 16 ? (static_cast<uint32_t>(a[row * k + d]) |
                           (static_cast<uint32_t>(a[row * k + d + 1]) << 16))
                        : 0u;
      }
      s = Elem<bf16_tag>::mfma32(k_frag<D>(tile, 0, ks, lane), u32x4{w[0], w[1], w[2], w[3]}, s);
    }
    if (row < 16) {
      for (int j = 0; j < 16; ++j) {
        const int key = acc_key(j, half);
        if (key < 16) c[row * 16 + key] = s[j];
      }
    }
  } else {
    // b [k, 16] is V (k keys x 16 dims), a [16, k] is P: O^T[d][row] = (a b)[row][d].
    for (int i = lane; i < k * 16; i += 64) tile[tile_offset<D>(i / 16, i % 16)] = b[i];
    __syncthreads();
    f32x16 s0 = f32x16{};
    f32x16 s1 = f32x16{};
    for (int j = 0; j < 16; ++j) {
      const int key = acc_key(j, half);
      s0[j] = (row < 16 && key < k) ? Elem<bf16_tag>::to_float(a[row * k + key]) : 0.f;
      s1[j] = (row < 16 && key + 32 < k) ? Elem<bf16_tag>::to_float(a[row * k + key + 32]) : 0.f;
    }
    const u32x4 p[4] = {p_frag<bf16_tag, 0>(s0), p_frag<bf16_tag, 1>(s0), p_frag<bf16_tag, 0>(s1),
                        p_frag<bf16_tag, 1>(s1)};
    f32x16 o = f32x16{};
    for (int kk = 0; kk < k / 16; ++kk) o = Elem<bf16_tag>::mfma32(v_frag<D>(tile, 0, kk, lane), p[kk], o);
    if (row < 16) {
      for (int j = 0; j < 16; ++j) {
        const int d = acc_key(j, half);
        if (d < 16) c[row * 16 + d] = o[j];
      }
    }
  }
}

template <typename Tag, int D>
hipError_t launch_typed(const PrefillArgs& args, hipStream_t stream) {
  const int blocks = args.q_blocks * args.batch * args.heads;
  hipLaunchKernelGGL((prefill_fwd_kernel<Tag, D>), dim3(blocks), dim3(kThreads), 0, stream, args);
  return hipGetLastError();
}

}  // namespace
}  // namespace prefill

static_assert(kPrefillBlockM == prefill::kBlockM, "host and kernel tile heights differ");
static_assert(kPrefillBlockN == prefill::kBlockN, "host and kernel tile widths differ");

hipError_t launch_prefill(const PrefillArgs& args, DType dtype, int head_dim, hipStream_t stream) {
  using namespace prefill;
  if (dtype == DType::bf16) {
    return head_dim == 64 ? launch_typed<bf16_tag, 64>(args, stream)
                          : launch_typed<bf16_tag, 128>(args, stream);
  }
  return head_dim == 64 ? launch_typed<f16_tag, 64>(args, stream)
                        : launch_typed<f16_tag, 128>(args, stream);
}

hipError_t launch_mfma_tile_test(const uint16_t* a, const uint16_t* b, float* c, int k, int trans_b,
                                 hipStream_t stream) {
  hipLaunchKernelGGL(prefill::mfma_tile_test_kernel, dim3(1), dim3(64), 0, stream, a, b, c, k,
                     trans_b);
  return hipGetLastError();
}

}  // namespace fl
