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
// Scheduling groups that keep the K fragment reads ahead of the score MFMAs.
#ifndef FL_PREFILL_QK_SCHED
#define FL_PREFILL_QK_SCHED 1
#endif
// K fragment reads issued ahead of their MFMAs.
#ifndef FL_PREFILL_K_AHEAD
#define FL_PREFILL_K_AHEAD 2
#endif
// Instruction classes of __builtin_amdgcn_sched_group_barrier.
constexpr int kSchedMfma = 0x008;
constexpr int kSchedDsRead = 0x100;

template <typename Tag, int D>
__global__ void __launch_bounds__(kThreads)
    __attribute__((amdgpu_waves_per_eu(FL_PREFILL_WAVES_PER_EU, FL_PREFILL_WAVES_PER_EU)))
    prefill_fwd_kernel(const PrefillArgs a) {
  using E = Elem<Tag>;
  constexpr int kTile = kTileElems<D>;
  // Two K and two V tile slots, each its own array: slot addresses are compile-time constants in
  // the unrolled loop below (every LDS read is one per-lane offset register plus an immediate),
  // and the compiler can tell that loads into one slot do not alias reads of another, so it does
  // not wait for the next tile's loads before reading this tile.
  __shared__ __attribute__((aligned(16))) uint16_t k_lds0[kTile];
  __shared__ __attribute__((aligned(16))) uint16_t k_lds1[kTile];
  __shared__ __attribute__((aligned(16))) uint16_t v_lds0[kTile];
  __shared__ __attribute__((aligned(16))) uint16_t v_lds1[kTile];

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

  // Per-lane LDS byte offsets within a tile (the swizzle makes them lane-dependent).
  int k_lds[D / 16];
#pragma unroll
  for (int ks = 0; ks < D / 16; ++ks) k_lds[ks] = k_lane_offset<D>(ks, lane);
  int v_lds[D / 32][2];
#pragma unroll
  for (int nb = 0; nb < D / 32; ++nb) {
    v_lds[nb][0] = v_lane_offset<D>(nb, 0, lane);
    v_lds[nb][1] = v_lane_offset<D>(nb, 1, lane);
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
  auto dma = [&](uint16_t* slot, const uint16_t* base, int64_t seq_stride,
                 const int (&off)[kDmaPerWave], int tile) {
    const int k0 = tile * kBlockN;
    const int rows = min(kBlockN, a.seqlen_k - k0);
    const auto rsrc =
        buffer_rsrc(base + k0 * seq_stride, static_cast<int>(((rows - 1) * seq_stride + D) * 2));
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

  // One tile: loads of the next tile into the other slots, then (for a wave that sees any of its
  // keys) scores, softmax and P V from slot kSlot, and a barrier after which the next tile's data
  // is in LDS and this tile's slots are free.
  auto tile_step = [&](int t, auto slot_tag) {
    constexpr int kSlot = decltype(slot_tag)::value;
    const char* kt = reinterpret_cast<const char*>(kSlot == 0 ? k_lds0 : k_lds1);
    const char* vt = reinterpret_cast<const char*>(kSlot == 0 ? v_lds0 : v_lds1);
    if (t + 1 < num_tiles) {
      dma(kSlot == 0 ? k_lds1 : k_lds0, kp, a.k_ss, k_off, t + 1);
      dma(kSlot == 0 ? v_lds1 : v_lds0, vp, a.v_ss, v_off, t + 1);
    }
    const int k0 = t * kBlockN;
    // A wave that sees no key of this tile sees none of the later ones either (causal).
    const bool active = !(a.causal && k0 > row0 + kRowsPerWave - 1 + a.causal_offset);
    if (active) {
      // S^T = K Q^T, K fragments read kAhead steps ahead of their MFMAs.
      constexpr int kSteps = D / 16;
      constexpr int kAhead = FL_PREFILL_K_AHEAD < kSteps ? FL_PREFILL_K_AHEAD : kSteps;
      f32x16 s0 = f32x16{};
      f32x16 s1 = f32x16{};
      {
        u32x4 a0[kSteps];
        u32x4 a1[kSteps];
#pragma unroll
        for (int ks = 0; ks < kAhead; ++ks) {
          a0[ks] = lds_load16(kt, k_lds[ks]);
          a1[ks] = lds_load16(kt + kKeyBlockBytes<D>, k_lds[ks]);
        }
#pragma unroll
        for (int ks = 0; ks < kSteps; ++ks) {
          if (ks + kAhead < kSteps) {
            a0[ks + kAhead] = lds_load16(kt, k_lds[ks + kAhead]);
            a1[ks + kAhead] = lds_load16(kt + kKeyBlockBytes<D>, k_lds[ks + kAhead]);
          }
          s0 = E::mfma32(a0[ks], qf[ks], s0);
          s1 = E::mfma32(a1[ks], qf[ks], s1);
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
      }
      // Keys past the end or above the diagonal: only edge and diagonal tiles (wave-uniform
      // branch; the empty asm keeps the compiler from turning it into selects on every tile).
      if ((k0 + kBlockN > a.seqlen_k) ||
          (a.causal && k0 + kBlockN - 1 > row0 + a.causal_offset)) {
        asm volatile("" ::: "memory");
        // acc_key(j, half) = acc_key(j, 0) + 4 half: fold the lane's part into the limit so every
        // comparison is against a compile-time constant (no per-key registers live in the loop).
        const int lim = last_key - k0 - 4 * half;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          constexpr int kBase = 0;
          const int kj = acc_key(j, kBase);
          if (kj > lim) s0[j] = -INFINITY;
          if (kj + 32 > lim) s1[j] = -INFINITY;
        }
      }
      // Online softmax in the exp2 domain on raw scores: with scale > 0,
      // max(scale * s) = scale * max(s), and p = 2^(s * scale_log2 - ref). The reference point
      // `ref` of o and l moves to the row's running max when it has grown by more than
      // kMoveSlack over it (prefill_tile.hpp), so probabilities stay at most 2^kMoveSlack and most
      // tiles of a long row skip the rescale of o.
      float mx = max_of(s0, s1);
      mx = max2_f32(mx, xor_lane(mx, 32));
      const float cand = mx * sl2;  // -inf while the row has seen only hidden keys
      const bool move = cand > ref + kMoveSlack;
      const float alpha = move ? exp2_fast(ref - cand) : 1.f;  // ref = -inf gives 0
      ref = move ? cand : ref;
      if (wave_any(move)) {
        asm volatile("" ::: "memory");
#pragma unroll
        for (int nb = 0; nb < D / 32; ++nb) o[nb] *= alpha;
      }
      // Rows without a visible key so far have only -inf scores: any finite shift gives p = 0.
      const float shift = ref == -INFINITY ? 0.f : ref;
      float rs0 = 0.f;
      float rs1 = 0.f;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        s0[j] = exp2_fast(fmaf(s0[j], sl2, -shift));
        s1[j] = exp2_fast(fmaf(s1[j], sl2, -shift));
        rs0 += s0[j];
        rs1 += s1[j];
      }
      l = fmaf(l, alpha, rs0 + rs1);
      const u32x4 pf[4] = {p_frag<Tag, 0>(s0), p_frag<Tag, 1>(s0), p_frag<Tag, 0>(s1),
                           p_frag<Tag, 1>(s1)};
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
#pragma unroll
        for (int nb = 0; nb < D / 32; ++nb) {
          const u32x4 vf = v_frag_at(vt + kk * kKeyStepBytes<D>, v_lds[nb][0], v_lds[nb][1]);
          o[nb] = E::mfma32(vf, pf[kk], o[nb]);
        }
      }
    }
    // The loads issued above have landed (the barrier waits for them) and every wave is done
    // with this tile's slots.
    __syncthreads();
  };

  if (num_tiles > 0) {
    dma(k_lds0, kp, a.k_ss, k_off, 0);
    dma(v_lds0, vp, a.v_ss, v_off, 0);
    __syncthreads();
  }
  for (int t = 0; t < num_tiles; t += 2) {
    tile_step(t, std::integral_constant<int, 0>{});
    if (t + 1 < num_tiles) tile_step(t + 1, std::integral_constant<int, 1>{});
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

// head_dim 128 and 64 run on the ping-pong kernel (prefill_pp.hip); FL_PREFILL_PINGPONG=0 keeps
// them on this one (for comparisons).
#ifndef FL_PREFILL_PINGPONG
#define FL_PREFILL_PINGPONG 1
#endif

// Which prefill kernel a call runs. Below 256 ping-pong workgroups non-causal, 128 causal (256 query
// rows each at head_dim 128, 384 at 64; causal blocks paired; one workgroup per CU), this kernel,
// whose 128-row workgroups (two per CU) spread a short prompt over more CUs. Measured on MI355X
// (TFLOP/s, ping-pong / this kernel, B=1, H=32, D = 128): S=1024 non-causal (128 workgroups)
// 532 / 552, S=2048 (256) 1,083 / 957; causal S=1024 (64) 242 / 261, S=2048 (128) 642 / 551; B=4
// causal S=512 (128) 270 / 269. Also this kernel: a non-causal call whose ping-pong blocks would be
// more than a quarter padding (at head_dim 64, S = 512 pads 256 of 768 rows) and that needs more
// than one round of workgroups, where the padded blocks take a round's time for a third of its
// rows: H=32, D = 64, S = 512, B=16 523 / 618, B=32 537 / 654; one round (B=4) 276 / 230; 11%
// padding (S = 2048, B=8, H=16) 931 / 819. The FL_KNOB_PREFILL_PP_MIN_WG knob replaces all of
// this with its own workgroup threshold (so tests can route one shape to either kernel).
bool prefill_on_pingpong(const PrefillArgs& args, int head_dim) {
  const int rows = prefill_pp_block_rows(head_dim);
  const int64_t pp_blocks = (args.seqlen_q + rows - 1) / rows;
  const int64_t pp_items = args.causal ? (pp_blocks + 1) / 2 : pp_blocks;
  const int64_t workgroups = pp_items * args.batch * args.heads;
  const int v = knob(FL_KNOB_PREFILL_PP_MIN_WG);
  if (v >= 0) return workgroups >= v;
  if (args.causal) return workgroups >= 128;
  const int64_t padding = pp_blocks * rows - args.seqlen_q;
  if (4 * padding > pp_blocks * rows && workgroups > 256) return false;
  return workgroups >= 256;
}

hipError_t launch_prefill(const PrefillArgs& args, DType dtype, int head_dim, hipStream_t stream) {
  using namespace prefill;
  if (FL_PREFILL_PINGPONG && prefill_on_pingpong(args, head_dim))
    return launch_prefill_pingpong(args, dtype, head_dim, stream);
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
