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

template <typename Tag, int D>
__global__ void __launch_bounds__(kThreads)
    __attribute__((amdgpu_waves_per_eu(FL_PREFILL_WAVES_PER_EU, FL_PREFILL_WAVES_PER_EU)))
    prefill_fwd_kernel(const PrefillArgs a) {
  using E = Elem<Tag>;
  constexpr int kTile = kTileElems<D>;
  // Two slots, each K then V.
  __shared__ __attribute__((aligned(16))) uint16_t smem[4 * kTile];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
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

  // Tile staging: each thread moves kPasses 16-byte pieces of K and of V per tile. Loads go
  // through buffer resources rebased on each tile and sized to its valid rows, so the per-thread
  // byte offsets are fixed for the whole kernel and, the sequence stride being at least D, rows
  // past the end of the sequence fall outside the resource and read as zeros (0 * V stays
  // finite) with no branch.
  constexpr int kChunks = D / 8;
  constexpr int kRowsPerPass = kThreads / kChunks;
  constexpr int kPasses = kBlockN / kRowsPerPass;
  const int st_row = tid / kChunks;
  const int st_col = (tid % kChunks) * 8;
  int k_off[kPasses];
  int v_off[kPasses];
#pragma unroll
  for (int p = 0; p < kPasses; ++p) {
    const int r = st_row + p * kRowsPerPass;
    k_off[p] = static_cast<int>((r * a.k_ss + st_col) * 2);
    v_off[p] = static_cast<int>((r * a.v_ss + st_col) * 2);
  }
  u32x4 kst[kPasses];
  u32x4 vst[kPasses];

  auto fetch = [&](int tile) {
    const int k0 = tile * kBlockN;
    const int rows = min(kBlockN, a.seqlen_k - k0);
    const auto krs = buffer_rsrc(kp + k0 * a.k_ss, static_cast<int>(((rows - 1) * a.k_ss + D) * 2));
    const auto vrs = buffer_rsrc(vp + k0 * a.v_ss, static_cast<int>(((rows - 1) * a.v_ss + D) * 2));
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
      kst[p] = buffer_load16(krs, k_off[p]);
      vst[p] = buffer_load16(vrs, v_off[p]);
    }
  };
  auto stash = [&](int slot) {
    uint16_t* kt = smem + 2 * slot * kTile;
    uint16_t* vt = kt + kTile;
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
      const int r = st_row + p * kRowsPerPass;
      *reinterpret_cast<u32x4*>(kt + r * kPitch<D> + st_col) = kst[p];
      *reinterpret_cast<u32x4*>(vt + r * kPitch<D> + st_col) = vst[p];
    }
  };

  f32x16 o[D / 32];
#pragma unroll
  for (int nb = 0; nb < D / 32; ++nb) o[nb] = f32x16{};
  float ref = -INFINITY;  // reference point of o and l, log2 units; -inf until a key is seen
  float l = 0.f;          // this lane's share of the running sum
  const float sl2 = a.scale_log2;
  // Last key my_row may see in the whole problem.
  const int last_key = a.causal ? min(a.seqlen_k - 1, my_row + a.causal_offset) : a.seqlen_k - 1;

  if (num_tiles > 0) fetch(0);
  for (int t = 0; t < num_tiles; ++t) {
    const int slot = t & 1;
    stash(slot);
    __syncthreads();
    if (t + 1 < num_tiles) fetch(t + 1);

    const int k0 = t * kBlockN;
    // Every key of this tile is hidden from every row of this wave (wave-uniform).
    if (a.causal && k0 > row0 + kRowsPerWave - 1 + a.causal_offset) continue;
    const uint16_t* kt = smem + 2 * slot * kTile;
    const uint16_t* vt = kt + kTile;

    f32x16 s0 = f32x16{};
    f32x16 s1 = f32x16{};
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
      const u32x4 a0 = k_frag<D>(kt, 0, ks, lane);
      const u32x4 a1 = k_frag<D>(kt, 1, ks, lane);
      s0 = E::mfma32(a0, qf[ks], s0);
      s1 = E::mfma32(a1, qf[ks], s1);
    }

    const bool need_mask = (k0 + kBlockN > a.seqlen_k) ||
                           (a.causal && k0 + kBlockN - 1 > row0 + a.causal_offset);
    if (need_mask) {
      const int lim = last_key - k0;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int kj = acc_key(j, half);
        if (kj > lim) s0[j] = -INFINITY;
        if (kj + 32 > lim) s1[j] = -INFINITY;
      }
    }

    // Online softmax in the exp2 domain on raw scores: with scale > 0,
    // max(scale * s) = scale * max(s), and p = 2^(s * scale_log2 - ref).
    float mx = max_of(s0, s1);
    mx = fmaxf(mx, xor_lane(mx, 32));
    // The reference point `ref` (log2 units) of o and l only moves when the row max has grown by
    // more than kRescaleSlack over it, so probabilities stay at most 2^kRescaleSlack: no overflow,
    // and a bf16/fp16 P keeps its relative precision. Most tiles then skip the rescale of o.
    const float cand = mx * sl2;  // -inf while the row has seen only hidden keys
    const bool move = cand > ref + kRescaleSlack;
    if (wave_any(move)) {
      const float alpha = move ? exp2_fast(ref - cand) : 1.f;  // ref = -inf gives 0
      ref = move ? cand : ref;
      l *= alpha;
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
    l += rs0 + rs1;

    const u32x4 p0 = p_frag<Tag, 0>(s0);
    const u32x4 p1 = p_frag<Tag, 1>(s0);
    const u32x4 p2 = p_frag<Tag, 0>(s1);
    const u32x4 p3 = p_frag<Tag, 1>(s1);
#pragma unroll
    for (int nb = 0; nb < D / 32; ++nb) {
      o[nb] = E::mfma32(v_frag<D>(vt, nb, 0, lane), p0, o[nb]);
      o[nb] = E::mfma32(v_frag<D>(vt, nb, 1, lane), p1, o[nb]);
      o[nb] = E::mfma32(v_frag<D>(vt, nb, 2, lane), p2, o[nb]);
      o[nb] = E::mfma32(v_frag<D>(vt, nb, 3, lane), p3, o[nb]);
    }
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
    for (int i = lane; i < 16 * k; i += 64) tile[(i / k) * kPitch<D> + i % k] = b[i];
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
    for (int i = lane; i < k * 16; i += 64) tile[(i / 16) * kPitch<D> + i % 16] = b[i];
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
