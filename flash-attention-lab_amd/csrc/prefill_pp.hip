// FlashAttention-2 forward (prefill) for gfx950 with explicit MFMA / softmax ping-pong between the
// two waves that share each SIMD. Same arithmetic and lane layouts as prefill_fwd.hip (see
// prefill_tile.hpp); what differs is how the work is laid out over time.
//
// Serves the attention_mma_pipelined and attention_mma ops of the reference
// (csrc/prefill/mma_pipelined.cu:54-183) at head_dim 128; the algorithm (tiling, online softmax
// with the -inf-safe reference point, bottom-right causal mask, 1/l epilogue) follows the
// reference's definitions (csrc/prefill/mma_tile.cuh:60-174, flash_lab/reference.py:90-152).
//
// Why: within one wave, VALU instructions issued between MFMAs do not overlap with them (on gfx950
// an MFMA followed by 8 independent FMAs takes as long as the two back to back), while an MFMA
// stream in one wave and a VALU stream in another wave of the same SIMD run concurrently at full
// MFMA rate. The softmax (about 150 VALU instructions per 32 x 64 tile, 32 of them exp) therefore
// only hides behind MFMAs if another wave on the same SIMD is in its MFMA phase at that moment.
//
//  * Workgroup: 8 waves x 32 query rows = 256 rows of one (batch, head). Waves w and w + 4 share a
//    SIMD (the dispatcher deals waves to SIMDs with period 4). Group 0 is waves 0-3, group 1 waves
//    4-7: one wave of each group per SIMD.
//  * Time is cut into half-periods by workgroup barriers. In half-period 2m group 0 runs
//    MFMA(m) = P V of tile m-1 then S = K Q^T of tile m (32 MFMAs) while group 1 runs the softmax
//    of tile m-1; in half-period 2m+1 the roles swap. Each MFMA phase is 32 MFMAs (1024 MFMA
//    cycles at D = 128), each softmax phase about 800 cycles of VALU issue, so the MFMA pipe of
//    every SIMD is fed by one wave or the other all the time.
//  * K and V tiles (64 keys) stream through a ring of kStages LDS slots each, filled by direct
//    global -> LDS loads (buffer_load ... lds) that group 1 issues at the start of its softmax
//    phases, 2 kStages - 3 half-periods before the data is needed. Load batch b = {K(b), V(b-1)}.
//    Loads past the last tile use an empty buffer resource (they write zeros into a free slot)
//    so every wave issues the same number of loads and the vmcnt accounting is uniform.
//  * Work order as in prefill_fwd.hip: XCD-contiguous (batch, head) ranges; causal query blocks
//    heaviest first.
#include <type_traits>

#include "launch.hpp"
#include "prefill_tile.hpp"

namespace fl {
namespace prefill {
namespace pp {
namespace {

constexpr int kPpWaves = 8;
constexpr int kPpThreads = 64 * kPpWaves;
constexpr int kPpBlockM = kRowsPerWave * kPpWaves;  // 256 query rows per workgroup
constexpr int kLoadWaves = 4;                       // group 1 issues the tile loads
constexpr int kXcds = 8;
constexpr float kLn2 = 0.693147180559945309f;
constexpr float kRescaleSlack = 8.f;

// LDS ring depth (K and V slots each). A load batch is issued 2 kStages - 2 half-periods before
// the half-period that first reads it, and must land 2 kStages - 3 half-periods after issue.
#ifndef FL_PP_STAGES
#define FL_PP_STAGES 3
#endif
constexpr int kStages = FL_PP_STAGES;
static_assert(kStages == 2 || kStages == 3 || kStages == 4, "2 to 4 ring stages");
// Raise the issue priority of the wave in its MFMA phase.
#ifndef FL_PP_SETPRIO
#define FL_PP_SETPRIO 1
#endif
// MFMAs whose A-operand fragments are in flight ahead of the one issuing.
#ifndef FL_PP_AHEAD
#define FL_PP_AHEAD 4
#endif

// f(integral_constant<int, i>) for i = I .. N - 1, unrolled at compile time.
template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

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

// max(x[l], x[l ^ 32]) on every lane: one v_permlane32_swap (lanes 32-63 of the first result and
// lanes 0-31 of the second are the other half's values).
__device__ __forceinline__ float max_halves(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_halves(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ int xcd_remap(int id, int n) {
  const int per = n / kXcds;
  if (id >= per * kXcds) return id;
  return (id % kXcds) * per + id / kXcds;
}

// Workgroup barrier without a memory fence: LDS reads are complete before it (lgkmcnt(0)); loads
// into LDS are waited for explicitly by the waves that issued them. The sched_barriers keep the
// compiler from moving any instruction across it.
__device__ __forceinline__ void phase_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

template <int kCount>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(kCount >= 0 && kCount <= 63, "vmcnt range");
  if constexpr (kCount == 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  if constexpr (kCount == 8) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
  if constexpr (kCount == 16) asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
}

template <typename Tag, int D>
__global__ void __launch_bounds__(kPpThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
    prefill_pp_kernel(const PrefillArgs a) {
  using E = Elem<Tag>;
  constexpr int kTile = kTileElems<D>;
  // One LDS array: the K ring (kStages slots) then the V ring. ds_read immediates reach 64 KiB, so
  // V reads go through per-lane offsets biased by the K ring's size and every slot offset is an
  // immediate (separate arrays past 64 KiB would each need their own address registers).
  __shared__ __attribute__((aligned(16))) uint16_t smem[2 * kStages * kTile];
  constexpr int kSlotBytes = 2 * kTile;
  constexpr int kVRingBytes = kStages * kSlotBytes;
  static_assert((kStages - 1) * kSlotBytes + kSlotBytes <= 65536, "K ring must fit the immediate range");
  auto k_slot = [&](auto s) -> uint16_t* { return smem + (decltype(s)::value % kStages) * kTile; };
  auto v_slot = [&](auto s) -> uint16_t* {
    return smem + (kStages + decltype(s)::value % kStages) * kTile;
  };
  // Byte offset of V slot s from the biased per-lane V offsets.
  auto v_slot_offset = [&](auto s) constexpr { return (decltype(s)::value % kStages) * kSlotBytes; };
  const char* lds_bytes = reinterpret_cast<const char*>(smem);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int group = wave >> 2;
  const int half = lane >> 5;

  const int work = xcd_remap(blockIdx.x, gridDim.x);
  const int bh = work / a.q_blocks;
  int qb = work - bh * a.q_blocks;
  if (a.causal) qb = a.q_blocks - 1 - qb;
  const int b = bh / a.heads;
  const int h = bh - b * a.heads;
  const int hkv = h / a.group;
  const int q0 = qb * kPpBlockM;
  const int row0 = q0 + wave * kRowsPerWave;
  const int my_row = row0 + (lane & 31);

  const uint16_t* qp = a.q + b * a.q_bs + h * a.q_hs;
  const uint16_t* kp = a.k + b * a.k_bs + hkv * a.k_hs;
  const uint16_t* vp = a.v + b * a.v_bs + hkv * a.v_hs;

  int kv_end = a.seqlen_k;
  if (a.causal) kv_end = min(kv_end, min(q0 + kPpBlockM, a.seqlen_q) + a.causal_offset);
  const int num_tiles = kv_end > 0 ? (kv_end + kBlockN - 1) / kBlockN : 0;
  // Tiles this wave sees any key of (a prefix of the workgroup's tiles).
  int my_tiles = num_tiles;
  if (a.causal) {
    const int last = row0 + kRowsPerWave - 1 + a.causal_offset;  // last key any of its rows sees
    my_tiles = last < 0 ? 0 : min(num_tiles, last / kBlockN + 1);
  }

  u32x4 qf[D / 16];
  {
    const bool ok = my_row < a.seqlen_q;
    const uint16_t* src = qp + static_cast<int64_t>(ok ? my_row : 0) * a.q_ss + 8 * half;
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) qf[ks] = ok ? load16(src + 16 * ks) : u32x4{0, 0, 0, 0};
    // Consume the Q registers here so the compiler's wait for them sits before the tile loads
    // (it does not see those, and would otherwise wait for all of them at the first use of Q).
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) asm volatile("" : "+v"(qf[ks]));
  }

  int k_lds[D / 16];
#pragma unroll
  for (int ks = 0; ks < D / 16; ++ks) k_lds[ks] = k_lane_offset<D>(ks, lane);
  int v_lds[D / 32][2];
  int v_bias = kVRingBytes;
  asm volatile("" : "+v"(v_bias));  // keep the bias in the registers, not in the immediates
#pragma unroll
  for (int nb = 0; nb < D / 32; ++nb) {
    v_lds[nb][0] = v_lane_offset<D>(nb, 0, lane) + v_bias;
    v_lds[nb][1] = v_lane_offset<D>(nb, 1, lane) + v_bias;
  }

  // Tile loads (group 1 only): each load wave moves kDmaPerWave 1 KiB blocks of a tile.
  constexpr int kChunksPerRow = D / 8;
  constexpr int kRowsPerBlock = 64 / kChunksPerRow;
  constexpr int kDmaPerWave = kBlockN / kRowsPerBlock / kLoadWaves;
  const int lw = wave & 3;
  int k_off[kDmaPerWave];
  int v_off[kDmaPerWave];
#pragma unroll
  for (int j = 0; j < kDmaPerWave; ++j) {
    const int row = (lw * kDmaPerWave + j) * kRowsPerBlock + lane / kChunksPerRow;
    const int chunk = (lane % kChunksPerRow) ^ swz<D>(row);
    k_off[j] = static_cast<int>((row * a.k_ss + 8 * chunk) * 2);
    v_off[j] = static_cast<int>((row * a.v_ss + 8 * chunk) * 2);
  }
  // Loads of one tensor's tile `tile` into `slot`; tiles outside [0, num_tiles) use an empty
  // resource and write zeros.
  // Loads of one tensor's tile `tile` into `slot` (inline assembly: ordered only by the explicit
  // waits and barriers of the schedule below); tiles outside [0, num_tiles) use an empty resource
  // and write zeros.
  auto dma = [&](uint16_t* slot, const uint16_t* base, int64_t seq_stride, const int (&off)[kDmaPerWave],
                 int tile) {
    const int k0 = tile * kBlockN;
    const int rows = (tile >= 0 && tile < num_tiles) ? min(kBlockN, a.seqlen_k - k0) : 0;
    const uint16_t* tile_base = rows > 0 ? base + k0 * seq_stride : base;
    const uint32_t bytes = rows > 0 ? static_cast<uint32_t>(((rows - 1) * seq_stride + D) * 2) : 0u;
    const u32x4s words = buffer_words(tile_base, bytes);
    const uint32_t lds0 = lds_address(slot) + lw * kDmaPerWave * 1024;
#pragma unroll
    for (int j = 0; j < kDmaPerWave; ++j) buffer_load16_to_lds_asm(words, lds0 + j * 1024, off[j]);
  };
  // Load batch bt = {K(bt), V(bt - 1)} into their ring slots.
  auto load_batch = [&](int bt, auto kslot_tag, auto vslot_tag) {
    dma(k_slot(kslot_tag), kp, a.k_ss, k_off, bt);
    dma(v_slot(vslot_tag), vp, a.v_ss, v_off, bt - 1);
  };

  f32x16 o[D / 32];
#pragma unroll
  for (int nb = 0; nb < D / 32; ++nb) o[nb] = f32x16{};
  f32x16 s0 = f32x16{};
  f32x16 s1 = f32x16{};
  u32x4 pf[4] = {};
  float ref = -INFINITY;
  float l = 0.f;
  const float sl2 = a.scale_log2;
  const int last_key = a.causal ? min(a.seqlen_k - 1, my_row + a.causal_offset) : a.seqlen_k - 1;

  // MFMA phase of period m: O += V(m-1) P(m-1), then S = K(m) Q^T.
  // MFMA phase of a period with slots kS = m % kStages: O += V(m-1) P(m-1) (16 MFMAs), then
  // S = K(m) Q^T (16 MFMAs). No branches: in period 0 the previous P and V are zeros (P starts at
  // 0, the V slot was filled from an empty resource), a skipped softmax leaves P = 0, and scores of
  // tiles nobody reads are never used. The 32 MFMAs form one software pipeline: the A-operand
  // fragment of MFMA i + kAhead is read from LDS right after MFMA i issues, and a scheduling
  // barrier after every step keeps that order (left to itself the scheduler reads each fragment
  // just before its MFMA and the LDS latency shows on every step).
  auto mfma_phase = [&](auto slot_tag) {
    constexpr int kS = decltype(slot_tag)::value;
    constexpr int kPv = 4 * (D / 32);  // P V MFMAs: key step kk = i / (D / 32), dim block nb
    constexpr int kQk = 2 * (D / 16);  // K Q^T MFMAs: dim step ks = j / 2, key block j % 2
    constexpr int kSteps = kPv + kQk;
    constexpr int kAhead = FL_PP_AHEAD;
    const char* vt = lds_bytes + v_slot_offset(std::integral_constant<int, kS + kStages - 1>{});
    const char* kt = reinterpret_cast<const char*>(k_slot(std::integral_constant<int, kS>{}));
    auto read_frag = [&](auto i_tag) -> u32x4 {
      constexpr int i = decltype(i_tag)::value;
      if constexpr (i < kPv) {
        constexpr int kk = i / (D / 32), nb = i % (D / 32);
        return v_frag_at(vt + kk * kKeyStepBytes<D>, v_lds[nb][0], v_lds[nb][1]);
      } else {
        constexpr int j = i - kPv, ks = j / 2, blk = j % 2;
        return lds_load16(kt + blk * kKeyBlockBytes<D>, k_lds[ks]);
      }
    };
    auto issue = [&](auto i_tag, const u32x4& f) {
      constexpr int i = decltype(i_tag)::value;
      if constexpr (i < kPv) {
        constexpr int kk = i / (D / 32), nb = i % (D / 32);
        o[nb] = E::mfma32(f, pf[kk], o[nb]);
      } else {
        constexpr int j = i - kPv, ks = j / 2, blk = j % 2;
        f32x16& acc = blk == 0 ? s0 : s1;
        acc = E::mfma32(f, qf[ks], ks == 0 ? f32x16{} : acc);
      }
    };
#if FL_PP_SETPRIO
    __builtin_amdgcn_s_setprio(1);
#endif
    u32x4 fr[kSteps];
    static_for<0, kAhead>([&](auto i) { fr[decltype(i)::value] = read_frag(i); });
    __builtin_amdgcn_sched_barrier(0);
    static_for<0, kSteps>([&](auto i) {
      constexpr int n = decltype(i)::value;
      issue(i, fr[n]);
      if constexpr (n + kAhead < kSteps) fr[n + kAhead] = read_frag(std::integral_constant<int, n + kAhead>{});
      __builtin_amdgcn_sched_barrier(0);
    });
#if FL_PP_SETPRIO
    __builtin_amdgcn_s_setprio(0);
#endif
  };

  // Softmax phase for tile t: S(t) -> P(t) (input type, packed as the next P V's B operand), the
  // lazily moved reference point, the O rescale and the running sum.
  auto softmax_phase = [&](int t) {
    if (t < 0 || t >= my_tiles) {
      // This wave sees no key of tile t: the P V that follows must add nothing.
#pragma unroll
      for (int i = 0; i < 4; ++i) pf[i] = u32x4{0, 0, 0, 0};
      return;
    }
    const int k0 = t * kBlockN;
    if ((k0 + kBlockN > a.seqlen_k) || (a.causal && k0 + kBlockN - 1 > row0 + a.causal_offset)) {
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
    const float mx = max_halves(max_of(s0, s1));
    const float cand = mx * sl2;
    const bool move = cand > ref + kRescaleSlack;
    const float alpha = move ? exp2_fast(ref - cand) : 1.f;
    ref = move ? cand : ref;
    if (wave_any(move)) {
      asm volatile("" ::: "memory");
#pragma unroll
      for (int nb = 0; nb < D / 32; ++nb) o[nb] *= alpha;
    }
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
    pf[0] = p_frag<Tag, 0>(s0);
    pf[1] = p_frag<Tag, 1>(s0);
    pf[2] = p_frag<Tag, 0>(s1);
    pf[3] = p_frag<Tag, 1>(s1);
  };

  // Vmcnt allowed before the barrier that publishes a batch: the kStages - 2 batches issued after it.
  constexpr int kLoadsPerBatch = 2 * kDmaPerWave;
  constexpr int kPendingAfter = (kStages - 2) * kLoadsPerBatch;

  // Prologue: group 1 loads batches 0 .. kStages - 2; batch 0 (K(0)) must be in LDS before the
  // first half-period.
  if (group == 1) {
    load_batch(0, std::integral_constant<int, 0>{}, std::integral_constant<int, kStages - 1>{});
    if constexpr (kStages > 2) load_batch(1, std::integral_constant<int, 1>{}, std::integral_constant<int, 0>{});
    if constexpr (kStages > 3) load_batch(2, std::integral_constant<int, 2>{}, std::integral_constant<int, 1>{});
    // Loads issued after batch 0: batches 1 .. kStages - 2.
    wait_vmcnt<(kStages - 2) * kLoadsPerBatch>();
  }
  phase_barrier();

  // Period m: half-period 2m then 2m + 1. Group 0: MFMA(m), softmax(m). Group 1: softmax(m - 1)
  // after issuing batch m + kStages - 1, then MFMA(m). Group 1 waits for batch m + 1 before the
  // barrier that ends half-period 2m (batch m + 1 is first read in half-period 2m + 2). Each group
  // runs its own straight-line loop, unrolled by kStages so that ring slots are compile-time
  // immediates; the periods % kStages left over run after it.
  const int periods = num_tiles + 1;  // the last one only finishes P V of the last tile
  auto run = [&](auto group_tag) {
    constexpr int kGroup = decltype(group_tag)::value;
    auto period = [&](int m, auto slot_tag) {
      constexpr int kS = decltype(slot_tag)::value;
      if constexpr (kGroup == 0) {
        mfma_phase(slot_tag);
        phase_barrier();
        softmax_phase(m);
        phase_barrier();
      } else {
        // Batch m + kStages - 1: K into slot (m - 1) % kStages, V into slot (m - 2) % kStages.
        load_batch(m + kStages - 1, std::integral_constant<int, kS + kStages - 1>{},
                   std::integral_constant<int, kS + kStages - 2>{});
        softmax_phase(m - 1);
        wait_vmcnt<kPendingAfter>();
        phase_barrier();
        mfma_phase(slot_tag);
        phase_barrier();
      }
    };
    int m = 0;
    for (; m + kStages <= periods; m += kStages) {
      period(m, std::integral_constant<int, 0>{});
      period(m + 1, std::integral_constant<int, 1>{});
      if constexpr (kStages > 2) period(m + 2, std::integral_constant<int, 2>{});
      if constexpr (kStages > 3) period(m + 3, std::integral_constant<int, 3>{});
    }
    const int rest = periods - m;
    if (rest > 0) period(m, std::integral_constant<int, 0>{});
    if (rest > 1) period(m + 1, std::integral_constant<int, 1>{});
    if constexpr (kStages > 3) {
      if (rest > 2) period(m + 2, std::integral_constant<int, 2>{});
    }
  };
  if (group == 0) {
    run(std::integral_constant<int, 0>{});
  } else {
    run(std::integral_constant<int, 1>{});
  }
  // Loads past the end may still be in flight into free slots; they must land before the
  // workgroup's LDS is handed to another workgroup.
  if (group == 1) wait_vmcnt<0>();

  const float lt = sum_halves(l);
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
      a.lse[(static_cast<int64_t>(b) * a.heads + h) * a.seqlen_q + my_row] =
          lt > 0.f ? ref * kLn2 + logf(lt) : -INFINITY;
    }
  }
}

template <typename Tag, int D>
hipError_t launch_typed(PrefillArgs args, hipStream_t stream) {
  args.q_blocks = (args.seqlen_q + kPpBlockM - 1) / kPpBlockM;
  const int blocks = args.q_blocks * args.batch * args.heads;
  hipLaunchKernelGGL((prefill_pp_kernel<Tag, D>), dim3(blocks), dim3(kPpThreads), 0, stream, args);
  return hipGetLastError();
}

}  // namespace
}  // namespace pp
}  // namespace prefill

hipError_t launch_prefill_pingpong(const PrefillArgs& args, DType dtype, int head_dim,
                                   hipStream_t stream) {
  using namespace prefill::pp;
  if (head_dim != 128) return hipErrorInvalidValue;
  return dtype == DType::bf16 ? launch_typed<bf16_tag, 128>(args, stream)
                              : launch_typed<f16_tag, 128>(args, stream);
}

}  // namespace fl
