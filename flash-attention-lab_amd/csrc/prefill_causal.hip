// Causal FlashAttention-2 forward (prefill) for gfx950: the ping-pong kernel of prefill_pp.hip with
// a causal pair of query blocks run as ONE stream of key tiles instead of two blocks.
//
// Serves the causal calls of the attention_mma_pipelined and attention_mma ops of the reference
// (csrc/prefill/mma_pipelined.cu:54-183) at head_dim 128 and 64; the arithmetic (tiling, online
// softmax with the -inf-safe reference point, bottom-right causal mask, 1/l epilogue) is the same
// as prefill_pp.hip's and follows the reference's definitions (csrc/prefill/mma_tile.cuh:60-174,
// flash_lab/reference.py:90-152).
//
// A workgroup takes the light block L and the heavy block H = q_blocks - 1 - L of one (batch,
// head), 256 query rows each. Its 8 waves (32 rows each) run one period per key tile with one
// workgroup barrier per period, as in prefill_pp.hip, but over a single stream of tiles: the light
// block's tiles in ascending order (0 .. nL - 1), then the heavy block's in DESCENDING order
// (nH - 1 .. 0). Wave w owns light rows 32 w .. 32 w + 31 of L and heavy rows 32 (7 - w) .. of H,
// so the waves whose light rows end early on L's diagonal are the ones whose heavy rows see H's
// diagonal tiles, which the heavy part starts with. Per wave the work is one light part, a few
// idle periods around the switch, then one heavy part:
//  * light part: periods 0 .. tiles(light rows) - 1, then the P V of its last tile, the light
//    rows' output and LSE (written straight from the accumulators, see store_rows) and a reset of
//    the softmax state;
//  * idle periods (tiles of the stream its rows do not see): only the wave's share of the tile
//    loads. Here it also finishes loading its heavy query rows (issued right after its last light
//    K Q^T, when the Q registers are free);
//  * heavy part: the last tiles(heavy rows) periods of the stream, then the final P V and output.
// At (4, 32, 32, 4096, 128) every wave has exactly 65 tiles in a stream of 68 (3 idle periods
// each, around the switch), one prologue and one drain per workgroup, against 68 tiles in 70
// periods with two prologues and drains when the pair runs as two blocks (prefill_pp.hip), where
// on each block's diagonal a wave's SIMD partner often has nothing to do.
//
// Every wave of a group issues the same tile loads in every period (a load outside the stream
// reads an empty buffer resource and writes zeros into a free slot), so the vmcnt accounting stays
// uniform; the compiler-visible memory instructions that a wave adds around its switch (the heavy
// query rows, the light output stores) are counted into the period-end waits they precede.
#include <type_traits>

#include "prefill_pp.hpp"

namespace fl {
namespace prefill {
namespace pp {
namespace {

template <typename Tag, int D>
__global__ void __launch_bounds__(kPpThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
    prefill_causal_kernel(const PrefillArgs a) {
  using E = Elem<Tag>;
  constexpr int kTile = kTileElems<D>;
  __shared__ __attribute__((aligned(16))) uint16_t smem[2 * kStages * kTile];
  constexpr int kSlotBytes = 2 * kTile;
  constexpr int kVRingBytes = kStages * kSlotBytes;
  const char* lds_bytes = reinterpret_cast<const char*>(smem);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // The lane index as a value the compiler cannot see through: address arithmetic that is only
  // needed around the switch (query rows, output rows) then stays where it is used instead of
  // being hoisted to the kernel's start and kept live through every period.
  auto opaque_lane = [&]() {
    int l = lane;
    asm volatile("" : "+v"(l));
    return l;
  };
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int group = wave >> 2;
  const int half = lane >> 5;

  // Work item: (batch, head) and the pair (light block lb, heavy block hb); the middle block of an
  // odd block count runs alone (no heavy part).
  const int work = xcd_remap(blockIdx.x, gridDim.x);
  const int items_per_bh = (a.q_blocks + 1) / 2;
  const int bh = work / items_per_bh;
  const int lb = work - bh * items_per_bh;
  const int hb = a.q_blocks - 1 - lb;
  const bool two = lb < hb;
  const int b = bh / a.heads;
  const int h = bh - b * a.heads;
  const int hkv = h / a.group;
  const uint16_t* qp = a.q + b * a.q_bs + h * a.q_hs;
  const uint16_t* kp = a.k + b * a.k_bs + hkv * a.k_hs;
  const uint16_t* vp = a.v + b * a.v_bs + hkv * a.v_hs;

  // Key tiles of a block: every key some row of it sees (bottom-right aligned).
  auto block_tiles = [&](int qb) {
    const int kv_end = min(a.seqlen_k, min((qb + 1) * kPpBlockM, a.seqlen_q) + a.causal_offset);
    return kv_end > 0 ? (kv_end + kBlockN - 1) / kBlockN : 0;
  };
  const int n_light = block_tiles(lb);
  const int n_heavy = two ? block_tiles(hb) : 0;
  const int stream = n_light + n_heavy;  // periods 0 .. stream - 1 multiply a tile's K; stream is P V only

  // A wave's rows in a block: the first of its 32 rows, how many of the block's tiles they see (a
  // prefix of the tile range; 0 for rows at or past S_q), and the first tile whose scores need
  // masking (it reaches past the sequence end or past the diagonal of the wave's first row).
  struct Rows {
    int row0;
    int tiles;
    int mask_from;
  };
  auto rows_of = [&](int qb, int chunk, int n_tiles) {
    Rows r;
    r.row0 = qb * kPpBlockM + chunk * kRowsPerWave;
    const int last = r.row0 + kRowsPerWave - 1 + a.causal_offset;  // last key any of its rows sees
    r.tiles = r.row0 >= a.seqlen_q || last < 0 ? 0 : min(n_tiles, last / kBlockN + 1);
    const int x = r.row0 + a.causal_offset - (kBlockN - 1);  // tile t needs masking iff 64 t > x
    r.mask_from = min(a.seqlen_k / kBlockN, x < 0 ? 0 : x / kBlockN + 1);
    return r;
  };
  const Rows light = rows_of(lb, wave, n_light);
  const Rows heavy = two ? rows_of(hb, kPpWaves - 1 - wave, n_heavy) : Rows{0, 0, 0};
  // The wave's heavy part is the last heavy.tiles periods of the stream: tile stream - 1 - p.
  const int heavy_start = stream - heavy.tiles;
  // Its heavy query rows replace the light ones in the Q registers: loaded after the MFMA phase of
  // its last light K Q^T (period q_issue), consumed at the start of period q_consume, the last idle
  // period before its first heavy K Q^T when there is one (a wait there costs nothing on the
  // critical path). Without light tiles the heavy rows are loaded in the prologue instead.
  const bool q_switch = two && heavy.tiles > 0 && light.tiles > 0;
  const int q_issue = q_switch ? light.tiles - 1 : -1;
  const int q_consume = q_switch ? max(light.tiles, heavy_start - 1) : -1;
  // The light rows' output is written after the P V of their last tile (period light.tiles).
  const int light_done = light.tiles;

  // Per-lane LDS byte offsets of the fragments within a ring slot; a period adds its slots' bases
  // (wave-uniform) at each read, so the offsets stay loop-invariant.
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

  // Tile loads (as in prefill_pp.hip): group 0 streams K, group 1 V; wave lw of a group moves
  // kDmaPerWave 1 KiB blocks of each tile into its part of the ring slot.
  constexpr int kChunksPerRow = D / 8;
  constexpr int kRowsPerBlock = 64 / kChunksPerRow;
  constexpr int kDmaPerWave = kBlockN / kRowsPerBlock / kLoadWaves;
  const int lw = wave & 3;
  const uint32_t lds_wave = __builtin_amdgcn_readfirstlane(
      lds_address(smem) + (group == 0 ? 0 : kVRingBytes) + lw * kDmaPerWave * 1024);
  const uint16_t* my_base = group == 0 ? kp : vp;
  const int64_t my_ss = group == 0 ? a.k_ss : a.v_ss;
  int my_off[kDmaPerWave];
#pragma unroll
  for (int j = 0; j < kDmaPerWave; ++j) {
    const int row = (lw * kDmaPerWave + j) * kRowsPerBlock + lane / kChunksPerRow;
    const int chunk = (lane % kChunksPerRow) ^ swz<D>(row);
    my_off[j] = static_cast<int>((row * my_ss + 8 * chunk) * 2);
  }
  const int64_t tile_bytes = static_cast<int64_t>(kBlockN) * my_ss * 2;
  const uint32_t full_bytes = static_cast<uint32_t>(((kBlockN - 1) * my_ss + D) * 2);
  // The last tile of a block's range may stop at the sequence end.
  auto last_bytes_of = [&](int n_tiles) {
    const int rows = n_tiles > 0 ? min(kBlockN, a.seqlen_k - (n_tiles - 1) * kBlockN) : 1;
    return static_cast<uint32_t>(((rows - 1) * my_ss + D) * 2);
  };
  const uint32_t light_last_bytes = last_bytes_of(n_light);
  const uint32_t heavy_last_bytes = last_bytes_of(n_heavy);
  // Buffer resource of the tile the stream multiplies in period q: light tile q, heavy tile
  // stream - 1 - q, or an empty resource outside the stream.
  auto tile_words = [&](int q) -> u32x4s {
    const bool in_light = q < n_light;
    const int t = in_light ? q : stream - 1 - q;
    const bool inside = q >= 0 && q < stream;
    const uint32_t last = in_light ? light_last_bytes : heavy_last_bytes;
    const int n_tiles = in_light ? n_light : n_heavy;
    const uint32_t bytes = !inside ? 0u : t == n_tiles - 1 ? last : full_bytes;
    const char* p = reinterpret_cast<const char*>(my_base) + (inside ? t * tile_bytes : 0);
    return buffer_words(p, bytes);
  };
  auto issue_block = [&](u32x4s w, int slot, auto j_tag) {
    constexpr int j = decltype(j_tag)::value;
    const uint32_t off = (static_cast<unsigned>(slot) % kStages) * kSlotBytes + j * 1024;
    buffer_load16_to_lds_asm(w, lds_wave + off, my_off[j]);
  };

  // The wave's query rows (lane (r, half) holds row row0 + r, dims 16 ks + 8 half .. + 7; zeros
  // past the sequence), the B operand of K Q^T.
  u32x4 qf[D / 16];
  auto load_q = [&](int row0) {
    const int r = row0 + (opaque_lane() & 31);
    const bool ok = r < a.seqlen_q;
    const uint16_t* src = qp + static_cast<int64_t>(ok ? r : 0) * a.q_ss + 8 * half;
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) qf[ks] = ok ? load16(src + 16 * ks) : u32x4{0, 0, 0, 0};
  };
  // Uses the Q registers, so that the compiler's wait for their loads sits here.
  auto consume_q = [&]() {
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) asm volatile("" : "+v"(qf[ks]));
  };

  // Softmax state of the rows the wave is on (light, then heavy).
  f32x16 o[D / 32];
#pragma unroll
  for (int nb = 0; nb < D / 32; ++nb) o[nb] = f32x16{};
  f32x16 s0 = f32x16{};
  f32x16 s1 = f32x16{};
  u32x4 pf[4] = {};
  float ref = kNoRef;
  float l = 0.f;
  const float sl2 = a.scale_log2;
  int cur_row0 = light.row0;
  int cur_mask_from = light.mask_from;
  // Last key of the lane's row, clamped to the sequence (rows past S_q keep a harmless value).
  auto last_key_of = [&](int row0) {
    return min(a.seqlen_k - 1, row0 + (opaque_lane() & 31) + a.causal_offset);
  };
  int last_key = last_key_of(light.row0);

  // Writes the wave's 32 output rows (normalized, rounded to the input type) and their LSE, then
  // resets the softmax state. Straight from the accumulators: lane l holds dims 32 nb + 8 g +
  // 4 half .. + 3 of row l % 32 (g = 0..3), i.e. half of each 16-byte piece; one permlane32 swap
  // per dword gives lanes 0-31 the whole even pieces and lanes 32-63 the odd ones, so every store
  // moves 16 bytes and each instruction writes 32 contiguous bytes of each of 32 rows.
  auto store_rows = [&](int row0) {
    const float lt = sum_halves(l);
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    const int lane_now = opaque_lane();
    const int r = row0 + (lane_now & 31);
    const bool ok = r < a.seqlen_q;
    uint16_t* orow = a.o + b * a.o_bs + h * a.o_hs + static_cast<int64_t>(ok ? r : 0) * a.o_ss + 8 * (lane_now >> 5);
#pragma unroll
    for (int nb = 0; nb < D / 32; ++nb) {
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        const uint32_t ax = E::pack2(o[nb][8 * m] * inv, o[nb][8 * m + 1] * inv);
        const uint32_t ay = E::pack2(o[nb][8 * m + 2] * inv, o[nb][8 * m + 3] * inv);
        const uint32_t bx = E::pack2(o[nb][8 * m + 4] * inv, o[nb][8 * m + 5] * inv);
        const uint32_t by = E::pack2(o[nb][8 * m + 6] * inv, o[nb][8 * m + 7] * inv);
        const auto rx = __builtin_amdgcn_permlane32_swap(ax, bx, false, false);
        const auto ry = __builtin_amdgcn_permlane32_swap(ay, by, false, false);
        const u32x4 piece{rx[0], ry[0], rx[1], ry[1]};
        if (ok) *reinterpret_cast<u32x4*>(orow + 32 * nb + 16 * m) = piece;
      }
    }
    if (ok && lane_now < 32) {
      a.lse[(static_cast<int64_t>(b) * a.heads + h) * a.seqlen_q + r] =
          lt > 0.f ? ref * kLn2 + logf(lt) : -INFINITY;
    }
#pragma unroll
    for (int nb = 0; nb < D / 32; ++nb) o[nb] = f32x16{};
    ref = kNoRef;
    l = 0.f;
  };
  // Memory instructions store_rows issues (2 D / 32 output pieces and one LSE word per lane). Its
  // rows inside the stream are always light rows of a full block (the light block of a pair is
  // never the last one), so every one of them is issued, each counted by vmcnt.
  constexpr int kStores = 2 * (D / 32) + 1;

  // MFMA phase of a period with slots kS = m % kStages, as in prefill_pp.hip: O += V(m-1) P(m-1),
  // then S = K(m) Q^T, one software pipeline with kAhead fragment reads in flight, hook(i) after
  // MFMA i.
  constexpr int kPv = 4 * (D / 32);
  constexpr int kQk = 2 * (D / 16);
  constexpr int kSteps = kPv + kQk;
  constexpr int kAhead = FL_PP_AHEAD;
  static_assert(kAhead >= 1 && kAhead <= kPv, "prefetched fragments are V fragments");
  static_assert(8 * (kDmaPerWave - 1) + 1 < kSteps, "one tile load every 8 MFMAs");
  // Fragment of MFMA i of period p's phase: V(p - 1) in V slot (p - 1) % kStages, K(p) in K slot
  // p % kStages. `slot` is p % kStages, a wave-uniform value.
  auto read_frag = [&](int slot, auto i_tag) -> u32x4 {
    constexpr int i = decltype(i_tag)::value;
    if constexpr (i < kPv) {
      constexpr int kk = i / (D / 32), nb = i % (D / 32);
      const int vs = (slot + kStages - 1) % kStages;
      return v_frag_at(lds_bytes + vs * kSlotBytes + kk * kKeyStepBytes<D>, v_lds[nb][0], v_lds[nb][1]);
    } else {
      constexpr int j = i - kPv, ks = j / 2, blk = j % 2;
      return lds_load16(lds_bytes + slot * kSlotBytes + blk * kKeyBlockBytes<D>, k_lds[ks]);
    }
  };
  u32x4 pre[kAhead];
  auto prefetch = [&](int slot) {
    static_for<0, kAhead>([&](auto i) { pre[decltype(i)::value] = read_frag(slot, i); });
  };
  auto prefetch_qk = [&](int slot) {
    static_for<0, kAhead>([&](auto i) {
      pre[decltype(i)::value] = read_frag(slot, std::integral_constant<int, kPv + decltype(i)::value>{});
    });
  };
  auto mfma_phase = [&](int slot, auto pv_tag, auto qk_tag, auto&& hook) {
    constexpr bool kDoPv = decltype(pv_tag)::value;
    constexpr bool kDoQk = decltype(qk_tag)::value;
    constexpr int kFirstStep = kDoPv ? 0 : kPv;
    u32x4 fr[kSteps];
    static_for<0, kAhead>([&](auto i) { fr[kFirstStep + decltype(i)::value] = pre[decltype(i)::value]; });
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
#if FL_PP_SETPRIO == 1
    __builtin_amdgcn_s_setprio(1);
#endif
    __builtin_amdgcn_sched_barrier(0);
    static_for<0, kSteps>([&](auto i) {
      constexpr int n = decltype(i)::value;
      constexpr bool kLive = n < kPv ? kDoPv : kDoQk;
      if constexpr (kLive) issue(i, fr[n]);
      if constexpr (n + kAhead < kSteps && (n + kAhead < kPv ? kDoPv : (kDoQk && (kDoPv || n >= kPv)))) {
        fr[n + kAhead] = read_frag(slot, std::integral_constant<int, n + kAhead>{});
      }
      hook(i);
      __builtin_amdgcn_sched_barrier(0);
    });
#if FL_PP_SETPRIO == 1
    __builtin_amdgcn_s_setprio(0);
#endif
  };
  auto loads_only = [&](auto&& hook) {
    static_for<0, kSteps>([&](auto i) { hook(i); });
  };

  // P(t) from S(t) against the reference point, packed as the P V operand; returns the lane's sum
  // of the unrounded probabilities.
  auto probabilities = [&](float neg_shift) -> float {
    f32x16 p0, p1;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      p0[j] = exp2_fast(fmaf(s0[j], sl2, neg_shift));
      p1[j] = exp2_fast(fmaf(s1[j], sl2, neg_shift));
    }
    float r0 = p0[0];  // (not 0 + p: the compiler keeps that add, for -0)
    float r1 = p1[0];
#pragma unroll
    for (int j = 1; j < 16; ++j) {
      r0 += p0[j];
      r1 += p1[j];
    }
    pf[0] = p_frag<Tag, 0>(p0);
    pf[1] = p_frag<Tag, 1>(p0);
    pf[2] = p_frag<Tag, 0>(p1);
    pf[3] = p_frag<Tag, 1>(p1);
    return r0 + r1;
  };
  // Softmax of key tile t for the rows the wave is on, with the reference point of prefill_pp.hip
  // (moved to the running max when a tile's max passes it by more than kMoveSlack).
  auto softmax_phase = [&](int t) {
#if FL_PP_SETPRIO == 2
    __builtin_amdgcn_s_setprio(1);
#endif
    if (t >= cur_mask_from) {
      asm volatile("" ::: "memory");
      const int lim = last_key - t * kBlockN - 4 * half;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int kj = acc_key(j, 0);
        s0[j] = kj > lim ? -INFINITY : s0[j];
        s1[j] = kj + 32 > lim ? -INFINITY : s1[j];
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    const float mx = max_halves(max_of(s0, s1)) * sl2;
    if (wave_any(mx > ref + kMoveSlack)) {
      asm volatile("" ::: "memory");
      const float moved = max2_f32(ref, mx);
      const float alpha = exp2_fast(ref - moved);
      ref = moved;
#pragma unroll
      for (int nb = 0; nb < D / 32; ++nb) o[nb] *= alpha;
      l *= alpha;
    }
    l += probabilities(-ref);
#if FL_PP_SETPRIO == 2
    __builtin_amdgcn_s_setprio(0);
#endif
  };

  // Ends the live range of values a period has consumed. A period's MFMA phase and softmax are
  // chosen at run time, and the compiler cannot tell that a period without K Q^T is never followed
  // by a softmax that reads its scores (or a P V that reads its probabilities), so without this
  // it keeps them live through every period and spills.
  auto dead = [&](auto& x) { x = __builtin_nondeterministic_value(x); };
  auto scores_dead = [&]() {
    dead(s0);
    dead(s1);
  };
  auto operands_dead = [&]() {
#pragma unroll
    for (int i = 0; i < 4; ++i) dead(pf[i]);
#pragma unroll
    for (int i = 0; i < kAhead; ++i) dead(pre[i]);
  };

  // Key tile of the stream in period p.
  auto tile_at = [&](int p) { return p < n_light ? p : stream - 1 - p; };
  // Light rows done: write them, and from now on the softmax state and masks are the heavy rows'.
  auto switch_to_heavy = [&]() {
    store_rows(light.row0);
    cur_row0 = heavy.row0;
    cur_mask_from = heavy.mask_from;
    last_key = last_key_of(heavy.row0);
  };

  // Period-end waits: group 0 waits for K(p + 1) with the kStages - 2 later K tiles in flight,
  // group 1 for V(p + 1) with kStages - 3 later V tiles. vmcnt retires a wave's vector-memory
  // instructions in issue order, so the exact count to wait for is the number issued after the
  // tile waited for: its later tiles' blocks, plus the heavy query rows (D / 16 loads after the
  // MFMA phase of period q_issue) and the light rows' output (kStores stores after the MFMA phase
  // of period store_period; the prologue counts as period -1) when those were issued in or after
  // the period that issued the tile. The tile waited for was issued in the MFMA phase of period
  // p - (kStages - 2) (group 0) or p - (kStages - 3) (group 1).
  constexpr int kPendingK = (kStages - 2) * kDmaPerWave;
  constexpr int kPendingV = (kStages - 3) * kDmaPerWave;
  const int store_period = light.tiles > 0 ? light.tiles : -1;
  auto period_end_wait = [&](int p, auto group_tag) {
    constexpr int kGroup = decltype(group_tag)::value;
    constexpr int kPending = kGroup == 0 ? kPendingK : kPendingV;
    const int issued = p - (kGroup == 0 ? kStages - 2 : kStages - 3);
    auto younger = [&](int e) { return e >= issued && e <= p; };
    const bool q_young = q_switch && younger(q_issue);
    const bool st_young = two && younger(store_period);
    if (q_young && st_young) {
      wait_vmcnt<kPending + D / 16 + kStores>();
    } else if (q_young) {
      wait_vmcnt<kPending + D / 16>();
    } else if (st_young) {
      wait_vmcnt<kPending + kStores>();
    } else {
      wait_vmcnt<kPending>();
    }
  };

  // Prologue: the query rows the wave starts with, then group 0 loads K(0 .. kStages - 2), group 1
  // V(-1 .. kStages - 3) (V(-1) stands for the P V that period 0 does not run).
  load_q(light.tiles > 0 || !two ? light.row0 : heavy.row0);
  consume_q();
  static_for<0, kStages - 1>([&](auto i_tag) {
    constexpr int i = decltype(i_tag)::value;
    if (group == 0) {
      const u32x4s w = tile_words(i);
      static_for<0, kDmaPerWave>([&](auto j) { issue_block(w, i, j); });
    } else {
      const u32x4s w = tile_words(i - 1);
      static_for<0, kDmaPerWave>([&](auto j) { issue_block(w, i + kStages - 1, j); });
    }
  });
  if (group == 0) {
    wait_vmcnt<(kStages - 2) * kDmaPerWave>();
  } else {
    wait_vmcnt<(kStages - 3) * kDmaPerWave>();
  }
  phase_barrier();
  // A wave with no light tiles starts on its heavy rows (their query rows were loaded above).
  if (!(light.tiles > 0 || !two)) switch_to_heavy();

  // Periods 0 .. stream, one barrier each. Group 0: MFMA(p), then the softmax of tile p. Group 1:
  // the softmax of tile p - 1, then MFMA(p). Group 0 loads K(p + kStages - 1) and group 1
  // V(p + kStages - 2) between the MFMAs of their phases. A wave's periods come in segments, each
  // with its own MFMA phase and events fixed at compile time (so every segment is straight-line
  // code):
  //  * light: K Q^T only (period 0), then full periods; after the last light K Q^T the heavy query
  //    rows are loaded;
  //  * switch: the P V of the last light tile and the light rows' output, idle periods (loads
  //    only), the first heavy K Q^T; or, with no idle period, one full period that does the P V of
  //    the last light tile and the K Q^T of the first heavy one with the output in between;
  //  * heavy: full periods, then the P V of the last heavy tile.
  // The heavy query rows are consumed (the compiler's wait for them) at a fixed point of each
  // switch path, before any loop: the compiler cannot see the tile loads, so a wait it had to
  // place inside a loop for loads that might still be in flight would drain the whole tile
  // pipeline every period. The loops also use the plain period-end wait; the first two heavy
  // periods, which the switch's extra memory instructions may still precede, use the counted one.
  using kFirstT = std::integral_constant<int, 0>;
  using kFullT = std::integral_constant<int, 1>;
  using kLastT = std::integral_constant<int, 2>;
  using kLoadsT = std::integral_constant<int, 3>;
  using T = std::true_type;
  using F = std::false_type;
  auto run = [&](auto group_tag) {
    constexpr int kGroup = decltype(group_tag)::value;
    constexpr int kLead = kGroup == 0 ? kStages - 1 : kStages - 2;
    // Event flags (compile-time): q_wait consumes the heavy query rows at the period's start;
    // q_load loads them after its MFMA phase; to_heavy writes the light rows and switches to the
    // heavy ones after its MFMA phase; counted selects the period-end wait that counts them.
    auto period = [&](int p, auto mode_tag, auto q_wait, auto q_load, auto to_heavy, auto counted) {
      constexpr int kMode = decltype(mode_tag)::value;
      constexpr bool kDoPv = kMode == kFullT::value || kMode == kLastT::value;
      constexpr bool kDoQk = kMode == kFirstT::value || kMode == kFullT::value;
      const int slot = __builtin_amdgcn_readfirstlane(p % kStages);
      u32x4s w;
      auto hook = [&](auto i_tag) {
        constexpr int i = decltype(i_tag)::value;
        if constexpr (i == 0) w = tile_words(p + kLead);
        if constexpr (i % 8 == 1 && i / 8 < kDmaPerWave) {
          issue_block(w, slot + kLead, std::integral_constant<int, i / 8>{});
        }
      };
      auto mfma = [&]() {
        if constexpr (kMode == kLoadsT::value) {
          loads_only(hook);
        } else {
          mfma_phase(slot, std::bool_constant<kDoPv>{}, std::bool_constant<kDoQk>{}, hook);
        }
      };
      auto after_mfma = [&]() {
        if constexpr (decltype(q_load)::value) load_q(heavy.row0);
        if constexpr (decltype(to_heavy)::value) switch_to_heavy();
      };
      if constexpr (decltype(q_wait)::value) consume_q();
      if constexpr (kMode == kFirstT::value) prefetch_qk(slot);
      if constexpr (kGroup == 0) {
        mfma();
        operands_dead();
        after_mfma();
        if constexpr (kDoQk) {
          prefetch((slot + 1) % kStages);  // V(p), for the P V of period p + 1
          softmax_phase(tile_at(p));
        }
        scores_dead();
      } else {
        if constexpr (kDoPv) {
          prefetch(slot);  // V(p - 1)
          softmax_phase(tile_at(p - 1));
        }
        scores_dead();
        mfma();
        operands_dead();
        after_mfma();
      }
      if constexpr (decltype(counted)::value) {
        period_end_wait(p, group_tag);
      } else {
        wait_vmcnt<kGroup == 0 ? kPendingK : kPendingV>();
      }
      phase_barrier();
    };
    int m = 0;
    // Light part: K Q^T of tiles 0 .. light.tiles - 1 (each P V one period later). The period
    // after which the heavy query rows load is its own instance, so no loop sees them in flight.
    if (light.tiles == 1) {
      if (q_switch) {
        period(0, kFirstT{}, F{}, T{}, F{}, T{});
      } else {
        period(0, kFirstT{}, F{}, F{}, F{}, T{});
      }
    } else if (light.tiles > 1) {
      period(0, kFirstT{}, F{}, F{}, F{}, F{});
      for (m = 1; m < light.tiles - 1; ++m) period(m, kFullT{}, F{}, F{}, F{}, F{});
      if (q_switch) {
        period(m, kFullT{}, F{}, T{}, F{}, T{});
      } else {
        period(m, kFullT{}, F{}, F{}, F{}, T{});
      }
    }
    m = light.tiles;
    if (!two) {
      if (light.tiles > 0) {
        period(m, kLastT{}, F{}, F{}, F{}, T{});
        ++m;
      }
      for (; m <= stream; ++m) period(m, kLoadsT{}, F{}, F{}, F{}, T{});
      return;
    }
    // Switch. Without light tiles the wave wrote its light rows (as zeros) before period 0 and
    // loaded its heavy query rows in the prologue.
    if (!q_switch) {
      if (light.tiles > 0) {
        period(m, kLastT{}, F{}, F{}, T{}, T{});
        ++m;
      }
      for (; m < heavy_start; ++m) period(m, kLoadsT{}, F{}, F{}, F{}, T{});
      if (heavy.tiles > 0) {
        period(m, kFirstT{}, F{}, F{}, F{}, T{});
        ++m;
      }
    } else if (heavy_start == light.tiles) {
      // No idle period: the query rows are consumed at the start of this one.
      period(m, kFullT{}, T{}, F{}, T{}, T{});
      ++m;
    } else if (heavy_start == light.tiles + 1) {
      period(m, kLastT{}, T{}, F{}, T{}, T{});
      period(m + 1, kFirstT{}, F{}, F{}, F{}, T{});
      m += 2;
    } else {
      period(m, kLastT{}, F{}, F{}, T{}, T{});
      for (++m; m < heavy_start - 1; ++m) period(m, kLoadsT{}, F{}, F{}, F{}, T{});
      period(m, kLoadsT{}, T{}, F{}, F{}, T{});  // the last idle period: consume the query rows
      period(m + 1, kFirstT{}, F{}, F{}, F{}, T{});
      m += 2;
    }
    // Heavy part: full periods up to the last heavy K Q^T (period stream - 1), then its P V.
    if (heavy.tiles > 0) {
      for (int i = 0; i < 2 && m < stream; ++i, ++m) period(m, kFullT{}, F{}, F{}, F{}, T{});
      for (; m < stream; ++m) period(m, kFullT{}, F{}, F{}, F{}, F{});
      period(m, kLastT{}, F{}, F{}, F{}, T{});
      ++m;
    }
    for (; m <= stream; ++m) period(m, kLoadsT{}, F{}, F{}, F{}, T{});
  };
  if (group == 0) {
    run(std::integral_constant<int, 0>{});
  } else {
    run(std::integral_constant<int, 1>{});
  }
  // The last rows: the heavy ones of a pair, or the light ones of a block that runs alone.
  store_rows(two ? heavy.row0 : light.row0);
  // Loads past the end of the stream may still be in flight into free slots.
  wait_vmcnt<0>();
}

template <typename Tag, int D>
hipError_t launch_typed(PrefillArgs args, hipStream_t stream) {
  args.q_blocks = (args.seqlen_q + kPpBlockM - 1) / kPpBlockM;
  const int blocks = (args.q_blocks + 1) / 2 * args.batch * args.heads;
  hipLaunchKernelGGL((prefill_causal_kernel<Tag, D>), dim3(blocks), dim3(kPpThreads), 0, stream, args);
  return hipGetLastError();
}

}  // namespace
}  // namespace pp
}  // namespace prefill

hipError_t launch_prefill_causal_stream(const PrefillArgs& args, DType dtype, int head_dim,
                                        hipStream_t stream) {
  using namespace prefill::pp;
  if (!args.causal) return hipErrorInvalidValue;
  if (head_dim == 64) {
    return dtype == DType::bf16 ? launch_typed<bf16_tag, 64>(args, stream)
                                : launch_typed<f16_tag, 64>(args, stream);
  }
  if (head_dim != 128) return hipErrorInvalidValue;
  return dtype == DType::bf16 ? launch_typed<bf16_tag, 128>(args, stream)
                              : launch_typed<f16_tag, 128>(args, stream);
}

}  // namespace fl
