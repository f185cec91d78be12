// FlashAttention-2 forward (prefill) for gfx950 with explicit MFMA / softmax ping-pong between the
// two waves that share each SIMD. Same arithmetic and lane layouts as prefill_fwd.hip (see
// prefill_tile.hpp); what differs is how the work is laid out over time.
//
// Serves the attention_mma_pipelined and attention_mma ops of the reference
// (csrc/prefill/mma_pipelined.cu:54-183) at head_dim 128 and 64; the algorithm (tiling, online softmax
// with the -inf-safe reference point, bottom-right causal mask, 1/l epilogue) follows the
// reference's definitions (csrc/prefill/mma_tile.cuh:60-174, flash_lab/reference.py:90-152).
//
// Why: within one wave, VALU instructions issued between MFMAs overlap with them only in part (on
// gfx950, 8 independent FMAs after each MFMA made a register-only loop 1.3x slower, and the
// exponential-heavy softmax, which also waits for its scores, overlaps less), while an MFMA stream
// in one wave and a VALU stream in another wave of the same SIMD run concurrently at full MFMA
// rate. A wave issues at most one instruction every 4-5 cycles whatever its kind, so the
// softmax wave's phase costs about 5 cycles per instruction (about 9.6 per exponential) and must
// stay below the MFMA phase's 1024 cycles: everything that is not softmax arithmetic (tile loads,
// their descriptors) is issued by the MFMA wave, which has idle issue slots while its MFMAs run.
// At head_dim 64 the MFMA phase is 16 MFMAs (512 cycles) against the same softmax as at 128, and
// a wave runs the two back to back in each period, so two waves per SIMD leave the matrix pipe
// idle most of the time: there the workgroup has a third group of four waves (168 VGPRs each, three
// waves per SIMD), which runs group 1's order and loads nothing. The VALU then bounds the period
// (one wave's softmax at a time keeps it busy; 32 of its ~90 instructions are exponentials), so at
// 64 the row sums are taken by the matrix cores and issue priorities order the three softmaxes.
//
//  * Workgroup: 8 waves x 32 query rows = 256 rows of one (batch, head) at head_dim 128, 12 waves
//    (384 rows) at 64. Waves w, w + 4 (and w + 8) share a SIMD (the dispatcher deals waves to
//    SIMDs with period 4). Group g is waves 4g .. 4g + 3: one wave of each group per SIMD.
//  * Time is cut into periods by workgroup barriers, one per tile. In the first half of period m
//    group 0 runs MFMA(m) = P V of tile m-1 then S = K Q^T of tile m (32 MFMAs) while group 1 runs
//    the softmax of tile m-1; in the second half the roles swap. Nothing holds the groups to the
//    half-period boundary: they keep the offset by themselves (contention for the MFMA pipe), and a
//    barrier in the middle of each period measured 1-1.6% slower.
//  * K and V tiles (64 keys) stream through a ring of kStages LDS slots each, filled by direct
//    global -> LDS loads (buffer_load ... lds) issued between the MFMAs of the MFMA phases: group 0
//    loads K(m + kStages - 1) in the first half of period m, group 1 V(m + kStages - 2) in the second
//    (4 loads per wave each at D = 128, 2 at D = 64; a load costs the issuing wave about 70
//    cycles, which the MFMA phase has to spare). Each group waits for its own tiles at the end of a
//    period, so the barrier that ends it publishes them before their first read. Loads past the
//    last tile use an empty buffer resource (they write zeros into a free slot) so every wave
//    issues the same number of loads and the vmcnt accounting is
//    uniform.
//  * Work order: XCD-contiguous (batch, head) ranges (workgroups are dealt round-robin over the 8
//    XCDs, each with its own L2); causal query blocks in heavy/light pairs per workgroup.
#include <type_traits>

#include "prefill_pp.hpp"

namespace fl {
namespace prefill {
namespace pp {
namespace {

template <typename Tag, int D>
__global__ void __launch_bounds__(64 * kPpWavesOf<D>)
    __attribute__((amdgpu_waves_per_eu(kPpGroups<D>, kPpGroups<D>))) prefill_pp_kernel(const PrefillArgs a) {
  using E = Elem<Tag>;
  constexpr int kGroups = kPpGroups<D>;
  constexpr int kBlockM = kPpBlockMOf<D>;
  constexpr int kTile = kTileElems<D>;
  // One LDS array: the K ring (kStages slots) then the V ring. ds_read immediates reach 64 KiB, so
  // V reads go through per-lane offsets biased by the K ring's size and every slot offset is an
  // immediate (separate arrays past 64 KiB would each need their own address registers).
  __shared__ __attribute__((aligned(16))) uint16_t smem[2 * kStages * kTile];
  constexpr int kSlotBytes = 2 * kTile;
  constexpr int kVRingBytes = kStages * kSlotBytes;
  static_assert(kVRingBytes <= 65536, "K ring must fit the immediate range");
  // Ring slots are ints: compile-time constants in the unrolled tile loop (folded into the LDS
  // instructions' immediates), run-time values only in a block's last period.
  auto k_slot = [&](int s) -> uint16_t* { return smem + (static_cast<unsigned>(s) % kStages) * kTile; };
  // Byte offset of V slot s from the biased per-lane V offsets.
  auto v_slot_offset = [&](int s) { return (static_cast<unsigned>(s) % kStages) * kSlotBytes; };
  const char* lds_bytes = reinterpret_cast<const char*>(smem);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int group = wave >> 2;
  const int half = lane >> 5;

  // Row sums on the matrix cores, at head_dim 64 only: there the softmax's VALU work bounds the
  // kernel and the matrix pipe has room. For key step kk, P^T's fragment pf[kk] (the 32x32x16 B
  // operand: lane l holds 8 of the step's keys of row l % 32) is also the B operand of one
  // v_mfma_f32_16x16x32, which reads it as B[k][n] in lane n + 16 (k / 8): lane group g = l / 16
  // holds row n + 16 (g % 2), half g / 2 of the step's keys. The A operand is a 0/1 selector,
  // A[m][k] = 1 iff (k / 8) % 2 == (m / 4) % 2, so D[m][n] is the step's sum of row
  // n + 16 ((m / 4) % 2), which lands in lane n + 16 (m / 4): every register of lane l holds the
  // sum of its own row l % 32 over both halves. Lane l holds A[l % 16][8 (l / 16) + e], e = 0..7,
  // all equal. This sums the probabilities as rounded for P V, so o and l agree exactly on them.
  constexpr bool kMfmaSums = D == 64;
  const uint32_t sel_word = ((lane >> 4) & 1) == ((lane >> 2) & 1) ? E::kOnePair : 0u;
  const u32x4 sum_sel{sel_word, sel_word, sel_word, sel_word};

  // Work item: (batch, head) and query blocks. Non-causal: one block per workgroup. Causal: the
  // blocks of a (batch, head) go in pairs (q_blocks - 1 - i, i), heavy first, so every workgroup
  // runs about the same number of tiles (a plain heaviest-first order still leaves a tail of heavy
  // blocks dealt late) and the light block's K and V are a prefix of the heavy one's.
  const int work = xcd_remap(blockIdx.x, gridDim.x);
  const int items_per_bh = a.causal ? (a.q_blocks + 1) / 2 : a.q_blocks;
  const int bh = work / items_per_bh;
  const int item = work - bh * items_per_bh;
  const int b = bh / a.heads;
  const int h = bh - b * a.heads;
  const int hkv = h / a.group;
  const uint16_t* qp = a.q + b * a.q_bs + h * a.q_hs;
  const uint16_t* kp = a.k + b * a.k_bs + hkv * a.k_hs;
  const uint16_t* vp = a.v + b * a.v_bs + hkv * a.v_hs;

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

  // Tile loads: group 0 streams the K tiles, group 1 the V tiles. Wave lw of a group moves
  // kDmaPerWave 1 KiB blocks of each tile; block j of a slot sits at LDS byte lds_wave + slot
  // offset + 1024 j, and its lane l covers row (lw kDmaPerWave + j) kRowsPerBlock + l /
  // kChunksPerRow, chunk l % kChunksPerRow (stored swizzled).
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
  // Buffer resource of tile t of the group's tensor: based at the tile's first row, sized to its
  // valid rows (full tiles before the last one, the last one up to the sequence end, none outside
  // [0, num_tiles): those read as zeros).
  const int64_t tile_bytes = static_cast<int64_t>(kBlockN) * my_ss * 2;
  // The wave's query rows of block qb, the B operand of K Q^T: lane (r, half) holds row
  // qb kPpBlockM + 32 wave + r, dims 16 ks + 8 half .. + 7 (zeros past the sequence).
  u32x4 qf[D / 16];
  auto load_q = [&](int qb) {
    const int r = qb * kBlockM + wave * kRowsPerWave + (lane & 31);
    const bool ok = r < a.seqlen_q;
    const uint16_t* src = qp + static_cast<int64_t>(ok ? r : 0) * a.q_ss + 8 * half;
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) qf[ks] = ok ? load16(src + 16 * ks) : u32x4{0, 0, 0, 0};
  };
  // Uses the Q registers, so that the compiler's wait for their loads sits here (it does not see
  // the tile loads, and would otherwise wait for every later one at the first use of Q).
  auto consume_q = [&]() {
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) asm volatile("" : "+v"(qf[ks]));
  };
  // The rows of the block to run next are in flight: the block before it loaded them in its last
  // MFMA period (P V only, so Q is no longer needed there), hiding their latency behind that
  // period and the epilogue. Measured per wave, loading them in the block's own prologue waited
  // 4,000-6,800 cycles (the second group's loads queue behind the first's).
  bool q_loaded = false;
  // One query block of kBlockM rows: its own tile range, pipeline and epilogue (and, when next_qb
  // >= 0, the query rows of block next_qb). Every wave has finished with the LDS ring and every
  // tile load has landed when it returns.
  auto process = [&](const int qb, const int next_qb) {
    const int q0 = qb * kBlockM;
    const int row0 = q0 + wave * kRowsPerWave;
    const int my_row = row0 + (lane & 31);

    int kv_end = a.seqlen_k;
    if (a.causal) kv_end = min(kv_end, min(q0 + kBlockM, a.seqlen_q) + a.causal_offset);
    const int num_tiles = kv_end > 0 ? (kv_end + kBlockN - 1) / kBlockN : 0;
    // Tiles this wave sees any key of (a prefix of the workgroup's tiles), and the first tile whose
    // scores need masking (it reaches past the sequence end or, causal, past the diagonal of the
    // wave's first row): every tile before it is fully visible to every row of the wave.
    int my_tiles = num_tiles;
    int mask_from = a.seqlen_k / kBlockN;
    if (a.causal) {
      const int last = row0 + kRowsPerWave - 1 + a.causal_offset;  // last key any of its rows sees
      my_tiles = last < 0 ? 0 : min(num_tiles, last / kBlockN + 1);
      const int x = row0 + a.causal_offset - (kBlockN - 1);  // tile t needs masking iff 64 t > x
      mask_from = min(mask_from, x < 0 ? 0 : x / kBlockN + 1);
    }
    // A wave whose rows all lie past the sequence (the last block of a ragged S_q) only keeps its
    // turn in the loads and barriers.
    if (row0 >= a.seqlen_q) my_tiles = 0;

    if (!q_loaded) {
      load_q(qb);
      consume_q();
    }
    q_loaded = false;

    const int last_rows = num_tiles > 0 ? min(kBlockN, a.seqlen_k - (num_tiles - 1) * kBlockN) : 1;
    const uint32_t full_bytes = static_cast<uint32_t>(((kBlockN - 1) * my_ss + D) * 2);
    const uint32_t last_bytes = static_cast<uint32_t>(((last_rows - 1) * my_ss + D) * 2);
    auto tile_words = [&](int t) -> u32x4s {
      const bool inside = t >= 0 && t < num_tiles;
      const uint32_t bytes = !inside ? 0u : t == num_tiles - 1 ? last_bytes : full_bytes;
      const char* p = reinterpret_cast<const char*>(my_base) + (inside ? t * tile_bytes : 0);
      return buffer_words(p, bytes);
    };
    // The same for a tile t >= 0 whose first row is at p = my_base + t tile_bytes, which the periods
    // carry from one to the next: half the scalar instructions, issued between two MFMAs. A tile
    // past the last one gets size 0, so its address is never formed.
    auto tile_words_at = [&](int t, const char* p) -> u32x4s {
      const int d = num_tiles - 1 - t;
      return buffer_words(p, d > 0 ? full_bytes : d == 0 ? last_bytes : 0u);
    };
    // Block j of the group's tile (descriptor `w`) into ring slot kSlot.
    auto issue_block = [&](u32x4s w, int slot, auto j_tag) {
      constexpr int j = decltype(j_tag)::value;
      const uint32_t off = (static_cast<unsigned>(slot) % kStages) * kSlotBytes + j * 1024;
      buffer_load16_to_lds_asm(w, lds_wave + off, my_off[j]);
    };
    auto load_tile = [&](int t, int slot) {
      const u32x4s w = tile_words(t);
      static_for<0, kDmaPerWave>([&](auto j) { issue_block(w, slot, j); });
    };

    f32x16 o[D / 32];
#pragma unroll
    for (int nb = 0; nb < D / 32; ++nb) o[nb] = f32x16{};
    f32x16 s0 = f32x16{};
    f32x16 s1 = f32x16{};
    u32x4 pf[4] = {};
    float ref = kNoRef;
    float l = 0.f;  // the lane's part of its row's sum; with kMfmaSums, the whole row's
    f32x4 ls = {};  // kMfmaSums: P's row sums from the last MFMA phase, added by the next softmax
    const float sl2 = a.scale_log2;
    const int last_key = a.causal ? min(a.seqlen_k - 1, my_row + a.causal_offset) : a.seqlen_k - 1;

    // MFMA phase of a period with slots kS = m % kStages: O += V(m-1) P(m-1) (16 MFMAs) and
    // S = K(m) Q^T (16 MFMAs). No branches: in period 0 the previous P and V are zeros (P starts at
    // 0, the V slot was filled from an empty resource), a skipped softmax leaves P = 0, and scores of
    // tiles nobody reads are never used. The 32 MFMAs form one software pipeline: the A-operand
    // fragment of the MFMA kAhead steps later is read from LDS right after an MFMA issues, and a
    // scheduling barrier after every step keeps that order (left to itself the scheduler reads each
    // fragment just before its MFMA and the LDS latency shows on every step). The first kAhead
    // fragments are read at the end of the wave's softmax phase (prefetch), so the MFMA phase
    // starts without waiting for LDS. hook(i) runs after the MFMA of phase step i (the tile loads
    // are issued there).
    // A phase with both parts runs the first kLeadPv P V steps, then K Q^T, then the rest of P V,
    // and computes the tile's row max (tile_mx, for the softmax that follows) between those last
    // P V MFMAs, from the scores K Q^T has just completed: the max tree then takes issue slots the
    // MFMA wave has free instead of lengthening the softmax phase, which sets the half-period. The
    // lead steps cover the latency of the first K fragment reads (K(m) is published by the barrier
    // that starts the phase, so its fragments cannot be prefetched).
    constexpr int kPv = 4 * (D / 32);  // P V MFMAs: key step kk = i / (D / 32), dim block nb
    constexpr int kQk = 2 * (D / 16);  // K Q^T MFMAs: dim step ks = j / 2, key block j % 2
    constexpr int kSteps = kPv + kQk;
    // (At head_dim 64 with one fragment ahead every MFMA waited for its LDS read: a phase took
    // ~1,200 cycles for 576 cycles of MFMAs, against ~650 with two.)
    constexpr int kAhead = FL_PP_AHEAD;
    constexpr int kLeadPv = kPv - 4;
    constexpr int kTail = kPv - kLeadPv;  // P V steps after K Q^T
    static_assert(kAhead >= 1 && kAhead <= kLeadPv, "prefetched fragments are V fragments");
    static_assert(kTail >= 2, "room for the max tree");
    static_assert(8 * (kDmaPerWave - 1) + 1 < kSteps, "one tile load every 8 MFMAs");
    // Logical step (i < kPv: P V step i; else K Q^T step i - kPv) of phase position n.
    auto step_at = [](auto n_tag, auto full_tag) constexpr {
      constexpr int n = decltype(n_tag)::value;
      if constexpr (!decltype(full_tag)::value) {
        return n;
      } else {
        return n < kLeadPv ? n : n < kLeadPv + kQk ? kPv + (n - kLeadPv) : n - kQk;
      }
    };
    // Fragment of logical step i of the phase with slots kS = m % kStages: V(m - 1) sits in V slot
    // kS + kStages - 1, K(m) in K slot kS.
    auto read_frag = [&](int slot, auto i_tag) -> u32x4 {
      constexpr int i = decltype(i_tag)::value;
      if constexpr (i < kPv) {
        constexpr int kk = i / (D / 32), nb = i % (D / 32);
        const char* vt = lds_bytes + v_slot_offset(slot + kStages - 1);
        return v_frag_at(vt + kk * kKeyStepBytes<D>, v_lds[nb][0], v_lds[nb][1]);
      } else {
        constexpr int j = i - kPv, ks = j / 2, blk = j % 2;
        const char* kt = reinterpret_cast<const char*>(k_slot(slot));
        return lds_load16(kt + blk * kKeyBlockBytes<D>, k_lds[ks]);
      }
    };
    // The first kAhead fragments of the next MFMA phase (P V's, or K Q^T's for a phase with K Q^T
    // only), read at the end of the wave's softmax phase. Only these cross from one phase to the
    // next: the rest of a phase's fragments live in that phase.
    u32x4 pre[kAhead];
    auto prefetch = [&](int slot) {
      static_for<0, kAhead>([&](auto i) { pre[decltype(i)::value] = read_frag(slot, i); });
    };
    auto prefetch_qk = [&](int slot) {
      static_for<0, kAhead>([&](auto i) {
        pre[decltype(i)::value] = read_frag(slot, std::integral_constant<int, kPv + decltype(i)::value>{});
      });
    };
    // Row max of the scores (log2 units, both halves of the row), computed by the MFMA phase that
    // produced them; the softmax of a masked tile computes its own.
    float tile_mx = kNoRef;
    float mx_t[10], mx_u[4], mx_w = 0.f;
    // Op k of the max tree over s0, s1 (18 ops: s0's leaves first, whose MFMAs finish first).
    auto max_op = [&](auto k_tag) {
      constexpr int k = decltype(k_tag)::value;
      if constexpr (k < 5) {
        mx_t[k] = max3_f32(s0[3 * k], s0[3 * k + 1], s0[3 * k + 2]);
      } else if constexpr (k < 10) {
        mx_t[k] = max3_f32(s1[3 * (k - 5)], s1[3 * (k - 5) + 1], s1[3 * (k - 5) + 2]);
      } else if constexpr (k < 13) {
        mx_u[k - 10] = max3_f32(mx_t[3 * (k - 10)], mx_t[3 * (k - 10) + 1], mx_t[3 * (k - 10) + 2]);
      } else if constexpr (k == 13) {
        mx_u[3] = max3_f32(mx_t[9], s0[15], s1[15]);
      } else if constexpr (k == 14) {
        mx_w = max3_f32(mx_u[0], mx_u[1], mx_u[2]);
      } else if constexpr (k == 15) {
        mx_w = max2_f32(mx_w, mx_u[3]);
      } else if constexpr (k == 16) {
        mx_w = max_halves(mx_w);
      } else {
        tile_mx = mx_w * sl2;  // scale_log2 > 0, so the max commutes with it
      }
    };
    constexpr int kMaxOps = 18;
    // Issue priorities (s_setprio): a wave in its MFMA phase outranks the others, so its MFMAs issue
    // as soon as their operands are ready. With three groups the softmax phases are ranked too,
    // group 1 over group 2 over group 0: one softmax at a time keeps the VALU busy (each is ~90
    // instructions, 32 of them exponentials, and a second wave's softmax only fills its gaps), and
    // waves of equal priority are served oldest first, which would put group 0's first. In this
    // order group 0's MFMA phase runs during group 1's softmax, group 1's during group 2's, and
    // group 2's during group 0's, which ends the period.
    constexpr int kMfmaPrio = kGroups == 3 ? 3 : 1;
    auto mfma_phase = [&](int slot, auto pv_tag, auto qk_tag, auto&& hook, auto prio_tag) {
      constexpr bool kDoPv = decltype(pv_tag)::value;
      constexpr bool kDoQk = decltype(qk_tag)::value;
      constexpr bool kFull = kDoPv && kDoQk;
      // Live phase positions are [kFirstLive, kEndLive); the first kAhead of them were prefetched.
      constexpr int kFirstLive = kDoPv ? 0 : kPv;
      constexpr int kEndLive = kDoQk ? kSteps : kPv;
      u32x4 fr[kSteps];  // by logical step
      static_for<0, kAhead>([&](auto i) {
        constexpr int n = kFirstLive + decltype(i)::value;
        fr[step_at(std::integral_constant<int, n>{}, std::bool_constant<kFull>{})] = pre[decltype(i)::value];
      });
      auto issue = [&](auto i_tag, const u32x4& f) {
        constexpr int i = decltype(i_tag)::value;
        if constexpr (i < kPv) {
          constexpr int kk = i / (D / 32), nb = i % (D / 32);
          o[nb] = E::mfma32(f, pf[kk], o[nb]);
          if constexpr (kMfmaSums && nb == D / 32 - 1) {
            ls = E::mfma16(sum_sel, pf[kk], kk == 0 ? f32x4{} : ls);
          }
        } else {
          constexpr int j = i - kPv, ks = j / 2, blk = j % 2;
          f32x16& acc = blk == 0 ? s0 : s1;
          acc = E::mfma32(f, qf[ks], ks == 0 ? f32x16{} : acc);
        }
      };
#if FL_PP_SETPRIO == 1
      __builtin_amdgcn_s_setprio(kMfmaPrio);
#endif
      __builtin_amdgcn_sched_barrier(0);
      static_for<0, kSteps>([&](auto n_tag) {
        constexpr int n = decltype(n_tag)::value;
        constexpr int i = step_at(n_tag, std::bool_constant<kFull>{});
        if constexpr (n >= kFirstLive && n < kEndLive) issue(std::integral_constant<int, i>{}, fr[i]);
        constexpr int nx = n + kAhead;
        if constexpr (nx >= kFirstLive + kAhead && nx < kEndLive) {
          constexpr int ix = step_at(std::integral_constant<int, nx>{}, std::bool_constant<kFull>{});
          fr[ix] = read_frag(slot, std::integral_constant<int, ix>{});
        }
        hook(n_tag);
        if constexpr (kFull && n >= kLeadPv + kQk) {
          constexpr int k = n - (kLeadPv + kQk);
          static_for<k * kMaxOps / kTail, (k + 1) * kMaxOps / kTail>([&](auto op) { max_op(op); });
        }
        __builtin_amdgcn_sched_barrier(0);
      });
#if FL_PP_SETPRIO == 1
      __builtin_amdgcn_s_setprio(decltype(prio_tag)::value);
#endif
      // A K Q^T-only phase (tile 0) has no P V MFMAs to hide the tree behind.
      if constexpr (kDoQk && !kDoPv) static_for<0, kMaxOps>([&](auto op) { max_op(op); });
    };
    // A phase whose MFMAs nobody in the group needs (causal tiles past the diagonal of all of the
    // group's rows): only its tile loads.
    auto loads_only = [&](auto&& hook) {
      static_for<0, kSteps>([&](auto i) { hook(i); });
    };

    // P(t) from S(t) against the reference point: p = 2^(s scale_log2 + neg_shift), packed (rounded
    // to the input type) as the P V operand; returns the lane's sum of the unrounded probabilities
    // (fp32 adds: v_dot2 on the packed values would be shorter, but on gfx950 it waits behind the
    // other wave's MFMAs, which more than doubles the phase), or 0 where the MFMA phase sums them.
    auto probabilities = [&](float neg_shift) -> float {
      f32x16 p0, p1;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        p0[j] = exp2_fast(fmaf(s0[j], sl2, neg_shift));
        p1[j] = exp2_fast(fmaf(s1[j], sl2, neg_shift));
      }
      if constexpr (kMfmaSums) {
        pf[0] = p_frag<Tag, 0>(p0);
        pf[1] = p_frag<Tag, 1>(p0);
        pf[2] = p_frag<Tag, 0>(p1);
        pf[3] = p_frag<Tag, 1>(p1);
        return 0.f;
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

    // Softmax phase for tile t: S(t) -> P(t) and the running sum. The reference point `ref` (log2
    // units, the same for both halves of a row) moves to the row's running max when the tile's max
    // passes it by more than kMoveSlack (a wave-uniform branch: the rescale of o runs only on tiles
    // where some row of the wave moved). A row without a key yet keeps kNoRef, so its masked scores
    // give p = 0.
    // It runs only for tiles t < my_tiles: a wave's periods past its last visible tile are
    // loads-only.
    auto softmax_body = [&](int t) {
      if constexpr (kMfmaSums) l += ls[0];  // P(t - 1)'s sums, relative to the current point
      float mx = tile_mx;
      if (t >= mask_from) {
        asm volatile("" ::: "memory");
        // acc_key(j, half) = acc_key(j, 0) + 4 half: fold the lane's part into the limit so every
        // comparison is against a compile-time constant (no per-key registers live in the loop).
        const int lim = last_key - t * kBlockN - 4 * half;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          constexpr int kBase = 0;
          const int kj = acc_key(j, kBase);
          s0[j] = kj > lim ? -INFINITY : s0[j];
          s1[j] = kj + 32 > lim ? -INFINITY : s1[j];
          // One compare and one select per score: left free, the scheduler kept all 32 compare
          // results live in scalar register pairs and chained them, which made the kernel spill
          // 86 scalar registers (reloaded on every masked tile).
          __builtin_amdgcn_sched_barrier(0);
        }
        mx = max_halves(max_of(s0, s1)) * sl2;  // -inf for a tile the row sees no key of
      }
      if (wave_any(mx > ref + kMoveSlack)) {
        asm volatile("" ::: "memory");
        const float moved = max2_f32(ref, mx);
        const float alpha = exp2_fast(ref - moved);  // 0 for a row's first key (ref = kNoRef)
        ref = moved;
#pragma unroll
        for (int nb = 0; nb < D / 32; ++nb) o[nb] *= alpha;
        l *= alpha;
      }
      if constexpr (kMfmaSums) {
        probabilities(-ref);
      } else {
        l += probabilities(-ref);
      }
    };
    auto softmax_phase = [&](int t) {
#if FL_PP_SETPRIO == 2
      __builtin_amdgcn_s_setprio(1);
#endif
      softmax_body(t);
#if FL_PP_SETPRIO == 2
      __builtin_amdgcn_s_setprio(0);
#endif
    };

    // Each group waits for its own loads at the end of period m: group 0 for K(m + 1) (first read
    // in period m + 1) with the kStages - 2 later K tiles still in flight, group 1 for V(m + 1)
    // (first read in period m + 1, by group 0's fragment prefetch) with the kStages - 3 later V
    // tiles.
    constexpr int kPendingK = (kStages - 2) * kDmaPerWave;
    constexpr int kPendingV = (kStages - 3) * kDmaPerWave;

    // Prologue: group 0 loads K(0 .. kStages - 2), group 1 V(-1 .. kStages - 3) (V(-1) stands for
    // the P V that period 0 does not run, so every wave issues the same loads); K(0) and V(0) must
    // be in LDS before period 0.
    static_for<0, kStages - 1>([&](auto i_tag) {
      constexpr int i = decltype(i_tag)::value;
      if (group == 0) {
        load_tile(i, i);
      } else if (group == 1) {
        load_tile(i - 1, i + kStages - 1);
      }
    });
    if (group == 0) {
      wait_vmcnt<(kStages - 2) * kDmaPerWave>();
    } else if (group == 1) {
      wait_vmcnt<(kStages - 3) * kDmaPerWave>();
    }
    phase_barrier();

    // Period m, one barrier at its end. Group 0: MFMA(m), softmax(m). Group 1 (and group 2 at
    // head_dim 64): softmax(m - 1), then MFMA(m). Each MFMA phase issues its group's next tile between its MFMAs (the descriptor
    // after MFMA 0, block j after MFMA 8j + 1). A group's periods run in four kinds:
    //  * first (m = 0): K Q^T only, as there is no tile -1 for a P V;
    //  * full, m = 1 .. G - 1, as a straight-line loop unrolled by kStages from slot 1 so that ring
    //    slots are compile-time immediates;
    //  * last (m = G): P V of tile G - 1 only, its slot G % kStages a run-time value;
    //  * loads only, m = G + 1 .. num_tiles: the group's tile loads and waits (the other group may
    //    still read those tiles) but no MFMAs,
    // where G is the number of tiles any row of the wave sees (my_tiles): num_tiles, or fewer for a
    // wave of earlier rows on a causal diagonal, whose tiles past those rows' diagonal it skips. The
    // waves of a group keep their turns on the MFMA pipes whatever their own G, and every wave runs
    // num_tiles + 1 periods of one barrier each.
    const int wave_tiles = my_tiles;
    using kFirstT = std::integral_constant<int, 0>;
    using kFullT = std::integral_constant<int, 1>;
    using kLastT = std::integral_constant<int, 2>;
    using kLoadsT = std::integral_constant<int, 3>;
    auto run = [&](auto group_tag) {
      constexpr int kGroup = decltype(group_tag)::value;
      // Group 2 (head_dim 64) runs group 1's order and loads nothing.
      constexpr bool kLoads = kGroup < 2;
      // The group's issue priority outside its MFMA phases, i.e. its softmax's (see kMfmaPrio).
      constexpr int kBasePrio =
          kGroups == 3 && FL_PP_SETPRIO == 1 ? (kGroup == 1 ? 2 : kGroup == 2 ? 1 : 0) : 0;
      using kPrioT = std::integral_constant<int, kBasePrio>;
      // Group 0 loads K(m + kStages - 1) into slot (m - 1) % kStages, group 1 V(m + kStages - 2)
      // into slot (m - 2) % kStages.
      constexpr int kLead = kGroup == 0 ? kStages - 1 : kStages - 2;
      // First row of tile m + kLead, the tile that period m loads.
      const char* lead_tile = reinterpret_cast<const char*>(my_base) + kLead * tile_bytes;
      auto period = [&](int m, int slot, auto mode_tag) {
        constexpr int kMode = decltype(mode_tag)::value;
        constexpr bool kDoPv = kMode == kFullT::value || kMode == kLastT::value;
        constexpr bool kDoQk = kMode == kFirstT::value || kMode == kFullT::value;
        u32x4s w;
        auto hook = [&](auto i_tag) {
          constexpr int i = decltype(i_tag)::value;
          if constexpr (kLoads && i == 0) {
            w = tile_words_at(m + kLead, lead_tile);
            lead_tile += tile_bytes;
          }
          if constexpr (kLoads && i % 8 == 1 && i / 8 < kDmaPerWave) {
            issue_block(w, slot + kLead, std::integral_constant<int, i / 8>{});
          }
        };
        auto mfma = [&]() {
          if constexpr (kMode == kLoadsT::value) {
            loads_only(hook);
          } else {
            mfma_phase(slot, std::bool_constant<kDoPv>{}, std::bool_constant<kDoQk>{}, hook, kPrioT{});
          }
        };
        // (Not with three groups: there the tile loops' registers are tight enough that the
        // compiler reuses registers these loads may still be writing, and then waits for every
        // load in flight inside the loops. The next block loads its rows in its prologue.)
        if constexpr (kMode == kLastT::value && kGroups == 2) {
          if (next_qb >= 0) {
            load_q(next_qb);
            q_loaded = true;
          }
        }
        if constexpr (kGroup == 0) {
          if constexpr (kMode == kFirstT::value) prefetch_qk(slot);
          mfma();
          if constexpr (kDoQk) {
            // The next MFMA phase's first fragments (V(m), published by the barrier that ended
            // period m - 1), read first so their latency hides behind the softmax.
            prefetch(slot + 1);
            softmax_phase(m);
          }
          if constexpr (kLoads) wait_vmcnt<kPendingK>();  // K(m + 1), first read in period m + 1
          phase_barrier();
        } else {
          if constexpr (kMode == kFirstT::value) prefetch_qk(slot);
          if constexpr (kDoPv) {
            prefetch(slot);
            softmax_phase(m - 1);
          }
          mfma();
          if constexpr (kLoads) wait_vmcnt<kPendingV>();  // V(m + 1), first read in period m + 1
          phase_barrier();
        }
      };
      if (num_tiles == 0) return;  // no key at all: nothing to multiply
      if constexpr (kBasePrio != 0) __builtin_amdgcn_s_setprio(kBasePrio);
      int m = 0;
      if (wave_tiles > 0) {
        period(0, 0, kFirstT{});
        for (m = 1; m < wave_tiles;) {
          bool done = false;
          static_for<0, kStages>([&](auto j) {
            if (done) return;
            period(m, (1 + decltype(j)::value) % kStages, kFullT{});
            done = ++m == wave_tiles;
          });
        }
        period(m, m % kStages, kLastT{});
        ++m;
      }
      for (; m <= num_tiles; ++m) period(m, m % kStages, kLoadsT{});
      if constexpr (kBasePrio != 0) __builtin_amdgcn_s_setprio(0);
    };
    if (group == 0) {
      run(std::integral_constant<int, 0>{});
    } else if (kGroups == 2 || group == 1) {
      run(std::integral_constant<int, 1>{});
    } else {
      if constexpr (kGroups == 3) run(std::integral_constant<int, 2>{});
    }
    // Loads past the end may still be in flight into free slots: each wave waits for its own here,
    // and the barrier below for the others', before the ring is reused.
    wait_vmcnt<0>();
    if (q_loaded) consume_q();

    const float lt = kMfmaSums ? l + ls[0] : sum_halves(l);
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    // Output rows go back whole, 16 bytes per lane (the accumulator layout would store 8 bytes per
    // lane into 32 rows a row stride apart): each wave stages its 32 rows in its own part of the
    // ring, rows padded by 16 bytes so that the row-per-lane writes spread over the banks, then
    // stores kRowsPerStore whole rows per instruction. Every staging address is one per-lane base
    // plus an immediate, so the addresses hold two registers (the bases are invariant across the
    // blocks of a causal workgroup and would otherwise stay live through the tile loop). With three
    // groups the lane index they derive from goes through an empty asm here, so the compiler
    // computes them here rather than before the tile loop (at 168 VGPRs, hoisted, they were
    // spilled).
    phase_barrier();
    int e_lane = lane;
    if constexpr (kGroups == 3) asm volatile("" : "+v"(e_lane));
    const int e_half = e_lane >> 5;
    const int e_row = row0 + (e_lane & 31);
    constexpr int kChunks = D / 8;
    constexpr int kStageRow = 2 * D + 16;
    constexpr int kRowsPerStore = 64 / kChunks;
    static_assert(kPpWavesOf<D> * kRowsPerWave * kStageRow <= static_cast<int>(sizeof(smem)), "staging fits");
    char* stage = reinterpret_cast<char*>(smem) + wave * kRowsPerWave * kStageRow;
    {
      char* wbase = stage + (e_lane & 31) * kStageRow + 8 * e_half;
#pragma unroll
      for (int nb = 0; nb < D / 32; ++nb) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          // Dims 32 nb + 8 g + 4 half .. + 3: half of 16-byte chunk 4 nb + g of this lane's row.
          const u32x2 packed{E::pack2(o[nb][4 * g] * inv, o[nb][4 * g + 1] * inv),
                             E::pack2(o[nb][4 * g + 2] * inv, o[nb][4 * g + 3] * inv)};
          *reinterpret_cast<u32x2*>(wbase + 16 * (4 * nb + g)) = packed;
        }
      }
    }
    {
      const int chunk = e_lane % kChunks;
      const char* rbase = stage + (e_lane / kChunks) * kStageRow + 16 * chunk;
      uint16_t* obase = a.o + b * a.o_bs + h * a.o_hs + 8 * chunk;
#pragma unroll
      for (int j = 0; j < kRowsPerWave / kRowsPerStore; ++j) {
        const int r = row0 + j * kRowsPerStore + e_lane / kChunks;
        const u32x4 v = *reinterpret_cast<const u32x4*>(rbase + j * kRowsPerStore * kStageRow);
        if (r < a.seqlen_q) *reinterpret_cast<u32x4*>(obase + static_cast<int64_t>(r) * a.o_ss) = v;
      }
    }
    if (e_row < a.seqlen_q && e_half == 0) {
      a.lse[(static_cast<int64_t>(b) * a.heads + h) * a.seqlen_q + e_row] =
          lt > 0.f ? ref * kLn2 + logf(lt) : -INFINITY;
    }
  };

  // One call site (a loop), so the block body is inlined once.
  const int heavy = a.q_blocks - 1 - item;
  const int blocks_here = a.causal && item < heavy ? 2 : 1;
  for (int i = 0; i < blocks_here; ++i) {
    // The next block's prologue refills the ring, which the epilogue's staging reads just used (no
    // memory fence: the output stores need not complete first).
    if (i > 0) phase_barrier();
    process(!a.causal ? item : i == 0 ? heavy : item, i + 1 < blocks_here ? item : -1);
  }
}

template <typename Tag, int D>
hipError_t launch_typed(PrefillArgs args, hipStream_t stream) {
  args.q_blocks = (args.seqlen_q + kPpBlockMOf<D> - 1) / kPpBlockMOf<D>;
  const int items_per_bh = args.causal ? (args.q_blocks + 1) / 2 : args.q_blocks;
  const int blocks = items_per_bh * args.batch * args.heads;
  hipLaunchKernelGGL((prefill_pp_kernel<Tag, D>), dim3(blocks), dim3(64 * kPpWavesOf<D>), 0, stream, args);
  return hipGetLastError();
}

}  // namespace
}  // namespace pp
}  // namespace prefill

int prefill_pp_block_rows(int head_dim) {
  return head_dim == 64 ? prefill::pp::kPpBlockMOf<64> : prefill::pp::kPpBlockMOf<128>;
}

hipError_t launch_prefill_pingpong(const PrefillArgs& args, DType dtype, int head_dim,
                                   hipStream_t stream) {
  using namespace prefill::pp;
  if (args.causal && knob(FL_KNOB_PREFILL_CAUSAL_STREAM) == 1)
    return launch_prefill_causal_stream(args, dtype, head_dim, stream);
  if (head_dim == 64) {
    return dtype == DType::bf16 ? launch_typed<bf16_tag, 64>(args, stream)
                                : launch_typed<f16_tag, 64>(args, stream);
  }
  if (head_dim != 128) return hipErrorInvalidValue;
  return dtype == DType::bf16 ? launch_typed<bf16_tag, 128>(args, stream)
                              : launch_typed<f16_tag, 128>(args, stream);
}

}  // namespace fl
