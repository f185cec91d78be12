// Pieces shared by the two ping-pong prefill kernels (prefill_pp.hip: one query block per
// workgroup, or a causal pair as two blocks; prefill_causal.hip: a causal pair as one stream of
// tiles): the workgroup shape, the ring depth, the online-softmax constants, and the barrier,
// wait and work-order helpers.
#pragma once

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
constexpr int kLoadWaves = 4;                       // waves per group: one group per tensor
// Groups of four waves in the ping-pong kernel (prefill_pp.hip): two at head_dim 128, three at 64,
// where a wave's softmax phase is much longer than its 16-MFMA phase and a third wave per SIMD
// keeps the matrix pipe fed while the others run their softmaxes.
template <int D>
constexpr int kPpGroups = D == 64 ? 3 : 2;
template <int D>
constexpr int kPpWavesOf = 4 * kPpGroups<D>;
template <int D>
constexpr int kPpBlockMOf = kRowsPerWave * kPpWavesOf<D>;  // 256 rows at D = 128, 384 at 64
constexpr int kXcds = 8;
constexpr float kLn2 = 0.693147180559945309f;
// Reference point of a row that has not seen a key yet: finite, so a masked score (-inf) still
// gives p = 2^(s scale_log2 - ref) = 0 and the first visible key always moves it, with no separate
// test for "no key yet".
constexpr float kNoRef = -1e30f;

// LDS ring depth (K and V slots each). A K tile is issued kStages - 1 periods before the period
// that first reads it, a V tile kStages - 2 (in the second half of its period).
#ifndef FL_PP_STAGES
#define FL_PP_STAGES 4
#endif
constexpr int kStages = FL_PP_STAGES;
static_assert(kStages == 3 || kStages == 4, "3 or 4 ring stages");
// Raise the issue priority of the wave in its MFMA phase (1) or in its softmax phase (2).
#ifndef FL_PP_SETPRIO
#define FL_PP_SETPRIO 1
#endif
// MFMAs whose A-operand fragments are in flight ahead of the one issuing. Two keep the MFMA phase
// as fast as four did and leave the registers that the peeled first and last periods need (with
// four, the kernel spilled at head_dim 128).
#ifndef FL_PP_AHEAD
#define FL_PP_AHEAD 2
#endif

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

// Waits until at most kCount of this wave's vector-memory loads are in flight.
template <int kCount>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(kCount >= 0 && kCount <= 63, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kCount) : "memory");
}

}  // namespace
}  // namespace pp
}  // namespace prefill
}  // namespace fl
