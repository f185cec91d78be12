// Matrix-pipe rate probe: a calibration kernel for the prefill roofline, with no counterpart in
// the reference. Built into its own library (calib/libfl_calib.so, by calib/build.py), which the
// product library does not contain; bench.py --only mfma builds and loads it.
//
// C ABI:
//   int flc_mfma_rate_probe(float* out, int32_t workgroups, int32_t iters, int32_t flags,
//                           hipStream_t stream);
//   const char* flc_last_error(void);
// `workgroups` workgroups of 8 waves (two per SIMD, one workgroup per CU) each run `iters`
// iterations of 16 v_mfma_f32_32x32x16_bf16 per wave. B operands come from registers; A operands
// from registers, or with FLC_PROBE_LDS_A (2) from an LDS read per MFMA (1 KiB per wave per MFMA,
// the prefill kernel's fragment traffic). Operands are pseudo-random bf16 shaped like N(0,1)
// draws, or zeros with FLC_PROBE_ZERO_OPERANDS (1). One float per thread is written to `out`
// (workgroups * 512 floats). FLOP per call: workgroups * 8 * iters * 16 * 32768. workgroups in
// [1, 65536], iters in [1, 2^20]. Returns 0, or 1 (bad argument) / 3 (launch error) with a
// message from flc_last_error().
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "gfx950.hpp"

namespace fl {
namespace {

// 16 pseudo-random bf16 values shaped like N(0,1) draws (random sign and mantissa, exponent
// 2^-3 .. 2^1), or zeros: one MFMA operand register.
__device__ __forceinline__ u32x4 probe_operand(uint32_t seed, bool zero) {
  u32x4 v;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t word = 0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      uint32_t x = seed * 8u + 2u * i + h;
      x ^= x >> 16;
      x *= 0x7feb352du;
      x ^= x >> 15;
      x *= 0x846ca68bu;
      x ^= x >> 16;
      const uint32_t bits = ((x >> 31) << 15) | ((124u + (x >> 8) % 5u) << 7) | (x & 0x7fu);
      word |= bits << (16 * h);
    }
    v[i] = zero ? 0u : word;
  }
  return v;
}

// Chains of v_mfma_f32_32x32x16_bf16, 8 waves per workgroup (two per SIMD, as in the prefill
// kernel) and one workgroup per CU (the 96 KiB LDS array): each wave issues 16 MFMAs per iteration
// on four accumulators with B operands from four registers and A operands either from four
// registers (kLdsA false: no memory traffic, LDS or VALU work beside the MFMAs) or read from LDS
// for every MFMA (kLdsA true: 1 KiB per wave per MFMA, the prefill kernel's fragment traffic, two
// reads in flight). The matrix pipes' sustained rate under the board's power limit, which depends
// on the operands' bits (random vs zero) and on the LDS traffic beside them.
constexpr int kProbeThreads = 512;
constexpr int kProbeFrags = 96;  // 1 KiB fragments in LDS
template <bool kLdsA>
__global__ void __launch_bounds__(kProbeThreads) mfma_rate_kernel(float* __restrict__ out,
                                                                  int iters, int zero) {
  __shared__ __attribute__((aligned(16))) u32x4 frags[kProbeFrags * 64];
  const uint32_t t = blockIdx.x * kProbeThreads + threadIdx.x;
  for (int i = threadIdx.x; i < kProbeFrags * 64; i += kProbeThreads)
    frags[i] = probe_operand(blockIdx.x * (kProbeFrags * 64u) + i + (1u << 30), zero != 0);
  __syncthreads();
  u32x4 a[4], b[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    a[i] = probe_operand(t * 16u + i, zero != 0);
    b[i] = probe_operand(t * 16u + 8u + i, zero != 0);
  }
  f32x16 c[4] = {};
  // Wave w reads fragments 8w .. 8w + 17 (at most 73 < kProbeFrags).
  const int lane = threadIdx.x & 63;
  const u32x4* mine = frags + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) * 8 * 64 + lane;
  for (int it = 0; it < iters; ++it) {
    if constexpr (!kLdsA) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          c[i] = Elem<bf16_tag>::mfma32(a[(i + j) & 3], b[(i + 2 * j) & 3], c[i]);
        }
      }
    } else {
      u32x4 f[18];
      f[0] = mine[0];
      f[1] = mine[64];
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        c[k & 3] = Elem<bf16_tag>::mfma32(f[k], b[(k + (k >> 2)) & 3], c[k & 3]);
        f[k + 2] = mine[(k + 2) * 64];
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
  // One LDS word in the result keeps the array (and so one workgroup per CU) in both forms.
  float s = __uint_as_float(frags[threadIdx.x][0]) * 1e-30f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int e = 0; e < 16; ++e) s += c[i][e];
  }
  out[t] = s;
}

}  // namespace
}  // namespace fl

namespace {
thread_local std::string g_last_error;
int fail(int code, const char* message) {
  g_last_error = message;
  return code;
}
}  // namespace

extern "C" {

const char* flc_last_error(void) { return g_last_error.c_str(); }

int flc_mfma_rate_probe(float* out, int32_t workgroups, int32_t iters, int32_t flags,
                        hipStream_t stream) {
  using namespace fl;
  if (workgroups < 1 || workgroups > 65536) return fail(1, "workgroups must be in [1, 65536]");
  if (iters < 1 || iters > (1 << 20)) return fail(1, "iters must be in [1, 2^20]");
  if (flags < 0 || flags > 3) return fail(1, "unknown probe flags");
  if (!out) return fail(1, "null output pointer");
  const int zero = (flags & 1) ? 1 : 0;
  if (flags & 2) {
    hipLaunchKernelGGL(mfma_rate_kernel<true>, dim3(workgroups), dim3(kProbeThreads), 0, stream,
                       out, iters, zero);
  } else {
    hipLaunchKernelGGL(mfma_rate_kernel<false>, dim3(workgroups), dim3(kProbeThreads), 0, stream,
                       out, iters, zero);
  }
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail(3, hipGetErrorString(err));
  return 0;
}

}  // extern "C"
