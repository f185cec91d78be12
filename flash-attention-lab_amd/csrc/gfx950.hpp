// gfx950 (CDNA4, MI355X) building blocks shared by the attention kernels: vector types, element
// conversions, the bf16/fp16 MFMA tiles the kernels use, the LDS transpose read, and 16-byte
// global loads. Nothing here is a translation of the reference's PTX wrappers (ptx.cuh); these are
// the CDNA4 instructions the kernels are built around.
//
// Fragment layouts, checked on the device by fl_mfma_tile_test and by a lane probe:
//   v_mfma_f32_32x32x16_{bf16,f16}: A[m][k] in lane m + 32 * (k / 8), element k % 8;
//     B[k][n] in lane n + 32 * (k / 8), element k % 8; D[m][n] in lane n + 32 * ((m / 4) % 2),
//     register 4 * (m / 8) + m % 4.
//   ds_read_b64_tr_b16: within each group of 16 lanes, lane i receives as element e the
//     16-bit value i % 4 of the 8 bytes addressed by lane 4 * e + i / 4 of the same group.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fl {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));

// Storage tags. bf16 and fp16 travel as raw 16-bit patterns; the tag picks conversions and the
// MFMA flavour.
struct bf16_tag {};
struct f16_tag {};
struct f32_tag {};

template <typename Tag>
struct Elem;

template <>
struct Elem<bf16_tag> {
  using storage = uint16_t;
  static __device__ __forceinline__ float to_float(uint16_t b) {
    return __uint_as_float(static_cast<uint32_t>(b) << 16);
  }
  // Round to nearest even (v_cvt_pk_bf16_f32 on gfx950).
  static __device__ __forceinline__ uint16_t from_float(float x) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(x));
  }
  // Two floats packed into one dword, lower address first.
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    return static_cast<uint32_t>(from_float(lo)) | (static_cast<uint32_t>(from_float(hi)) << 16);
  }
  static __device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};

template <>
struct Elem<f16_tag> {
  using storage = uint16_t;
  static __device__ __forceinline__ float to_float(uint16_t b) {
    return static_cast<float>(__builtin_bit_cast(_Float16, b));
  }
  static __device__ __forceinline__ uint16_t from_float(float x) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
  }
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    return static_cast<uint32_t>(from_float(lo)) | (static_cast<uint32_t>(from_float(hi)) << 16);
  }
  static __device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};

template <>
struct Elem<f32_tag> {
  using storage = float;
  static __device__ __forceinline__ float to_float(float x) { return x; }
  static __device__ __forceinline__ float from_float(float x) { return x; }
};

// 16-byte global load and store. The pointers must be 16-byte aligned (the host checks row
// alignment before any launch).
__device__ __forceinline__ u32x4 load16(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}
// Streaming variant for data read exactly once (the decode KV cache): non-temporal hint.
__device__ __forceinline__ u32x4 load16_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

// ds_read_b64_tr_b16 on an LDS address given as a generic pointer into __shared__ memory.
__device__ __forceinline__ i16x4 lds_read_tr16(const void* p) {
  typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(const_cast<void*>(p)));
}

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// Butterfly exchange with lane ^ mask through ds_bpermute (works across the 32-lane halves).
__device__ __forceinline__ float xor_lane(float v, int mask) {
  const int lane = __lane_id();
  return __int_as_float(
      __builtin_amdgcn_ds_bpermute((lane ^ mask) << 2, __float_as_int(v)));
}

}  // namespace fl
