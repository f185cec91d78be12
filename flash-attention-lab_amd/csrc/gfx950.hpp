// gfx950 (CDNA4, MI355X) building blocks shared by the attention kernels: vector types, element
// conversions, the bf16/fp16 MFMA tiles the kernels use, the LDS transpose read, and 16-byte
// global loads. Nothing here is a translation of the reference's PTX wrappers (ptx.cuh); these are
// the CDNA4 instructions the kernels are built around.
//
// Fragment layouts, checked on the device by fl_mfma_tile_test and by a lane probe:
//   v_mfma_f32_32x32x16_{bf16,f16}: A[m][k] in lane m + 32 * (k / 8), element k % 8;
//     B[k][n] in lane n + 32 * (k / 8), element k % 8; D[m][n] in lane n + 32 * ((m / 4) % 2),
//     register 4 * (m / 8) + m % 4.
//   v_mfma_f32_16x16x32_{bf16,f16}: A[m][k] in lane m + 16 * (k / 8), element k % 8;
//     B[k][n] in lane n + 16 * (k / 8), element k % 8; D[m][n] in lane n + 16 * (m / 4),
//     register m % 4. (Not covered by fl_mfma_tile_test: the head_dim 64 prefill takes every row
//     sum with it, so the prefill parity tests at head_dim 64 pin it; tests/test_row_sum_layout.py
//     checks the row-sum selector against this layout on the CPU.)
//   ds_read_b64_tr_b16: within each group of 16 lanes, lane i receives as element e the
//     16-bit value i % 4 of the 8 bytes addressed by lane 4 * e + i / 4 of the same group.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace fl {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
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
  // Two floats packed into one dword, lower address first (one v_cvt_pk_bf16_f32, RNE).
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
  }
  static __device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  static constexpr uint32_t kOnePair = 0x3F803F80u;  // {1.0, 1.0}
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
  // One v_cvt_pk_f16_f32 (RNE).
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, f16x2));
  }
  static __device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  static constexpr uint32_t kOnePair = 0x3C003C00u;  // {1.0, 1.0}
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

// Buffer resource over `bytes` bytes from `base` (raw addressing, no stride). A buffer load whose
// offset is at or past `bytes` returns zeros without touching memory, which is how tile loads past
// the end of a sequence are zero-filled without branches.
constexpr int kBufferRsrcWord3 = 0x00020000;  // gfx9-family raw buffer configuration
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, kBufferRsrcWord3);
}
// buffer_load_dwordx4 ... lds: each lane's 16 bytes go to LDS at `lds_block` + 16 * lane (the
// block address is wave-uniform); offsets past the resource write zeros.
__device__ __forceinline__ void buffer_load16_to_lds(__amdgpu_buffer_rsrc_t rsrc, void* lds_block,
                                                     int offset) {
  typedef __attribute__((address_space(3))) void lds_void;
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void*)(lds_block), 16, offset, 0, 0, 0);
}

// The same load issued from inline assembly: the compiler does not see it, so it inserts no
// waits of its own for later LDS reads. The caller orders it with explicit s_waitcnt vmcnt and
// barriers. `words` is a raw buffer resource (base, num_records, kBufferRsrcWord3), `lds_addr` the
// wave-uniform LDS byte address of the 1 KiB block (lane l writes 16 bytes at lds_addr + 16 l).
typedef uint32_t u32x4s __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x4s buffer_words(const void* base, uint32_t bytes) {
  const uint64_t addr = reinterpret_cast<uint64_t>(base);
  return u32x4s{static_cast<uint32_t>(addr), static_cast<uint32_t>(addr >> 32) & 0xffffu, bytes,
                static_cast<uint32_t>(kBufferRsrcWord3)};
}
__device__ __forceinline__ void buffer_load16_to_lds_asm(u32x4s words, uint32_t lds_addr,
                                                         int offset) {
  // The address and resource are wave-uniform by contract; readfirstlane makes that explicit to
  // the compiler so they are always given scalar registers (a no-op when they already are).
  auto uniform = [](uint32_t x) {
    return static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(x)));
  };
  const u32x4s w{uniform(words[0]), uniform(words[1]), uniform(words[2]), uniform(words[3])};
  const uint32_t m0 = uniform(lds_addr);
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %2, 0 offen lds"
               :
               : "v"(offset), "s"(m0), "s"(w)
               : "memory", "m0");
}
// 32-bit LDS address of a __shared__ object.
__device__ __forceinline__ uint32_t lds_address(const void* p) {
  typedef __attribute__((address_space(3))) const void lds_cvoid;
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_cvoid*)(p)));
}

// True on every lane when `pred` holds on any active lane (a wave-uniform branch condition).
__device__ __forceinline__ bool wave_any(bool pred) {
  return __builtin_amdgcn_ballot_w64(pred) != 0;
}

// ds_read_b64_tr_b16 on an LDS address given as a generic pointer into __shared__ memory.
__device__ __forceinline__ i16x4 lds_read_tr16(const void* p) {
  typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(const_cast<void*>(p)));
}

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// DPP lane moves within rows of 16 lanes (pure VALU, no LDS traffic).
template <int kCtrl>
__device__ __forceinline__ float dpp_move(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kCtrl, 0xF, 0xF, false));
}
constexpr int kDppQuadSwap1 = 0xB1;     // quad_perm [1, 0, 3, 2]: lane ^ 1
constexpr int kDppQuadSwap2 = 0x4E;     // quad_perm [2, 3, 0, 1]: lane ^ 2
constexpr int kDppRowHalfMirror = 0x141;  // lane i <- lane 7 - i within each 8
constexpr int kDppRowMirror = 0x140;      // lane i <- lane 15 - i within each 16

// Sum over aligned groups of kLanes lanes (4, 8, 16, 32 or 64); every lane of a group gets the
// same bits (each step adds a pair of equal partial sums in either order).
template <int kLanes>
__device__ __forceinline__ float group_sum(float x) {
  static_assert(kLanes == 4 || kLanes == 8 || kLanes == 16 || kLanes == 32 || kLanes == 64, "");
  x += dpp_move<kDppQuadSwap1>(x);
  x += dpp_move<kDppQuadSwap2>(x);
  if constexpr (kLanes >= 8) x += dpp_move<kDppRowHalfMirror>(x);
  if constexpr (kLanes >= 16) x += dpp_move<kDppRowMirror>(x);
  if constexpr (kLanes >= 32) x += __shfl_xor(x, 16);
  if constexpr (kLanes >= 64) x += __shfl_xor(x, 32);
  return x;
}

// Maxes the compiler turns into v_maximum3_f32, gfx950's NaN-propagating maximum (IEEE 754-2019
// `maximum`). fmaxf's NaN-ignoring semantics cost a self-max (NaN quieting) on every operand the
// compiler cannot prove quiet, such as a value read back from another lane; here a NaN can only
// come from NaN inputs, which give a NaN output either way. (Not inline assembly: an asm statement
// that reads an MFMA result is invisible to the compiler's wait-state insertion for the
// MFMA -> VALU read hazard.)
__device__ __forceinline__ float max2_f32(float a, float b) { return __builtin_elementwise_maximum(a, b); }
__device__ __forceinline__ float max3_f32(float a, float b, float c) {
  return __builtin_elementwise_maximum(__builtin_elementwise_maximum(a, b), c);
}

// max(x[l], x[l ^ 32]) and x[l] + x[l ^ 32] on every lane: one v_permlane32_swap (lanes 32-63 of
// the first result and lanes 0-31 of the second are the other half's values).
__device__ __forceinline__ float max_halves(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return max2_f32(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_halves(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// f(integral_constant<int, i>) for i = I .. N - 1, unrolled at compile time.
template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

// Butterfly exchange with lane ^ mask through ds_bpermute (works across the 32-lane halves).
__device__ __forceinline__ float xor_lane(float v, int mask) {
  const int lane = __lane_id();
  return __int_as_float(
      __builtin_amdgcn_ds_bpermute((lane ^ mask) << 2, __float_as_int(v)));
}

}  // namespace fl
