// Fragment-level pieces of the prefill kernel, shared with the MFMA tile test so the lane
// layouts are checked in isolation.
//
// Each wave owns 32 query rows. Scores are computed transposed, S^T = K Q^T, on
// v_mfma_f32_32x32x16: K (keys x dims) is the A operand read from LDS, Q^T the B operand held in
// registers for the whole kernel. In the accumulator layout lane l then holds query row l % 32
// and 16 of the 32 keys of a key block, the other 16 being in lane l ^ 32; a row's max and sum
// need one exchange between the two halves of the wave and no other cross-lane traffic.
//
// The output is accumulated transposed too, O^T = V^T P^T, so lane l keeps query row l % 32 and
// the per-row rescale is a per-lane multiply. P^T is the B operand: lane l must supply 8 keys of
// its own row, and it supplies exactly the ones it holds. For key step kk (16 keys) the B
// operand's k index 8 * half + 4 * a + b (half = l / 32) is key 16 * kk + 8 * a + 4 * half + b,
// which are accumulator registers 8 * (kk % 2) + 0..7 of key block kk / 2. V^T, the A operand,
// is read with that same key order: two ds_read_b64_tr_b16 per operand, each returning 4
// consecutive keys of one column.
#pragma once

#include "gfx950.hpp"

namespace fl::prefill {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kRowsPerWave = 32;
constexpr int kBlockM = kRowsPerWave * kWaves;  // query rows per workgroup
constexpr int kBlockN = 64;                     // keys per tile

// LDS tiles hold 64 rows of D elements with no padding. Within a row, 16-byte chunk c is stored
// at chunk c ^ swz(r), an XOR swizzle chosen so that both LDS read patterns of the kernel are free
// of bank conflicts on gfx950's 64 banks x 4 bytes (256 bytes per cycle):
//  * K operand (ds_read_b128): 16 lanes read 16 consecutive rows at one logical chunk; swz is a
//    bijection on each run of 16 rows, so they hit 16 distinct chunk positions.
//  * V operand (ds_read_b64_tr_b16): 32 lanes read 4 consecutive rows x 4 chunks (an aligned
//    group 4g..4g+3); swz moves each of the 4 rows to a different aligned group.
// At D = 64 two rows share a 256-byte bank window, so the row parity takes part.
template <int D>
constexpr int kPitch = D;
template <int D>
constexpr int kTileElems = kBlockN * kPitch<D>;

template <int D>
__device__ __forceinline__ constexpr int swz(int r) {
  return D == 128 ? 4 * (r & 3) + ((r >> 2) & 3) : 4 * ((r >> 1) & 1) + ((r >> 2) & 3);
}

// Element offset of (row, col) in a swizzled tile.
template <int D>
__device__ __forceinline__ constexpr int tile_offset(int r, int col) {
  return r * kPitch<D> + 8 * ((col >> 3) ^ swz<D>(r)) + (col & 7);
}

// Byte offset in a tile of lane l's K operand piece for dim step ks: row l % 32, dims
// 16 ks + 8 (l / 32) .. + 7 (key block mb adds 32 rows, a fixed offset since swz(r + 32) = swz(r)).
template <int D>
__device__ __forceinline__ int k_lane_offset(int ks, int lane) {
  return 2 * tile_offset<D>(lane & 31, 16 * ks + 8 * (lane >> 5));
}
template <int D>
constexpr int kKeyBlockBytes = 32 * kPitch<D> * 2;

// Byte offset of lane l's first transpose read of the V operand for dim block nb (the second read,
// 8 rows further, is `hi`). Within each 16-lane group, lane i addresses row i / 4 and columns
// 4 (i % 4) .. + 3 of a 4 x 16 block (8 contiguous bytes, which the swizzle keeps together), so
// that the transpose read hands lane i column i of all 4 rows. Key step kk adds 16 rows, a fixed
// offset since swz(r + 16) = swz(r).
template <int D>
__device__ __forceinline__ int v_lane_offset(int nb, int hi, int lane) {
  const int i = lane & 15;
  const int r = 4 * (lane >> 5) + (i >> 2) + 8 * hi;
  const int col = 32 * nb + 16 * ((lane >> 4) & 1) + 4 * (i & 3);
  return 2 * tile_offset<D>(r, col);
}
template <int D>
constexpr int kKeyStepBytes = 16 * kPitch<D> * 2;

__device__ __forceinline__ u32x4 lds_load16(const void* base, int byte_offset) {
  return *reinterpret_cast<const u32x4*>(static_cast<const char*>(base) + byte_offset);
}

// A operand of S^T += K Q^T for key block mb (32 keys) and dim step ks (16 dims):
// lane l reads K[32 mb + l % 32][16 ks + 8 (l / 32) .. + 7], one 16-byte LDS read.
template <int D>
__device__ __forceinline__ u32x4 k_frag(const uint16_t* k_tile, int mb, int ks, int lane) {
  return lds_load16(k_tile, mb * kKeyBlockBytes<D> + k_lane_offset<D>(ks, lane));
}

// A operand of O^T += V^T P^T for dim block nb (32 dims) and key step kk (16 keys): lane l needs
// V[16 kk + 4 half + e][32 nb + l % 32] for e = 0..3, then the same for the 4 keys 8 rows on.
__device__ __forceinline__ u32x4 v_frag_at(const void* v_tile, int lo_offset, int hi_offset) {
  const u32x2 lo = __builtin_bit_cast(u32x2, lds_read_tr16(static_cast<const char*>(v_tile) + lo_offset));
  const u32x2 hi = __builtin_bit_cast(u32x2, lds_read_tr16(static_cast<const char*>(v_tile) + hi_offset));
  return u32x4{lo.x, lo.y, hi.x, hi.y};
}
template <int D>
__device__ __forceinline__ u32x4 v_frag(const uint16_t* v_tile, int nb, int kk, int lane) {
  return v_frag_at(v_tile, kk * kKeyStepBytes<D> + v_lane_offset<D>(nb, 0, lane),
                   kk * kKeyStepBytes<D> + v_lane_offset<D>(nb, 1, lane));
}

// B operand of O^T += V^T P^T for key step kk from the probabilities of key block kk / 2:
// registers 8 * (kk % 2) .. + 7, rounded to the input type.
template <typename Tag, int kHalf>
__device__ __forceinline__ u32x4 p_frag(const f32x16& s) {
  using E = Elem<Tag>;
  constexpr int j = 8 * kHalf;
  return u32x4{E::pack2(s[j], s[j + 1]), E::pack2(s[j + 2], s[j + 3]), E::pack2(s[j + 4], s[j + 5]),
               E::pack2(s[j + 6], s[j + 7])};
}

// Key offset within a 32-key block of accumulator register j in a lane of the given half.
__device__ __forceinline__ constexpr int acc_key(int j, int half) {
  return 8 * (j >> 2) + 4 * half + (j & 3);
}

// Online softmax reference point of a row (log2 units; o and l are kept relative to it): it moves
// to the row's running max when a tile's max passes it by more than kMoveSlack, so every
// probability is at most 2^kMoveSlack, and the key that set it has p = 1 exactly. What this
// trades: a key's p is rounded to the input type (2^-8 relative in bf16) unless it is exactly a
// power of two, and the reference's exact running max keeps the largest key of a row at p = 1,
// exact, whatever its share of the row. A point that moved only when a lane's probabilities summed
// past 2^15 left a dominant key that arrives after the point at p >> 1 and rounded; on a row where
// one key holds 16% of the weight that was 1.8e-3 of error before the output rounding, against
// 2.5e-4 with the exact max, and broke the reference's tolerance. With a slack of 3 a key stays
// rounded only while it is within 8x of the weight of the exact key that set the point, and a key
// that dominates its row moves it. In CPU emulations of this arithmetic (randn inputs at three
// score scales, and rows with a planted dominant key at a random position) slacks 0 to 3 gave the
// exact max's error to within 10% and the 2^15 rule up to 1.7x of it. Cost against the 2^15 rule,
// headline shape: slack 0 (the exact max: a new max in any of a wave's 32 rows on 42 of 64 tiles,
// each a 64-multiply rescale of o, and the workgroup barrier makes every wave wait for the
// slowest) -17%; slack 1 -8% / -12% (non-causal / causal); 2 -4% / -6%; 3 -3.5% / -3%.
constexpr float kMoveSlack = 3.f;

// Max of the 32 scores a lane holds (a tile's 64 keys of its row, split with the other half),
// as 16 three-input maxes.
__device__ __forceinline__ float max_of(const f32x16& x, const f32x16& y) {
  float t[12];
#pragma unroll
  for (int i = 0; i < 5; ++i) t[i] = max3_f32(x[3 * i], x[3 * i + 1], x[3 * i + 2]);
#pragma unroll
  for (int i = 0; i < 5; ++i) t[5 + i] = max3_f32(y[3 * i], y[3 * i + 1], y[3 * i + 2]);
  t[10] = x[15];
  t[11] = y[15];
  const float u0 = max3_f32(t[0], t[1], t[2]);
  const float u1 = max3_f32(t[3], t[4], t[5]);
  const float u2 = max3_f32(t[6], t[7], t[8]);
  const float u3 = max3_f32(t[9], t[10], t[11]);
  return max2_f32(max3_f32(u0, u1, u2), u3);
}

}  // namespace fl::prefill
