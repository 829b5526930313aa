// Device-side helpers shared by the gfx950 kernels (64-lane wavefronts).
#pragma once

#include "q35_hip_api.h"

#include <cstdint>

namespace q35 {

__device__ __forceinline__ float half_bits_to_float(uint16_t h) {
  return __half2float(__ushort_as_half(h));
}
// Round to nearest even, as float_to_half (src/cpu/q8_0.cpp:18-55) for finite values.
// The value is pinned in an fp32 register first: otherwise the compiler may
// fold the multiply that produced it into the conversion (v_fma_mixlo_f16,
// which rounds the exact product to binary16 once), and the result would
// depend on the surrounding code instead of on the fp32 value.
__device__ __forceinline__ uint16_t float_to_half_bits(float f) {
  q35_materialize(f);
  return __half_as_ushort(__float2half_rn(f));
}

// Q4 DOT4 GEMMs: int8 -8 in every byte (the offset-binary correction
// operand), and a body word of a Q4_0BlockX8 tile (eight nibbles: columns
// j and j + 4 of one row) unpacked to eight int8 values, low nibbles first.
constexpr long kMinus8 = static_cast<long>(0xF8F8F8F8F8F8F8F8ull);
__device__ __forceinline__ long unpack_word(uint32_t w) {
  const uint32_t lo = w & 0x0f0f0f0fu;
  const uint32_t hi = (w >> 4) & 0x0f0f0f0fu;
  return static_cast<long>((static_cast<uint64_t>(hi) << 32) | lo);
}

// Stores four consecutive rows of one token (vectorized when `vec`).
__device__ __forceinline__ void store_row4(float *dst, bool vec, float v0, float v1, float v2, float v3) {
  if (vec) {
    *reinterpret_cast<q35_f32x4 *>(dst) = q35_f32x4{v0, v1, v2, v3};
  } else {
    dst[0] = v0;
    dst[1] = v1;
    dst[2] = v2;
    dst[3] = v3;
  }
}

// Row words of a DOT4 tile for a lane covering RM consecutive rows
// (RM = 1 or 2): the lane's body word(s) and binary16 row scale(s).
template <int RM>
struct RowWords;
template <>
struct RowWords<1> {
  typedef uint32_t Q;
  typedef uint16_t D;
  static __device__ __forceinline__ uint32_t word(const Q &q, int) { return q; }
  static __device__ __forceinline__ uint16_t scale(const D &d, int) { return d; }
};
template <>
struct RowWords<2> {
  typedef q35_u32x2 Q;
  typedef uint32_t D;
  static __device__ __forceinline__ uint32_t word(const Q &q, int i) { return q[i]; }
  static __device__ __forceinline__ uint16_t scale(const D &d, int i) { return static_cast<uint16_t>(d >> (16 * i)); }
};
template <>
struct RowWords<4> {
  typedef q35_u32x4 Q;
  typedef q35_u32x2 D;
  static __device__ __forceinline__ uint32_t word(const Q &q, int i) { return q[i]; }
  static __device__ __forceinline__ uint16_t scale(const D &d, int i) {
    return static_cast<uint16_t>(d[i >> 1] >> (16 * (i & 1)));
  }
};
// XOR-butterfly reductions over groups of `Width` lanes (Width <= 64, power of 2).
template <int Width>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int m = Width / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}
template <int Width>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
  for (int m = Width / 2; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}
template <int Width>
__device__ __forceinline__ int group_sum_int(int v) {
#pragma unroll
  for (int m = Width / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

// Sum over each 16-lane DPP row, every lane of the row getting the total:
// the butterfly xor 1, 2, 4, 8. After the xor 1 and xor 2 steps all four
// lanes of a quad hold the same partial, so the xor-4 step takes the other
// quad's partial from the mirror lane (7 - i inside each half row): the value
// the xor-4 exchange brings, added in the same operand order, through one DPP
// add instead of two DPP moves and a select.
__device__ __forceinline__ float row_sum16(float v) {
  v += q35_row_xor(v, 1);
  v += q35_row_xor(v, 2);
  v += q35_row_half_mirror(v);
  return v + q35_row_xor(v, 8);
}

// Wavefront-wide sum: the 16-lane row sums, then the two cross-row steps;
// every lane gets the total.
__device__ __forceinline__ float wave_sum(float v) {
  v = row_sum16(v);
  v += __shfl_xor(v, 16, 64);
  v += __shfl_xor(v, 32, 64);
  return v;
}

// Sum over a whole workgroup of `Waves` wavefronts; every thread gets the result.
template <int Waves>
__device__ __forceinline__ float block_sum(float v, float *scratch) {
  v = group_sum<64>(v);
  const int wave = threadIdx.x >> 6;
  lds_barrier();  // an earlier call's readers are done with scratch
  if ((threadIdx.x & 63) == 0) scratch[wave] = v;
  lds_barrier();
  float total = 0.0F;
#pragma unroll
  for (int w = 0; w < Waves; ++w) total += scratch[w];
  return total;
}

// The RMSNorm's sum of squares, one tree shared by every kernel that
// normalizes a residual row (so their norms round identically): the squares
// x*x are summed per 16-column group as a butterfly over the columns in lane
// order (exchanges xor 1, 2, 4, 8), then lane l of one wavefront takes the
// group sums l, l + 64, l + 128, ... in order and wave_sum adds the lanes.
//
// A group held by four consecutive lanes, lane k with columns 4k..4k+3 (the
// xor 1, 2 steps in registers, xor 4, 8 as lane exchanges 1, 2):
__device__ __forceinline__ float sq_group16_quad(q35_f32x4 v) {
#pragma clang fp contract(off)
  const float s0 = v[0] * v[0], s1 = v[1] * v[1], s2 = v[2] * v[2], s3 = v[3] * v[3];
  float s = (s0 + s1) + (s2 + s3);
  s += q35_row_xor(s, 1);
  s += q35_row_xor(s, 2);
  return s;
}
// A group held by sixteen consecutive lanes (one DPP row), one column each:
__device__ __forceinline__ float sq_group16_lanes(float x) {
#pragma clang fp contract(off)
  return row_sum16(x * x);
}
// The row total from its n group sums (every lane of one wavefront calls it).
__device__ __forceinline__ float norm_total_groups(const float *gp, int n) {
  const int l = threadIdx.x & 63;
  float v = l < n ? gp[l] : 0.0F;
  for (int g = l + 64; g < n; g += 64) v += gp[g];
  return wave_sum(v);
}

// splitmix64 sign words of the randomized-sign H128 basis (src/cpu/q4_h128.cpp:16-33).
__device__ __forceinline__ uint64_t splitmix64(uint64_t v) {
  v += 0x9e3779b97f4a7c15ull;
  v = (v ^ (v >> 30)) * 0xbf58476d1ce4e5b9ull;
  v = (v ^ (v >> 27)) * 0x94d049bb133111ebull;
  return v ^ (v >> 31);
}
__device__ __forceinline__ uint64_t h128_sign_word(uint64_t block, uint64_t word, uint64_t seed) {
  return splitmix64(seed + block * 0x9e3779b97f4a7c15ull + word * 0xd1b54a32d192ed03ull);
}

// Logistic functions with the reference's branch structure
// (src/runtime/weights.inl:656-678, src/cpu/activation.cpp:329-357).
__device__ __forceinline__ float sigmoid_stable(float x) {
  if (x >= 0.0F) return 1.0F / (1.0F + expf(-x));
  const float z = expf(x);
  return z / (1.0F + z);
}
__device__ __forceinline__ float silu_times(float g, float u) {
  const float e = expf(-fabsf(g));
  const float s = g >= 0.0F ? 1.0F / (1.0F + e) : e / (1.0F + e);
  return g * s * u;
}
__device__ __forceinline__ float softplus_stable(float x) {
  if (x > 20.0F) return x;
  if (x < -20.0F) return expf(x);
  return log1pf(expf(x));
}

// Monotone 64-bit key: larger value first, then lower index (ties go to the
// lowest token, src/runtime/cpu_engine_greedy.inl:53-56).
__device__ __forceinline__ unsigned long long argmax_key(float value, uint32_t index) {
  uint32_t u = __float_as_uint(value);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return (static_cast<unsigned long long>(u) << 32) | static_cast<uint32_t>(0xffffffffu - index);
}
__device__ __forceinline__ float argmax_key_value(unsigned long long key) {
  uint32_t u = static_cast<uint32_t>(key >> 32);
  u = (u & 0x80000000u) ? (u & 0x7fffffffu) : ~u;
  return __uint_as_float(u);
}
__device__ __forceinline__ uint32_t argmax_key_index(unsigned long long key) {
  return 0xffffffffu - static_cast<uint32_t>(key & 0xffffffffu);
}

}  // namespace q35
