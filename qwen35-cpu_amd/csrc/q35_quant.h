// Device routine shared by every kernel that prepares projection inputs: the
// randomized-sign Hadamard-128 rotation and per-32 int8 quantization of one
// 128-column block of one token, and the stores of the result in the layouts
// the DOT4 GEMM (A16) and the reference kernels (X4/X1) read.
//
// Reference semantics (bit-exact given the same FP32 input):
//   signs + FWHT stage order 1,2,...,64     src/cpu/q4_h128.cpp:35-61
//   absmax/127, unrounded 1/scale, round half away from zero, clamp +-127,
//   stored scale = binary16(scale) * 1/sqrt(128)   q4_0.cpp:212-235, q4_h128.cpp:319-321
// With h128 == false it is the identity-basis quantizer q8_0_quantize_vector_1
// (q4_0.cpp:212-235).
//
// Layout: a 16-lane row of the wavefront holds the block, lane j = lane % 16
// holding columns 8j .. 8j+7. FWHT strides 1, 2, 4 run in registers and
// strides 8, 16, 32, 64 exchange with lane j^1, j^2, j^4, j^8 through DPP row
// moves, in the reference's stage order with the reference's (a+b, a-b)
// butterflies; a 32-column group is four lanes, so its absmax and code sum
// finish with two quad exchanges, and each lane's eight codes are exactly
// one A16 word (token t, k-group j % 4 of block 4*blk + j/4).
#pragma once

#include "q35_device.h"
#include "q35_internal.h"

namespace q35 {

struct QuantOut {
  uint64_t *codes = nullptr;        // A16 [token_tile][nb][64]
  float *scales = nullptr;          // [token_tile][nb][16]
  q35_q8_0_block_x4 *x4 = nullptr;  // reference X4 layout (optional)
  q35_q8_0_block_x1 *x1 = nullptr;  // reference X1 layout (optional)
};

// Int8 quantization of one 32-value block held by four consecutive lanes,
// eight values each (q8_0_quantize_vector_1, q4_0.cpp:212-235): absmax over
// the block, scale = absmax / 127, codes round(x / scale) clamped to +-127
// (packed little-endian into `word`), the block's code sum, and the
// binary16-rounded scale as stored. Every lane of the row calls it. (The
// same steps as the quantization in h128_quantize_row16, kept separate so
// that the hot preparation kernels compile as they are.)
__device__ __forceinline__ void q8_block_codes8(const float v[8], uint64_t &word, int &sum, float &stored) {
  float amax = 0.0F;
#pragma unroll
  for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(v[e]));
  amax = fmaxf(amax, q35_row_xor(amax, 1));
  amax = fmaxf(amax, q35_row_xor(amax, 2));
  const float scale = amax / 127.0F;
  const float inv = scale == 0.0F ? 0.0F : 1.0F / scale;
  word = 0;
  sum = 0;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float r = roundf(v[e] * inv);
    r = fminf(fmaxf(r, -127.0F), 127.0F);
    const int code = static_cast<int>(r);
    sum += code;
    word |= static_cast<uint64_t>(static_cast<uint8_t>(static_cast<int8_t>(code))) << (8 * e);
  }
  sum += q35_row_xor_i(sum, 1);
  sum += q35_row_xor_i(sum, 2);
  stored = half_bits_to_float(float_to_half_bits(scale));
}

// The rotation and quantization of one (token, 128-column block) item held
// by L lanes (L = 16, 32 or 64), lane j = lane % L holding the V = 128 / L
// columns V*j .. V*j+V-1: `bits` receives the lane's V int8 codes (bytes
// V*j % 8 .. of one A16 word: k-group (V*j % 32) / 8 of block 4*blk + V*j/32),
// `sum` their 32-column block's code sum and `stored` that block's
// binary16-rounded scale (times 1/sqrt(128) in the H128 basis). The FWHT runs
// its strides 1 .. V/2 in registers and V .. 64 as exchanges with lane j^1 ..
// j^(L/2), every stage with the reference's (a + b, a - b) butterflies, so
// each value sees the same additions whatever L is: the codes and scales do
// not depend on L, and a kernel picks the L that keeps its lanes busy. All 64
// lanes of the wavefront call it (the exchanges need every lane).
template <int L>
__device__ __forceinline__ void h128_quantize_core_l(float v[128 / L], int blk, bool h128, uint64_t seed,
                                                     uint64_t &bits, int &sum, float &stored) {
  static_assert(L == 16 || L == 32 || L == 64, "16, 32 or 64 lanes per item");
  constexpr int V = 128 / L, G = 32 / V;  // values per lane, lanes per 32-column block
  const int j = __lane_id() & (L - 1), c0 = V * j;
  if (h128) {
    const uint64_t w = h128_sign_word(blk, c0 >> 6, seed);
    const unsigned sb = static_cast<unsigned>(w >> (c0 & 63));
#pragma unroll
    for (int e = 0; e < V; ++e)
      if ((sb >> e) & 1u) v[e] = -v[e];
#pragma unroll
    for (int s = 1; s < V; s <<= 1)
#pragma unroll
      for (int e = 0; e < V; ++e)
        if (!(e & s)) {
          const float a = v[e], b = v[e + s];
          v[e] = a + b;
          v[e + s] = a - b;
        }
    // the partner's value p: a lower lane keeps v + p, an upper lane p - v,
    // both as one exact fma(v, +-1, p)
#pragma unroll
    for (int m = 1; m < L; m <<= 1) {
      const float sgn = (j & m) != 0 ? -1.0F : 1.0F;
#pragma unroll
      for (int e = 0; e < V; ++e) v[e] = fmaf(v[e], sgn, q35_lane_xor(v[e], m));
    }
  }
  float amax = 0.0F;
#pragma unroll
  for (int e = 0; e < V; ++e) amax = fmaxf(amax, fabsf(v[e]));
#pragma unroll
  for (int m = 1; m < G; m <<= 1) amax = fmaxf(amax, q35_row_xor(amax, m));
  const float scale = amax / 127.0F;
  const float inv = scale == 0.0F ? 0.0F : 1.0F / scale;
  bits = 0;
  sum = 0;
#pragma unroll
  for (int e = 0; e < V; ++e) {
    float r = roundf(v[e] * inv);
    r = fminf(fmaxf(r, -127.0F), 127.0F);
    const int code = static_cast<int>(r);
    sum += code;
    bits |= static_cast<uint64_t>(static_cast<uint8_t>(static_cast<int8_t>(code))) << (8 * e);
  }
#pragma unroll
  for (int m = 1; m < G; m <<= 1) sum += q35_row_xor_i(sum, m);
  stored = half_bits_to_float(float_to_half_bits(scale));
  if (h128) stored *= kH128InvSqrt;
}

__device__ __forceinline__ void h128_quantize_core(float v[8], int blk, bool h128, uint64_t seed, uint64_t &word,
                                                   int &sum, float &stored) {
  h128_quantize_core_l<16>(v, blk, h128, seed, word, sum, stored);
}

// V code bytes at p (aligned to V bytes).
template <int V>
__device__ __forceinline__ void store_code_bytes(uint8_t *p, uint64_t bits) {
  if constexpr (V == 8)
    *reinterpret_cast<uint64_t *>(p) = bits;
  else if constexpr (V == 4)
    *reinterpret_cast<uint32_t *>(p) = static_cast<uint32_t>(bits);
  else
    *reinterpret_cast<uint16_t *>(p) = static_cast<uint16_t>(bits);
}

// One item per L lanes (h128_quantize_core_l) and the stores of its codes and
// scales; all 64 lanes call it, items whose `active` is false store nothing.
template <int L>
__device__ __forceinline__ void h128_quantize_lanes(float v[128 / L], int t, int blk, int nb, bool h128,
                                                    uint64_t seed, const QuantOut &o, bool active) {
  constexpr int V = 128 / L;
  const int c0 = V * (__lane_id() & (L - 1));
  uint64_t bits;
  int sum;
  float stored;
  h128_quantize_core_l<L>(v, blk, h128, seed, bits, sum, stored);
  if (!active) return;
  const int b = blk * 4 + (c0 >> 5), kg = (c0 & 31) >> 3, byte0 = c0 & 7;
  const bool first = (c0 & 31) == 0;  // the 32-column block's first lane
  const int tile = t >> 4, tok = t & 15;
  if (o.codes != nullptr) {
    store_code_bytes<V>(reinterpret_cast<uint8_t *>(o.codes + (static_cast<size_t>(tile) * nb + b) * 64 + tok + 16 * kg) +
                            byte0,
                        bits);
    if (first) o.scales[(static_cast<size_t>(tile) * nb + b) * 16 + tok] = stored;
  }
  if (o.x4 != nullptr) {
    q35_q8_0_block_x4 &bx = o.x4[static_cast<size_t>(t >> 2) * nb + b];
    store_code_bytes<V>(reinterpret_cast<uint8_t *>(&bx.qs[(t & 3) * 32 + (c0 & 31)]), bits);
    if (first) {
      bx.scales[t & 3] = stored;
      bx.sums[t & 3] = static_cast<int16_t>(sum);
    }
  }
  if (o.x1 != nullptr) {
    q35_q8_0_block_x1 &b1 = o.x1[static_cast<size_t>(t) * nb + b];
    uint8_t *q = reinterpret_cast<uint8_t *>(b1.qs) + (c0 & 31);
#pragma unroll
    for (int e = 0; e < V; ++e) q[e] = static_cast<uint8_t>(bits >> (8 * e));
    if (first) {
      b1.scales[0] = stored;
      b1.sums[0] = static_cast<int16_t>(sum);
      b1.pad = 0;
    }
  }
}

__device__ __forceinline__ void h128_quantize_row16(float v[8], int t, int blk, int nb, bool h128, uint64_t seed,
                                                    const QuantOut &o, bool active) {
  h128_quantize_lanes<16>(v, t, blk, nb, h128, seed, o, active);
}

}  // namespace q35
