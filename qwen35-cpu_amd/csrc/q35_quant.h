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
#pragma once

#include "q35_device.h"
#include "q35_internal.h"

namespace q35 {

struct QuantOut {
  uint64_t *codes = nullptr;        // A16 [token_tile][nb][64]
  float *scales = nullptr;       // [token_tile][nb][16]
  q35_q8_0_block_x4 *x4 = nullptr;  // reference X4 layout (optional)
  q35_q8_0_block_x1 *x1 = nullptr;  // reference X1 layout (optional)
};

// One wavefront holds the block as v0 = column lane, v1 = column 64 + lane of
// 128-column block `blk` of token t (nb = 32-column blocks per row).
__device__ __forceinline__ void h128_quantize_block(float v0, float v1, int lane, int t, int blk, int nb,
                                                    bool h128, uint64_t seed, const QuantOut &o) {
  if (h128) {
    const uint64_t w0 = h128_sign_word(blk, 0, seed), w1 = h128_sign_word(blk, 1, seed);
    if ((w0 >> lane) & 1ull) v0 = -v0;
    if ((w1 >> lane) & 1ull) v1 = -v1;
#pragma unroll
    for (int s = 1; s < 64; s <<= 1) {
      const float p0 = __shfl_xor(v0, s, 64), p1 = __shfl_xor(v1, s, 64);
      if (lane & s) {
        v0 = p0 - v0;
        v1 = p1 - v1;
      } else {
        v0 = v0 + p0;
        v1 = v1 + p1;
      }
    }
    const float lhs = v0;
    v0 = lhs + v1;
    v1 = lhs - v1;
  }
  const int tile = t >> 4, tok = t & 15;
  // Two 32-value groups per value slot: group(v0) = lane/32, group(v1) = 2 + lane/32.
  const float vals[2] = {v0, v1};
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    const float v = vals[half];
    const float amax = group_max<32>(fabsf(v));
    const float scale = amax / 127.0F;
    const float inv = scale == 0.0F ? 0.0F : 1.0F / scale;
    float r = roundf(v * inv);
    r = fminf(fmaxf(r, -127.0F), 127.0F);
    const int code = static_cast<int>(r);
    const int sum = group_sum_int<32>(code);
    float stored = half_bits_to_float(float_to_half_bits(scale));
    if (h128) stored *= kH128InvSqrt;
    const int b = blk * 4 + half * 2 + (lane >> 5);
    const int k = lane & 31;
    if (o.codes != nullptr) {
      uint8_t *dst = reinterpret_cast<uint8_t *>(o.codes);
      const size_t word = (static_cast<size_t>(tile) * nb + b) * 64 + tok + 16 * (k >> 3);
      dst[word * 8 + (k & 7)] = static_cast<uint8_t>(static_cast<int8_t>(code));
      if (k == 0) o.scales[(static_cast<size_t>(tile) * nb + b) * 16 + tok] = stored;
    }
    if (o.x4 != nullptr) {
      q35_q8_0_block_x4 &blkx = o.x4[static_cast<size_t>(t >> 2) * nb + b];
      blkx.qs[(t & 3) * 32 + k] = static_cast<int8_t>(code);
      if (k == 0) {
        blkx.scales[t & 3] = stored;
        blkx.sums[t & 3] = static_cast<int16_t>(sum);
      }
    }
    if (o.x1 != nullptr) {
      q35_q8_0_block_x1 &blk1 = o.x1[static_cast<size_t>(t) * nb + b];
      blk1.qs[k] = static_cast<int8_t>(code);
      if (k == 0) {
        blk1.scales[0] = stored;
        blk1.sums[0] = static_cast<int16_t>(sum);
        blk1.pad = 0;
      }
    }
  }
}

}  // namespace q35
