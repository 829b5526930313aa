// Activation preparation for the Q4-G32-DOT4 projections: optional producer
// (RMSNorm, SiLU*mul, split-K attention merge), then the randomized-sign
// Hadamard-128 rotation and per-32 int8 quantization.
//
// Reference semantics (bit-exact given the same FP32 input):
//   signs + FWHT stage order 1,2,...,64     src/cpu/q4_h128.cpp:35-61
//   absmax/127, unrounded 1/scale, round half away from zero, clamp +-127,
//   stored scale = binary16(scale) * 1/sqrt(128)   q4_0.cpp:212-235, q4_h128.cpp:319-321
// One wavefront per (token, 128-column block), four per workgroup, so a
// 16-token step spreads over 16 x K/128 wavefronts; two values per lane, the
// first six FWHT stages are lane shuffles and the last one is in-lane. An
// RMSNorm source recomputes its row's sum of squares in each wavefront.
#include "q35_quant.h"

namespace q35 {
namespace {

constexpr int kPrepThreads = 256;

// Merge of split-K attention partials for one (token, head, dim), pairwise in
// split order with the zero-sum identity (merge_attention_partial,
// src/cpu/full_attention_tiled.cpp:66-78), then normalised and gated
// (full_attention.cpp:104-127).
__device__ float attention_merge_value(const PrepArgs &a, int t, int c) {
  const int h = c / a.head_dim, d = c - h * a.head_dim;
  const int seq = a.seq_lens[t];
  const int splits = (seq + a.split_tokens - 1) / a.split_tokens;
  const size_t hs = (static_cast<size_t>(t) * a.heads + h) * a.max_splits;
  float m = 0.0F, l = 0.0F, v = 0.0F;
  for (int s = 0; s < splits; ++s) {
    const float om = a.part_ml[(hs + s) * 2], ol = a.part_ml[(hs + s) * 2 + 1];
    const float ov = a.part_o[(hs + s) * a.head_dim + d];
    if (ol == 0.0F) continue;
    if (l == 0.0F) {
      m = om; l = ol; v = ov;
      continue;
    }
    const float mm = fmaxf(m, om);
    const float x = expf(m - mm), y = expf(om - mm);
    v = x * v + y * ov;
    l = x * l + y * ol;
    m = mm;
  }
  const float inv = 1.0F / (l > 0.0F ? l : 1.0F);
  const float g = a.gates[(static_cast<size_t>(t) * a.heads + h) * a.head_dim + d];
  return (v * inv) * sigmoid_stable(g);
}

template <int SRC>
__device__ __forceinline__ float load_source(const PrepArgs &a, int t, int c, float rms_inv) {
  const float *row = a.x + static_cast<size_t>(t) * a.x_stride;
  if constexpr (SRC == kPrepPlain) {
    return row[c];
  } else if constexpr (SRC == kPrepRmsNorm) {
    return row[c] * rms_inv * (a.weight[c] + a.weight_offset);
  } else if constexpr (SRC == kPrepSiluMul) {
    return silu_times(row[c], row[c + a.K]);
  } else {
    return attention_merge_value(a, t, c);
  }
}

template <int SRC>
__global__ __launch_bounds__(kPrepThreads) void prep_kernel(PrepArgs a) {
  const int K = a.K, nb = K >> 5, nblk = K >> 7;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int item = blockIdx.x * (kPrepThreads / 64) + wave;
  if (item >= a.tokens * nblk) return;  // whole wavefronts only; no workgroup barrier below
  const int t = item / nblk, blk = item - t * nblk;

  float rms_inv = 1.0F;
  if constexpr (SRC == kPrepRmsNorm) {
    // the row's sum of squares, four 16-byte loads per lane in flight
    // (x_stride and K are multiples of 128)
    const q35_f32x4 *row4 = reinterpret_cast<const q35_f32x4 *>(a.x + static_cast<size_t>(t) * a.x_stride);
    const int n4 = K >> 2;
    float ss = 0.0F;
    for (int i0 = lane; i0 < n4; i0 += 256) {
      q35_f32x4 v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int i = i0 + 64 * u;
        v[u] = i < n4 ? row4[i] : q35_f32x4{0.0F, 0.0F, 0.0F, 0.0F};
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) ss += v[u][0] * v[u][0] + v[u][1] * v[u][1] + v[u][2] * v[u][2] + v[u][3] * v[u][3];
    }
    ss = group_sum<64>(ss);
    rms_inv = 1.0F / sqrtf(ss / static_cast<float>(K) + a.eps);
  }

  {
    const int c0 = blk * 128 + lane, c1 = c0 + 64;
    float v0 = load_source<SRC>(a, t, c0, rms_inv);
    float v1 = load_source<SRC>(a, t, c1, rms_inv);
    if (a.normed_out != nullptr) {
      a.normed_out[static_cast<size_t>(t) * K + c0] = v0;
      a.normed_out[static_cast<size_t>(t) * K + c1] = v1;
    }
    QuantOut o;
    o.codes = a.codes;
    o.params = a.params;
    o.x4 = a.x4;
    o.x1 = a.x1;
    h128_quantize_block(v0, v1, lane, t, blk, nb, a.h128, a.seed, o);
  }
}

// X4 (reference prefill layout) -> A16.
__global__ void x4_to_a16_kernel(const q35_q8_0_block_x4 *x4, int tokens, int nb, uint64_t *codes,
                                 ActParam *params) {
  const int b = blockIdx.x, tile = blockIdx.y, lane = threadIdx.x;
  const int tok = tile * 16 + (lane & 15), g = lane >> 4;
  uint64_t word = 0;
  ActParam p{0.0F, 0};
  if (tok < tokens) {
    const q35_q8_0_block_x4 &src = x4[static_cast<size_t>(tok >> 2) * nb + b];
    const uint8_t *q = reinterpret_cast<const uint8_t *>(src.qs) + (tok & 3) * 32 + g * 8;
    for (int i = 0; i < 8; ++i) word |= static_cast<uint64_t>(q[i]) << (8 * i);
    p = ActParam{src.scales[tok & 3], -8 * static_cast<int32_t>(src.sums[tok & 3])};
  }
  codes[(static_cast<size_t>(tile) * nb + b) * 64 + lane] = word;
  if (g == 0) params[(static_cast<size_t>(tile) * nb + b) * 16 + (lane & 15)] = p;
}

__global__ void x1_to_a16_kernel(const q35_q8_0_block_x1 *x1, int nb, uint64_t *codes,
                                 ActParam *params) {
  const int b = blockIdx.x, lane = threadIdx.x;
  const int tok = lane & 15, g = lane >> 4;
  uint64_t word = 0;
  ActParam p{0.0F, 0};
  if (tok == 0) {
    const uint8_t *q = reinterpret_cast<const uint8_t *>(x1[b].qs) + g * 8;
    for (int i = 0; i < 8; ++i) word |= static_cast<uint64_t>(q[i]) << (8 * i);
    p = ActParam{x1[b].scales[0], -8 * static_cast<int32_t>(x1[b].sums[0])};
  }
  codes[static_cast<size_t>(b) * 64 + lane] = word;
  if (g == 0) params[static_cast<size_t>(b) * 16 + tok] = p;
}

}  // namespace

hipError_t launch_prep(const PrepArgs &a, hipStream_t stream) {
  if (a.tokens <= 0) return hipSuccess;
  const int items = a.tokens * (a.K >> 7);
  const dim3 grid((items + kPrepThreads / 64 - 1) / (kPrepThreads / 64)), block(kPrepThreads);
  switch (a.source) {
    case kPrepPlain: Q35_LAUNCH((prep_kernel<kPrepPlain>), grid, block, 0, stream, a); break;
    case kPrepRmsNorm: Q35_LAUNCH((prep_kernel<kPrepRmsNorm>), grid, block, 0, stream, a); break;
    case kPrepSiluMul: Q35_LAUNCH((prep_kernel<kPrepSiluMul>), grid, block, 0, stream, a); break;
    default: Q35_LAUNCH((prep_kernel<kPrepAttnMerge>), grid, block, 0, stream, a); break;
  }
  return hipGetLastError();
}

hipError_t launch_x4_to_a16(const q35_q8_0_block_x4 *x4, int tokens, int nb, uint64_t *codes,
                            ActParam *params, hipStream_t stream) {
  const dim3 grid(nb, (tokens + 15) / 16);
  Q35_LAUNCH((x4_to_a16_kernel), grid, 64, 0, stream, x4, tokens, nb, codes, params);
  return hipGetLastError();
}

hipError_t launch_x1_to_a16(const q35_q8_0_block_x1 *x1, int nb, uint64_t *codes,
                            ActParam *params, hipStream_t stream) {
  Q35_LAUNCH((x1_to_a16_kernel), nb, 64, 0, stream, x1, nb, codes, params);
  return hipGetLastError();
}

}  // namespace q35
