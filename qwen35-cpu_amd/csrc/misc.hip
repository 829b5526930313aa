// Small kernels: embedding gather, stand-alone activation ops used by the
// kernel-level ABI entries, and the reference-shaped DeltaNet row update.
#include "q35_device.h"
#include "q35_internal.h"

namespace q35 {
namespace {

// dequantize_embedding_row for the identity-basis DOT4 head
// (src/runtime/gguf_matrix.inl:21-26, q4_dot4.cpp:31-40): x = half(d[r]) * (u - 8).
__global__ void embed_kernel(const q35_q4_0_block_x8 *embed, int nb, const int32_t *tokens,
                             float *x, int hidden, int32_t *counts, long long counts_stride,
                             const int32_t *slots, const uint8_t *count_input, bool g16) {
  const int r = blockIdx.x;
  const int token = tokens[r];
  const int rt = token >> 3, row = token & 7;
  for (int k = threadIdx.x; k < hidden; k += blockDim.x) {
    const int b = k >> 5, kk = k & 31;
    if (g16) {
      // Q4G16Tile: d[half][row] then the DOT4 codes (q4_g16_dequantize_row, q4_g16.cpp:98-103)
      const uint8_t *tile = reinterpret_cast<const uint8_t *>(embed) + (static_cast<size_t>(rt) * nb + b) * 160;
      const uint16_t dh = *reinterpret_cast<const uint16_t *>(tile + 2 * (8 * (kk >> 4) + row));
      const int u = (tile[32 + 32 * (kk >> 3) + 4 * row + (kk & 3)] >> (4 * ((kk & 7) >> 2))) & 15;
      x[static_cast<size_t>(r) * hidden + k] = half_bits_to_float(dh) * static_cast<float>(u - 8);
      continue;
    }
    const q35_q4_0_block_x8 &w = embed[static_cast<size_t>(rt) * nb + b];
    const int u = (w.qs[32 * (kk >> 3) + 4 * row + (kk & 3)] >> (4 * ((kk & 7) >> 2))) & 15;
    x[static_cast<size_t>(r) * hidden + k] = half_bits_to_float(w.d[row]) * static_cast<float>(u - 8);
  }
  if (threadIdx.x == 0 && counts != nullptr && count_input != nullptr && count_input[r])
    counts[static_cast<long long>(slots[r]) * counts_stride + token] += 1;
}

__global__ void rms_norm_kernel(const float *x, const float *w, float *y, int width, float eps,
                                float offset) {
  __shared__ float scratch[8];
  const int r = blockIdx.x;
  const float *xr = x + static_cast<size_t>(r) * width;
  float ss = 0.0F;
  for (int i = threadIdx.x; i < width; i += 256) ss += xr[i] * xr[i];
  ss = block_sum<4>(ss, scratch);
  const float inv = 1.0F / sqrtf(ss / static_cast<float>(width) + eps);
  for (int i = threadIdx.x; i < width; i += 256)
    y[static_cast<size_t>(r) * width + i] = xr[i] * inv * (w[i] + offset);
}

__global__ void l2_normalize_kernel(float *x, int width, float eps, float scale) {
  __shared__ float scratch[8];
  float *xr = x + static_cast<size_t>(blockIdx.x) * width;
  float ss = 0.0F;
  for (int i = threadIdx.x; i < width; i += 256) ss += xr[i] * xr[i];
  ss = block_sum<4>(ss, scratch);
  const float m = scale / sqrtf(ss + eps);
  __syncthreads();
  for (int i = threadIdx.x; i < width; i += 256) xr[i] *= m;
}

// causal_conv1d_silu_f32 (activation.cpp:164-222): one thread per channel of
// [begin, end) walks the batch's tokens in order, each token advancing the
// ring (the oldest slot is `ring`); kernel-major weights [kernel][channels].
__global__ void conv1d_silu_kernel(float *state, int ring, const float *input, long long stride, const float *w,
                                   float *out, int batch, int channels, int kernel, int begin, int end) {
  const int c = begin + static_cast<int>(blockIdx.x * blockDim.x + threadIdx.x);
  if (c >= end) return;
  const int hist = kernel - 1;
  for (int t = 0; t < batch; ++t) {
    const float x = input[t * stride + c];
    float sum = x * w[static_cast<size_t>(hist) * channels + c];
    for (int k = 0; k < hist; ++k)
      sum += state[static_cast<size_t>((ring + k) % hist) * channels + c] * w[static_cast<size_t>(k) * channels + c];
    if (hist) state[static_cast<size_t>(ring) * channels + c] = x;
    out[static_cast<size_t>(t) * channels + c] = silu_times(sum, 1.0F);
    if (hist) ring = (ring + 1) % hist;
  }
}

__global__ void silu_mul_kernel(const float *g, const float *u, float *out, long long n) {
  const long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) out[i] = silu_times(g[i], u[i]);
}

__global__ void rope_kernel(float *x, int head_dim, int rope_dim, const float *c, const float *s) {
  const int h = blockIdx.x, i = threadIdx.x, half = rope_dim / 2;
  if (i >= half) return;
  float *a = x + static_cast<size_t>(h) * head_dim;
  const float x0 = a[i], x1 = a[i + half];
  a[i] = x0 * c[i] - x1 * s[i];
  a[i + half] = x1 * c[i] + x0 * s[i];
}

__global__ void store_f16_kernel(const float *x, uint16_t *y, long long n) {
  const long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float v = x[i];
  // NaN stores the quiet pattern like attention_float_to_half (full_attention.cpp:22-25)
  y[i] = isnan(v) ? static_cast<uint16_t>((__float_as_uint(v) >> 16 & 0x8000u) | 0x7e00u)
                  : float_to_half_bits(v);
}

}  // namespace

hipError_t launch_embed(const q35_q4_0_block_x8 *embed, int nb, const int32_t *tokens, int batch,
                        float *x, int hidden, int32_t *counts, long long counts_stride,
                        const int32_t *slots, const uint8_t *count_input, hipStream_t stream, bool g16) {
  if (batch <= 0) return hipSuccess;
  Q35_LAUNCH((embed_kernel), batch, 256, 0, stream, embed, nb, tokens, x, hidden, counts, counts_stride,
                                          slots, count_input, g16);
  return hipGetLastError();
}

hipError_t launch_rms_norm(const float *x, const float *w, float *y, int rows, int width,
                           float eps, float offset, hipStream_t stream) {
  if (rows <= 0) return hipSuccess;
  Q35_LAUNCH((rms_norm_kernel), rows, 256, 0, stream, x, w, y, width, eps, offset);
  return hipGetLastError();
}

hipError_t launch_l2_normalize(float *x, int rows, int width, float eps, float scale,
                               hipStream_t stream) {
  if (rows <= 0) return hipSuccess;
  Q35_LAUNCH((l2_normalize_kernel), rows, 256, 0, stream, x, width, eps, scale);
  return hipGetLastError();
}

hipError_t launch_conv1d_silu(float *state, int ring, const float *input, long long stride, const float *w,
                              float *out, int batch, int channels, int kernel, int begin, int end, hipStream_t stream) {
  if (batch <= 0 || begin >= end) return hipSuccess;
  Q35_LAUNCH((conv1d_silu_kernel), (end - begin + 255) / 256, 256, 0, stream, state, ring, input, stride, w, out,
                                                                 batch, channels, kernel, begin, end);
  return hipGetLastError();
}

hipError_t launch_silu_mul(const float *g, const float *u, float *out, long long n,
                           hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  Q35_LAUNCH((silu_mul_kernel), static_cast<unsigned>((n + 255) / 256), 256, 0, stream, g, u, out, n);
  return hipGetLastError();
}

hipError_t launch_rope(float *x, int heads, int head_dim, int rope_dim, const float *c,
                       const float *s, hipStream_t stream) {
  if (heads <= 0) return hipSuccess;
  Q35_LAUNCH((rope_kernel), heads, 256, 0, stream, x, head_dim, rope_dim, c, s);
  return hipGetLastError();
}

hipError_t launch_store_f16(const float *x, uint16_t *y, long long n, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  Q35_LAUNCH((store_f16_kernel), static_cast<unsigned>((n + 255) / 256), 256, 0, stream, x, y, n);
  return hipGetLastError();
}

}  // namespace q35
