/* q35_oracle.c -- plain-C restatement of the reference's scalar semantics for
 * the batched-decode path. TEST INFRASTRUCTURE ONLY: loaded by tests/, by
 * __graft_entry__.smoke() and by bench.py's cpu_baseline leg as the checker,
 * never shipped or measured as the product.
 *
 * Parity pins (tests/test_oracle_*.py):
 *   - half conversions: exhaustive 65536-value round trip, and against the
 *     reference build (oracle/_ref) on 2^20 seeded floats incl. subnormals;
 *   - q8 quantizers, H128 transform/prepare: bit-exact against golden vectors
 *     written by the reference build (tests/golden/), plus the reference's own
 *     H128 basis known answer (tests/q4_quantizer_test.cpp:12-19 output) and
 *     orthogonality / Sylvester closed forms;
 *   - DOT4 pack/unpack: bijection round trip, brute-force int32 block dots on
 *     tiny inputs against an FP64 dequantized product;
 *   - matvec/matmul/argmax: bit-exact against golden vectors of the reference's
 *     avx2 path (same fma order, q4_dot4_simd.inl:91-94);
 *   - DeltaNet, attention, activation ops, whole decode step: within tolerance
 *     of the reference build's outputs (golden vectors) and FP64 brute force.
 * Compiled with -ffp-contract=off so that separate multiply/add steps stay
 * separate, as in the reference scalar code. */
#include "q35_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* src/cpu/q8_0.cpp:18-55 (round to nearest even, subnormals, NaN payload) */
uint16_t q35o_float_to_half(float value) {
  const uint32_t bits = f2u(value);
  const uint32_t sign = (bits >> 16) & 0x8000u;
  const uint32_t mag = bits & 0x7fffffffu;
  if (mag >= 0x7f800000u) {
    if (mag == 0x7f800000u) return (uint16_t)(sign | 0x7c00u);
    const uint16_t payload = (uint16_t)((mag >> 13) & 0x03ffu);
    return (uint16_t)(sign | 0x7c00u | payload | (payload == 0));
  }
  if (mag > 0x477fefffu) return (uint16_t)(sign | 0x7c00u);
  if (mag < 0x38800000u) {
    if (mag < 0x33000000u) return (uint16_t)sign;
    const uint32_t exponent = mag >> 23;
    const uint32_t mantissa = (mag & 0x007fffffu) | 0x00800000u;
    const uint32_t shift = 126u - exponent;
    uint32_t hm = mantissa >> shift;
    const uint32_t rem = mantissa & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (hm & 1u))) ++hm;
    return (uint16_t)(sign | hm);
  }
  const uint32_t rounded = mag + 0x00000fffu + ((mag >> 13) & 1u);
  return (uint16_t)(sign | ((rounded - 0x38000000u) >> 13));
}

/* src/cpu/q8_0.cpp:57-83 */
float q35o_half_to_float(uint16_t value) {
  const uint32_t sign = (uint32_t)(value & 0x8000u) << 16;
  const uint32_t exponent = (value >> 10) & 0x1fu;
  uint32_t mantissa = value & 0x03ffu;
  uint32_t bits;
  if (exponent == 0) {
    if (mantissa == 0) {
      bits = sign;
    } else {
      uint32_t e = 113u;
      while ((mantissa & 0x0400u) == 0) { mantissa <<= 1; --e; }
      mantissa &= 0x03ffu;
      bits = sign | (e << 23) | (mantissa << 13);
    }
  } else if (exponent == 0x1fu) {
    bits = sign | 0x7f800000u | (mantissa << 13);
  } else {
    bits = sign | ((exponent + 112u) << 23) | (mantissa << 13);
  }
  return u2f(bits);
}

/* src/cpu/full_attention.cpp:18-46 (KV store rounding; quiet NaN) */
uint16_t q35o_attention_float_to_half(float value) {
  const uint32_t bits = f2u(value);
  const uint32_t sign = (bits >> 16) & 0x8000u;
  const uint32_t mag = bits & 0x7fffffffu;
  if (mag >= 0x7f800000u) return (uint16_t)(sign | (mag > 0x7f800000u ? 0x7e00u : 0x7c00u));
  if (mag > 0x477fefffu) return (uint16_t)(sign | 0x7c00u);
  if (mag < 0x33000001u) return (uint16_t)sign;
  if (mag < 0x38800000u) {
    const uint32_t exponent = mag >> 23;
    const uint32_t mantissa = (mag & 0x7fffffu) | 0x800000u;
    const uint32_t shift = 113u - exponent;
    uint32_t hm = mantissa >> (shift + 13u);
    const uint32_t rem = mantissa & ((1u << (shift + 13u)) - 1u);
    const uint32_t half = 1u << (shift + 12u);
    if (rem > half || (rem == half && (hm & 1u))) ++hm;
    return (uint16_t)(sign | hm);
  }
  const uint32_t rounded = mag + 0x00000fffu + ((mag >> 13) & 1u);
  return (uint16_t)(sign | ((rounded - 0x38000000u) >> 13));
}

/* attention_cache_store_f16 (full_attention.cpp:201-217), scalar branch: the
 * conversion above over n values */
void q35o_attention_store_f16(const float *x, uint16_t *out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = q35o_attention_float_to_half(x[i]);
}

/* One 32-value block: src/cpu/q4_0.cpp:212-235 (scalar quantizer). The code
 * uses the unrounded 1/scale; the stored scale is the binary16-rounded one;
 * std::round rounds half away from zero (C roundf). */
static void quantize_block(const float *src, float *scale_out, int16_t *sum_out, int8_t *codes) {
  float amax = 0.0f;
  for (int i = 0; i < 32; ++i) {
    const float a = fabsf(src[i]);
    amax = amax > a ? amax : a;  /* std::max(amax, a) keeps amax on ties/NaN */
  }
  const float scale = amax / 127.0f;
  const float inv = scale == 0.0f ? 0.0f : 1.0f / scale;
  *scale_out = q35o_half_to_float(q35o_float_to_half(scale));
  int32_t sum = 0;
  for (int i = 0; i < 32; ++i) {
    float r = roundf(src[i] * inv);
    r = r < -127.0f ? -127.0f : (r > 127.0f ? 127.0f : r);
    codes[i] = (int8_t)r;
    sum += codes[i];
  }
  *sum_out = (int16_t)sum;
}

/* q4_0.cpp:212-235 */
void q35o_q8_quantize_vector_1(const float *x, q35o_q8x1 *out, size_t blocks) {
  for (size_t b = 0; b < blocks; ++b) {
    memset(&out[b], 0, sizeof(out[b]));
    quantize_block(x + b * 32, &out[b].scales[0], &out[b].sums[0], out[b].qs);
  }
}

/* q4_0.cpp:149-180 */
void q35o_q8_quantize_vectors_4(const float *x, q35o_q8x4 *out, size_t vectors, size_t blocks) {
  const size_t width = blocks * 32;
  for (size_t tile = 0; tile < vectors / 4; ++tile)
    for (size_t b = 0; b < blocks; ++b) {
      q35o_q8x4 *dst = &out[tile * blocks + b];
      for (size_t t = 0; t < 4; ++t)
        quantize_block(x + (tile * 4 + t) * width + b * 32, &dst->scales[t], &dst->sums[t],
                       dst->qs + t * 32);
    }
}

/* q4_h128.cpp:16-33 */
static uint64_t splitmix64(uint64_t v) {
  v += 0x9e3779b97f4a7c15ull;
  v = (v ^ (v >> 30)) * 0xbf58476d1ce4e5b9ull;
  v = (v ^ (v >> 27)) * 0x94d049bb133111ebull;
  return v ^ (v >> 31);
}
uint64_t q35o_h128_sign_word(size_t block, size_t word, uint64_t seed) {
  const uint64_t key = seed + (uint64_t)block * 0x9e3779b97f4a7c15ull;
  return splitmix64(key + (uint64_t)word * 0xd1b54a32d192ed03ull);
}

/* q4_h128.cpp:35-61, 77-84: signs, then Sylvester FWHT with strides 1..64 */
void q35o_h128_transform_unscaled(const float *x, float *y, size_t block, uint64_t seed) {
  memcpy(y, x, 128 * sizeof(float));
  for (size_t w = 0; w < 2; ++w) {
    const uint64_t s = q35o_h128_sign_word(block, w, seed);
    for (size_t bit = 0; bit < 64; ++bit)
      if ((s >> bit) & 1u) y[w * 64 + bit] = -y[w * 64 + bit];
  }
  for (size_t stride = 1; stride < 128; stride *= 2)
    for (size_t base = 0; base < 128; base += 2 * stride)
      for (size_t lane = 0; lane < stride; ++lane) {
        const float lhs = y[base + lane], rhs = y[base + stride + lane];
        y[base + lane] = lhs + rhs;
        y[base + stride + lane] = lhs - rhs;
      }
}

/* q4_h128.cpp:63-75 */
void q35o_h128_transform(const float *x, float *y, size_t block, uint64_t seed) {
  q35o_h128_transform_unscaled(x, y, block, seed);
  for (int i = 0; i < 128; ++i) y[i] *= 0.08838834764831844055f;
}

/* q4_h128.cpp:259-324 (scalar branch) */
int q35o_h128_prepare_activation_1(const float *x, q35o_q8x1 *out, size_t cols, uint64_t seed) {
  if (!x || !out || cols == 0 || cols % 128) return 0;
  float y[128];
  for (size_t blk = 0; blk < cols / 128; ++blk) {
    q35o_h128_transform_unscaled(x + blk * 128, y, blk, seed);
    q35o_q8_quantize_vector_1(y, out + blk * 4, 4);
    for (int g = 0; g < 4; ++g) out[blk * 4 + g].scales[0] *= 0.08838834764831844055f;
  }
  return 1;
}

/* q4_h128.cpp:326-401 */
int q35o_h128_prepare_activations_4(const float *x, q35o_q8x4 *out, size_t vectors, size_t cols,
                                    uint64_t seed) {
  if (!x || !out || vectors == 0 || vectors % 4 || cols == 0 || cols % 128) return 0;
  const size_t blocks = cols / 32;
  float y[4 * 128];
  for (size_t tile = 0; tile < vectors / 4; ++tile)
    for (size_t blk = 0; blk < cols / 128; ++blk) {
      for (size_t t = 0; t < 4; ++t)
        q35o_h128_transform_unscaled(x + (tile * 4 + t) * cols + blk * 128, y + t * 128, blk, seed);
      q35o_q8x4 *dst = out + tile * blocks + blk * 4;
      q35o_q8_quantize_vectors_4(y, dst, 4, 4);
      for (int g = 0; g < 4; ++g)
        for (int t = 0; t < 4; ++t) dst[g].scales[t] *= 0.08838834764831844055f;
    }
  return 1;
}

/* q4_h128.cpp:195-222 (weight quantizer: absmax/7, binary16 scale) */
void q35o_q4_quantize_transformed(const float *x, q35o_q4_0 *out, size_t blocks) {
  for (size_t b = 0; b < blocks; ++b) {
    const float *v = x + b * 32;
    float amax = 0.0f;
    for (int i = 0; i < 32; ++i) { const float a = fabsf(v[i]); amax = amax > a ? amax : a; }
    const float scale = amax / 7.0f;
    out[b].d = q35o_float_to_half(scale);
    const float stored = q35o_half_to_float(out[b].d);
    const float inv = stored == 0.0f ? 0.0f : 1.0f / stored;
    for (int i = 0; i < 16; ++i) {
      float lo = roundf(v[i] * inv), hi = roundf(v[i + 16] * inv);
      lo = lo < -7.0f ? -7.0f : (lo > 7.0f ? 7.0f : lo);
      hi = hi < -7.0f ? -7.0f : (hi > 7.0f ? 7.0f : hi);
      out[b].qs[i] = (uint8_t)(((int)lo + 8) | (((int)hi + 8) << 4));
    }
  }
}

/* q4_h128.cpp:224-252 */
int q35o_h128_quantize_matrix(const float *x, q35o_q4_0 *out, size_t rows, size_t cols,
                              uint64_t seed) {
  if (!x || !out || cols == 0 || cols % 128) return 0;
  float y[128];
  for (size_t r = 0; r < rows; ++r)
    for (size_t blk = 0; blk < cols / 128; ++blk) {
      q35o_h128_transform(x + r * cols + blk * 128, y, blk, seed);
      q35o_q4_quantize_transformed(y, out + r * (cols / 32) + blk * 4, 4);
    }
  return 1;
}

/* q4_dot4.cpp:5-18: qs[32t+4r+j] = u[r][8t+j] | u[r][8t+4+j] << 4 */
void q35o_dot4_pack_rows_8(const q35o_q4_0 *src, q35o_q4x8 *dst, size_t rows, size_t blocks) {
  for (size_t rt = 0; rt < rows / 8; ++rt)
    for (size_t b = 0; b < blocks; ++b) {
      q35o_q4x8 *o = &dst[rt * blocks + b];
      for (size_t r = 0; r < 8; ++r) {
        const q35o_q4_0 *s = &src[(rt * 8 + r) * blocks + b];
        o->d[r] = s->d;
        for (size_t t = 0; t < 4; ++t)
          for (size_t j = 0; j < 4; ++j) {
            const size_t k0 = 8 * t + j, k1 = 8 * t + 4 + j;
            const int n0 = (s->qs[k0 % 16] >> (4 * (k0 / 16))) & 15;
            const int n1 = (s->qs[k1 % 16] >> (4 * (k1 / 16))) & 15;
            o->qs[32 * t + 4 * r + j] = (uint8_t)(n0 | (n1 << 4));
          }
      }
    }
}

static int dot4_code(const q35o_q4x8 *w, size_t r, size_t k) {
  return (w->qs[32 * (k / 8) + 4 * r + k % 4] >> (4 * ((k % 8) / 4))) & 15;
}

/* q4_dot4.cpp:19-30 */
void q35o_dot4_unpack_rows_8(const q35o_q4x8 *src, q35o_q4_0 *dst, size_t rows, size_t blocks) {
  for (size_t row = 0; row < rows; ++row)
    for (size_t b = 0; b < blocks; ++b) {
      const q35o_q4x8 *s = &src[(row / 8) * blocks + b];
      q35o_q4_0 *o = &dst[row * blocks + b];
      memset(o, 0, sizeof(*o));
      o->d = s->d[row % 8];
      for (size_t k = 0; k < 32; ++k)
        o->qs[k % 16] |= (uint8_t)(dot4_code(s, row % 8, k) << (4 * (k / 16)));
    }
}

/* q4_dot4.cpp:31-40 */
void q35o_dot4_dequantize_row(const q35o_q4x8 *m, size_t row, float *out, size_t blocks) {
  for (size_t b = 0; b < blocks; ++b) {
    const q35o_q4x8 *w = &m[(row / 8) * blocks + b];
    const float scale = q35o_half_to_float(w->d[row % 8]);
    for (size_t k = 0; k < 32; ++k) out[b * 32 + k] = scale * (float)(dot4_code(w, row % 8, k) - 8);
  }
}

/* Integer part of q4_dot4.cpp:46-52: dot = sum_k (u-8)*a, one int32 per
 * (row, block). codes is [blocks][32], sums unused by the definition but the
 * SIMD form sum u*a - 8*sum_a must agree (tests check both). */
void q35o_dot4_block_dots(const q35o_q4x8 *m, const int8_t *codes, const int16_t *sums,
                          int32_t *out, size_t rows, size_t blocks) {
  (void)sums;
  for (size_t r = 0; r < rows; ++r)
    for (size_t b = 0; b < blocks; ++b) {
      const q35o_q4x8 *w = &m[(r / 8) * blocks + b];
      int32_t dot = 0;
      for (size_t k = 0; k < 32; ++k) dot += (dot4_code(w, r % 8, k) - 8) * (int32_t)codes[b * 32 + k];
      out[r * blocks + b] = dot;
    }
}

/* q4_dot4.cpp:43-56 scalar_row: result = fma(float(dot), d_w*s_a, result) */
static float scalar_row(const q35o_q4x8 *m, const int8_t *qs, size_t qstride, const float *scales,
                        size_t sstride, size_t row, size_t blocks) {
  float result = 0.0f;
  for (size_t b = 0; b < blocks; ++b) {
    const q35o_q4x8 *w = &m[(row / 8) * blocks + b];
    const int8_t *a = qs + b * qstride;
    int dot = 0;
    for (size_t k = 0; k < 32; ++k) dot += (dot4_code(w, row % 8, k) - 8) * (int)a[k];
    const float s = q35o_half_to_float(w->d[row % 8]) * scales[b * sstride];
    result = fmaf((float)dot, s, result);
  }
  return result;
}

/* q4_dot4.cpp:58-72 */
void q35o_dot4_matvec(const q35o_q4x8 *m, const q35o_q8x1 *v, float *out, size_t rows,
                      size_t blocks) {
  for (size_t r = 0; r < rows; ++r)
    out[r] = scalar_row(m, v[0].qs, sizeof(q35o_q8x1), &v[0].scales[0],
                        sizeof(q35o_q8x1) / sizeof(float), r, blocks);
}

/* q4_dot4.cpp:87-106 */
void q35o_dot4_matmul(const q35o_q4x8 *m, const q35o_q8x4 *v, float *out, size_t rows,
                      size_t count, size_t blocks, size_t stride) {
  for (size_t t = 0; t < count; ++t) {
    const q35o_q8x4 *base = v + (t / 4) * blocks;
    for (size_t r = 0; r < rows; ++r)
      out[t * stride + r] = scalar_row(m, base[0].qs + (t % 4) * 32, sizeof(q35o_q8x4),
                                       &base[0].scales[t % 4], sizeof(q35o_q8x4) / sizeof(float), r,
                                       blocks);
  }
}

/* q4_dot4.cpp:107-124 */
void q35o_dot4_argmax(const q35o_q4x8 *m, const q35o_q8x1 *v, const int *counts, float penalty,
                      size_t offset, size_t rows, size_t blocks, float *value, size_t *index) {
  float best = -INFINITY;
  size_t at = offset;
  for (size_t r = 0; r < rows; ++r) {
    float x = scalar_row(m, v[0].qs, sizeof(q35o_q8x1), &v[0].scales[0],
                         sizeof(q35o_q8x1) / sizeof(float), r, blocks);
    if (counts && counts[offset + r] > 0 && penalty > 1.0f) x = x > 0 ? x / penalty : x * penalty;
    if (x > best) { best = x; at = offset + r; }
  }
  *value = best;
  *index = at;
}

/* src/cpu/delta_net.cpp:63-98; state layout [head][value_row][key_col] */
void q35o_delta_net_update_rows(float *state, const float *q, const float *k, const float *v,
                                const float *alpha, const float *beta, float *out, size_t kdim,
                                size_t vdim, size_t row_begin, size_t row_end) {
  for (size_t flat = row_begin; flat < row_end; ++flat) {
    const size_t head = flat / vdim, vrow = flat - head * vdim;
    float *s = state + flat * kdim;
    const float *qh = q + head * kdim, *kh = k + head * kdim;
    float sk = 0.0f;
    for (size_t c = 0; c < kdim; ++c) {
      const float decayed = s[c] * alpha[head];
      s[c] = decayed;
      sk += decayed * kh[c];
    }
    const float delta = (v[head * vdim + vrow] - sk) * beta[head];
    float sq = 0.0f;
    for (size_t c = 0; c < kdim; ++c) {
      const float updated = s[c] + delta * kh[c];
      s[c] = updated;
      sq += updated * qh[c];
    }
    out[head * vdim + vrow] = sq;
  }
}

/* src/cpu/full_attention.cpp:48-54 */
static float attention_sigmoid(float x) {
  if (x >= 0.0f) return 1.0f / (1.0f + expf(-x));
  const float e = expf(x);
  return e / (1.0f + e);
}

/* src/cpu/full_attention.cpp:56-128 (scalar decode rows), KV given as one
 * FP16 row pointer per context token (AttentionKvRows, full_attention.h:10-20).
 * Rows are flattened [query_head] of a single decode token; scores holds
 * sequence_length floats per row. */
void q35o_attention_decode(const float *q, const float *gates, const uint16_t *const *key_rows,
                           const uint16_t *const *value_rows, float *scores, float *out,
                           size_t query_width, int sequence_length, int heads, int kv_heads,
                           int head_dim, float scale, size_t row_begin, size_t row_end) {
  (void)query_width;
  const int per_kv = heads / kv_heads;
  for (size_t row = row_begin; row < row_end; ++row) {
    const int head = (int)row;
    const int kvh = head / per_kv;
    const float *qh = q + (size_t)head * head_dim;
    const float *gh = gates + (size_t)head * head_dim;
    float *srow = scores + row * (size_t)sequence_length;
    float mx = -INFINITY;
    for (int c = 0; c < sequence_length; ++c) {
      const uint16_t *kr = key_rows[c] + (size_t)kvh * head_dim;
      float dot = 0.0f;
      for (int i = 0; i < head_dim; ++i) dot += qh[i] * q35o_half_to_float(kr[i]);
      dot *= scale;
      srow[c] = dot;
      mx = mx > dot ? mx : dot;
    }
    float denom = 0.0f;
    for (int c = 0; c < sequence_length; ++c) {
      const float p = expf(srow[c] - mx);
      srow[c] = p;
      denom += p;
    }
    const float inv = 1.0f / (denom > 0.0f ? denom : 1.0f);
    float *oh = out + (size_t)head * head_dim;
    for (int i = 0; i < head_dim; ++i) oh[i] = 0.0f;
    for (int c = 0; c < sequence_length; ++c) {
      const float p = srow[c] * inv;
      const uint16_t *vr = value_rows[c] + (size_t)kvh * head_dim;
      for (int i = 0; i < head_dim; ++i) oh[i] += p * q35o_half_to_float(vr[i]);
    }
    for (int i = 0; i < head_dim; ++i) oh[i] *= attention_sigmoid(gh[i]);
  }
}

/* src/cpu/activation.cpp:224-262 */
void q35o_rms_norm(const float *x, const float *w, float *y, size_t rows, size_t width, float eps,
                   float offset) {
  for (size_t r = 0; r < rows; ++r) {
    const float *xr = x + r * width;
    float *yr = y + r * width;
    float ss = 0.0f;
    for (size_t c = 0; c < width; ++c) ss += xr[c] * xr[c];
    const float inv = 1.0f / sqrtf(ss / (float)width + eps);
    for (size_t c = 0; c < width; ++c) yr[c] = xr[c] * inv * (w[c] + offset);
  }
}

/* src/cpu/activation.cpp:264-298 */
void q35o_l2_normalize(float *x, size_t rows, size_t width, float eps, float scale) {
  for (size_t r = 0; r < rows; ++r) {
    float *xr = x + r * width;
    float ss = 0.0f;
    for (size_t c = 0; c < width; ++c) ss += xr[c] * xr[c];
    const float m = scale / sqrtf(ss + eps);
    for (size_t c = 0; c < width; ++c) xr[c] *= m;
  }
}

/* src/cpu/activation.cpp:164-222, batch 1: sum = x*w[hist] + sum_k state[(ring+k)%hist]*w[k] */
void q35o_conv1d_silu(float *state, size_t ring, const float *input, const float *kernel_major,
                      float *out, size_t channels, size_t kernel) {
  const size_t hist = kernel - 1;
  for (size_t c = 0; c < channels; ++c) {
    const float x = input[c];
    float sum = x * kernel_major[hist * channels + c];
    for (size_t k = 0; k < hist; ++k)
      sum += state[((ring + k) % hist) * channels + c] * kernel_major[k * channels + c];
    if (hist) state[ring * channels + c] = x;
    const float e = expf(-fabsf(sum));
    const float sg = sum >= 0.0f ? 1.0f / (1.0f + e) : e / (1.0f + e);
    out[c] = sum * sg;
  }
}

/* src/cpu/activation.cpp:329-357 */
void q35o_silu_mul(const float *gate, const float *up, float *out, size_t n) {
  for (size_t i = 0; i < n; ++i) {
    const float v = gate[i];
    const float e = expf(-fabsf(v));
    const float sg = v >= 0.0f ? 1.0f / (1.0f + e) : e / (1.0f + e);
    out[i] = v * sg * up[i];
  }
}

/* src/cpu/activation.cpp:124-162 (split-half rotation of the first rope_dim) */
void q35o_rope(float *x, size_t heads, size_t head_dim, size_t rope_dim, const float *cosine,
               const float *sine) {
  const size_t half = rope_dim / 2;
  for (size_t h = 0; h < heads; ++h) {
    float *a = x + h * head_dim, *b = a + half;
    for (size_t i = 0; i < half; ++i) {
      const float x0 = a[i], x1 = b[i];
      a[i] = x0 * cosine[i] - x1 * sine[i];
      b[i] = x1 * cosine[i] + x0 * sine[i];
    }
  }
}

/* src/runtime/weights.inl:656-678 */
float q35o_sigmoid(float x) {
  if (x >= 0.0f) { const float z = expf(-x); return 1.0f / (1.0f + z); }
  const float z = expf(x);
  return z / (1.0f + z);
}
float q35o_softplus(float x) {
  if (x > 20.0f) return x;
  if (x < -20.0f) return expf(x);
  return log1pf(expf(x));
}

/* src/runtime/cpu_engine.inl:343-355 */
void q35o_rope_tables(float theta, int rope_dim, size_t positions, float *cosine, float *sine) {
  const size_t half = (size_t)rope_dim / 2;
  float *inv = (float *)malloc(half * sizeof(float));
  for (size_t i = 0; i < half; ++i) inv[i] = powf(theta, -(float)(2 * i) / (float)rope_dim);
  for (size_t p = 0; p < positions; ++p)
    for (size_t i = 0; i < half; ++i) {
      const float angle = (float)p * inv[i];
      cosine[p * half + i] = cosf(angle);
      sine[p * half + i] = sinf(angle);
    }
  free(inv);
}

static int g16_code(const q35o_g16 *t, int row, int i) {
  return ((t->qs[32 * (i / 8) + 4 * row + i % 4] >> (i % 8 < 4 ? 0 : 4)) & 15) - 8;
}

void q35o_g16_dequantize_row(const q35o_g16 *m, size_t row, float *out, size_t blocks) {
  for (size_t b = 0; b < blocks; ++b) {
    const q35o_g16 *t = &m[(row / 8) * blocks + b];
    for (int i = 0; i < 32; ++i)
      out[b * 32 + i] = q35o_half_to_float(t->d[i / 16][row % 8]) * (float)g16_code(t, (int)(row % 8), i);
  }
}

void q35o_g16_matmul(const q35o_g16 *m, const q35o_q8x1 *v, float *out, size_t rows, size_t count,
                     size_t blocks, size_t stride) {
  for (size_t t = 0; t < count; ++t)
    for (size_t r = 0; r < rows; ++r) {
      float acc = 0.0f;
      for (size_t b = 0; b < blocks; ++b) {
        const q35o_g16 *tile = &m[(r / 8) * blocks + b];
        const q35o_q8x1 *a = &v[t * blocks + b];
        for (int half = 0; half < 2; ++half) {
          int32_t dot = 0;
          for (int i = 16 * half; i < 16 * half + 16; ++i) dot += g16_code(tile, (int)(r % 8), i) * a->qs[i];
          acc = fmaf((float)dot, q35o_half_to_float(tile->d[half][r % 8]) * a->scales[0], acc);
        }
      }
      out[t * stride + r] = acc;
    }
}

void q35o_q8_matmul(const q35o_q8_0 *m, const float *mscales, const q35o_q8x1 *v, float *out, size_t rows,
                    size_t count, size_t blocks, size_t stride) {
  for (size_t t = 0; t < count; ++t)
    for (size_t r = 0; r < rows; ++r) {
      float acc = 0.0f;
      for (size_t b = 0; b < blocks; ++b) {
        int32_t dot = 0;
        for (int i = 0; i < 32; ++i) dot += (int32_t)m[r * blocks + b].qs[i] * v[t * blocks + b].qs[i];
        acc = fmaf((float)dot, mscales[r * blocks + b] * v[t * blocks + b].scales[0], acc);
      }
      out[t * stride + r] = acc;
    }
}

/* One projection row: matmul_2d_quantized_batch (weights.inl:1297-1502) per
 * row is prepare (H128 or identity) then the DOT4 fma chain. */
static void project_row(const q35o_q4x8 *w, size_t rows, size_t cols, const float *x, int h128,
                        uint64_t seed, float *out, q35o_q8x1 *scratch) {
  if (h128)
    q35o_h128_prepare_activation_1(x, scratch, cols, seed);
  else
    q35o_q8_quantize_vector_1(x, scratch, cols / 32);
  q35o_dot4_matvec(w, scratch, out, rows, cols / 32);
}

/* run_linear_attention_step (layers.inl:36-217) for one row */
static void linear_step(const q35o_dims *d, const q35o_layer *L, float *conv_state, size_t *ring,
                        float *recurrent, const float *projected, float *core, float *tmp) {
  const size_t q_dim = (size_t)d->lin_k_heads * d->lin_k_dim;
  const size_t v_dim = (size_t)d->lin_v_heads * d->lin_v_dim;
  const size_t ch = 2 * q_dim + v_dim;
  const size_t K = (size_t)d->lin_kernel;
  const float *z = projected + ch, *bv = z + v_dim, *av = bv + d->lin_v_heads;
  float *beta = tmp, *alpha = beta + d->lin_v_heads, *conv_out = alpha + d->lin_v_heads;
  float *kmajor = conv_out + ch, *gq = kmajor + K * ch, *gk = gq + (size_t)d->lin_v_heads * d->lin_k_dim;
  for (int h = 0; h < d->lin_v_heads; ++h) {
    beta[h] = q35o_sigmoid(bv[h]);
    const float pre = q35o_softplus(av[h] + L->dt_bias[h]);
    alpha[h] = expf(pre * -expf(L->a_log[h]));
  }
  /* pack_conv1d_kernel_major (weights.inl:532-544) */
  for (size_t k = 0; k < K; ++k)
    for (size_t c = 0; c < ch; ++c) kmajor[k * ch + c] = L->conv_w[c * K + k];
  q35o_conv1d_silu(conv_state, *ring, projected, kmajor, conv_out, ch, K);
  *ring = (*ring + 1) % (K - 1);
  float *q = conv_out, *k = conv_out + q_dim, *v = conv_out + 2 * q_dim;
  q35o_l2_normalize(q, (size_t)d->lin_k_heads, (size_t)d->lin_k_dim, 1.0e-6f,
                    1.0f / sqrtf((float)d->lin_k_dim));
  q35o_l2_normalize(k, (size_t)d->lin_k_heads, (size_t)d->lin_k_dim, 1.0e-6f, 1.0f);
  const float *sq = q, *sk = k;
  if (d->lin_k_heads != d->lin_v_heads) {
    const int per = d->lin_v_heads / d->lin_k_heads;
    for (int h = 0; h < d->lin_v_heads; ++h) {
      memcpy(gq + (size_t)h * d->lin_k_dim, q + (size_t)(h / per) * d->lin_k_dim, d->lin_k_dim * sizeof(float));
      memcpy(gk + (size_t)h * d->lin_k_dim, k + (size_t)(h / per) * d->lin_k_dim, d->lin_k_dim * sizeof(float));
    }
    sq = gq;
    sk = gk;
  }
  float *delta_out = gk + (size_t)d->lin_v_heads * d->lin_k_dim;
  q35o_delta_net_update_rows(recurrent, sq, sk, v, alpha, beta, delta_out, (size_t)d->lin_k_dim,
                             (size_t)d->lin_v_dim, 0, (size_t)d->lin_v_heads * d->lin_v_dim);
  q35o_rms_norm(delta_out, L->lin_norm, core, (size_t)d->lin_v_heads, (size_t)d->lin_v_dim,
                d->rms_eps, 0.0f);
  q35o_silu_mul(z, core, core, v_dim);
}

/* prepare_full_attention_row + run_full_attention_step (layers.inl:221-395) */
static void full_step(const q35o_dims *d, const q35o_layer *L, uint16_t *keys, uint16_t *values,
                      size_t position, const float *cosine, const float *sine,
                      const float *projected, float *core, float *tmp) {
  const size_t hd = (size_t)d->head_dim, nh = (size_t)d->n_heads, kvh = (size_t)d->n_kv_heads;
  const size_t kvw = kvh * hd;
  float *q = tmp, *gate = q + nh * hd, *qn = gate + nh * hd, *kn = qn + nh * hd;
  float *scores = kn + kvw;
  for (size_t h = 0; h < nh; ++h) {
    memcpy(q + h * hd, projected + h * 2 * hd, hd * sizeof(float));
    memcpy(gate + h * hd, projected + h * 2 * hd + hd, hd * sizeof(float));
  }
  const float *kin = projected + nh * hd * 2, *vin = kin + kvw;
  q35o_rms_norm(q, L->q_norm, qn, nh, hd, d->rms_eps, 1.0f);
  q35o_rms_norm(kin, L->k_norm, kn, kvh, hd, d->rms_eps, 1.0f);
  q35o_rope(qn, nh, hd, (size_t)d->rope_dim, cosine, sine);
  q35o_rope(kn, kvh, hd, (size_t)d->rope_dim, cosine, sine);
  for (size_t i = 0; i < kvw; ++i) {
    keys[position * kvw + i] = q35o_attention_float_to_half(kn[i]);
    values[position * kvw + i] = q35o_attention_float_to_half(vin[i]);
  }
  const int seq = (int)position + 1;
  const uint16_t **krow = (const uint16_t **)malloc((size_t)seq * sizeof(void *));
  const uint16_t **vrow = (const uint16_t **)malloc((size_t)seq * sizeof(void *));
  for (int c = 0; c < seq; ++c) {
    krow[c] = keys + (size_t)c * kvw;
    vrow[c] = values + (size_t)c * kvw;
  }
  q35o_attention_decode(qn, gate, krow, vrow, scores, core, nh * hd, seq, (int)nh, (int)kvh,
                        (int)hd, 1.0f / sqrtf((float)hd), 0, nh);
  free(krow);
  free(vrow);
}

/* Stage entry points for stage-wise parity: one row of one layer's
 * attention block from given inputs (the same routines the whole step runs). */
int q35o_linear_attention_row(const q35o_dims *d, const q35o_layer *L, float *conv_state, size_t *ring,
                              float *recurrent, const float *projected, float *core) {
  const size_t q_dim = (size_t)d->lin_k_heads * d->lin_k_dim;
  const size_t v_dim = (size_t)d->lin_v_heads * d->lin_v_dim;
  const size_t ch = 2 * q_dim + v_dim;
  const size_t n = 16 * (ch + 2 * v_dim) + (size_t)d->lin_kernel * ch + 4 * v_dim + 64;
  float *tmp = (float *)malloc(n * sizeof(float));
  if (!tmp) return -1;
  linear_step(d, L, conv_state, ring, recurrent, projected, core, tmp);
  free(tmp);
  return 0;
}

int q35o_full_attention_row(const q35o_dims *d, const q35o_layer *L, uint16_t *keys, uint16_t *values,
                            size_t position, const float *cosine, const float *sine, const float *projected,
                            float *core) {
  const size_t full_core = (size_t)d->n_heads * d->head_dim;
  const size_t n = 4 * full_core + (size_t)d->n_kv_heads * d->head_dim + (size_t)d->n_heads * (position + 1) + 64;
  float *tmp = (float *)malloc(n * sizeof(float));
  if (!tmp) return -1;
  full_step(d, L, keys, values, position, cosine, sine, projected, core, tmp);
  free(tmp);
  return 0;
}

int q35o_forward_batch(const q35o_dims *d, const q35o_weights *w, q35o_state *const *states,
                       const int32_t *tokens, size_t batch, float penalty, int32_t *out_tokens,
                       float *out_logits, float *out_hidden) {
  const size_t H = (size_t)d->hidden, I = (size_t)d->intermediate, V = (size_t)d->vocab;
  const size_t q_dim = (size_t)d->lin_k_heads * d->lin_k_dim;
  const size_t v_dim = (size_t)d->lin_v_heads * d->lin_v_dim;
  const size_t ch = 2 * q_dim + v_dim;
  const size_t lin_in = ch + v_dim + 2 * (size_t)d->lin_v_heads;
  const size_t hd = (size_t)d->head_dim;
  const size_t full_in = (size_t)d->n_heads * hd * 2 + 2 * (size_t)d->n_kv_heads * hd;
  const size_t full_core = (size_t)d->n_heads * hd;
  size_t maxw = lin_in > full_in ? lin_in : full_in;
  if (2 * I > maxw) maxw = 2 * I;
  size_t maxk = H > I ? H : I;
  if (v_dim > maxk) maxk = v_dim;
  if (full_core > maxk) maxk = full_core;
  size_t max_pos = 0;
  for (size_t r = 0; r < batch; ++r)
    if (states[r]->position + 1 > max_pos) max_pos = states[r]->position + 1;
  const size_t half = (size_t)d->rope_dim / 2;
  const size_t tmp_n = 16 * maxw + (size_t)d->lin_kernel * ch + 4 * full_core +
                       (size_t)d->n_heads * max_pos + 64;
  float *x = (float *)malloc(H * sizeof(float));
  float *normed = (float *)malloc(maxk * sizeof(float));
  float *proj = (float *)malloc(maxw * sizeof(float));
  float *core = (float *)malloc(maxk * sizeof(float));
  float *resid = (float *)malloc(H * sizeof(float));
  float *hbuf = (float *)malloc(maxk * sizeof(float));
  float *tmp = (float *)malloc(tmp_n * sizeof(float));
  float *logits = (float *)malloc(V * sizeof(float));
  float *cosine = (float *)malloc(max_pos * half * sizeof(float));
  float *sine = (float *)malloc(max_pos * half * sizeof(float));
  q35o_q8x1 *prep = (q35o_q8x1 *)malloc((maxk / 32 + 1) * sizeof(q35o_q8x1));
  int ok = x && normed && proj && core && resid && hbuf && tmp && logits && cosine && sine && prep;
  if (ok) q35o_rope_tables(d->rope_theta, d->rope_dim, max_pos, cosine, sine);
  for (size_t r = 0; ok && r < batch; ++r) {
    q35o_state *s = states[r];
    if (w->embed_g16)
      q35o_g16_dequantize_row(w->embed_g16, (size_t)tokens[r], x, H / 32);
    else
      q35o_dot4_dequantize_row(w->embed, (size_t)tokens[r], x, H / 32);
    size_t li = 0, fi = 0;
    for (int l = 0; l < d->n_layers; ++l) {
      const q35o_layer *L = &w->layers[l];
      q35o_rms_norm(x, L->input_norm, normed, 1, H, d->rms_eps, 1.0f);
      if (L->is_linear) {
        /* a Q8 gate tail: the Q4 rows, then the gate rows from the
         * identity-basis input (run_q8_gate_tail, weights.inl:1015-1034) */
        project_row(L->in_proj, lin_in - (size_t)L->gate_rows, H, normed, 1, d->sign_seed, proj, prep);
        if (L->gate_rows > 0) {
          q35o_q8_quantize_vector_1(normed, prep, H / 32);
          q35o_q8_matmul(L->gate_q8, L->gate_scales, prep, proj + lin_in - (size_t)L->gate_rows,
                         (size_t)L->gate_rows, 1, H / 32, 0);
        }
        linear_step(d, L, s->conv_state[li], &s->conv_ring[li], s->recurrent[li], proj, core, tmp);
        project_row(L->out_proj, H, v_dim, core, 1, d->sign_seed, hbuf, prep);
        ++li;
      } else {
        project_row(L->in_proj, full_in, H, normed, 1, d->sign_seed, proj, prep);
        full_step(d, L, s->keys[fi], s->values[fi], s->position, cosine + s->position * half,
                  sine + s->position * half, proj, core, tmp);
        project_row(L->out_proj, H, full_core, core, 1, d->sign_seed, hbuf, prep);
        ++fi;
      }
      for (size_t i = 0; i < H; ++i) resid[i] = x[i] + hbuf[i];
      q35o_rms_norm(resid, L->post_norm, normed, 1, H, d->rms_eps, 1.0f);
      project_row(L->gate_up, 2 * I, H, normed, 1, d->sign_seed, proj, prep);
      q35o_silu_mul(proj, proj + I, core, I);
      project_row(L->down, H, I, core, 1, d->sign_seed, hbuf, prep);
      for (size_t i = 0; i < H; ++i) x[i] = resid[i] + hbuf[i];
    }
    q35o_rms_norm(x, w->final_norm, normed, 1, H, d->rms_eps, 1.0f);
    if (out_hidden) memcpy(out_hidden + r * H, normed, H * sizeof(float));
    if (w->embed_g16) {
      /* g16_matmul (gguf_matrix.inl:105-138): identity-basis X1 activations */
      q35o_q8_quantize_vector_1(normed, prep, H / 32);
      q35o_g16_matmul(w->embed_g16, prep, logits, V, 1, H / 32, V);
    } else {
      project_row(w->embed, V, H, normed, 0, 0, logits, prep);
    }
    if (out_logits) memcpy(out_logits + r * V, logits, V * sizeof(float));
    /* cpu_engine_greedy.inl:45-57 and :115-124: penalty, lowest index on ties */
    float best = -INFINITY;
    int32_t at = 0;
    for (size_t t = 0; t < V; ++t) {
      float val = logits[t];
      if (penalty > 1.0f && s->counts && s->counts[t] > 0) val = val > 0 ? val / penalty : val * penalty;
      if (val > best) { best = val; at = (int32_t)t; }
    }
    out_tokens[r] = at;
    ++s->position;
  }
  free(x); free(normed); free(proj); free(core); free(resid); free(hbuf); free(tmp);
  free(logits); free(cosine); free(sine); free(prep);
  return ok ? 0 : -1;
}
