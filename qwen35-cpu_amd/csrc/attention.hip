// Gated GQA full-attention decode over a paged FP16 KV pool.
//
// attn_prep: per (request, head) -- de-interleave [q | gate] (layers.inl:226-236),
//   per-head RMSNorm with (1 + w) (weights.inl:1517-1527), split-half RoPE on the
//   first rope_dim dims (activation.cpp:124-162), and the FP16 round-to-nearest
//   KV append of normalised K and raw V (full_attention.cpp:18-46, kv_pages.h:40-69).
// attention: split-K flash-decoding. One workgroup per (split of 256 context
//   tokens, KV head, request) serves all query heads of the GQA group, so each
//   K/V byte is read once. It walks the request's page table, scores with FP32
//   math over FP16 keys (full_attention.cpp:82-93), keeps the split's ungated
//   partial (max, sum, sum p*V); the splits are merged in order with the
//   reference rule merge_attention_partial (full_attention_tiled.cpp:66-78),
//   then normalised and multiplied by sigmoid(gate).
#include "q35_device.h"
#include "q35_internal.h"

namespace q35 {
namespace {

constexpr int kHeadDim = 256;
constexpr int kAttnThreads = 256;
constexpr int kMaxGroup = 8;  // query heads per KV head

__global__ __launch_bounds__(kAttnThreads) void attn_prep_kernel(AttnPrepArgs a) {
  __shared__ float scratch[8];
  __shared__ float ybuf[kHeadDim];
  const int r = blockIdx.x, slot = blockIdx.y, d = threadIdx.x;
  const int hd = a.head_dim;
  const bool is_q = slot < a.heads;
  const float *prow = a.proj + static_cast<size_t>(r) * a.proj_stride;
  float x = 0.0F;
  if (d < hd) {
    if (is_q) {
      x = prow[static_cast<size_t>(slot) * 2 * hd + d];
      a.gate_out[(static_cast<size_t>(r) * a.heads + slot) * hd + d] =
          prow[static_cast<size_t>(slot) * 2 * hd + hd + d];
    } else {
      x = prow[static_cast<size_t>(a.heads) * 2 * hd + static_cast<size_t>(slot - a.heads) * hd + d];
    }
  }
  const float ss = block_sum<kAttnThreads / 64>(x * x, scratch);
  const float inv = 1.0F / sqrtf(ss / static_cast<float>(hd) + a.eps);
  const float *w = is_q ? a.q_norm : a.k_norm;
  float y = d < hd ? x * inv * (w[d] + 1.0F) : 0.0F;
  if (d < hd) ybuf[d] = y;
  __syncthreads();
  const int pos = a.positions[r];
  const int half = a.rope_dim / 2;
  if (d < a.rope_dim) {
    const float cs = a.rope_cos[static_cast<size_t>(pos) * half + (d % half)];
    const float sn = a.rope_sin[static_cast<size_t>(pos) * half + (d % half)];
    if (d < half) {
      const float x0 = ybuf[d], x1 = ybuf[d + half];
      y = x0 * cs - x1 * sn;
    } else {
      const float x0 = ybuf[d - half], x1 = ybuf[d];
      y = x1 * cs + x0 * sn;
    }
  }
  if (d >= hd) return;
  if (is_q) {
    a.q_out[(static_cast<size_t>(r) * a.heads + slot) * hd + d] = y;
  } else {
    const int g = slot - a.heads;
    const int page = a.page_table[static_cast<size_t>(r) * a.max_pages + pos / a.page_tokens];
    const size_t row = (static_cast<size_t>(page) * a.page_tokens + pos % a.page_tokens) * a.kv_heads + g;
    a.k_pool[row * hd + d] = float_to_half_bits(y);
    const float v = prow[static_cast<size_t>(a.heads) * 2 * hd + static_cast<size_t>(a.kv_heads) * hd +
                         static_cast<size_t>(g) * hd + d];
    a.v_pool[row * hd + d] = float_to_half_bits(v);
  }
}

__device__ __forceinline__ void load_half16(const uint16_t *p, float out[16]) {
  const uint4 u0 = reinterpret_cast<const uint4 *>(p)[0];
  const uint4 u1 = reinterpret_cast<const uint4 *>(p)[1];
  const uint32_t w[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    out[2 * i] = half_bits_to_float(static_cast<uint16_t>(w[i] & 0xffffu));
    out[2 * i + 1] = half_bits_to_float(static_cast<uint16_t>(w[i] >> 16));
  }
}

// GQA group size QPK (query heads per KV head) is a template parameter.
template <int QPK>
__global__ __launch_bounds__(kAttnThreads) void attention_kernel(AttnArgs a) {
  Q35_DYNAMIC_SHARED(float, smem);  // scores [QPK][split_tokens], then reduction
  const int sp = blockIdx.x, g = blockIdx.y, r = blockIdx.z;
  const int seq = a.seq_lens != nullptr ? a.seq_lens[r] : a.positions[r] + 1;
  const int t0 = sp * a.split_tokens;
  if (t0 >= seq) return;
  const int t1 = min(seq, t0 + a.split_tokens);
  const int n = t1 - t0;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int kvw = a.kv_heads * kHeadDim;
  const int32_t *pt = a.page_table + static_cast<size_t>(r) * a.max_pages;
  float *scores = smem;  // [QPK][split_tokens]

  // ---- QK: 16 lanes per token, 16 dims per lane, four tokens per wave step
  const int sub = lane & 15, tslot = lane >> 4;
  float qv[QPK][16];
#pragma unroll
  for (int u = 0; u < QPK; ++u) {
    const float *qh = a.q + (static_cast<size_t>(r) * a.heads + g * QPK + u) * kHeadDim + 16 * sub;
#pragma unroll
    for (int i = 0; i < 16; ++i) qv[u][i] = qh[i];
  }
  for (int base = wave * 4; base < n; base += 16) {
    const int i = base + tslot;
    float part[QPK];
#pragma unroll
    for (int u = 0; u < QPK; ++u) part[u] = 0.0F;
    if (i < n) {
      const int tok = t0 + i;
      const int page = pt[tok / a.page_tokens];
      const uint16_t *krow =
          a.k_pool + (static_cast<size_t>(page) * a.page_tokens + tok % a.page_tokens) * kvw +
          static_cast<size_t>(g) * kHeadDim + 16 * sub;
      float kf[16];
      load_half16(krow, kf);
#pragma unroll
      for (int u = 0; u < QPK; ++u)
#pragma unroll
        for (int e = 0; e < 16; ++e) part[u] += qv[u][e] * kf[e];
    }
#pragma unroll
    for (int u = 0; u < QPK; ++u) {
      const float s = group_sum<16>(part[u]);
      if (sub == 0 && i < n) scores[u * a.split_tokens + i] = s * a.scale;
    }
  }
  __syncthreads();

  // ---- softmax statistics per query head (wave u owns head u, u += 4)
  __shared__ float s_max[kMaxGroup], s_sum[kMaxGroup];
  for (int u = wave; u < QPK; u += kAttnThreads / 64) {
    float m = -INFINITY;
    for (int i = lane; i < n; i += 64) m = fmaxf(m, scores[u * a.split_tokens + i]);
    m = group_max<64>(m);
    float l = 0.0F;
    for (int i = lane; i < n; i += 64) {
      const float p = expf(scores[u * a.split_tokens + i] - m);
      scores[u * a.split_tokens + i] = p;
      l += p;
    }
    l = group_sum<64>(l);
    if (lane == 0) {
      s_max[u] = m;
      s_sum[u] = l;
    }
  }
  __syncthreads();

  // ---- PV: lane owns 4 dims, waves split the tokens
  float acc[QPK][4];
#pragma unroll
  for (int u = 0; u < QPK; ++u) acc[u][0] = acc[u][1] = acc[u][2] = acc[u][3] = 0.0F;
  for (int i = wave; i < n; i += kAttnThreads / 64) {
    const int tok = t0 + i;
    const int page = pt[tok / a.page_tokens];
    const uint16_t *vrow =
        a.v_pool + (static_cast<size_t>(page) * a.page_tokens + tok % a.page_tokens) * kvw +
        static_cast<size_t>(g) * kHeadDim + 4 * lane;
    const uint2 raw = *reinterpret_cast<const uint2 *>(vrow);
    const float v0 = half_bits_to_float(raw.x & 0xffffu), v1 = half_bits_to_float(raw.x >> 16);
    const float v2 = half_bits_to_float(raw.y & 0xffffu), v3 = half_bits_to_float(raw.y >> 16);
#pragma unroll
    for (int u = 0; u < QPK; ++u) {
      const float p = scores[u * a.split_tokens + i];
      acc[u][0] += p * v0; acc[u][1] += p * v1; acc[u][2] += p * v2; acc[u][3] += p * v3;
    }
  }
  __syncthreads();  // scores no longer needed: reuse smem for the wave reduction
  float *red = smem;  // [4 waves][QPK][256]
#pragma unroll
  for (int u = 0; u < QPK; ++u)
#pragma unroll
    for (int e = 0; e < 4; ++e) red[(wave * QPK + u) * kHeadDim + 4 * lane + e] = acc[u][e];
  __syncthreads();
  for (int idx = tid; idx < QPK * kHeadDim; idx += kAttnThreads) {
    const int u = idx / kHeadDim, dd = idx % kHeadDim;
    float v = 0.0F;
#pragma unroll
    for (int w = 0; w < kAttnThreads / 64; ++w) v += red[(w * QPK + u) * kHeadDim + dd];
    const size_t hs = (static_cast<size_t>(r) * a.heads + g * QPK + u) * a.max_splits + sp;
    a.part_o[hs * kHeadDim + dd] = v;
    if (dd == 0) {
      a.part_ml[hs * 2] = s_max[u];
      a.part_ml[hs * 2 + 1] = s_sum[u];
    }
  }
}

__global__ void attention_merge_kernel(AttnArgs a, const float *gates, float *out) {
  const int h = blockIdx.x, r = blockIdx.y, d = threadIdx.x;
  const int seq = a.seq_lens != nullptr ? a.seq_lens[r] : a.positions[r] + 1;
  const int splits = (seq + a.split_tokens - 1) / a.split_tokens;
  const size_t hs = (static_cast<size_t>(r) * a.heads + h) * a.max_splits;
  float m = 0.0F, l = 0.0F, v = 0.0F;
  for (int s = 0; s < splits; ++s) {
    const float om = a.part_ml[(hs + s) * 2], ol = a.part_ml[(hs + s) * 2 + 1];
    const float ov = a.part_o[(hs + s) * kHeadDim + d];
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
  const size_t o = (static_cast<size_t>(r) * a.heads + h) * kHeadDim + d;
  out[o] = (v * inv) * sigmoid_stable(gates[o]);
}

}  // namespace

hipError_t launch_attn_prep(const AttnPrepArgs &a, hipStream_t stream) {
  if (a.batch <= 0) return hipSuccess;
  if (a.head_dim > kHeadDim || a.rope_dim > a.head_dim) return hipErrorInvalidValue;
  Q35_LAUNCH((attn_prep_kernel), dim3(a.batch, a.heads + a.kv_heads), kAttnThreads, 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_attention(const AttnArgs &a, hipStream_t stream) {
  if (a.batch <= 0) return hipSuccess;
  if (a.head_dim != kHeadDim || a.heads % a.kv_heads != 0) return hipErrorInvalidValue;
  const int qpk = a.heads / a.kv_heads;
  const size_t score_bytes = static_cast<size_t>(qpk) * a.split_tokens * sizeof(float);
  const size_t red_bytes = static_cast<size_t>(4) * qpk * kHeadDim * sizeof(float);
  const size_t smem = score_bytes > red_bytes ? score_bytes : red_bytes;
  const dim3 grid(a.max_splits, a.kv_heads, a.batch), block(kAttnThreads);
  switch (qpk) {
    case 1: Q35_LAUNCH((attention_kernel<1>), grid, block, smem, stream, a); break;
    case 2: Q35_LAUNCH((attention_kernel<2>), grid, block, smem, stream, a); break;
    case 4: Q35_LAUNCH((attention_kernel<4>), grid, block, smem, stream, a); break;
    case 8: Q35_LAUNCH((attention_kernel<8>), grid, block, smem, stream, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_attention_merge(const AttnArgs &a, const float *gates, float *out,
                                  hipStream_t stream) {
  Q35_LAUNCH((attention_merge_kernel), dim3(a.heads, a.batch), kHeadDim, 0, stream, a, gates, out);
  return hipGetLastError();
}

}  // namespace q35
