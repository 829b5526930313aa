// Gated GQA full-attention decode over a paged FP16 KV pool.
//
// attn_prep: per (request, head) -- de-interleave [q | gate] (layers.inl:226-236),
//   per-head RMSNorm with (1 + w) (weights.inl:1517-1527), split-half RoPE on the
//   first rope_dim dims (activation.cpp:124-162), and the FP16 round-to-nearest
//   KV append of normalised K and raw V (full_attention.cpp:18-46, kv_pages.h:40-69).
// attention: split-K flash-decoding over chunks of 64 context tokens (one
//   workgroup per chunk, KV head and request -- or, for the rows of a prefill
//   segment, per chunk, KV head and tile of up to kAttnTileRows positions,
//   which then share one load of the chunk's K and V; see attention_kernel), then
//   attention_merge_kernel: log-sum-exp merge of the chunks, normalisation and
//   sigmoid(gate), written as FP32 or prepared as the o projection's A16
//   activations.
#include <algorithm>

#include "q35_quant.h"

namespace q35 {
namespace {

constexpr int kHeadDim = 256;
constexpr int kAttnThreads = 256;

template <int MS>  // bound on the qkv projection's K splits
__global__ __launch_bounds__(kAttnThreads) void attn_prep_kernel(AttnPrepArgs a) {
  __shared__ float scratch[8];
  __shared__ float ybuf[kHeadDim];
  const int r = blockIdx.x, slot = blockIdx.y, d = threadIdx.x;
  const int hd = a.head_dim;
  const bool is_q = slot < a.heads;
  const int g = max(slot - a.heads, 0);
  const int dd = min(d, hd - 1);  // threads past head_dim mirror a valid column and store nothing
  // every load that does not depend on the projection is issued first, so
  // the kernel waits on one round trip (the position's page and RoPE row
  // behind the position itself)
  const int pos = a.positions[r];
  const float *w = is_q ? a.q_norm : a.k_norm;
  const float w1 = w[dd] + 1.0F;
  const int half = a.rope_dim / 2;
  const int rd = min(d, a.rope_dim - 1) % half;
  const float cs = a.rope_cos[static_cast<size_t>(pos) * half + rd];
  const float sn = a.rope_sin[static_cast<size_t>(pos) * half + rd];
  const int pshift = __builtin_ctz(static_cast<unsigned>(a.page_tokens));  // a power of two
  const int prow = a.row_seg != nullptr ? a.row_seg[r] : r;
  const int page = a.page_table[static_cast<size_t>(prow) * a.max_pages + (pos >> pshift)];
  // q head: [q | gate] of the head; k head: its K row and its V row
  const int col_x = is_q ? slot * 2 * hd + dd : a.heads * 2 * hd + g * hd + dd;
  const int col_2 = is_q ? slot * 2 * hd + hd + dd : a.heads * 2 * hd + a.kv_heads * hd + g * hd + dd;
  const float x = d < hd ? a.proj.template sum<MS>(r, col_x) : 0.0F;
  const float second = a.proj.template sum<MS>(r, col_2);
  if (is_q && d < hd) a.gate_out[(static_cast<size_t>(r) * a.heads + slot) * hd + d] = second;
  const float ss = block_sum<kAttnThreads / 64>(x * x, scratch);
  const float inv = 1.0F / sqrtf(ss / static_cast<float>(hd) + a.eps);
  float y = d < hd ? x * inv * w1 : 0.0F;
  if (d < hd) ybuf[d] = y;
  lds_barrier();
  if (d < a.rope_dim) {
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
    const size_t row = ((static_cast<size_t>(page) << pshift) + (pos & (a.page_tokens - 1))) * a.kv_heads + g;
    a.k_pool[row * hd + d] = float_to_half_bits(y);
    a.v_pool[row * hd + d] = float_to_half_bits(second);
  }
}

// ---------------------------------------------------------------- attention
// One workgroup of 512 threads per (chunk of kChunkTokens context tokens, KV
// head, request) serves the QPK query heads of the GQA group, so every K/V
// byte is read once. Thread t scores token t/8 over dims 32*(t%8)..+31 (four
// 16-byte K loads) and accumulates P*V for dims 4*(t%64)..+3 over tokens
// t/64 + 8j (eight 8-byte V loads). The page-table entries are loaded together
// with the context length (a slot past the context reads the chunk's first
// page and gets probability zero), so K and V are issued after one round
// trip. Scores are FP32 dot products over FP16 keys (full_attention.cpp:82-93);
// the chunk leaves its partial (max, sum, sum p*V) for the merge.
constexpr int kChunkTokens = 64;
constexpr int kScoreThreads = 512;
constexpr int kScoreWaves = kScoreThreads / 64;
constexpr int kQStride = 36;  // 32 dims + 4: the eight dim slices land on distinct LDS banks

template <int QPK, bool TILED>
__global__ __launch_bounds__(kScoreThreads) __attribute__((amdgpu_waves_per_eu(4))) void attention_kernel(AttnArgs a) {
  constexpr int NQ = (QPK * kHeadDim + kScoreThreads - 1) / kScoreThreads;  // query values staged per thread
  __shared__ float qs[QPK * 8 * kQStride];
  __shared__ float probs[QPK][kChunkTokens];
  __shared__ float s_m[QPK], s_l[QPK];
  __shared__ float red[kScoreWaves][QPK][kHeadDim];
  const int sp = blockIdx.x, g = blockIdx.y;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int kq = tid & 7, ti = tid >> 3;
  const int t0 = sp * kChunkTokens;
  const int kvw = a.kv_heads * kHeadDim;
  // the rows of this workgroup: one request row, or a tile of consecutive
  // positions of one segment (they share its page table, and the last row
  // has the longest context)
  const int r0 = TILED ? a.tile_row0[blockIdx.z] : static_cast<int>(blockIdx.z);
  const int nrows = TILED ? a.tile_rows[blockIdx.z] : 1;
  const int32_t *pt = a.page_table + static_cast<size_t>(a.row_seg != nullptr ? a.row_seg[r0] : r0) * a.max_pages;
  const int last_page = a.max_pages - 1;
  // page_tokens is a power of two: shifts and masks, not integer division
  const int pshift = __builtin_ctz(static_cast<unsigned>(a.page_tokens)), pmask = a.page_tokens - 1;
  auto seq_of = [&](int r) { return a.seq_lens != nullptr ? a.seq_lens[r] : a.positions[r] + 1; };
  auto load_q = [&](int r, float qv[NQ]) {
#pragma unroll
    for (int k = 0; k < NQ; ++k) {
      const int e = min(tid + k * kScoreThreads, QPK * kHeadDim - 1);
      qv[k] = a.q[(static_cast<size_t>(r) * a.heads + g * QPK + e / kHeadDim) * kHeadDim + e % kHeadDim];
    }
  };
  // one round trip: the query heads, the context length and the page-table
  // entries of every token slot (clamped into the row)
  float qv[NQ];
  load_q(r0, qv);
  const int seq_tile = seq_of(r0 + nrows - 1);
  const int pfirst = pt[min(t0 >> pshift, last_page)];
  const int pk = pt[min((t0 + ti) >> pshift, last_page)];
  int pv[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) pv[j] = pt[min((t0 + wave + 8 * j) >> pshift, last_page)];
  if (t0 >= seq_tile) return;  // whole workgroup
  const int n_tile = min(seq_tile - t0, kChunkTokens);

  // K, then V (the memory counter retires loads in issue order); slots past
  // the tile's context read the chunk's first token
  const bool kload = ti < n_tile;
  const int ktok = kload ? t0 + ti : t0;
  const q35_u32x4 *krow = reinterpret_cast<const q35_u32x4 *>(
      a.k_pool + ((static_cast<size_t>(kload ? pk : pfirst) << pshift) + (ktok & pmask)) * kvw +
      static_cast<size_t>(g) * kHeadDim + 32 * kq);
  q35_u32x4 kraw[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) kraw[i] = Q35_LOAD_NT(krow + i);
  q35_u32x2 vraw[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const bool vin = wave + 8 * j < n_tile;
    const int vt = vin ? t0 + wave + 8 * j : t0;
    vraw[j] = Q35_LOAD_NT(reinterpret_cast<const q35_u32x2 *>(
        a.v_pool + ((static_cast<size_t>(vin ? pv[j] : pfirst) << pshift) + (vt & pmask)) * kvw +
        static_cast<size_t>(g) * kHeadDim + 4 * lane));
  }

  for (int i = 0; i < nrows; ++i) {
    const int r = r0 + i;
    const int seq = TILED ? seq_of(r) : seq_tile;
    if (t0 >= seq) {  // this row's context ends before the chunk (uniform)
      if (TILED && i + 1 < nrows) load_q(r + 1, qv);
      continue;
    }
    // tokens past the row's context score -inf and get probability exactly 0
    // (their V rows are finite), so a row's partial does not depend on the
    // tile it runs in
    const int n = min(seq - t0, kChunkTokens);
    const bool kin = ti < n;

    // the group's query heads into LDS, in eight padded 32-dim slices (the
    // previous row's readers passed the barriers of its softmax and P*V)
#pragma unroll
    for (int k = 0; k < NQ; ++k) {
      const int e = tid + k * kScoreThreads;
      if (e < QPK * kHeadDim) {
        const int u = e / kHeadDim, d = e % kHeadDim;
        qs[(u * 8 + d / 32) * kQStride + d % 32] = qv[k];
      }
    }
    if (TILED && i + 1 < nrows) load_q(r + 1, qv);  // the next row's query, in flight meanwhile
    lds_barrier();

    // ---- scores: 32 dims per thread, then the 8 lanes of the token
    float part[QPK];
#pragma unroll
    for (int u = 0; u < QPK; ++u) part[u] = 0.0F;
#pragma unroll
    for (int i4 = 0; i4 < 4; ++i4) {
      float kf[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        kf[2 * e] = half_bits_to_float(static_cast<uint16_t>(kraw[i4][e] & 0xffffu));
        kf[2 * e + 1] = half_bits_to_float(static_cast<uint16_t>(kraw[i4][e] >> 16));
      }
#pragma unroll
      for (int u = 0; u < QPK; ++u) {
        const float *qp = qs + (u * 8 + kq) * kQStride + 8 * i4;
        const q35_f32x4 qa = *reinterpret_cast<const q35_f32x4 *>(qp);
        const q35_f32x4 qb = *reinterpret_cast<const q35_f32x4 *>(qp + 4);
        part[u] += qa[0] * kf[0] + qa[1] * kf[1] + qa[2] * kf[2] + qa[3] * kf[3] + qb[0] * kf[4] +
                   qb[1] * kf[5] + qb[2] * kf[6] + qb[3] * kf[7];
      }
      // one iteration at a time: no hoisted query reads, no sunk dot products
#pragma unroll
      for (int u = 0; u < QPK; ++u) q35_materialize(part[u]);
      q35_compiler_fence();
    }
#pragma unroll
    for (int u = 0; u < QPK; ++u) {
      part[u] += q35_row_xor(part[u], 1);
      part[u] += q35_row_xor(part[u], 2);
      part[u] += q35_row_xor(part[u], 4);
      if (kq == 0) probs[u][ti] = kin ? part[u] * a.scale : -INFINITY;
    }
    lds_barrier();

    // ---- chunk softmax statistics (wave u handles head u)
    for (int u = wave; u < QPK; u += kScoreWaves) {
      const float s = probs[u][lane];
      const float m = group_max<64>(s);
      const float p = lane < n ? expf(s - m) : 0.0F;
      const float l = group_sum<64>(p);
      probs[u][lane] = p;
      if (lane == 0) {
        s_m[u] = m;
        s_l[u] = l;
      }
    }
    lds_barrier();

    // ---- P*V over this wave's tokens, then the fixed-order wave sum
    float acc[QPK][4];
#pragma unroll
    for (int u = 0; u < QPK; ++u) acc[u][0] = acc[u][1] = acc[u][2] = acc[u][3] = 0.0F;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int t = wave + 8 * j;
      const float v0 = half_bits_to_float(static_cast<uint16_t>(vraw[j][0] & 0xffffu));
      const float v1 = half_bits_to_float(static_cast<uint16_t>(vraw[j][0] >> 16));
      const float v2 = half_bits_to_float(static_cast<uint16_t>(vraw[j][1] & 0xffffu));
      const float v3 = half_bits_to_float(static_cast<uint16_t>(vraw[j][1] >> 16));
#pragma unroll
      for (int u = 0; u < QPK; ++u) {
        const float p = probs[u][t];  // 0 past the row's tokens
        acc[u][0] += p * v0;
        acc[u][1] += p * v1;
        acc[u][2] += p * v2;
        acc[u][3] += p * v3;
      }
#pragma unroll
      for (int u = 0; u < QPK; ++u)
#pragma unroll
        for (int k = 0; k < 4; ++k) q35_materialize(acc[u][k]);
      q35_compiler_fence();
    }
#pragma unroll
    for (int u = 0; u < QPK; ++u)
      *reinterpret_cast<q35_f32x4 *>(&red[wave][u][4 * lane]) = q35_f32x4{acc[u][0], acc[u][1], acc[u][2], acc[u][3]};
    lds_barrier();
    for (int e = tid; e < QPK * kHeadDim; e += kScoreThreads) {
      const int u = e / kHeadDim, d = e % kHeadDim;
      float v = red[0][u][d];
#pragma unroll
      for (int w = 1; w < kScoreWaves; ++w) v += red[w][u][d];
      const size_t hs = (static_cast<size_t>(r) * a.heads + g * QPK + u) * a.max_splits + sp;
      a.part_o[hs * kHeadDim + d] = v;
      if (d == 0) {
        a.part_ml[hs * 2] = s_m[u];
        a.part_ml[hs * 2 + 1] = s_l[u];
      }
    }
  }
}

// Merge of the chunk partials of one (request, head): log-sum-exp weights
// exp(m_s - M) over all chunks (the same result as merging them pairwise with
// merge_attention_partial, full_attention_tiled.cpp:66-78, up to rounding),
// normalisation, and the sigmoid output gate (full_attention.cpp:104-127).
// One wavefront per (128-dim block b, head h, request): lane j = lane % 16
// holds dims 128b + 8j .. +7 -- one H128 block of the o projection's input --
// and the result is stored as FP32 and/or prepared as A16 activations (the
// four 16-lane rows compute the same values; row 0 stores). The gate row and
// the partial rows of the first kMergeBatch chunks are loaded together with
// the chunk statistics, right after the context length.
constexpr int kMergeBatch = 16;

__global__ __launch_bounds__(64) void attention_merge_kernel(AttnArgs a, const float *gates, float *out,
                                                            QuantOut qo, uint64_t seed) {
  const int b = blockIdx.x & 1, h = blockIdx.x >> 1, r = blockIdx.y;
  const int lane = threadIdx.x, j = lane & 15;
  const size_t hs = (static_cast<size_t>(r) * a.heads + h) * a.max_splits;
  const int d0 = 128 * b + 8 * j;
  const size_t o = (static_cast<size_t>(r) * a.heads + h) * kHeadDim + d0;
  const q35_f32x4 gate_lo = *reinterpret_cast<const q35_f32x4 *>(gates + o);
  const q35_f32x4 gate_hi = *reinterpret_cast<const q35_f32x4 *>(gates + o + 4);
  const int seq = a.seq_lens != nullptr ? a.seq_lens[r] : a.positions[r] + 1;
  const int splits = (seq + kChunkTokens - 1) / kChunkTokens;
  q35_f32x4 rows[kMergeBatch][2];
  auto load_rows = [&](int s0) {
#pragma unroll
    for (int u = 0; u < kMergeBatch; ++u) {
      const q35_f32x4 *src = reinterpret_cast<const q35_f32x4 *>(a.part_o + (hs + min(s0 + u, splits - 1)) * kHeadDim + d0);
      rows[u][0] = src[0];
      rows[u][1] = src[1];
    }
  };
  // chunk statistics of chunks lane, lane + 64, ...: the first batch of 64
  // stays in registers
  float m0 = -INFINITY, l0 = 0.0F;
  {
    const int s = min(lane, splits - 1);
    m0 = a.part_ml[(hs + s) * 2];
    l0 = a.part_ml[(hs + s) * 2 + 1];
    if (lane >= splits) m0 = -INFINITY;
  }
  load_rows(0);
  float M = m0;
  for (int s = lane + 64; s < splits; s += 64) M = fmaxf(M, a.part_ml[(hs + s) * 2]);
  M = group_max<64>(M);
  float acc[8] = {0.0F, 0.0F, 0.0F, 0.0F, 0.0F, 0.0F, 0.0F, 0.0F};
  float L = 0.0F;
  for (int s0 = 0; s0 < splits; s0 += 64) {
    const int cnt = min(64, splits - s0);
    float m = m0, l = l0;
    if (s0 > 0 && lane < cnt) {
      m = a.part_ml[(hs + s0 + lane) * 2];
      l = a.part_ml[(hs + s0 + lane) * 2 + 1];
    }
    float w = 0.0F, lw = 0.0F;
    if (lane < cnt) {
      w = expf(m - M);
      lw = w * l;
    }
    L += group_sum<64>(lw);
    for (int s = 0; s < cnt; s += kMergeBatch) {
      if (s0 + s > 0) load_rows(s0 + s);
#pragma unroll
      for (int u = 0; u < kMergeBatch; ++u) {
        if (s + u >= cnt) break;
        const float ws = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), s + u));
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          acc[e] += ws * rows[u][0][e];
          acc[4 + e] += ws * rows[u][1][e];
        }
      }
    }
  }
  const float inv = 1.0F / (L > 0.0F ? L : 1.0F);
  float y[8];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    y[e] = (acc[e] * inv) * sigmoid_stable(gate_lo[e]);
    y[4 + e] = (acc[4 + e] * inv) * sigmoid_stable(gate_hi[e]);
  }
  if (out != nullptr && lane < 16)
#pragma unroll
    for (int e = 0; e < 8; ++e) out[o + e] = y[e];
  if (qo.codes != nullptr) h128_quantize_row16(y, r, 2 * h + b, a.heads * kHeadDim / 32, true, seed, qo, lane < 16);
}

}  // namespace

hipError_t launch_attn_prep(const AttnPrepArgs &a, hipStream_t stream) {
  if (a.batch <= 0) return hipSuccess;
  if (a.head_dim > kHeadDim || a.rope_dim > a.head_dim) return hipErrorInvalidValue;
  const dim3 grid(a.batch, a.heads + a.kv_heads);
  switch (split_bound(a.proj.splits)) {
    case 1: Q35_LAUNCH((attn_prep_kernel<1>), grid, kAttnThreads, 0, stream, a); break;
    case 4: Q35_LAUNCH((attn_prep_kernel<4>), grid, kAttnThreads, 0, stream, a); break;
    case 8: Q35_LAUNCH((attn_prep_kernel<8>), grid, kAttnThreads, 0, stream, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_attention(const AttnArgs &a, hipStream_t stream) {
  if (a.batch <= 0) return hipSuccess;
  if (a.head_dim != kHeadDim || a.heads % a.kv_heads != 0 || a.split_tokens != kChunkTokens)
    return hipErrorInvalidValue;
  const int qpk = a.heads / a.kv_heads;
  const bool tiled = a.tile_row0 != nullptr;
  const int gs = a.grid_splits > 0 ? std::min(a.grid_splits, a.max_splits) : a.max_splits;
  const dim3 grid(gs, a.kv_heads, tiled ? a.tiles : a.batch), block(kScoreThreads);
#define Q35_ATTN(Q)                                                             \
  if (tiled)                                                                    \
    Q35_LAUNCH((attention_kernel<Q, true>), grid, block, 0, stream, a);        \
  else                                                                          \
    Q35_LAUNCH((attention_kernel<Q, false>), grid, block, 0, stream, a);
  switch (qpk) {
    case 1: Q35_ATTN(1) break;
    case 2: Q35_ATTN(2) break;
    case 4: Q35_ATTN(4) break;
    case 8: Q35_ATTN(8) break;
    default: return hipErrorInvalidValue;
  }
#undef Q35_ATTN
  return hipGetLastError();
}

hipError_t launch_attention_merge(const AttnArgs &a, const float *gates, float *out, uint64_t *codes,
                                  float *scales, uint64_t seed, hipStream_t stream) {
  if (a.batch <= 0) return hipSuccess;
  if (a.head_dim != kHeadDim || a.split_tokens != kChunkTokens) return hipErrorInvalidValue;
  QuantOut qo;
  qo.codes = codes;
  qo.scales = scales;
  Q35_LAUNCH((attention_merge_kernel), dim3(2 * a.heads, a.batch), 64, 0, stream, a, gates, out, qo, seed);
  return hipGetLastError();
}

}  // namespace q35
