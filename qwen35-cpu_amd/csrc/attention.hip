// Gated GQA full-attention decode over a paged FP16 KV pool.
//
// attn_prep: per (request, head) -- de-interleave [q | gate] (layers.inl:226-236),
//   per-head RMSNorm with (1 + w) (weights.inl:1517-1527), split-half RoPE on the
//   first rope_dim dims (activation.cpp:124-162), and the FP16 round-to-nearest
//   KV append of normalised K and raw V (full_attention.cpp:18-46, kv_pages.h:40-69).
// attention: split-K flash-decoding over chunks of 64 context tokens, one
//   workgroup per chunk, KV head and request (attention_kernel); the rows of
//   prompt segments run as tiles of up to kAttnTileRows positions, one
//   workgroup per tile and KV head walking the chunks and merging them itself
//   (attention_flash_kernel). Then attention_merge_kernel: log-sum-exp merge
//   of the chunks, normalisation and sigmoid(gate), written as FP32 or
//   prepared as the o projection's A16 activations (attention_finish_kernel
//   for the prompt rows, whose chunks are merged already).
#include <algorithm>

#include "q35_quant.h"

namespace q35 {
namespace {

constexpr int kHeadDim = 256;
constexpr int kAttnThreads = 256;

// The head preparation's roundings, contraction off: the squares of the
// per-head RMSNorm, its 1 / sqrt(mean square + eps) over 256 dims (the mean a
// rounding of its own: a constant divisor would otherwise fold into an fma
// with eps), and the split-half RoPE pair (d < half: x0 = y[d],
// x1 = y[d + half]; the upper dim of the pair: x0 = y[d - half], x1 = y[d]).
__device__ __forceinline__ float head_sq(float x) {
#pragma clang fp contract(off)
  return x * x;
}
__device__ __forceinline__ float head_rms_inv(float ss, float eps) {
#pragma clang fp contract(off)
  return 1.0F / sqrtf(ss / static_cast<float>(kHeadDim) + eps);
}
__device__ __forceinline__ float rope_lower(float x0, float x1, float cs, float sn) {
#pragma clang fp contract(off)
  return x0 * cs - x1 * sn;
}
__device__ __forceinline__ float rope_upper(float x0, float x1, float cs, float sn) {
#pragma clang fp contract(off)
  return x1 * cs + x0 * sn;
}

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
  const float ss = block_sum<kAttnThreads / 64>(head_sq(x), scratch);
  const float inv = head_rms_inv(ss, a.eps);  // head_dim is 256 (launch_attn_prep)
  float y = d < hd ? x * inv * w1 : 0.0F;
  if (d < hd) ybuf[d] = y;
  lds_barrier();
  if (d < a.rope_dim) y = d < half ? rope_lower(ybuf[d], ybuf[d + half], cs, sn) : rope_upper(ybuf[d - half], ybuf[d], cs, sn);
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
// Scores and P*V run on v_mfma_f32_16x16x32_f16 over 64-token chunks of the
// paged FP16 cache (full_attention.cpp:82-127 computes them as FP32 dot
// products over FP16 keys and values). An M tile holds 16 query vectors:
//   S[m][t] = sum_d q[m][d] k[t][d]: A = the queries, B = the keys (lane l
//     holds dims 32kk + 8(l/16) .. +7 of token l%16 -- 16 contiguous bytes of
//     its cache row), the eight 32-dim steps accumulated in order;
//   O[m][d] = sum_t p[m][t] v[t][d]: A = the probabilities, B = V^T staged
//     in LDS, the two 32-token steps accumulated in order.
// The FP32 queries and probabilities enter as two FP16 operands each,
// hi = binary16(x) and lo = binary16(x - hi), so every product with an FP16
// key or value is exact in FP32 and x is carried to 22 significant bits
// (|q| below 65504; probabilities are in [0, 1]). Each output element of an
// MFMA depends only on its own A row, B column and C element, so a query's
// scores, statistics and partial do not depend on which M row it occupies or
// what else shares the tile: the decode kernel (one request row, its QPK
// heads in an M tile) and the tiled prefill kernel (16 positions of a head
// in an M tile) give every row the same bits.
// Per chunk and query the softmax takes the maximum over the chunk's tokens,
// p = exp(s - max) (0 past the row's context), and the sum of p as a tree
// over each 16-token tile (the xor-1/2/4/8 exchange) added tile by tile;
// the partial (max, sum, sum p*V) goes to attention_merge_kernel.
constexpr int kChunkTokens = 64;
constexpr int kKStride = kHeadDim + 8;  // halfs per staged K row: the lanes' 16-byte key reads spread over the banks
constexpr int kPStride = kChunkTokens + 4;  // floats per probability row in LDS

// The query operands of one lane (query l % 16): dims 32kk + 8(l/16) .. +7
// of the query for kk = 0..7, as hi and lo parts (zeros when !live).
struct QOps {
  q35_f16x8 hi[8], lo[8];
};
__device__ __forceinline__ void load_q_ops(const float *q, bool live, int lane, QOps &o) {
  const int kg = lane >> 4;
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) {
    float x[8];
    if (live) {
      const q35_f32x4 a = *reinterpret_cast<const q35_f32x4 *>(q + 32 * kk + 8 * kg);
      const q35_f32x4 b = *reinterpret_cast<const q35_f32x4 *>(q + 32 * kk + 8 * kg + 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        x[i] = a[i];
        x[4 + i] = b[i];
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) x[i] = 0.0F;
    }
    q35_split_f16(x, o.hi[kk], o.lo[kk]);
  }
}

// Scores of a 16-token tile; key(kk) is the lane's key operand of step kk.
// Lane l receives S[4(l/16) + j][l % 16], j = 0..3.
template <typename Key>
__device__ __forceinline__ q35_f32x4 qk_tile(const QOps &q, Key key) {
  q35_f32x4 c = {0.0F, 0.0F, 0.0F, 0.0F};
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) {
    const q35_f16x8 k = key(kk);
    c = Q35_MFMA_F32_16X16X32_F16(q.hi[kk], k, c);
    c = Q35_MFMA_F32_16X16X32_F16(q.lo[kk], k, c);
  }
  return c;
}

__device__ __forceinline__ float tile_max(float v) {
  v = fmaxf(v, q35_row_xor(v, 1));
  v = fmaxf(v, q35_row_xor(v, 2));
  v = fmaxf(v, q35_row_xor(v, 4));
  return fmaxf(v, q35_row_xor(v, 8));
}
__device__ __forceinline__ float tile_sum(float v) { return row_sum16(v); }

// The probability operands of one lane (query l % 16): tokens
// 32ks + 8(l/16) .. +7 of the row in `pl` for ks = 0, 1.
__device__ __forceinline__ void load_p_ops(const float *pl, int lane, q35_f16x8 hi[2], q35_f16x8 lo[2]) {
  const float *row = pl + (lane & 15) * kPStride + 8 * (lane >> 4);
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    const q35_f32x4 a = *reinterpret_cast<const q35_f32x4 *>(row + 32 * ks);
    const q35_f32x4 b = *reinterpret_cast<const q35_f32x4 *>(row + 32 * ks + 4);
    float x[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[i] = a[i];
      x[4 + i] = b[i];
    }
    q35_split_f16(x, hi[ks], lo[ks]);
  }
}

// P*V of dims 16dt .. 16dt+15 from a V chunk staged transposed in LDS
// (vt[dim][token], row stride kVTStride): the value operand of lane l is the
// 16 bytes of dim 16dt + l%16, tokens 32ks + 8(l/16) .. +7 (token
// 32ks + 8(l/16) + i at k index 8(l/16) + i, as in the decode kernel's
// register operands), read whole by one 16-byte LDS load.
constexpr int kVTStride = kChunkTokens + 8;  // halfs per staged dim row: 16 rows of an operand read on distinct banks
__device__ __forceinline__ q35_f32x4 pvt_tile(const q35_f16x8 phi[2], const q35_f16x8 plo[2], const uint16_t *vt,
                                              int dt, int lane) {
  const uint16_t *row = vt + (16 * dt + (lane & 15)) * kVTStride + 8 * (lane >> 4);
  q35_f32x4 c = {0.0F, 0.0F, 0.0F, 0.0F};
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    const q35_f16x8 v = q35_f16x8_bits(*reinterpret_cast<const q35_u32x4 *>(row + 32 * ks));
    c = Q35_MFMA_F32_16X16X32_F16(phi[ks], v, c);
    c = Q35_MFMA_F32_16X16X32_F16(plo[ks], v, c);
  }
  return c;
}

// The value operands of P*V taken straight from global memory: lane l
// (column n = l % 16, token group tg = l / 16) of wavefront w loads 8 bytes,
// dims 64w + 4n .. +3, of tokens 32ks + 8tg + i (i = 0..7) per 32-token step
// ks -- each group of 16 lanes reads 128 contiguous bytes of a cache row --
// and regroups them in registers: operand (ks, j) holds dim 64w + 4n + j of
// its eight tokens, two per dword. Token 32ks + 8tg + i sits at k index
// 8tg + i of step ks, as in the LDS-staged form (pv_tile), so every output
// element sees the same products in the same order; only the dim a column
// stands for changes.
struct VOps {
  q35_u32x2 raw[2][8];  // [ks][i]: 4 dims of one token
};
__device__ __forceinline__ q35_f16x8 v_operand(const VOps &v, int ks, int j) {
  // binary16 j of each token: low half of dword j/2 for even j, high half for odd
  const unsigned sel = (j & 1) ? 0x07060302u : 0x05040100u;
  q35_u32x4 d;
#pragma unroll
  for (int p = 0; p < 4; ++p)
    d[p] = __builtin_amdgcn_perm(v.raw[ks][2 * p + 1][j >> 1], v.raw[ks][2 * p][j >> 1], sel);
  return q35_f16x8_bits(d);
}

// Decode: one workgroup of 4 wavefronts per (chunk, KV head, request row);
// the row's QPK heads are the live rows of one M tile. Wavefront w scores
// token tile w (its keys loaded straight into operands); the tile maxima and
// sums meet in LDS; wavefront w then forms P*V for dims 64w .. 64w+63 from
// value operands loaded straight into registers (VOps). The loads are issued
// queries (staged in LDS), keys, values, so the scores and the softmax run
// while the values are still in flight. Occupancy floor 2 keeps the MFMA
// results in VGPRs. GROUPS: pages hold whole 8-token groups (8 or more
// tokens per page), so one page-table entry serves a lane's 8 value tokens
// (2 entry loads per thread instead of 16).
template <int QPK, bool GROUPS>
__global__ __launch_bounds__(256) Q35_WAVES_PER_EU(2) void attention_kernel(AttnArgs a) {
  constexpr int kQStride = kHeadDim + 4;  // floats per staged query row (rows start on different banks)
  __shared__ __align__(16) float qs[QPK * kQStride];
  __shared__ __align__(16) float pl[16 * kPStride];
  __shared__ float tmax[4][16], tsum[4][16];
  const int sp = blockIdx.x, g = blockIdx.y;
  const int ord = static_cast<int>(blockIdx.z);  // partial rows are indexed by the ordinal
  const int r = a.row_list != nullptr ? a.row_list[ord] : ord;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int t0 = sp * kChunkTokens;
  const int kvw = a.kv_heads * kHeadDim;
  const int32_t *pt = a.page_table + static_cast<size_t>(a.row_seg != nullptr ? a.row_seg[r] : r) * a.max_pages;
  const int last_page = a.max_pages - 1;
  // page_tokens is a power of two: shifts and masks, not integer division
  const int pshift = __builtin_ctz(static_cast<unsigned>(a.page_tokens)), pmask = a.page_tokens - 1;
  const int kt = 16 * wave + (lane & 15);  // this lane's key token within the chunk
  const int tg = lane >> 4;                // this lane's value token group
  // one round trip: the row's QPK query heads (QPK x 256 floats, one 16-byte
  // load per thread), the context length and the page-table entries of the
  // lane's key token and of its 16 value tokens (pages of 8 or more tokens
  // hold whole 8-token groups: the group's first entry serves all 8)
  constexpr int kQ4 = QPK * kHeadDim / 4, kQLoads = (kQ4 + 255) / 256;
  const q35_f32x4 *qsrc = reinterpret_cast<const q35_f32x4 *>(a.q + (static_cast<size_t>(r) * a.heads + g * QPK) * kHeadDim);
  q35_f32x4 qraw[kQLoads];
#pragma unroll
  for (int u = 0; u < kQLoads; ++u) {
    const int e = tid + 256 * u;
    if (e < kQ4) qraw[u] = qsrc[e];
  }
  const int seq = a.seq_lens != nullptr ? a.seq_lens[r] : a.positions[r] + 1;
  const int pfirst = pt[min(t0 >> pshift, last_page)];
  const int pk = pt[min((t0 + kt) >> pshift, last_page)];
  constexpr int istep = GROUPS ? 0 : 1;
  int pv[2][8];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks)
#pragma unroll
    for (int i = 0; i < 8; ++i)
      pv[ks][i] = (GROUPS && i > 0) ? pv[ks][0] : pt[min((t0 + 32 * ks + 8 * tg + i * istep) >> pshift, last_page)];
  // the page-table loads go out before the context length is waited for
  // (otherwise the compiler sinks them below the early return)
  q35_compiler_fence();
  if (t0 >= seq) return;  // whole workgroup
  const int n = min(seq - t0, kChunkTokens);
  // keys of tile `wave` (slots past the context read the chunk's first token)
  const bool kin = kt < n;
  const uint16_t *krow = a.k_pool + ((static_cast<size_t>(kin ? pk : pfirst) << pshift) + ((kin ? t0 + kt : t0) & pmask)) * kvw +
                         static_cast<size_t>(g) * kHeadDim + 8 * (lane >> 4);
  q35_u32x4 kraw[8];
#pragma unroll
  for (int kk = 0; kk < 8; ++kk) kraw[kk] = Q35_LOAD_NT(reinterpret_cast<const q35_u32x4 *>(krow + 32 * kk));
  q35_compiler_fence();  // the keys go out before the values
  // values (slots past the context read the chunk's first token: p = 0 there)
  VOps v;
  const size_t vcol = static_cast<size_t>(g) * kHeadDim + 64 * wave + 4 * (lane & 15);
#pragma unroll
  for (int ks = 0; ks < 2; ++ks)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int vt = 32 * ks + 8 * tg + i;
      const bool vin = vt < n;
      v.raw[ks][i] = Q35_LOAD_NT(reinterpret_cast<const q35_u32x2 *>(
          a.v_pool + ((static_cast<size_t>(vin ? pv[ks][i] : pfirst) << pshift) + ((vin ? t0 + vt : t0) & pmask)) * kvw +
          vcol));
    }

  q35_compiler_fence();  // every load above is in flight before the first wait
#pragma unroll
  for (int u = 0; u < kQLoads; ++u) {
    const int e = tid + 256 * u;
    if (e < kQ4) *reinterpret_cast<q35_f32x4 *>(qs + (e >> 6) * kQStride + 4 * (e & 63)) = qraw[u];
  }
  lds_barrier();
  // query m = lane % 16 is head g*QPK + m
  const int m = lane & 15;
  QOps q;
  load_q_ops(qs + min(m, QPK - 1) * kQStride, m < QPK, lane, q);

  const q35_f32x4 s = qk_tile(q, [&](int kk) { return q35_f16x8_bits(kraw[kk]); });
  float sc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    sc[j] = kin ? s[j] * a.scale : -INFINITY;
    const float mx = tile_max(sc[j]);
    if ((lane & 15) == 0) tmax[wave][4 * (lane >> 4) + j] = mx;
  }
  lds_barrier();
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int mm = 4 * (lane >> 4) + j;
    const float mx = fmaxf(fmaxf(fmaxf(tmax[0][mm], tmax[1][mm]), tmax[2][mm]), tmax[3][mm]);
    const float p = kin ? expf(sc[j] - mx) : 0.0F;
    pl[mm * kPStride + kt] = p;
    const float ps = tile_sum(p);
    if ((lane & 15) == 0) tsum[wave][mm] = ps;
  }
  lds_barrier();

  q35_f16x8 phi[2], plo[2];
  load_p_ops(pl, lane, phi, plo);
  // lane l receives O[4(l/16) + jj][column l % 16] of operand j: dim
  // 64w + 4(l % 16) + j of query head g*QPK + 4(l/16) + jj
  q35_f32x4 o[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    q35_f32x4 c = {0.0F, 0.0F, 0.0F, 0.0F};
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const q35_f16x8 vo = v_operand(v, ks, j);
      c = Q35_MFMA_F32_16X16X32_F16(phi[ks], vo, c);
      c = Q35_MFMA_F32_16X16X32_F16(plo[ks], vo, c);
    }
    o[j] = c;
  }
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) {
    const int mm = 4 * (lane >> 4) + jj;
    if (mm < QPK) {
      const size_t hs = (static_cast<size_t>(ord) * a.heads + g * QPK + mm) * a.max_splits + sp;
      const q35_f32x4 out = {o[0][jj], o[1][jj], o[2][jj], o[3][jj]};
      *reinterpret_cast<q35_f32x4 *>(a.part_o + hs * kHeadDim + 64 * wave + 4 * (lane & 15)) = out;
    }
  }
  if (wave == 0 && lane < QPK) {
    const float mx = fmaxf(fmaxf(fmaxf(tmax[0][lane], tmax[1][lane]), tmax[2][lane]), tmax[3][lane]);
    const size_t hs = (static_cast<size_t>(ord) * a.heads + g * QPK + lane) * a.max_splits + sp;
    a.part_ml[hs * 2] = mx;
    a.part_ml[hs * 2 + 1] = ((tsum[0][lane] + tsum[1][lane]) + tsum[2][lane]) + tsum[3][lane];
  }
}

// Prefill and packed steps: one workgroup per (tile of up to kAttnTileRows
// consecutive positions of one segment of two or more rows, KV head), two
// wavefronts per query head of the group: wavefront w serves head
// g*QPK + w/2 of the tile's rows (its M tile), scores the chunk's token tiles
// 2(w%2) and 2(w%2)+1, and forms P*V for dims 128(w%2) .. +127, as the decode
// kernel splits a chunk over its wavefronts (the tile maxima and sums meet in
// LDS and combine in the same order). The rows share the segment's page
// table. The workgroup walks the tile's 64-token chunks in order, twice:
//   pass 1 scores every chunk and keeps each row's largest chunk maximum, M
//     (the merge's maximum over the row's chunks);
//   pass 2 runs each chunk as the decode kernel does (scores, the chunk
//     maximum m_s, p = exp(s - m_s) with 0 past the row's context, l_s, the
//     P*V partial o_s) and folds it at once as attention_merge_kernel folds
//     the decode kernel's partials: acc = fma(exp(m_s - M), o_s, acc) in chunk
//     order, and per batch of 64 chunks L += the merge's 64-lane tree over
//     exp(m_s - M) * l_s.
// The row's one partial (M, L, acc) then goes through the merge's
// one-partial case (attention_finish_kernel), whose weight for it is
// exp(0) = 1, so every row gets the bits of the decode kernel's chunk
// partials merged, while no chunk partial leaves the
// workgroup. A chunk's K rows are staged in LDS for the scores, then its V,
// transposed to one 64-token row per dim (pvt_tile reads each value operand
// whole), takes their place for P*V. Workgroups start longest tile first
// (the last tiles of a segment have the longest contexts).
constexpr int kFlashBatch = 64;  // chunks per merge tree (the merge's 64 lanes)

template <int QPK>
__global__ __launch_bounds__(128 * QPK) Q35_WAVES_PER_EU(2) void attention_flash_kernel(AttnArgs a) {
  constexpr int kThreads = 128 * QPK;
  constexpr int NP = kChunkTokens * 32 / kThreads;  // 16-byte pieces of a K (or V) chunk per thread
  constexpr int kDimTiles = kHeadDim / 32;          // 16-dim P*V tiles per wavefront
  // a chunk's K rows [token][kKStride], then its V transposed [dim][kVTStride]
  constexpr int kKVHalfs = kChunkTokens * kKStride > kHeadDim * kVTStride ? kChunkTokens * kKStride : kHeadDim * kVTStride;
  __shared__ __align__(16) uint16_t kv[kKVHalfs];
  __shared__ __align__(16) float pls[QPK][16 * kPStride];
  __shared__ float tmax[QPK][4][16], tsum[QPK][4][16];
  __shared__ float lwb[QPK][16][kFlashBatch];
  __shared__ float lsum_rows[QPK][16];
  __shared__ int rows_lds[2][kChunkTokens];
  // workgroup p (linear) runs on XCD p % 8: where the KV heads divide the 8
  // XCDs evenly, each head's tiles go to its own 8 / kv_heads XCDs, whose L2s
  // then hold that head's K/V chunks for all of its tiles; the longest tiles
  // still start first
  int z, g;
  {
    const int nt = static_cast<int>(gridDim.x), nh = static_cast<int>(gridDim.y);
    const int p = static_cast<int>(blockIdx.x) + nt * static_cast<int>(blockIdx.y);
    if (8 % nh == 0 && (nt * nh) % 8 == 0) {
      const int xph = 8 / nh;  // XCDs per KV head
      g = (p & 7) / xph;
      z = nt - 1 - ((p >> 3) * xph + (p & 7) % xph);
    } else {
      z = nt - 1 - static_cast<int>(blockIdx.x);
      g = static_cast<int>(blockIdx.y);
    }
  }
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int u = wave >> 1, hf = wave & 1;  // query head in the group, half of the chunk
  const int kvw = a.kv_heads * kHeadDim;
  const int r0 = a.tile_row0[z], nrows = a.tile_rows[z];
  const int32_t *pt = a.page_table + static_cast<size_t>(a.row_seg != nullptr ? a.row_seg[r0] : r0) * a.max_pages;
  const int last_page = a.max_pages - 1;
  const int pshift = __builtin_ctz(static_cast<unsigned>(a.page_tokens)), pmask = a.page_tokens - 1;
  auto seq_of = [&](int r) { return a.seq_lens != nullptr ? a.seq_lens[r] : a.positions[r] + 1; };
  const int seq_tile = seq_of(r0 + nrows - 1);  // the tile's last row has the longest context
  const int nch = (seq_tile + kChunkTokens - 1) / kChunkTokens;
  // rows 4(l/16) + j of this lane: their context lengths (0 past the tile)
  int seq_r[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int mm = 4 * (lane >> 4) + j;
    seq_r[j] = mm < nrows ? seq_of(r0 + mm) : 0;
  }
  const int m = lane & 15;
  QOps q;
  load_q_ops(a.q + (static_cast<size_t>(r0 + min(m, nrows - 1)) * a.heads + g * QPK + u) * kHeadDim, m < nrows, lane,
             q);
  if (hf == 0 && lane < 16) lsum_rows[u][lane] = 0.0F;

  // Piece i of a thread is token tid/32 + i*kThreads/32 of a chunk, dims
  // 8(tid%32) .. +7 (one base address plus a constant in LDS). The cache rows
  // of a chunk's tokens (page resolved; tokens past the tile's context read
  // the chunk's first token) are resolved one chunk ahead by the first 64
  // threads into rows_lds[chunk % 2]. Each load is issued one compute phase
  // ahead of its use: a chunk's K during the previous chunk's P*V (pass 2)
  // or scores (pass 1), its V during its own scores.
  const uint16_t *k_col = a.k_pool + static_cast<size_t>(g) * kHeadDim + 8 * (tid & 31);
  uint16_t *kv_piece = kv + (tid >> 5) * kKStride + 8 * (tid & 31);
  auto piece_token = [&](int i) { return (tid >> 5) + (kThreads >> 5) * i; };
  auto fill_rows = [&](int sp) {  // past the last chunk: its last chunk again
    if (tid < kChunkTokens) {
      const int t0 = min(sp, nch - 1) * kChunkTokens;
      const bool in = t0 + tid < seq_tile;
      const int page = pt[min((in ? t0 + tid : t0) >> pshift, last_page)];
      rows_lds[sp & 1][tid] = (page << pshift) + ((in ? t0 + tid : t0) & pmask);
    }
  };
  auto load = [&](const uint16_t *col, int sp, q35_u32x4 raw[NP]) {
#pragma unroll
    for (int i = 0; i < NP; ++i)
      raw[i] = *reinterpret_cast<const q35_u32x4 *>(col + static_cast<size_t>(rows_lds[sp & 1][piece_token(i)]) * kvw);
  };
  auto store = [&](const q35_u32x4 raw[NP]) {
#pragma unroll
    for (int i = 0; i < NP; ++i) *reinterpret_cast<q35_u32x4 *>(kv_piece + (kThreads >> 5) * i * kKStride) = raw[i];
  };
  // V goes to LDS transposed: item it (of 512 per chunk) is tokens
  // 8(it % 8) .. +7 at dims 4(it / 8) .. +3, eight 8-byte loads regrouped in
  // registers (v_operand's regrouping) into four 16-byte dim-row pieces, so
  // the eight items of a dim group fill one row's 128 contiguous bytes
  constexpr int kVItems = kThreads >= 512 ? 1 : 512 / kThreads;
  const bool v_item = tid < 512;  // 1024-thread workgroups: half the threads
  auto load_v = [&](int sp, q35_u32x2 vr[kVItems][8]) {
#pragma unroll
    for (int s2 = 0; s2 < kVItems; ++s2) {
      const int it = min(tid + kThreads * s2, 511), tgp = it & 7, dg = it >> 3;
      const uint16_t *col = a.v_pool + static_cast<size_t>(g) * kHeadDim + 4 * dg;
#pragma unroll
      for (int i = 0; i < 8; ++i)
        vr[s2][i] = *reinterpret_cast<const q35_u32x2 *>(col + static_cast<size_t>(rows_lds[sp & 1][8 * tgp + i]) * kvw);
    }
  };
  auto store_v = [&](const q35_u32x2 vr[kVItems][8]) {
#pragma unroll
    for (int s2 = 0; s2 < kVItems; ++s2) {
      const int it = min(tid + kThreads * s2, 511), tgp = it & 7, dg = it >> 3;
      if (!v_item) break;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const unsigned sel = (j & 1) ? 0x07060302u : 0x05040100u;
        q35_u32x4 d;
#pragma unroll
        for (int p2 = 0; p2 < 4; ++p2) d[p2] = __builtin_amdgcn_perm(vr[s2][2 * p2 + 1][j >> 1], vr[s2][2 * p2][j >> 1], sel);
        *reinterpret_cast<q35_u32x4 *>(kv + (4 * dg + j) * kVTStride + 8 * tgp) = d;
      }
    }
  };
  // this wavefront's two token tiles of chunk sp (K staged): masked, scaled
  // scores, and each tile's per-row maximum into tmax
  auto scores = [&](int sp, float sc[2][4]) {
    const int t0 = sp * kChunkTokens;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int tt = 2 * hf + k;
      const uint16_t *krow = kv + (16 * tt + (lane & 15)) * kKStride + 8 * (lane >> 4);
      const q35_f32x4 s =
          qk_tile(q, [&](int kk) { return q35_f16x8_bits(*reinterpret_cast<const q35_u32x4 *>(krow + 32 * kk)); });
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        sc[k][j] = t0 + 16 * tt + (lane & 15) < seq_r[j] ? s[j] * a.scale : -INFINITY;
        const float t = tile_max(sc[k][j]);
        if ((lane & 15) == 0) tmax[u][tt][4 * (lane >> 4) + j] = t;
      }
    }
  };
  // the chunk's per-row maximum over its four tiles, in tile order
  auto chunk_max = [&](float mx[4]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int mm = 4 * (lane >> 4) + j;
      mx[j] = fmaxf(fmaxf(fmaxf(tmax[u][0][mm], tmax[u][1][mm]), tmax[u][2][mm]), tmax[u][3][mm]);
    }
  };

  q35_u32x4 raw[NP];  // one chunk's K or V pieces in flight
  // pass 1: M
  float M[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
  fill_rows(0);
  lds_barrier();
  load(k_col, 0, raw);
  for (int sp = 0; sp < nch; ++sp) {
    fill_rows(sp + 1);
    store(raw);
    lds_barrier();
    load(k_col, sp + 1, raw);  // past the last chunk: re-reads it, unused
    float sc[2][4], mx[4];
    scores(sp, sc);
    lds_barrier();  // the tile maxima are in; every wavefront is done with K
    chunk_max(mx);
#pragma unroll
    for (int j = 0; j < 4; ++j) M[j] = fmaxf(M[j], mx[j]);
  }

  // pass 2: the chunks folded in order
  float acc[kDimTiles][4];
#pragma unroll
  for (int dt = 0; dt < kDimTiles; ++dt)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[dt][j] = 0.0F;
  float *pl = pls[u];
  lds_barrier();  // pass 1's last reads of tmax and rows_lds are done
  fill_rows(0);
  lds_barrier();
  load(k_col, 0, raw);
  q35_u32x2 vraw[kVItems][8];  // one chunk's V items in flight
  for (int sp = 0; sp < nch; ++sp) {
    const int t0 = sp * kChunkTokens;
    store(raw);
    load_v(sp, vraw);  // this chunk's V, behind its scores
    fill_rows(sp + 1);
    lds_barrier();
    float sc[2][4], mx[4];
    scores(sp, sc);
    lds_barrier();  // the tile maxima are in
    chunk_max(mx);
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int tt = 2 * hf + k;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int t = 16 * tt + (lane & 15);
        const float p = t0 + t < seq_r[j] ? expf(sc[k][j] - mx[j]) : 0.0F;
        pl[(4 * (lane >> 4) + j) * kPStride + t] = p;
        const float ps = tile_sum(p);
        if ((lane & 15) == 0) tsum[u][tt][4 * (lane >> 4) + j] = ps;
      }
    }
    lds_barrier();  // every wavefront is done with K; p and the tile sums are in
    store_v(vraw);
    lds_barrier();
    load(k_col, sp + 1, raw);  // the next chunk's K, behind this chunk's P*V
    // the chunk's weight in the merge; rows whose context ends before the
    // chunk have no partial for it
    float w[4], lsum[4];
    bool live[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int mm = 4 * (lane >> 4) + j;
      lsum[j] = ((tsum[u][0][mm] + tsum[u][1][mm]) + tsum[u][2][mm]) + tsum[u][3][mm];
      live[j] = t0 < seq_r[j];
      w[j] = live[j] ? expf(mx[j] - M[j]) : 0.0F;
    }
    q35_f16x8 phi[2], plo[2];
    load_p_ops(pl, lane, phi, plo);
#pragma unroll
    for (int dt = 0; dt < kDimTiles; ++dt) {
      const q35_f32x4 o = pvt_tile(phi, plo, kv, kDimTiles * hf + dt, lane);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (live[j]) acc[dt][j] = fmaf(w[j], o[j], acc[dt][j]);
    }
    if (hf == 0) {
      if ((lane & 15) == 0) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          lwb[u][4 * (lane >> 4) + j][sp % kFlashBatch] = live[j] ? __fmul_rn(w[j], lsum[j]) : 0.0F;
      }
      if (sp % kFlashBatch == kFlashBatch - 1 || sp == nch - 1) {
        // the merge's tree over the batch's chunks (lane = chunk), row by row
        wave_lds_sync();
        const int cnt = sp % kFlashBatch + 1;
        for (int rr = 0; rr < 16; ++rr) {
          const float v = group_sum<kFlashBatch>(lane < cnt ? lwb[u][rr][lane] : 0.0F);
          if (lane == 0) lsum_rows[u][rr] += v;
        }
        wave_lds_sync();
      }
    }
    lds_barrier();  // every wavefront is done with V, p and the tile sums
  }

  // the row's merged partial
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int mm = 4 * (lane >> 4) + j;
    if (mm >= nrows) continue;
    const size_t hs = static_cast<size_t>(r0 + mm) * a.heads + g * QPK + u;
#pragma unroll
    for (int dt = 0; dt < kDimTiles; ++dt)
      a.prompt_o[hs * kHeadDim + 16 * (kDimTiles * hf + dt) + (lane & 15)] = acc[dt][j];
    if (hf == 0 && (lane & 15) == 0) {
      a.prompt_ml[hs * 2] = M[j];
      a.prompt_ml[hs * 2 + 1] = lsum_rows[u][mm];
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
  const int b = blockIdx.x & 1, h = blockIdx.x >> 1;
  const int ord = static_cast<int>(blockIdx.y);  // the decode kernel's ordinal of the row
  const int r = a.row_list != nullptr ? a.row_list[ord] : ord;
  // lane l holds dims 128b + 2l, +1 of the head (an H128 item of 64 lanes)
  const int lane = threadIdx.x;
  const size_t hs = (static_cast<size_t>(ord) * a.heads + h) * a.max_splits;
  const int d0 = 128 * b + 2 * lane;
  const size_t o = (static_cast<size_t>(r) * a.heads + h) * kHeadDim + d0;
  const q35_f32x2 gate = *reinterpret_cast<const q35_f32x2 *>(gates + o);
  const int seq = a.seq_lens != nullptr ? a.seq_lens[r] : a.positions[r] + 1;
  // the first statistics and partial rows are read at indices bounded by the
  // row's partial slots, not by the chunk count, so they do not wait for the
  // context length; chunks past the context are masked below and never used
  const int bound = a.max_splits;
  q35_f32x2 rows[kMergeBatch];
  auto load_rows = [&](int s0, int bound) {
#pragma unroll
    for (int u = 0; u < kMergeBatch; ++u)
      rows[u] = *reinterpret_cast<const q35_f32x2 *>(a.part_o + (hs + min(s0 + u, bound - 1)) * kHeadDim + d0);
  };
  // chunk statistics of chunks lane, lane + 64, ...: the first batch of 64
  // stays in registers
  float m0 = -INFINITY, l0 = 0.0F;
  {
    const int s = min(lane, bound - 1);
    m0 = a.part_ml[(hs + s) * 2];
    l0 = a.part_ml[(hs + s) * 2 + 1];
  }
  load_rows(0, bound);
  const int splits = (seq + kChunkTokens - 1) / kChunkTokens;
  if (lane >= splits) m0 = -INFINITY;
  float M = m0;
  for (int s = lane + 64; s < splits; s += 64) M = fmaxf(M, a.part_ml[(hs + s) * 2]);
  M = group_max<64>(M);
  float acc[2] = {0.0F, 0.0F};
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
      lw = __fmul_rn(w, l);
    }
    L += group_sum<64>(lw);
    for (int s = 0; s < cnt; s += kMergeBatch) {
      if (s0 + s > 0) load_rows(s0 + s, splits);
#pragma unroll
      for (int u = 0; u < kMergeBatch; ++u) {
        if (s + u >= cnt) break;
        const float ws = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), s + u));
#pragma unroll
        for (int e = 0; e < 2; ++e) acc[e] = fmaf(ws, rows[u][e], acc[e]);
      }
    }
  }
  const float inv = 1.0F / (L > 0.0F ? L : 1.0F);
  float y[2];
#pragma unroll
  for (int e = 0; e < 2; ++e) y[e] = (acc[e] * inv) * sigmoid_stable(gate[e]);
  if (out != nullptr) *reinterpret_cast<q35_f32x2 *>(out + o) = q35_f32x2{y[0], y[1]};
  if (qo.codes != nullptr) h128_quantize_lanes<64>(y, r, 2 * h + b, a.heads * kHeadDim / 32, true, seed, qo, true);
}

// The rows of the segments of two or more rows in a tiled launch (prompt
// rows): attention_flash_kernel has merged all their chunks into one partial
// per (row, head) in prompt_o / prompt_ml, so their merge is
// attention_merge_kernel's one-partial case --
// weight w = expf(m - M) with M = m, L = w * l, acc = fma(w, o, 0) -- done
// here with the same operations (the same bits as that kernel on such a row),
// then the normalisation, gate and quantisation. Each 16-lane row serves its
// own (row, 128-dim block, head) item, kFinishItems per workgroup, so the
// loads of an item do not wait on the row's context length.
constexpr int kFinishItems = 16;

__global__ __launch_bounds__(16 * kFinishItems) void attention_finish_kernel(AttnArgs a, const float *gates,
                                                                            float *out, QuantOut qo, uint64_t seed) {
  const int pairs = 2 * a.heads, total = a.prompt_row_count * pairs;
  const int want = blockIdx.x * kFinishItems + (threadIdx.x >> 4);
  const bool active = want < total;
  const int item = active ? want : total - 1;  // spare rows redo the last item and store nothing
  const int i = item / pairs, p = item - i * pairs;
  const int b = p & 1, h = p >> 1, r = a.prompt_rows[i], j = threadIdx.x & 15;
  const size_t hs = static_cast<size_t>(r) * a.heads + h;
  const int d0 = 128 * b + 8 * j;
  const size_t o = hs * kHeadDim + d0;
  const q35_f32x4 gate_lo = *reinterpret_cast<const q35_f32x4 *>(gates + o);
  const q35_f32x4 gate_hi = *reinterpret_cast<const q35_f32x4 *>(gates + o + 4);
  const q35_f32x4 *src = reinterpret_cast<const q35_f32x4 *>(a.prompt_o + o);
  const q35_f32x4 o_lo = src[0], o_hi = src[1];
  const float m = a.prompt_ml[hs * 2], l = a.prompt_ml[hs * 2 + 1];
  const float M = m;
  const float w = expf(m - M);
  const float L = __fmul_rn(w, l);
  const float inv = 1.0F / (L > 0.0F ? L : 1.0F);
  float y[8];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    y[e] = (fmaf(w, o_lo[e], 0.0F) * inv) * sigmoid_stable(gate_lo[e]);
    y[4 + e] = (fmaf(w, o_hi[e], 0.0F) * inv) * sigmoid_stable(gate_hi[e]);
  }
  if (out != nullptr && active)
#pragma unroll
    for (int e = 0; e < 8; ++e) out[o + e] = y[e];
  if (qo.codes != nullptr) h128_quantize_row16(y, r, 2 * h + b, a.heads * kHeadDim / 32, true, seed, qo, active);
}

}  // namespace

hipError_t launch_attn_prep(const AttnPrepArgs &a, hipStream_t stream) {
  if (a.batch <= 0) return hipSuccess;
  if (a.head_dim != kHeadDim || a.rope_dim > a.head_dim) return hipErrorInvalidValue;
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
  // tiled: the prompt tiles, then the one-row segments' rows as decode rows
  const int decode_rows = tiled ? a.row_count : a.batch;
  if (tiled && a.tiles > 0 && (a.prompt_o == nullptr || a.prompt_ml == nullptr)) return hipErrorInvalidValue;
#define Q35_ATTN(Q)                                                                                    \
  if (tiled && a.tiles > 0)                                                                            \
    Q35_LAUNCH((attention_flash_kernel<Q>), dim3(a.tiles, a.kv_heads), dim3(128 * (Q)), 0, stream, a); \
  if (decode_rows > 0 && a.page_tokens >= 8)                                                          \
    Q35_LAUNCH((attention_kernel<Q, true>), dim3(gs, a.kv_heads, decode_rows), dim3(256), 0, stream, a); \
  else if (decode_rows > 0)                                                                            \
    Q35_LAUNCH((attention_kernel<Q, false>), dim3(gs, a.kv_heads, decode_rows), dim3(256), 0, stream, a);
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
  // tiled: the one-row segments' rows (decode rows) here, the prompt rows below
  const bool tiled = a.tile_row0 != nullptr;
  const int rows = tiled ? a.row_count : a.batch;
  if (rows > 0) Q35_LAUNCH((attention_merge_kernel), dim3(2 * a.heads, rows), 64, 0, stream, a, gates, out, qo, seed);
  if (tiled && a.prompt_row_count > 0) {
    if (a.prompt_o == nullptr || a.prompt_ml == nullptr) return hipErrorInvalidValue;
    const int items = a.prompt_row_count * 2 * a.heads;
    Q35_LAUNCH((attention_finish_kernel), dim3((items + kFinishItems - 1) / kFinishItems), 16 * kFinishItems, 0, stream,
               a, gates, out, qo, seed);
  }
  return hipGetLastError();
}

}  // namespace q35
