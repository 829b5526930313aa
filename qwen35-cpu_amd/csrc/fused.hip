// Decode projections with their neighbours folded in, for steps of one token
// tile (at most 16 rows). Each removes a kernel boundary from the layer:
//
//   gemm_norm_kernel   RMSNorm(1 + w) of the residual rows + H128
//                      preparation (prefill.inl:3-14, q4_h128.cpp:326-401)
//                      as the prologue of the split-K projection that
//                      consumes them (the in / qkv and gate_up projections).
//   gemm_resid_kernel  a projection whose workgroup owns all K splits of a
//                      16-row group, summed in split order in LDS, plus the
//                      residual: x_out = x + proj (the out / o and down
//                      projections, cpu_engine.inl:266-300).
//
// Both keep the arithmetic of the split launch and its consumer bit for bit,
// so a step that runs them gives the rows the general path gives:
// - the projection partials are gemm_rows_kernel's: the exact int32 block dot
//   from v_mfma_i32_16x16x32_i8 (a -8 correction MFMA seeding C) and
//   acc = fma(float(dot), half(d) * s, acc) in block order per K split
//   (q4_dot4.cpp:53), splits as gemm_plan cuts them;
// - the split sum is ((p0 + p1) + p2) + ..., then x + sum (rms_prep_kernel);
// - the norm's sum of squares is rms_prep_kernel's: thread i of 256 adds the
//   float4s i, i + 256, ... (sq_accum), a 64-lane butterfly per wavefront,
//   then (w0 + w1) + (w2 + w3); y = (x * rms_inv) * (1 + w);
// - the H128 codes come from the shared h128_quantize_core.
#include <algorithm>

#include "q35_quant.h"

namespace q35 {
namespace {

typedef Q35_V4I v4i;

constexpr int kNormWaves = 8;      // wavefronts per gemm_norm workgroup (512 threads)
constexpr int kNormMaxGroups = 5;  // H128 groups one K split touches (staged in LDS)
constexpr int kResidMaxSplits = 32;
constexpr int kResidMaxBlocks = 512;  // K / 32 of a residual projection (activation scales in LDS)
// staged scale slots: every block's 16, plus room for the clamped copies a
// staging batch of 4 x 1024 threads writes past them
constexpr int kResidScaleSlots = kResidMaxBlocks * 16 + 4 * 1024;

// The int32 block dots of one block for RM rows and 4 tokens (the -8
// correction MFMA seeds C, so D is the reference's exact dot).
template <int RM>
__device__ __forceinline__ void block_dots(long act, const typename RowWords<RM>::Q &q, v4i D[RM]) {
  typedef RowWords<RM> RW;
  const v4i zero = {0, 0, 0, 0};
  const v4i corr = Q35_MFMA_I32_16X16X32_I8(act, kMinus8, zero, 0, 0, 0);
#pragma unroll
  for (int r = 0; r < RM; ++r) D[r] = Q35_MFMA_I32_16X16X32_I8(act, unpack_word(RW::word(q, r)), corr, 0, 0, 0);
}
// acc = fma(float(dot), half(d) * s, acc) for one block (q4_dot4.cpp:53); a
// padded slot (valid false) adds exactly +0.
template <int RM>
__device__ __forceinline__ void block_chain(const v4i D[RM], const q35_f32x4 &sa, const typename RowWords<RM>::D &d,
                                            bool valid, float acc[RM][4]) {
  typedef RowWords<RM> RW;
#pragma unroll
  for (int r = 0; r < RM; ++r) {
    const float dw = valid ? half_bits_to_float(RW::scale(d, r)) : 0.0F;
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[r][j] = fmaf(static_cast<float>(D[r][j]), dw * sa[j], acc[r][j]);
  }
}

// Workgroup: 8 wavefronts of 16·RM rows each, one K split (grid.y). The
// prologue takes the rows' norms from the group sums of squares the residual
// projection left (sq_groups), normalizes and prepares the split's H128
// groups for all 16 token slots into LDS (32 items of 16 lanes per pass);
// then each wavefront issues the MFMAs of all BPS blocks of the split before
// the block-order fp32 chain.
template <int RM, int NQ, int BPS>
__global__ __launch_bounds__(64 * kNormWaves) void gemm_norm_kernel(NormGemmArgs a) {
  typedef RowWords<RM> RW;
  constexpr int kLanesPerTile = 8 / RM, kGroupRows = 16 * RM;
  constexpr int kPasses = (16 * NQ + 31) / 32;
  __shared__ uint64_t lcodes[NQ * 4 * 64];
  __shared__ __align__(16) float lscales[NQ * 4 * 16];
  __shared__ float totals[16];
  const GemmArgs &g = a.g;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int G = lane >> 4, c = lane & 15, j = lane & 15;
  const int nb = g.nb, K = nb * 32, ntiles = g.rows >> 3, ng = K >> 4;
  const int tokens = g.tokens;
  const int S = gridDim.y, split = blockIdx.y;
  const int b0 = (split * nb) / S, b1 = ((split + 1) * nb) / S, bl = b1 - 1;
  const int q0 = b0 >> 2, nq = ((b1 + 3) >> 2) - q0;  // H128 groups the split touches
  const int lb0 = 4 * q0;                              // first staged block

  // 1. loads, in the order they are waited for: the group sums of token
  // slots 2w and 2w + 1 (lane l: groups l, l + 64, ...), the items' values
  // and norm weights, then the split's weights
  float gv[2][4];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const float *gp = a.sq_groups + static_cast<size_t>(min(2 * wave + u, tokens - 1)) * ng;
#pragma unroll
    for (int k = 0; k < 4; ++k) gv[u][k] = gp[min(lane + 64 * k, ng - 1)];
  }
  q35_f32x4 xq[kPasses][2], wq[kPasses][2];
#pragma unroll
  for (int p = 0; p < kPasses; ++p) {
    const int it = p * 32 + (tid >> 4);
    const int col = (q0 + min(it >> 4, nq - 1)) * 128 + 8 * j;
    const q35_f32x4 *xp =
        reinterpret_cast<const q35_f32x4 *>(a.x + static_cast<size_t>(min(it & 15, tokens - 1)) * K + col);
    const q35_f32x4 *wp = reinterpret_cast<const q35_f32x4 *>(a.weight + col);
    xq[p][0] = xp[0];
    xq[p][1] = xp[1];
    wq[p][0] = wp[0];
    wq[p][1] = wp[1];
  }
  const int gi = blockIdx.x * kNormWaves + wave;  // this wavefront's row group
  const int rt = min(gi * (kGroupRows / 8) + c / kLanesPerTile, ntiles - 1);
  const int r0 = RM * (c % kLanesPerTile);
  const uint8_t *tile = reinterpret_cast<const uint8_t *>(g.w) + static_cast<size_t>(rt) * nb * 144;
  const uint8_t *qrow = tile + 16 + 32 * G + 4 * r0;
  const uint8_t *drow = tile + 2 * r0;
  typename RW::Q q[BPS];
  typename RW::D d[BPS];
#pragma unroll
  for (int i = 0; i < BPS; ++i) {
    const size_t b = static_cast<size_t>(min(b0 + i, bl));
    // streamed: read once per step (gemm_rows_kernel's reason)
    q[i] = Q35_LOAD_NT(reinterpret_cast<const typename RW::Q *>(qrow + b * 144));
    d[i] = Q35_LOAD_NT(reinterpret_cast<const typename RW::D *>(drow + b * 144));
  }

  // 2. the rows' sums of squares (norm_total_groups' tree)
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    float v = lane < ng ? gv[u][0] : 0.0F;
#pragma unroll
    for (int k = 1; k < 4; ++k) v = lane + 64 * k < ng ? v + gv[u][k] : v;
    const float total = wave_sum(v);
    if (lane == 0) totals[2 * wave + u] = total;
  }
  lds_barrier();

  // 3. the split's H128 groups: item it = (token slot it % 16, group q0 +
  // it / 16) on the 16 lanes of one DPP row; slots past the batch are
  // prepared from zeros
  const bool publish = blockIdx.x == 0;  // trace copies: one row group writes them
#pragma unroll
  for (int p = 0; p < kPasses; ++p) {
    if (p * 32 >= 16 * nq) break;  // uniform over the workgroup
    const int it = p * 32 + (tid >> 4), tq = it & 15, gq = it >> 4;
    const bool item = gq < nq, real = tq < tokens;
    const float rms_inv = 1.0F / sqrtf(totals[tq] / static_cast<float>(K) + a.eps);
    float v[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[e] = xq[p][0][e] * rms_inv * (wq[p][0][e] + 1.0F);
      v[4 + e] = xq[p][1][e] * rms_inv * (wq[p][1][e] + 1.0F);
    }
    const int grp = q0 + min(gq, nq - 1);
    if (publish && item && real && a.normed_out != nullptr)
#pragma unroll
      for (int e = 0; e < 8; ++e) a.normed_out[static_cast<size_t>(tq) * K + grp * 128 + 8 * j + e] = v[e];
    if (!real)
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = 0.0F;
    uint64_t word;
    int sum;
    float stored;
    h128_quantize_core(v, grp, true, a.seed, word, sum, stored);
    const int b = grp * 4 + (j >> 2), kg = j & 3, lb = b - lb0;
    if (item) {
      lcodes[lb * 64 + tq + 16 * kg] = word;
      if (kg == 0) lscales[lb * 16 + tq] = stored;
      if (publish && real && a.codes_out != nullptr) {
        a.codes_out[static_cast<size_t>(b) * 64 + tq + 16 * kg] = word;
        if (kg == 0) a.scales_out[static_cast<size_t>(b) * 16 + tq] = stored;
      }
    }
  }
  lds_barrier();

  // 4. the split's chain (gemm_rows_kernel's arithmetic), activations from LDS
  float acc[RM][4];
#pragma unroll
  for (int i = 0; i < RM; ++i)
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[i][t] = 0.0F;
  v4i D[BPS][RM];
#pragma unroll
  for (int i = 0; i < BPS; ++i) {
    const int lb = min(b0 + i, bl) - lb0;
    block_dots<RM>(static_cast<long>(lcodes[lb * 64 + lane]), q[i], D[i]);
  }
#pragma unroll
  for (int i = 0; i < BPS; ++i) {
    const int lb = min(b0 + i, bl) - lb0;
    const q35_f32x4 sa = *reinterpret_cast<const q35_f32x4 *>(&lscales[lb * 16 + 4 * G]);
    block_chain<RM>(D[i], sa, d[i], b0 + i < b1, acc);
  }
  // rows RM·c .. RM·c + RM-1 of tokens 4G..4G+3
  const int row = gi * kGroupRows + RM * c;
  if (row >= g.rows) return;
#pragma unroll
  for (int t4 = 0; t4 < 4; ++t4) {
    const int tok = 4 * G + t4;
    if (tok >= tokens) continue;
    float *dst = S > 1 ? g.partials + (static_cast<size_t>(split) * tokens + tok) * g.rows + row
                       : g.out + static_cast<size_t>(tok) * g.stride + row;
#pragma unroll
    for (int r = 0; r < RM; ++r) dst[r] = acc[r][t4];
  }
}

// Workgroup = one 16-row group (lane (G, c): row c, tokens 4G..4G+3), all S
// K splits: wavefront w runs splits w, w + W, ..., the loads of all (at most
// BPS) blocks of a split issued together; the activation scales are staged
// once in LDS. The split sums meet in LDS and are added in split order, then
// the residual; each token's 16 new residual values leave their group sum of
// squares (sq_group16_lanes) for the next norm.
template <int BPS, int MAXW>
__global__ __launch_bounds__(64 * MAXW) void gemm_resid_kernel(ResidGemmArgs a) {
  typedef RowWords<1> RW;
  __shared__ float part[kResidMaxSplits * 256];  // [split][token slot][row]
  __shared__ __align__(16) float lsc[kResidScaleSlots];
  const GemmArgs &g = a.g;
  const int W = static_cast<int>(blockDim.x) >> 6;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int G = lane >> 4, c = lane & 15;
  const int nb = g.nb, ntiles = g.rows >> 3, S = a.splits;
  const int grp = blockIdx.x;
  const int rt = min(grp * 2 + (c >> 3), ntiles - 1);
  const uint8_t *tile = reinterpret_cast<const uint8_t *>(g.w) + static_cast<size_t>(rt) * nb * 144;
  const uint8_t *qrow = tile + 16 + 32 * G + 4 * (c & 7);
  const uint8_t *drow = tile + 2 * (c & 7);
  const uint64_t *acodes = g.codes + lane;
  const int nsc = nb * 16, bd = static_cast<int>(blockDim.x);
  // the first batch of activation scales, then the first split's weights
  // and codes, then the scales into LDS (which waits for the scales only)
  float sc[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) sc[k] = g.scales[min(k * bd + tid, nsc - 1)];
  // the residual values of this thread's outputs (e = tid, tid + bd, ...
  // below 256), loaded now so the epilogue waits on no memory; unconditional
  // loads at clamped indices (a load under a branch holds every later wait)
  float res[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int e = min(tid + k * bd, 255);
    res[k] = a.residual[static_cast<size_t>(min(e >> 4, g.tokens - 1)) * g.rows + grp * 16 + (e & 15)];
  }
  RW::Q q[BPS];
  RW::D d[BPS];
  long act[BPS];
  auto load = [&](int s) {
    const int b0 = (s * nb) / S, bl = ((s + 1) * nb) / S - 1;
#pragma unroll
    for (int i = 0; i < BPS; ++i) {
      const size_t b = static_cast<size_t>(min(b0 + i, bl));
      // streamed: read once per step (gemm_rows_kernel's reason)
      q[i] = Q35_LOAD_NT(reinterpret_cast<const RW::Q *>(qrow + b * 144));
      d[i] = Q35_LOAD_NT(reinterpret_cast<const RW::D *>(drow + b * 144));
      act[i] = static_cast<long>(acodes[b * 64]);
    }
  };
  int s = wave;
  if (s < S) load(s);
  // the staged copies past nsc land in LDS padding (no store under a branch,
  // which would wait for every load in flight, the split's weights included)
#pragma unroll
  for (int k = 0; k < 4; ++k) lsc[min(k * bd + tid, kResidScaleSlots - 1)] = sc[k];
  for (int base = 4 * bd; base < nsc; base += 4 * bd) {  // wider K: more batches
#pragma unroll
    for (int k = 0; k < 4; ++k) sc[k] = g.scales[min(base + k * bd + tid, nsc - 1)];
#pragma unroll
    for (int k = 0; k < 4; ++k) lsc[min(base + k * bd + tid, kResidScaleSlots - 1)] = sc[k];
  }
  lds_barrier();
  while (s < S) {
    const int b0 = (s * nb) / S, b1 = ((s + 1) * nb) / S, bl = b1 - 1;
    v4i D[BPS][1];
#pragma unroll
    for (int i = 0; i < BPS; ++i) block_dots<1>(act[i], q[i], D[i]);
    float acc[1][4] = {{0.0F, 0.0F, 0.0F, 0.0F}};
#pragma unroll
    for (int i = 0; i < BPS; ++i) {
      const q35_f32x4 sa = *reinterpret_cast<const q35_f32x4 *>(&lsc[min(b0 + i, bl) * 16 + 4 * G]);
      block_chain<1>(D[i], sa, d[i], b0 + i < b1, acc);
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) part[(s * 16 + 4 * G + t) * 16 + c] = acc[0][t];
    s += W;
    if (s < S) load(s);
  }
  __syncthreads();
  const int ng = g.rows >> 4;
#pragma unroll
  for (int k = 0; k < 4; ++k) {  // 16-lane rows: token t's 16 columns
    const int e = tid + k * bd;
    if (e >= 256) break;
    const int t = e >> 4, r = e & 15;
    float sum = part[t * 16 + r];
    for (int u = 1; u < S; ++u) sum += part[(u * 16 + t) * 16 + r];
    const int row = grp * 16 + r;
    const size_t o = static_cast<size_t>(min(t, g.tokens - 1)) * g.rows + row;
    const float x = res[k] + sum;
    const float gs = sq_group16_lanes(x);
    if (t < g.tokens) {
      if (a.proj_out != nullptr) a.proj_out[o] = sum;
      a.x_out[o] = x;
      if (r == 0) a.sq_groups[static_cast<size_t>(t) * ng + grp] = gs;
    }
  }
}

}  // namespace

namespace {
// Most H128 groups one K split of the plan touches (0: the shape is not supported).
int norm_groups(int rows, int nb, int tokens, int cu_count, int max_split) {
  if (tokens < 1 || tokens > 16 || rows % 8 != 0 || nb < 4 || nb % 4 != 0 || nb * 32 > 4096) return 0;
  const GemmPlan p = gemm_plan(rows, nb, false, false, cu_count, 0, 0, max_split);
  int most = 0;
  for (int s = 0; s < p.split; ++s) {
    const int b0 = (s * nb) / p.split, b1 = ((s + 1) * nb) / p.split;
    most = std::max(most, ((b1 + 3) >> 2) - (b0 >> 2));
  }
  return most <= kNormMaxGroups ? most : 0;
}
}  // namespace

bool gemm_norm_fits(int rows, int nb, int tokens, int cu_count, int max_split) {
  if (norm_groups(rows, nb, tokens, cu_count, max_split) == 0) return false;
  const GemmPlan p = gemm_plan(rows, nb, false, false, cu_count, 0, 0, max_split);
  return (nb + p.split - 1) / p.split <= 16 && nb * 32 / 16 <= 256;  // blocks per split; group sums per lane
}

hipError_t launch_gemm_norm(const NormGemmArgs &a, SplitRows *out_rows, hipStream_t stream) {
  const GemmArgs &g = a.g;
  if (!gemm_norm_fits(g.rows, g.nb, g.tokens, g.cu_count, a.max_split) || a.x == nullptr || a.weight == nullptr ||
      a.sq_groups == nullptr)
    return hipErrorInvalidValue;
  const GemmPlan p = gemm_plan(g.rows, g.nb, false, false, g.cu_count, 0, 0, a.max_split);
  if ((p.split > 1 && g.partials == nullptr) || (p.split == 1 && g.out == nullptr)) return hipErrorInvalidValue;
  if (a.codes_out != nullptr && a.scales_out == nullptr) return hipErrorInvalidValue;
  const int cus = g.cu_count > 0 ? g.cu_count : 256;
  // 32-row wavefronts unless that leaves fewer workgroups than half the compute units
  const int groups32 = ((g.rows >> 3) + 3) / 4;
  const bool rm2 = (groups32 + kNormWaves - 1) / kNormWaves * p.split >= cus / 2;
  const int groups = rm2 ? groups32 : ((g.rows >> 3) + 1) / 2;
  const dim3 grid((groups + kNormWaves - 1) / kNormWaves, p.split), block(64 * kNormWaves);
  const bool nq2 = norm_groups(g.rows, g.nb, g.tokens, g.cu_count, a.max_split) <= 2;
  const bool bps8 = (g.nb + p.split - 1) / p.split <= 8;
#define Q35_NORM(RM, NQ)                                                            \
  if (bps8)                                                                         \
    Q35_LAUNCH((gemm_norm_kernel<RM, NQ, 8>), grid, block, 0, stream, a);           \
  else                                                                              \
    Q35_LAUNCH((gemm_norm_kernel<RM, NQ, 16>), grid, block, 0, stream, a);
  if (rm2) {
    if (nq2) { Q35_NORM(2, 2) } else { Q35_NORM(2, kNormMaxGroups) }
  } else {
    if (nq2) { Q35_NORM(1, 2) } else { Q35_NORM(1, kNormMaxGroups) }
  }
#undef Q35_NORM
  if (out_rows != nullptr) {
    out_rows->p = p.split > 1 ? g.partials : g.out;
    out_rows->splits = p.split;
    out_rows->split_stride = p.split > 1 ? static_cast<long long>(g.tokens) * g.rows : 0;
    out_rows->width = g.rows;
  }
  return hipGetLastError();
}

bool gemm_resid_fits(int rows, int nb, int tokens, int cu_count) {
  if (tokens < 1 || tokens > 16 || rows % 16 != 0 || nb < 1 || nb > kResidMaxBlocks) return false;
  const int S = gemm_plan(rows, nb, false, false, cu_count, 0, 0, kResidMaxSplits).split;
  return S <= kResidMaxSplits && (nb + S - 1) / S <= 16;
}

hipError_t launch_gemm_resid(const ResidGemmArgs &in, hipStream_t stream) {
  ResidGemmArgs a = in;
  const GemmArgs &g = a.g;
  if (!gemm_resid_fits(g.rows, g.nb, g.tokens, g.cu_count) || a.residual == nullptr || a.x_out == nullptr ||
      a.sq_groups == nullptr || g.codes == nullptr || g.scales == nullptr)
    return hipErrorInvalidValue;
  const int S = gemm_plan(g.rows, g.nb, false, false, g.cu_count, 0, 0, kResidMaxSplits).split;
  a.splits = S;
  const int bps = (g.nb + S - 1) / S;  // most blocks of one split
  if (bps <= 8) {
    Q35_LAUNCH((gemm_resid_kernel<8, 16>), dim3(g.rows / 16), dim3(64 * std::min(S, 16)), 0, stream, a);
  } else {
    Q35_LAUNCH((gemm_resid_kernel<16, 8>), dim3(g.rows / 16), dim3(64 * std::min(S, 8)), 0, stream, a);
  }
  return hipGetLastError();
}

}  // namespace q35
