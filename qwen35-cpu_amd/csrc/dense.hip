// Dense Q4-G32-DOT4 projection GEMM for many tokens (prefill chunks and
// packed steps). Built with the MFMA results in VGPRs (-amdgpu-mfma-vgpr-form):
// the fp32 epilogue reads every result, so AGPR results would cost a read
// per value.
#include "q35_device.h"
#include "q35_internal.h"

namespace q35 {

// Dense projection GEMM for many tokens (prefill chunks and packed steps
// beyond one split launch): one wavefront per (64-row group, NT·16-token
// group) walks every K block in order, so each weight tile is unpacked once
// for NT token tiles and no partial rows go to memory. The K split that the
// split launch uses for the same shape (gemm_plan with the consumer's bound)
// is kept as the summation structure: the fma chain restarts from 0 at each
// split boundary (b0 = s·nb/S) and the finished split sums are added in split
// order, out = ((p_0 + p_1) + p_2) + ..., which is what a consumer of the
// split partials computes (SplitRows::reduce). Per block the int8 MFMAs and
// the fp32 chain acc = fma(float(dot), d·s, acc) are gemm_kernel's. The
// multipliers d·s of a token tile (4 rows x 4 tokens per lane) come from one
// v_mfma_f32_16x16x1_4b outer product (block b: the tile's 16 token scales
// times the scales of rows 4n + b) instead of 16 VALU products per lane: an
// fp32 product with one live term, bit-identical to the VALU product
// whenever it is zero or in the normal range, so every output carries the
// split launch's bits unless some weight-scale x activation-scale product is
// subnormal (below 2^-126: scales of order 1e-19 each). Workgroup i runs on
// XCD i % 8; the logical order puts the token groups of one row group on one
// XCD, where they share its L2.
namespace {
typedef Q35_V4I v4i;
typedef q35_f32x16 v16f;
constexpr int kRowsPerGroup = 64;

template <int NT>
__global__ __launch_bounds__(256) void gemm_dense_kernel(GemmArgs a, int S, int token_groups, int units) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int G = lane >> 4, c = lane & 15, h = c & 1, T = c >> 1;
  const int nwg = static_cast<int>(gridDim.x);  // a multiple of 8
  const int logical = (static_cast<int>(blockIdx.x) & 7) * (nwg >> 3) + (static_cast<int>(blockIdx.x) >> 3);
  const int unit = logical * 4 + wave;
  if (unit >= units) return;
  const int g = unit / token_groups, tg = unit - g * token_groups;
  const int nb = a.nb, ntiles = a.rows >> 3, tiles = (a.tokens + 15) >> 4;
  // rows past the matrix read a valid tile (the last); token tiles past the
  // chunk read the last valid tile; neither is stored
  const int rt = min(g * 8 + T, ntiles - 1);
  const uint8_t *wt = reinterpret_cast<const uint8_t *>(a.w) + static_cast<size_t>(rt) * nb * 144;
  const q35_u32x4 *qp = reinterpret_cast<const q35_u32x4 *>(wt + 16 + 16 * (2 * G + h));
  const q35_u32x2 *dp = reinterpret_cast<const q35_u32x2 *>(wt + 8 * h);
  const uint64_t *ap[NT];
  const float *sp[NT];  // the scale of token lane%16 of each tile
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int tile = min(tg * NT + t, tiles - 1);
    ap[t] = a.codes + static_cast<size_t>(tile) * nb * 64 + lane;
    sp[t] = a.scales + static_cast<size_t>(tile) * nb * 16 + c;
  }
  struct Block {
    q35_u32x4 q;
    q35_u32x2 d;
    long act[NT];
    float sa[NT];
  };
  // block b (clamped into the matrix: a load past the end re-reads the last
  // block, an L2 hit, instead of branching)
  auto load = [&](Block &k, int b) {
    b = min(b, nb - 1);
    k.q = qp[static_cast<size_t>(b) * 9];  // 144-byte tiles: 9 x 16 bytes
    k.d = dp[static_cast<size_t>(b) * 18];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      k.act[t] = static_cast<long>(ap[t][static_cast<size_t>(b) * 64]);
      k.sa[t] = sp[t][static_cast<size_t>(b) * 16];
    }
  };
  float acc[NT][4][4], tot[NT][4][4];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[t][r][j] = tot[t][r][j] = 0.0F;
  auto compute = [&](const Block &k) {
    const v4i zero = {0, 0, 0, 0};
    const float dw[4] = {half_bits_to_float(static_cast<uint16_t>(k.d[0] & 0xffffu)),
                         half_bits_to_float(static_cast<uint16_t>(k.d[0] >> 16)),
                         half_bits_to_float(static_cast<uint16_t>(k.d[1] & 0xffffu)),
                         half_bits_to_float(static_cast<uint16_t>(k.d[1] >> 16))};
    const long w0 = unpack_word(k.q[0]), w1 = unpack_word(k.q[1]), w2 = unpack_word(k.q[2]), w3 = unpack_word(k.q[3]);
    // the B operand of the multiplier outer product: lane 16b + n holds the
    // scale of row 4n + b (this lane's row 4c + G)
    const float dsel = G == 0 ? dw[0] : G == 1 ? dw[1] : G == 2 ? dw[2] : dw[3];
    v16f zero16;
#pragma unroll
    for (int e = 0; e < 16; ++e) zero16[e] = 0.0F;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const v4i corr = Q35_MFMA_I32_16X16X32_I8(k.act[t], kMinus8, zero, 0, 0, 0);
      v4i D[4];
      D[0] = Q35_MFMA_I32_16X16X32_I8(k.act[t], w0, corr, 0, 0, 0);
      D[1] = Q35_MFMA_I32_16X16X32_I8(k.act[t], w1, corr, 0, 0, 0);
      D[2] = Q35_MFMA_I32_16X16X32_I8(k.act[t], w2, corr, 0, 0, 0);
      D[3] = Q35_MFMA_I32_16X16X32_I8(k.act[t], w3, corr, 0, 0, 0);
      // element 4r + j: token 4G + j's scale times row 4c + r's (the layout
      // of D[r][j])
      const v16f m = Q35_MFMA_F32_16X16X1_4B(k.sa[t], dsel, zero16);
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[t][r][j] = fmaf(static_cast<float>(D[r][j]), m[4 * r + j], acc[t][r][j]);
    }
  };
  // splits s = 0..S-1 over blocks [s·nb/S, (s+1)·nb/S); a finished chain is
  // added to the running sum (which starts at +0, and no chain is -0, so the
  // first addition is exact: tot = p_0). The loads run two blocks ahead of
  // the compute across split boundaries (ping-pong buffers, the loop unrolled
  // by two), and a boundary only folds the chain: a uniform branch.
  Block buf[2];
  load(buf[0], 0);
  int s = 0, be = nb / S;  // the end of split s: ((s + 1) * nb) / S
  for (int b = 0; b < nb; b += 2) {
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      load(buf[k ^ 1], b + k + 1);  // past the last block: re-reads it, unused
      if (b + k < nb) {
        compute(buf[k]);
        if (b + k + 1 == be) {
#pragma unroll
          for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
              for (int j = 0; j < 4; ++j) {
                tot[t][r][j] += acc[t][r][j];
                acc[t][r][j] = 0.0F;
              }
          ++s;
          be = ((s + 1) * nb) / S;
        }
      }
    }
  }
  // rows 4c..4c+3 of the group (one per MFMA) for tokens 4G..4G+3 of each tile
  const int row = g * kRowsPerGroup + 4 * c;
  if (row >= a.rows) return;
  const bool vec_out = (a.stride & 3) == 0;
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int tok = (tg * NT + t) * 16 + 4 * G + j;
      if (tok >= a.tokens) continue;
      store_row4(a.out + static_cast<size_t>(tok) * a.stride + row, vec_out, tot[t][0][j], tot[t][1][j], tot[t][2][j],
                 tot[t][3][j]);
    }
}

}  // namespace

int gemm_dense_splits(int rows, int nb, int cu_count, int max_split) {
  return gemm_plan(rows, nb, false, false, cu_count, 0, 0, max_split > 0 ? max_split : 32).split;
}

bool gemm_dense_fits(int rows, int tokens, int cu_count) {
  const long long waves = static_cast<long long>((rows / 8 + 7) / 8) * ((tokens + 31) / 32);  // two-tile units
  return tokens > kMaxTokens && waves >= 2LL * (cu_count > 0 ? cu_count : 256);
}

hipError_t launch_gemm_dense(const GemmArgs &a, hipStream_t stream) {
  if (a.tokens <= 0 || a.rows <= 0) return hipSuccess;
  if (a.out == nullptr || a.rows % 8 != 0 || a.stride < a.rows || a.residual != nullptr) return hipErrorInvalidValue;
  // four token tiles per wavefront (228 VGPRs, two wavefronts per SIMD: half
  // the weight unpacking per token) on matrices of 16384 rows or more while
  // the grid keeps a wavefront per SIMD; two tiles (144 VGPRs, three per
  // SIMD) below (4B at 2048 tokens: gate_up 411 against 434 us with two
  // tiles; in_proj 295, qkv 230, out/o 103 and down 237 us with two tiles
  // against 304, 231, 128 and 276 with four)
  const int groups = (a.rows / 8 + 7) / 8;
  const int cus = a.cu_count > 0 ? a.cu_count : 256;
  const int nt = a.rows >= 16384 && static_cast<long long>(groups) * ((a.tokens + 63) / 64) >= 4LL * cus ? 4 : 2;
  const int S = gemm_dense_splits(a.rows, a.nb, a.cu_count, a.max_split);
  const int token_groups = (a.tokens + 16 * nt - 1) / (16 * nt);
  const int units = groups * token_groups;
  const int wgs = ((units + 3) / 4 + 7) / 8 * 8;
  if (nt == 4)
    Q35_LAUNCH((gemm_dense_kernel<4>), dim3(wgs), dim3(256), 0, stream, a, S, token_groups, units);
  else
    Q35_LAUNCH((gemm_dense_kernel<2>), dim3(wgs), dim3(256), 0, stream, a, S, token_groups, units);
  return hipGetLastError();
}

}  // namespace q35
