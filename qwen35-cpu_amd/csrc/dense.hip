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
// XCD i % 8; the logical order gives each XCD about an eighth of the row
// groups with every token group, walked row groups fastest, so that its L2
// holds its row groups' weights and the few token groups in flight.
namespace {
typedef Q35_V4I v4i;

// Occupancy floor 2 (at most 256 VGPRs): the MFMA results then land in VGPRs;
// above 256 the compiler places them in AGPRs and copies each element out
// with a VALU move (64 per K block here), in a kernel whose VALU issue --
// the int32-to-fp32 conversion and fma of every block dot -- is its limit.
template <int NT, int R>
__global__ __launch_bounds__(256) Q35_WAVES_PER_EU(2) void gemm_dense_kernel(GemmArgs a, int S, int token_groups, int units) {
  constexpr int RM = 4;  // rows (MFMAs) per lane: 64-row groups
  typedef RowWords<4> RWv;
  constexpr int kLanesPerTile = 8 / RM, kGroupRows = 16 * RM;
  // the wavefront index is read into a scalar register so that every base
  // below is wave-uniform: the loads are raw buffer loads from wave-uniform
  // resources with a fixed per-lane voffset and the block's offset in a
  // scalar register, so the loop holds no per-lane address arithmetic
  const int wave = q35_uniform(static_cast<int>(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63;
  const int G = lane >> 4, c = lane & 15;
  const int nwg = static_cast<int>(gridDim.x);  // a multiple of 8
  const int logical = (static_cast<int>(blockIdx.x) & 7) * (nwg >> 3) + (static_cast<int>(blockIdx.x) >> 3);
  const int unit = logical * 4 + wave;
  if (unit >= units) return;
  // units in blocks of gx row groups (an XCD's share of the rows) x every
  // token group, the row groups fastest within a block: the units resident on
  // an XCD at once span its row groups and a few token groups, whose weights
  // and activations then stay in its L2 while the token groups advance
  const int groups = units / token_groups, gx = (groups + 7) >> 3;
  const int blk = unit / (gx * token_groups), k = unit - blk * gx * token_groups;
  const int rb = min(gx, groups - blk * gx);  // row groups of this block
  const int g = blk * gx + k % rb, tg = k / rb;
  const int nb = a.nb, ntiles = a.rows >> 3, tiles = (a.tokens + 15) >> 4;
  // rows past the matrix read a valid tile (the last); token tiles past the
  // chunk read the last valid tile; neither is stored. Lane c holds rows
  // r0 .. r0+3 of tile rt: per block their 16 code bytes of k-group G and
  // their four fp16 scales, of which it supplies row r0 + G's to the
  // multipliers' MFMA. (All four k-group lanes of a row pair read the same
  // 8 scale bytes: loading only the 2 or 4 bytes a lane uses made the
  // kernel 20% slower.) Every offset is below its resource's extent (the
  // launcher bounds the extents by 2^31 bytes).
  const int rt0 = g * (kGroupRows / 8);  // < ntiles: g < ceil(ntiles / 8)
  const int rt = min(rt0 + c / kLanesPerTile, ntiles - 1);
  const int r0 = RM * (c % kLanesPerTile);
  const q35_buffer wres = q35_make_buffer(reinterpret_cast<const uint8_t *>(a.w) + static_cast<size_t>(rt0) * nb * 144,
                                          (ntiles - rt0) * nb * 144);
  const int woff = (rt - rt0) * nb * 144;
  const int qoff = woff + 16 + 32 * G + 4 * r0, doff = woff + 2 * r0;
  const int tile0 = min(tg * NT, tiles - 1);
  const q35_buffer ares = q35_make_buffer(a.codes + static_cast<size_t>(tile0) * nb * 64, (tiles - tile0) * nb * 512);
  const q35_buffer sres = q35_make_buffer(a.scales + static_cast<size_t>(tile0) * nb * 16, (tiles - tile0) * nb * 64);
  int aoff[NT], soff[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int dt = min(tg * NT + t, tiles - 1) - tile0;
    aoff[t] = dt * nb * 512 + 8 * lane;
    soff[t] = dt * nb * 64 + 4 * c;
  }
  // v_perm_b32 selector moving the fp16 scale of row r0 + G (bytes 2G, 2G+1
  // of the tile's four scales) to the low half, zeros above
  const uint32_t dsel_bytes = 0x0C0C0000u | (static_cast<uint32_t>(2 * G + 1) << 8) | static_cast<uint32_t>(2 * G);
  struct Block {
    typename RWv::Q q;
    typename RWv::D d;
    long act[NT];
    float s1[NT];  // the scale of token lane%16 of each tile
  };
  auto load = [&](Block &k, int b) {
    b = min(b, nb - 1);
    k.q = q35_buffer_load16(wres, qoff, b * 144);
    k.d = q35_buffer_load8(wres, doff, b * 144);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      k.act[t] = __builtin_bit_cast(long, q35_buffer_load8(ares, aoff[t], b * 512));
      k.s1[t] = __builtin_bit_cast(float, q35_buffer_load4(sres, soff[t], b * 64));
    }
  };
  float acc[NT][RM][4], tot[NT][RM][4];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int r = 0; r < RM; ++r)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[t][r][j] = tot[t][r][j] = 0.0F;
  auto compute = [&](const Block &k) {
    const v4i zero = {0, 0, 0, 0};
    long wq[RM];
#pragma unroll
    for (int r = 0; r < RM; ++r) wq[r] = unpack_word(RWv::word(k.q, r));
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const v4i corr = Q35_MFMA_I32_16X16X32_I8(k.act[t], kMinus8, zero, 0, 0, 0);
      v4i D[RM];
#pragma unroll
      for (int r = 0; r < RM; ++r) D[r] = Q35_MFMA_I32_16X16X32_I8(k.act[t], wq[r], corr, 0, 0, 0);
      {
        // the multipliers as one outer-product MFMA: element 4r + j is token
        // 4G + j's scale times row 4c + r's (the layout of D[r][j]); lane
        // 16b + n supplies row 4n + b's scale, every lane token lane%16's
        const float dsel = half_bits_to_float(static_cast<uint16_t>(__builtin_amdgcn_perm(k.d[1], k.d[0], dsel_bytes)));
        q35_f32x16 zero16;
#pragma unroll
        for (int e = 0; e < 16; ++e) zero16[e] = 0.0F;
        const q35_f32x16 mm = Q35_MFMA_F32_16X16X1_4B(k.s1[t], dsel, zero16);
#pragma unroll
        for (int r = 0; r < RM; ++r)
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[t][r][j] = fmaf(static_cast<float>(D[r][j]), mm[4 * r + j], acc[t][r][j]);
      }
    }
  };
  // splits s = 0..S-1 over blocks [s·nb/S, (s+1)·nb/S); a finished chain is
  // added to the running sum (which starts at +0, and no chain is -0, so the
  // first addition is exact: tot = p_0). The loads run R-1 blocks ahead of
  // the compute (a ring of R register buffers, the loop unrolled by R) across
  // split boundaries, where a uniform branch folds the chain.
  Block buf[R];
#pragma unroll
  for (int k = 0; k < R - 1; ++k) load(buf[k], k);
  int s = 0, be = nb / S;  // end of split 0: ((s + 1) * nb) / S
  for (int b = 0; b < nb; b += R) {
#pragma unroll
    for (int k = 0; k < R; ++k) {
      load(buf[(k + R - 1) % R], b + k + R - 1);
      if (b + k < nb) {
        compute(buf[k]);
        if (b + k + 1 == be) {
#pragma unroll
          for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int r = 0; r < RM; ++r)
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
  const int row = g * kGroupRows + RM * c;
  if (row >= a.rows) return;
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int tok = (tg * NT + t) * 16 + 4 * G + j;
      if (tok >= a.tokens) continue;
#pragma unroll
      for (int r = 0; r < RM; ++r) a.out[static_cast<size_t>(tok) * a.stride + row + r] = tot[t][r][j];
    }
}

}  // namespace

int gemm_dense_splits(int rows, int nb, int cu_count, int max_split) {
  return gemm_plan(rows, nb, false, false, cu_count, 0, 0, max_split > 0 ? max_split : 32).split;
}

bool gemm_dense_fits(int rows, int tokens, int cu_count) {
  const long long waves = static_cast<long long>((rows / 8 + 7) / 8) * ((tokens + 31) / 32);  // two-tile units
  return tokens >= kMaxTokens && waves >= 2LL * (cu_count > 0 ? cu_count : 256);
}

hipError_t launch_gemm_dense(const GemmArgs &a, hipStream_t stream) {
  if (a.tokens <= 0 || a.rows <= 0) return hipSuccess;
  if (a.out == nullptr || a.rows % 8 != 0 || a.stride < a.rows || a.residual != nullptr) return hipErrorInvalidValue;
  // the kernel addresses the matrix and the activations through buffer
  // resources with 32-bit extents
  const long long tiles = (a.tokens + 15) / 16;
  if (static_cast<long long>(a.rows / 8) * a.nb * 144 >= (1LL << 31) || tiles * a.nb * 512 >= (1LL << 31))
    return hipErrorInvalidValue;
  // two token tiles per wavefront (137 VGPRs, three wavefronts per SIMD):
  // four tiles (217 VGPRs, two per SIMD) measure 5% slower on the config-5
  // projections, and rings of three or four blocks are no faster either. At
  // one split launch's rows (64) each wavefront takes one tile: twice the
  // wavefronts for a grid that would leave most SIMDs with none (the 4B
  // gate_up at 64 rows: 1152 instead of 576)
  const int groups = (a.rows / 8 + 7) / 8;
  const int nt = a.tokens <= kMaxTokens ? 1 : 2;
  const int S = gemm_dense_splits(a.rows, a.nb, a.cu_count, a.max_split);
  const int token_groups = (a.tokens + 16 * nt - 1) / (16 * nt);
  const int units = groups * token_groups;
  const int wgs = ((units + 3) / 4 + 7) / 8 * 8;
  if (nt == 1)
    Q35_LAUNCH((gemm_dense_kernel<1, 2>), dim3(wgs), dim3(256), 0, stream, a, S, token_groups, units);
  else
    Q35_LAUNCH((gemm_dense_kernel<2, 2>), dim3(wgs), dim3(256), 0, stream, a, S, token_groups, units);
  return hipGetLastError();
}

}  // namespace q35
