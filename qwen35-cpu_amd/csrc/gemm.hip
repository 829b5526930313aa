// Q4-G32-DOT4 grouped GEMV/GEMM on CDNA4 int8 MFMA.
//
// Reads the reference's 144-byte Q4_0BlockX8 DOT4 tiles in place (no repack):
//   qs[32t+4r+j] = u[r][8t+j] | u[r][8t+4+j] << 4          (q4_dot4.h:5-6)
// so the 32-bit word 8t+r of a tile body holds row r's columns 8t..8t+3 (low
// nibbles) and 8t+4..8t+7 (high nibbles).
//
// Work decomposition (gemm_kernel; the single-token-tile split path of the
// decode step runs gemm_rows_kernel below, the same scheme with 16- or
// 32-row groups). The rows form 64-row groups (eight 8-row tiles). A
// workgroup owns one group and one of S contiguous K ranges (split-K across
// workgroups, grid.y); its W wavefronts split that range, and every wavefront
// issues the loads of all blocks of a chunk (KS blocks: weights, row scales,
// activation codes and activation scales) before its first MFMA, so a launch
// keeps groups x S x W x KS x 1.2 KB in flight and no wavefront waits on a
// second round trip. The wavefronts of a workgroup are summed in fixed order
// through LDS; with S > 1 each workgroup writes its partial sums to
// partials[s][token][row] and the consumer kernel adds the S partials in split
// order, so every result is deterministic.
//
// Lane l = (G = l/16, c = l%16) loads, per 32-column block, the 16-byte body
// segment 2G + (c%2) of tile c/2 -- four words = rows 4(c%2)..4(c%2)+3 of
// tile c/2, columns 8G..8G+7 -- plus the four FP16 scales of those rows (8
// bytes at tile offset 8(c%2)). Word i, unpacked to int8, is the B operand of
// v_mfma_i32_16x16x32_i8 #i for B column c (= output row 4c+i) and k-group G;
// the A operand is the prepared activation word of token c, k-group G (the
// "A16" layout). One extra MFMA against a constant -8 B operand yields
// -8 * sum(a) per token, which seeds the C operand of the four real MFMAs, so
//   D_i[4G+j][c] = sum_k (u - 8) * a      (q4_dot4_simd.inl:66-89)
// is the reference's exact int32 block dot for row 4c+i and token 4G+j. The
// FP32 epilogue per block is the reference's
//   acc = fma(float(dot), half(d_row) * s_tok, acc)   (q4_dot4.cpp:53)
// in block order within each wavefront. With one wavefront and one split per
// group (exact mode) every output is the reference's single fma chain.
//
// The greedy head (argmax epilogue) runs a grid-stride loop over row groups
// and leaves one 64-bit (value, lowest index) key per workgroup and token;
// argmax_finalize_kernel reduces those keys per token. No atomics anywhere.
#include "q35_device.h"
#include "q35_internal.h"

namespace q35 {
namespace {

typedef Q35_V4I v4i;

constexpr int kRowsPerGroup = 64;
constexpr int kMaxWaves = 4;

// Occupancy floor 2 (at most 256 VGPRs) keeps the MFMA results in VGPRs
// (above 256 the compiler places them in AGPRs and copies every element
// out); the DOTS form needs more registers and keeps floor 1.
template <int KS, bool ARGMAX, bool DOTS>
__global__ __launch_bounds__(256) Q35_WAVES_PER_EU(DOTS ? 1 : 2) void gemm_kernel(GemmArgs a) {
  Q35_DYNAMIC_SHARED(float, red);  // [W][16][64] wave partials, then [16] argmax keys
  const int W = static_cast<int>(blockDim.x) >> 6;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int G = lane >> 4, c = lane & 15, h = c & 1, T = c >> 1;
  const int nb = a.nb, ntiles = a.rows >> 3;
  const int groups = (ntiles + 7) >> 3;
  const int S = gridDim.y, split = blockIdx.y;
  unsigned long long *best = reinterpret_cast<unsigned long long *>(red + W * 16 * 64);

  // this wavefront's block range: split of the K range, then 1/W of it
  const int sb0 = (split * nb) / S, sb1 = ((split + 1) * nb) / S;
  const int per = (sb1 - sb0 + W - 1) / W;
  const int b0 = min(sb1, sb0 + wave * per), b1 = min(sb1, b0 + per);
  // a wavefront with an empty range (never planned, kept safe) reads block 0
  // and contributes nothing
  const bool has_blocks = b0 < b1;
  const int bl = has_blocks ? b1 - 1 : 0;
  const int token_tiles = (a.tokens + 15) >> 4;
  const uint8_t *wbase = reinterpret_cast<const uint8_t *>(a.w);
  const bool vec_out = (a.stride & 3) == 0;

  // token tiles: one per grid.z slice (the argmax path walks them all)
  for (int tt = blockIdx.z; tt < token_tiles; tt += gridDim.z) {
    const uint64_t *acodes = a.codes + static_cast<size_t>(tt) * nb * 64 + lane;
    const float *ascale = a.scales + static_cast<size_t>(tt) * nb * 16 + 4 * G;
    unsigned long long run_best[4] = {0ull, 0ull, 0ull, 0ull};  // single-wave argmax
    if (ARGMAX && W > 1) {
      __syncthreads();
      if (threadIdx.x < 16) best[threadIdx.x] = 0ull;
    }
    for (int g = blockIdx.x; g < groups; g += gridDim.x) {
      float acc[4][4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = 0.0F;
      // rows past the matrix read a valid tile (the last); their outputs are
      // never stored
      const int rt = min(g * 8 + T, ntiles - 1);
      const uint8_t *qrow = wbase + static_cast<size_t>(rt) * nb * 144 + 16 + 16 * (2 * G + h);
      const uint8_t *drow = wbase + static_cast<size_t>(rt) * nb * 144 + 8 * h;

      for (int cb = has_blocks ? b0 : 0; cb < (has_blocks ? b1 : 1); cb += KS) {
        // all loads of the chunk first (indices clamped into the wave's
        // range, so no load is predicated), then the MFMAs
        q35_u32x4 q[KS];
        q35_u32x2 d[KS];
        long act[KS];
        q35_f32x4 sa[KS];
#pragma unroll
        for (int i = 0; i < KS; ++i) {
          const size_t b = static_cast<size_t>(min(cb + i, bl));
          q[i] = *reinterpret_cast<const q35_u32x4 *>(qrow + b * 144);
          d[i] = *reinterpret_cast<const q35_u32x2 *>(drow + b * 144);
          act[i] = static_cast<long>(acodes[b * 64]);
          sa[i] = *reinterpret_cast<const q35_f32x4 *>(ascale + b * 16);
        }
#pragma unroll
        for (int i = 0; i < KS; ++i) {
          // a padded slot past the wave's range re-reads its last block; a
          // zero row scale makes its contribution exactly +0 (acc is never -0)
          const bool valid = has_blocks && cb + i < b1;
          if (!valid) d[i] = q35_u32x2{0u, 0u};
          const v4i zero = {0, 0, 0, 0};
          const v4i corr = Q35_MFMA_I32_16X16X32_I8(act[i], kMinus8, zero, 0, 0, 0);
          v4i D[4];
          D[0] = Q35_MFMA_I32_16X16X32_I8(act[i], unpack_word(q[i][0]), corr, 0, 0, 0);
          D[1] = Q35_MFMA_I32_16X16X32_I8(act[i], unpack_word(q[i][1]), corr, 0, 0, 0);
          D[2] = Q35_MFMA_I32_16X16X32_I8(act[i], unpack_word(q[i][2]), corr, 0, 0, 0);
          D[3] = Q35_MFMA_I32_16X16X32_I8(act[i], unpack_word(q[i][3]), corr, 0, 0, 0);
          const float dw[4] = {half_bits_to_float(static_cast<uint16_t>(d[i][0] & 0xffffu)),
                               half_bits_to_float(static_cast<uint16_t>(d[i][0] >> 16)),
                               half_bits_to_float(static_cast<uint16_t>(d[i][1] & 0xffffu)),
                               half_bits_to_float(static_cast<uint16_t>(d[i][1] >> 16))};
#pragma unroll
          for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int j = 0; j < 4; ++j)
              acc[r][j] = fmaf(static_cast<float>(D[r][j]), dw[r] * sa[i][j], acc[r][j]);
          if constexpr (DOTS) {
            if (!valid) continue;
            const int b = cb + i;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const int tok = tt * 16 + 4 * G + j;
              if (tok >= a.tokens) continue;
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                const int row = g * kRowsPerGroup + 4 * c + r;
                if (row < a.rows)
                  a.block_dots[(static_cast<size_t>(tok) * a.rows + row) * nb + b] = D[r][j];
              }
            }
          }
        }
      }

      if (ARGMAX && W == 1) {
        // one wavefront: penalty, then the best key of tokens 4G..4G+3 over
        // this lane's four rows and the 16 lanes sharing G
        const int row0 = g * kRowsPerGroup + 4 * c;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int tok = tt * 16 + 4 * G + j;
          unsigned long long key = 0ull;
          if (tok < a.tokens) {
            const float pen = a.penalties != nullptr ? a.penalties[tok] : 1.0F;
            const long long crow = a.count_rows != nullptr ? a.count_rows[tok] : tok;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int row = row0 + r;
              if (row >= a.rows) continue;
              float val = acc[r][j];
              if (pen > 1.0F && a.counts != nullptr && a.counts[crow * a.counts_stride + row] > 0)
                val = val > 0.0F ? val / pen : val * pen;
              const unsigned long long k = argmax_key(val, static_cast<uint32_t>(row));
              key = k > key ? k : key;
            }
          }
#pragma unroll
          for (int m = 1; m < 16; m <<= 1) {
            const unsigned long long o = __shfl_xor(key, m, 64);
            key = o > key ? o : key;
          }
          run_best[j] = key > run_best[j] ? key : run_best[j];
        }
        continue;
      }
      if (!ARGMAX && W == 1) {
        // one wavefront: store straight from registers (rows 4c..4c+3 of
        // tokens 4G..4G+3)
        const int row = g * kRowsPerGroup + 4 * c;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int tok = tt * 16 + 4 * G + j;
          if (tok >= a.tokens || row >= a.rows) continue;
          if (S > 1) {
            float *dst = a.partials + (static_cast<size_t>(split) * a.tokens + tok) * a.rows + row;
            store_row4(dst, true, acc[0][j], acc[1][j], acc[2][j], acc[3][j]);
          } else if (a.out != nullptr) {
            const size_t o = static_cast<size_t>(tok) * a.stride + row;
            float v[4] = {acc[0][j], acc[1][j], acc[2][j], acc[3][j]};
            if (a.residual != nullptr)
#pragma unroll
              for (int r = 0; r < 4; ++r) v[r] = a.residual[o + r] + v[r];
            store_row4(a.out + o, vec_out, v[0], v[1], v[2], v[3]);
          }
        }
        continue;
      }

      // Fixed-order sum of the wavefronts' partials, then the epilogue.
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float *dst = red + (static_cast<size_t>(wave) * 16 + (4 * G + j)) * 64 + 4 * c;
        *reinterpret_cast<q35_f32x4 *>(dst) = q35_f32x4{acc[0][j], acc[1][j], acc[2][j], acc[3][j]};
      }
      __syncthreads();
      for (int e = threadIdx.x; e < 16 * 64; e += blockDim.x) {
        const int t = e >> 6, r = e & 63;
        float s = red[static_cast<size_t>(t) * 64 + r];
        for (int w = 1; w < W; ++w) s += red[(static_cast<size_t>(w) * 16 + t) * 64 + r];
        const int tok = tt * 16 + t, row = g * kRowsPerGroup + r;
        if constexpr (!ARGMAX) {
          if (tok < a.tokens && row < a.rows) {
            if (S > 1) {
              a.partials[(static_cast<size_t>(split) * a.tokens + tok) * a.rows + row] = s;
            } else if (a.out != nullptr) {
              const size_t o = static_cast<size_t>(tok) * a.stride + row;
              a.out[o] = a.residual != nullptr ? a.residual[o] + s : s;
            }
          }
        } else {
          // greedy head: repetition penalty, then the per-token best key of
          // this group (all 64 lanes of a wave share t)
          unsigned long long key = 0ull;
          if (tok < a.tokens && row < a.rows) {
            float val = s;
            const float pen = a.penalties != nullptr ? a.penalties[tok] : 1.0F;
            if (pen > 1.0F && a.counts != nullptr) {
              const long long crow = a.count_rows != nullptr ? a.count_rows[tok] : tok;
              if (a.counts[crow * a.counts_stride + row] > 0) val = val > 0.0F ? val / pen : val * pen;
            }
            key = argmax_key(val, static_cast<uint32_t>(row));
          }
#pragma unroll
          for (int m = 32; m >= 1; m >>= 1) {
            const unsigned long long o = __shfl_xor(key, m, 64);
            key = o > key ? o : key;
          }
          if (lane == 0 && key > best[t]) best[t] = key;
        }
      }
      __syncthreads();
    }
    if (ARGMAX && W == 1) {
      if (c == 0) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int tok = tt * 16 + 4 * G + j;
          if (tok < a.tokens) a.cand[static_cast<size_t>(blockIdx.x) * a.cand_stride + tok] = run_best[j];
        }
      }
    } else if (ARGMAX) {
      __syncthreads();
      if (threadIdx.x < 16) {
        const int tok = tt * 16 + threadIdx.x;
        if (tok < a.tokens) a.cand[static_cast<size_t>(blockIdx.x) * a.cand_stride + tok] = best[threadIdx.x];
      }
    }
  }
}

// Split-K projection kernel with 16·RM-row groups (RM = 1 or 2 MFMAs per
// block): one wavefront per (row group, K split, token tile). Fewer rows per
// wavefront shorten each wavefront's serial epilogue (the fp32 chain is 3
// VALU ops per output and block) at the same split partials.
// Lane l = (G = l/16, c = l%16) covers rows r0 .. r0+RM-1 of tile c/(8/RM),
// r0 = RM·(c % (8/RM)): per block it loads the body words 8G + r0 .. +RM-1
// (k-group G) and those rows' FP16 scales; word i is the B operand of MFMA #i
// for column c, i.e. output row RM·c + i of the group. The int32 block dot
// and the fp32 chain per block are gemm_kernel's.
// Occupancy floor 2 keeps the MFMA results in VGPRs (no AGPR copies).
template <int KS, int RM>
__global__ __launch_bounds__(64) Q35_WAVES_PER_EU(2) void gemm_rows_kernel(GemmArgs a) {
  typedef RowWords<RM> RW;
  constexpr int kLanesPerTile = 8 / RM, kGroupRows = 16 * RM;
  const int lane = threadIdx.x;
  const int G = lane >> 4, c = lane & 15;
  const int nb = a.nb, ntiles = a.rows >> 3;
  const int S = gridDim.y, split = blockIdx.y, g = blockIdx.x, tt = blockIdx.z;
  const int b0 = (split * nb) / S, b1 = ((split + 1) * nb) / S;
  const int bl = b1 - 1;
  const uint64_t *acodes = a.codes + static_cast<size_t>(tt) * nb * 64 + lane;
  const float *ascale = a.scales + static_cast<size_t>(tt) * nb * 16 + 4 * G;
  // rows past the matrix read a valid tile (the last); they are never stored
  const int rt = min(g * (kGroupRows / 8) + c / kLanesPerTile, ntiles - 1);
  const int r0 = RM * (c % kLanesPerTile);
  const uint8_t *tile = reinterpret_cast<const uint8_t *>(a.w) + static_cast<size_t>(rt) * nb * 144;
  const uint8_t *qrow = tile + 16 + 32 * G + 4 * r0;
  const uint8_t *drow = tile + 2 * r0;
  float acc[RM][4];
#pragma unroll
  for (int i = 0; i < RM; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.0F;
  for (int cb = b0; cb < b1; cb += KS) {
    typename RW::Q q[KS];
    typename RW::D d[KS];
    long act[KS];
    q35_f32x4 sa[KS];
#pragma unroll
    for (int i = 0; i < KS; ++i) {
      const size_t b = static_cast<size_t>(min(cb + i, bl));
      // read once per step: streamed (non-temporal), so that they do not
      // evict the vocabulary head's weights from the Infinity Cache between
      // steps (the head then reads much of its 143 MB from there)
      q[i] = Q35_LOAD_NT(reinterpret_cast<const typename RW::Q *>(qrow + b * 144));
      d[i] = Q35_LOAD_NT(reinterpret_cast<const typename RW::D *>(drow + b * 144));
      act[i] = static_cast<long>(acodes[b * 64]);
      sa[i] = *reinterpret_cast<const q35_f32x4 *>(ascale + b * 16);
    }
#pragma unroll
    for (int i = 0; i < KS; ++i) {
      // a slot past the range re-reads its last block; a zero row scale makes
      // its contribution exactly +0 (acc is never -0)
      const bool valid = cb + i < b1;
      const v4i zero = {0, 0, 0, 0};
      const v4i corr = Q35_MFMA_I32_16X16X32_I8(act[i], kMinus8, zero, 0, 0, 0);
#pragma unroll
      for (int r = 0; r < RM; ++r) {
        const v4i D = Q35_MFMA_I32_16X16X32_I8(act[i], unpack_word(RW::word(q[i], r)), corr, 0, 0, 0);
        const float dw = valid ? half_bits_to_float(RW::scale(d[i], r)) : 0.0F;
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[r][j] = fmaf(static_cast<float>(D[j]), dw * sa[i][j], acc[r][j]);
      }
    }
  }
  // rows RM·c .. RM·c + RM-1 of tokens 4G..4G+3
  const int row = g * kGroupRows + RM * c;
  if (row >= a.rows) return;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int tok = tt * 16 + 4 * G + j;
    if (tok >= a.tokens) continue;
    if (S > 1) {
      float *dst = a.partials + (static_cast<size_t>(split) * a.tokens + tok) * a.rows + row;
      if constexpr (RM == 1)
        *dst = acc[0][j];
      else
        *reinterpret_cast<q35_f32x2 *>(dst) = q35_f32x2{acc[0][j], acc[1][j]};
    } else {
      const size_t o = static_cast<size_t>(tok) * a.stride + row;
#pragma unroll
      for (int r = 0; r < RM; ++r) a.out[o + r] = a.residual != nullptr ? a.residual[o + r] + acc[r][j] : acc[r][j];
    }
  }
}

// Streaming Q4 GEMV for the vocabulary head: a tall matrix, one K split.
//
// Each wavefront owns a contiguous run of `gpw` 64-row groups and walks it
// chunk by chunk (KS blocks per chunk, all K blocks of a group before the
// next group). A ring of R register buffers keeps the weight loads of the
// next R-1 chunks in flight while the MFMAs of the current chunk run, so the
// wavefronts never alternate between a load phase and a compute phase. Every
// weight load is unconditional: past the wavefront's last chunk the ring
// re-loads that chunk (an L2 hit) instead of branching, since a load under a
// branch makes the compiler wait for every outstanding load at the join. The
// A16 codes and scales of all NT token tiles are staged once per workgroup in
// LDS, so the weights are the only HBM stream. Per block, row and token the
// arithmetic is gemm_kernel's: the exact int32 block dot and the reference's
// fp32 fma chain in block order (q4_dot4.cpp:53). ARGMAX leaves one best key
// per wavefront and token in cand[wave][token] (0 for a wavefront past the
// last group); otherwise the rows are stored to out[token][row].
constexpr int kHeadWaves = 4;  // wavefronts per workgroup
constexpr int kHeadKS = 4;     // blocks per chunk
constexpr int kHeadRing = 3;   // chunks per wavefront: one computing, the rest in flight
constexpr size_t kHeadMaxLds = 64 * 1024;
// wavefronts per SIMD the register budget (and the grid) are sized for: the
// accumulators of more token tiles need more registers
constexpr int head_waves_per_simd(int nt) { return nt == 1 ? 3 : 2; }

template <int KS, bool G16>
struct HeadChunk {
  q35_u32x4 q[KS];
  q35_u32x2 d[KS];
  q35_u32x2 d2[G16 ? KS : 1];  // G16: the scales of columns 16-31
};

// G16: Q4G16Tile weights (q4_g16.h:5-6, 160-byte tiles: d[2][8] then the
// DOT4 codes). Each block's two 16-column halves are separate int8 dots:
// MFMAs over the activations with the other half's K lanes zeroed, chained
// per block as half 0 then half 1, acc = fma(float(dot), d_half * s, acc)
// (q4_g16_matmul_wide, q4_g16_evex.cpp:25-49). G16 launches use a two-chunk
// ring: with three, the second scale words spill at the head's occupancy.
template <int KS, int R, int NT, bool ARGMAX, int OCC, bool G16>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(OCC, OCC))) void head_kernel(GemmArgs a,
                                                                                               int gpw) {
  static_assert(R >= 2, "the ring loads the next chunk before computing the current one");
  Q35_DYNAMIC_SHARED(uint64_t, lcodes);  // [NT][nb][64] A16 words, then float [NT][nb][16]
  const int nb = a.nb;
  float *lscales = reinterpret_cast<float *>(lcodes + static_cast<size_t>(NT) * nb * 64);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int G = lane >> 4, c = lane & 15, h = c & 1, T = c >> 1;
  const int ntiles = a.rows >> 3, groups = (ntiles + 7) >> 3;
  const int gw = blockIdx.x * kHeadWaves + wave;
  const int g0 = min(groups, gw * gpw), g1 = min(groups, g0 + gpw);
  const int cpg = (nb + KS - 1) / KS;
  const int iters = (g1 - g0) * cpg;
  const uint8_t *wbase = reinterpret_cast<const uint8_t *>(a.w);
  constexpr int kTile = G16 ? 160 : 144, kCodes = G16 ? 32 : 16;
  const size_t tile_bytes = static_cast<size_t>(nb) * kTile;

  // next chunk to load: group lg, chunk lch (advanced after every load);
  // past the last chunk the last one is loaded again
  int lg = g0, lch = 0;
  auto load = [&](HeadChunk<KS, G16> &buf) {
    const bool past = lg >= g1;
    const int gl = max(past ? g1 - 1 : lg, 0), cl = past ? cpg - 1 : lch;
    const int rt = min(gl * 8 + T, ntiles - 1);
    const uint8_t *tile = wbase + static_cast<size_t>(rt) * tile_bytes;
#pragma unroll
    for (int i = 0; i < KS; ++i) {
      const size_t b = static_cast<size_t>(min(cl * KS + i, nb - 1));
      buf.q[i] = *reinterpret_cast<const q35_u32x4 *>(tile + b * kTile + kCodes + 16 * (2 * G + h));
      buf.d[i] = *reinterpret_cast<const q35_u32x2 *>(tile + b * kTile + 8 * h);
      if constexpr (G16) buf.d2[i] = *reinterpret_cast<const q35_u32x2 *>(tile + b * kTile + 16 + 8 * h);
    }
    if (++lch == cpg) {
      lch = 0;
      ++lg;
    }
  };

  // per-token penalty and counts row (loop invariant; loaded before the
  // weights so that the group epilogues never wait on a load)
  float pen[NT][4];
  int crow[NT][4];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int tok = min(t * 16 + 4 * G + j, a.tokens - 1);
      pen[t][j] = ARGMAX && a.penalties != nullptr ? a.penalties[tok] : 1.0F;
      crow[t][j] = ARGMAX && a.count_rows != nullptr ? a.count_rows[tok] : tok;
    }

  HeadChunk<KS, G16> buf[R];
  load(buf[0]);
  // stage the activations; the first pass is issued before chunks 1..R-2, so
  // waiting for it leaves those chunks in flight
  {
    const int n16 = NT * nb * 32;  // 16-byte words of codes
    const int s16 = NT * nb * 4;   // 16-byte words of scales
    const q35_u32x4 *gc = reinterpret_cast<const q35_u32x4 *>(a.codes);
    const q35_u32x4 *gs = reinterpret_cast<const q35_u32x4 *>(a.scales);
    q35_u32x4 *lc = reinterpret_cast<q35_u32x4 *>(lcodes);
    q35_u32x4 *ls = reinterpret_cast<q35_u32x4 *>(lscales);
    auto pass = [&](int i0, bool first) {
      q35_u32x4 v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int i = min(i0 + u * 256, n16 + s16 - 1);
        v[u] = i < n16 ? gc[i] : gs[i - n16];
      }
      if (first) {
#pragma unroll
        for (int k = 1; k < R - 1; ++k) load(buf[k]);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int i = i0 + u * 256;
        if (i < n16) lc[i] = v[u];
        else if (i < n16 + s16) ls[i - n16] = v[u];
      }
    };
    pass(threadIdx.x, true);
    for (int i0 = threadIdx.x + 4 * 256; i0 < n16 + s16; i0 += 4 * 256) pass(i0, false);
  }
  lds_barrier();

  float acc[NT][4][4];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[t][i][j] = 0.0F;
  unsigned long long run_best[NT][4];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int j = 0; j < 4; ++j) run_best[t][j] = 0ull;
  const bool vec_out = (a.stride & 3) == 0;

  // group cg, chunk cch of the next compute
  int cg = g0, cch = 0;
  auto epilogue = [&]() {
    const int row0 = cg * kRowsPerGroup + 4 * c;
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int tok = t * 16 + 4 * G + j;
        if constexpr (ARGMAX) {
          unsigned long long key = 0ull;
          if (tok < a.tokens) {
            const float p = pen[t][j];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int row = row0 + r;
              if (row >= a.rows) continue;
              float val = acc[t][r][j];
              if (p > 1.0F && a.counts != nullptr &&
                  a.counts[static_cast<long long>(crow[t][j]) * a.counts_stride + row] > 0)
                val = val > 0.0F ? val / p : val * p;
              const unsigned long long k = argmax_key(val, static_cast<uint32_t>(row));
              key = k > key ? k : key;
            }
          }
#pragma unroll
          for (int m = 1; m < 16; m <<= 1) {
            const unsigned long long o = __shfl_xor(key, m, 64);
            key = o > key ? o : key;
          }
          run_best[t][j] = key > run_best[t][j] ? key : run_best[t][j];
        } else {
          if (tok < a.tokens && row0 < a.rows)
            store_row4(a.out + static_cast<size_t>(tok) * a.stride + row0, vec_out, acc[t][0][j], acc[t][1][j],
                       acc[t][2][j], acc[t][3][j]);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[t][r][j] = 0.0F;
      }
  };
  auto compute = [&](HeadChunk<KS, G16> &cur) {
#pragma unroll
    for (int i = 0; i < KS; ++i) {
      const int b = cch * KS + i;
      // a slot past the last block re-reads it; a zero row scale makes its
      // contribution exactly +0 (acc is never -0)
      if (b >= nb) {
        cur.d[i] = q35_u32x2{0u, 0u};
        if constexpr (G16) cur.d2[i] = q35_u32x2{0u, 0u};
      }
      const int bl = min(b, nb - 1);
      const long w0 = unpack_word(cur.q[i][0]), w1 = unpack_word(cur.q[i][1]);
      const long w2 = unpack_word(cur.q[i][2]), w3 = unpack_word(cur.q[i][3]);
      const float dw[4] = {half_bits_to_float(static_cast<uint16_t>(cur.d[i][0] & 0xffffu)),
                           half_bits_to_float(static_cast<uint16_t>(cur.d[i][0] >> 16)),
                           half_bits_to_float(static_cast<uint16_t>(cur.d[i][1] & 0xffffu)),
                           half_bits_to_float(static_cast<uint16_t>(cur.d[i][1] >> 16))};
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const long act = static_cast<long>(lcodes[(static_cast<size_t>(t) * nb + bl) * 64 + lane]);
        const q35_f32x4 sa =
            *reinterpret_cast<const q35_f32x4 *>(lscales + (static_cast<size_t>(t) * nb + bl) * 16 + 4 * G);
        const v4i zero = {0, 0, 0, 0};
        if constexpr (G16) {
          // lanes G = 0, 1 hold columns 0-15 of the block, G = 2, 3 columns 16-31
          const long lo = G < 2 ? act : 0l, hi = G < 2 ? 0l : act;
          const float dh[4] = {half_bits_to_float(static_cast<uint16_t>(cur.d2[i][0] & 0xffffu)),
                               half_bits_to_float(static_cast<uint16_t>(cur.d2[i][0] >> 16)),
                               half_bits_to_float(static_cast<uint16_t>(cur.d2[i][1] & 0xffffu)),
                               half_bits_to_float(static_cast<uint16_t>(cur.d2[i][1] >> 16))};
          const v4i corr_lo = Q35_MFMA_I32_16X16X32_I8(lo, kMinus8, zero, 0, 0, 0);
          const v4i corr_hi = Q35_MFMA_I32_16X16X32_I8(hi, kMinus8, zero, 0, 0, 0);
          const long wr[4] = {w0, w1, w2, w3};
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const v4i Dl = Q35_MFMA_I32_16X16X32_I8(lo, wr[r], corr_lo, 0, 0, 0);
            const v4i Dh = Q35_MFMA_I32_16X16X32_I8(hi, wr[r], corr_hi, 0, 0, 0);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              acc[t][r][j] = fmaf(static_cast<float>(Dl[j]), dw[r] * sa[j], acc[t][r][j]);
              acc[t][r][j] = fmaf(static_cast<float>(Dh[j]), dh[r] * sa[j], acc[t][r][j]);
            }
          }
        } else {
          const v4i corr = Q35_MFMA_I32_16X16X32_I8(act, kMinus8, zero, 0, 0, 0);
          v4i D[4];
          D[0] = Q35_MFMA_I32_16X16X32_I8(act, w0, corr, 0, 0, 0);
          D[1] = Q35_MFMA_I32_16X16X32_I8(act, w1, corr, 0, 0, 0);
          D[2] = Q35_MFMA_I32_16X16X32_I8(act, w2, corr, 0, 0, 0);
          D[3] = Q35_MFMA_I32_16X16X32_I8(act, w3, corr, 0, 0, 0);
#pragma unroll
          for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int j = 0; j < 4; ++j)
              acc[t][r][j] = fmaf(static_cast<float>(D[r][j]), dw[r] * sa[j], acc[t][r][j]);
        }
      }
    }
    if (++cch == cpg) {
      epilogue();
      cch = 0;
      ++cg;
    }
  };

  // at the top of each round chunks it .. it+R-2 are in flight in
  // buf[0 .. R-2]; step k issues chunk it+k+R-1 into the buffer freed by
  // step k-1, then computes chunk it+k
  for (int it = 0; it < iters; it += R) {
#pragma unroll
    for (int k = 0; k < R; ++k) {
      load(buf[(k + R - 1) % R]);
      if (it + k < iters) compute(buf[k]);
    }
  }

  if constexpr (ARGMAX) {
    if (c == 0) {
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int tok = t * 16 + 4 * G + j;
          if (tok < a.tokens) a.cand[static_cast<size_t>(gw) * a.cand_stride + tok] = run_best[t][j];
        }
    }
  }
}

// One workgroup per token: the best key over all workgroups' candidates,
// eight loads per thread in flight, then the wave and workgroup maxima.
constexpr int kFinalizeThreads = 256;
__global__ __launch_bounds__(kFinalizeThreads) void argmax_finalize_kernel(const unsigned long long *cand, int ncand,
                                                                           int cand_stride, int tokens,
                                                                           int32_t *index, float *value) {
  __shared__ unsigned long long wbest[kFinalizeThreads / 64];
  const int tok = blockIdx.x, tid = threadIdx.x;
  unsigned long long key = 0ull;
  for (int i0 = tid; i0 < ncand; i0 += 8 * kFinalizeThreads) {
    unsigned long long k[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = i0 + u * kFinalizeThreads;
      k[u] = i < ncand ? cand[static_cast<size_t>(i) * cand_stride + tok] : 0ull;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) key = k[u] > key ? k[u] : key;
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const unsigned long long o = __shfl_xor(key, m, 64);
    key = o > key ? o : key;
  }
  if ((tid & 63) == 0) wbest[tid >> 6] = key;
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < kFinalizeThreads / 64; ++w) key = wbest[w] > key ? wbest[w] : key;
    if (index != nullptr) index[tok] = static_cast<int32_t>(argmax_key_index(key));
    if (value != nullptr) value[tok] = argmax_key_value(key);
  }
}

// out[t][row] = (residual +) the split partial rows summed in split order;
// used where no consumer kernel folds the reduction in (kernel-level entries).
__global__ void split_reduce_kernel(SplitRows src, int tokens, float *out, int stride, const float *residual) {
  const int row = blockIdx.x * blockDim.x + threadIdx.x, t = blockIdx.y;
  if (row >= src.width || t >= tokens) return;
  const size_t o = static_cast<size_t>(t) * stride + row;
  const float *q = src.p + static_cast<long long>(t) * src.width + row;
  float v = q[0];
  for (int s = 1; s < src.splits; ++s) v += q[s * src.split_stride];
  out[o] = residual != nullptr ? residual[o] + v : v;
}

}  // namespace

hipError_t launch_split_reduce(const SplitRows &src, int tokens, float *out, int stride, const float *residual,
                               hipStream_t stream) {
  if (tokens <= 0 || src.width <= 0) return hipSuccess;
  Q35_LAUNCH((split_reduce_kernel), dim3((src.width + 255) / 256, tokens), dim3(256), 0, stream, src, tokens, out,
             stride, residual);
  return hipGetLastError();
}

GemmPlan gemm_plan(int rows, int nb, bool exact, bool argmax, int cu_count, int force_ks, int force_split,
                   int max_split) {
  GemmPlan p{};
  const int groups = (rows / 8 + 7) / 8;
  const int cus = cu_count > 0 ? cu_count : 256;
  if (exact) {
    p.ks = 8;
    p.waves = 1;
    p.split = 1;
    p.grid = groups;
  } else if (argmax) {
    // one wavefront per workgroup walking whole row groups (all K chunks),
    // several workgroups per CU to hide the chunk latency
    p.ks = 8;
    p.waves = 1;
    p.split = 1;
    p.grid = std::min(groups, 8 * cus);
  } else {
    // one wavefront per workgroup; K split across workgroups in chunks of 8
    // blocks. (Chunks of 4 for narrow outputs give the GEMM more workgroups,
    // but twice the split partials for the consumer to read: the decode step
    // measured faster with 8 throughout.)
    p.ks = force_ks > 0 ? force_ks : 8;
    const int chunks = (nb + p.ks - 1) / p.ks;
    p.split = force_split > 0 ? std::min(force_split, chunks) : std::min({chunks, 32, std::max(1, max_split)});
    const int per_split = (chunks + p.split - 1) / p.split;
    p.waves = force_split > 0 ? std::min(kMaxWaves, per_split) : 1;
    p.grid = groups;
  }
  p.smem = (static_cast<size_t>(p.waves) * 16 * 64) * 4 + 16 * 8;
  return p;
}

namespace {
// Launch shape of head_kernel: token tiles, 64-row groups per wavefront,
// workgroups and LDS bytes; `use` is false when the staged activations do
// not fit (gemm_kernel then runs the shape).
struct HeadPlan {
  bool use;
  int nt, gpw, grid;
  size_t smem;
};
HeadPlan head_plan(int rows, int nb, int tokens, int cu_count, int force_gpw) {
  HeadPlan p{};
  const int groups = (rows / 8 + 7) / 8;
  const int cus = cu_count > 0 ? cu_count : 256;
  p.nt = (tokens + 15) / 16;
  p.smem = static_cast<size_t>(p.nt) * nb * (64 * sizeof(uint64_t) + 16 * sizeof(float));
  p.use = p.nt >= 1 && p.nt <= 4 && p.smem <= kHeadMaxLds;
  // as few groups per wavefront as keep every wavefront resident at once
  const int resident = cus * 4 * head_waves_per_simd(std::max(1, std::min(p.nt, 4)));
  p.gpw = force_gpw > 0 ? force_gpw : std::max(1, (groups + resident - 1) / resident);
  const int waves = (groups + p.gpw - 1) / p.gpw;
  p.grid = (waves + kHeadWaves - 1) / kHeadWaves;
  return p;
}
}  // namespace

// Token tiles whose staged activations fit one head workgroup's LDS.
int head_fit_tiles(int nb) {
  int nt = 4;
  while (nt > 0 && static_cast<size_t>(nt) * nb * (64 * sizeof(uint64_t) + 16 * sizeof(float)) > kHeadMaxLds) --nt;
  return nt;
}

int gemm_argmax_cands(int rows, int nb, int tokens, int cu_count, int force_gpw, bool g16) {
  const HeadPlan hp = head_plan(rows, nb, tokens, cu_count, force_gpw);
  if (hp.use) return hp.grid * kHeadWaves;
  // G16: launches of head_fit_tiles token tiles at one plan's grid
  if (g16) return head_plan(rows, nb, 16 * std::max(1, head_fit_tiles(nb)), cu_count, force_gpw).grid * kHeadWaves;
  return gemm_plan(rows, nb, false, true, cu_count, 0, 0).grid;
}

int gemm_argmax_cand_capacity(int rows, int cu_count) {
  return std::max(head_plan(rows, 1, 16, cu_count, 0).grid * kHeadWaves,
                  gemm_plan(rows, 32, false, true, cu_count, 0, 0).grid);
}

size_t gemm_partial_floats(int rows, int nb, int tokens, int cu_count) {
  const GemmPlan p = gemm_plan(rows, nb, false, false, cu_count, 0, 0);
  return p.split > 1 ? static_cast<size_t>(p.split) * tokens * rows : 0;
}

hipError_t launch_gemm(const GemmArgs &a, hipStream_t stream) {
  if (a.tokens <= 0 || a.rows <= 0) return hipSuccess;
  const bool argmax = a.cand != nullptr;
  const bool exact = a.exact || a.block_dots != nullptr;
  if (a.g16 && (!(argmax || a.head) || exact || (!argmax && a.out == nullptr))) return hipErrorInvalidValue;
  if ((argmax || a.head) && !exact && (argmax || a.out != nullptr)) {
    const HeadPlan hp = head_plan(a.rows, a.nb, a.tokens, a.cu_count, a.force_gpw);
    if (!hp.use && (a.g16 || !argmax)) {
      // G16 has only the staged-activation kernel, and a logits head must
      // keep its single fma chain per output at every batch size (the split
      // fallback would sum several wavefronts' chains): launches over groups
      // of token tiles that fit, all at one grid so that the candidate rows
      // (G16 argmax) line up with gemm_argmax_cands
      const int fit = head_fit_tiles(a.nb);
      if (fit < 1) {
        // rows too wide for even one staged token tile (more than 113 K
        // blocks): the logits head runs the exact-mode GEMM, one wavefront
        // per row group over all K blocks -- the same single block-order
        // chain per output. G16 has no other kernel.
        if (a.g16) return hipErrorInvalidValue;
        GemmArgs c = a;
        c.exact = true;
        return launch_gemm(c, stream);
      }
      const int gpw = head_plan(a.rows, a.nb, 16 * fit, a.cu_count, a.force_gpw).gpw;
      for (int t0 = 0; t0 < a.tokens; t0 += 16 * fit) {
        GemmArgs c = a;
        c.tokens = std::min(16 * fit, a.tokens - t0);
        c.force_gpw = gpw;
        c.codes = a.codes + static_cast<size_t>(t0 / 16) * a.nb * 64;
        c.scales = a.scales + static_cast<size_t>(t0 / 16) * a.nb * 16;
        if (a.out != nullptr) c.out = a.out + static_cast<size_t>(t0) * a.stride;
        if (a.cand != nullptr) c.cand = a.cand + t0;
        if (a.penalties != nullptr) c.penalties = a.penalties + t0;
        if (a.count_rows != nullptr)
          c.count_rows = a.count_rows + t0;
        else if (a.counts != nullptr)
          c.counts = a.counts + static_cast<long long>(t0) * a.counts_stride;
        const hipError_t e = launch_gemm(c, stream);
        if (e != hipSuccess) return e;
      }
      return hipSuccess;
    }
    if (hp.use) {
      const dim3 grid(hp.grid), block(64 * kHeadWaves);
#define Q35_HEAD_G(NT, G16)                                                                                     \
  if (argmax) {                                                                                                 \
    Q35_LAUNCH((head_kernel<kHeadKS, (G16 ? 2 : kHeadRing), NT, true, head_waves_per_simd(NT), G16>), grid, block, hp.smem,  \
               stream, a, hp.gpw);                                                                              \
  } else {                                                                                                      \
    Q35_LAUNCH((head_kernel<kHeadKS, (G16 ? 2 : kHeadRing), NT, false, head_waves_per_simd(NT), G16>), grid, block, hp.smem, \
               stream, a, hp.gpw);                                                                              \
  }
#define Q35_HEAD(NT)         \
  if (a.g16) {               \
    Q35_HEAD_G(NT, true)     \
  } else {                   \
    Q35_HEAD_G(NT, false)    \
  }
      switch (hp.nt) {
        case 1: Q35_HEAD(1) break;
        case 2: Q35_HEAD(2) break;
        case 3: Q35_HEAD(3) break;
        default: Q35_HEAD(4) break;
      }
#undef Q35_HEAD
#undef Q35_HEAD_G
      return hipGetLastError();
    }
  }
  const GemmPlan p = gemm_plan(a.rows, a.nb, exact, argmax, a.cu_count, a.force_ks, a.force_split,
                               a.max_split > 0 ? a.max_split : 32);
  // a split plan writes [split][tokens][rows] partials; a single split writes `out`
  if ((p.split > 1 && a.partials == nullptr) || (p.split == 1 && a.out == nullptr && !argmax && a.block_dots == nullptr))
    return hipErrorInvalidValue;
  const dim3 grid(p.grid, p.split, argmax ? 1 : (a.tokens + 15) / 16), block(64 * p.waves);
  if (!argmax && a.block_dots == nullptr && !exact && p.waves == 1 && (a.tokens <= 16 || a.group_rows > 0)) {
    // one token tile: row groups of 16·RM rows per wavefront -- 32 rows, or
    // 16 where 32-row groups would leave fewer than two wavefronts per CU
    // (narrow outputs). Several token tiles (4B-sized chunks at B = 64)
    // measured faster with gemm_kernel's 64-row groups.
    const int cus = a.cu_count > 0 ? a.cu_count : 256;
    const int waves32 = ((a.rows >> 3) + 3) / 4 * p.split * ((a.tokens + 15) / 16);
    const int rm = a.group_rows == 32 ? 2 : a.group_rows == 16 ? 1 : (waves32 < 2 * cus ? 1 : 2);
    const dim3 grid_r(((a.rows >> 3) + 2 * rm - 1) / (2 * rm), p.split, (a.tokens + 15) / 16);
#define Q35_ROWS(KS, RM) Q35_LAUNCH((gemm_rows_kernel<KS, RM>), grid_r, dim3(64), 0, stream, a)
    if (p.ks == 4) {
      if (rm == 1) Q35_ROWS(4, 1); else Q35_ROWS(4, 2);
    } else {
      if (rm == 1) Q35_ROWS(8, 1); else Q35_ROWS(8, 2);
    }
#undef Q35_ROWS
    return hipGetLastError();
  }
  if (argmax) {
    Q35_LAUNCH((gemm_kernel<8, true, false>), grid, block, p.smem, stream, a);
  } else if (a.block_dots != nullptr) {
    Q35_LAUNCH((gemm_kernel<8, false, true>), grid, block, p.smem, stream, a);
  } else if (p.ks == 4) {
    Q35_LAUNCH((gemm_kernel<4, false, false>), grid, block, p.smem, stream, a);
  } else {
    Q35_LAUNCH((gemm_kernel<8, false, false>), grid, block, p.smem, stream, a);
  }
  return hipGetLastError();
}

hipError_t launch_argmax_finalize(const unsigned long long *cand, int ncand, int cand_stride, int tokens,
                                  int32_t *index, float *value, hipStream_t stream) {
  Q35_LAUNCH((argmax_finalize_kernel), dim3(tokens), dim3(kFinalizeThreads), 0, stream, cand, ncand, cand_stride,
             tokens, index, value);
  return hipGetLastError();
}

}  // namespace q35
