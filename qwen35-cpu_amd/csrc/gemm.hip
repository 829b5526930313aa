// Q4-G32-DOT4 grouped GEMV/GEMM on CDNA4 int8 MFMA.
//
// Reads the reference's 144-byte Q4_0BlockX8 DOT4 tiles in place (no repack):
//   qs[32t+4r+j] = u[r][8t+j] | u[r][8t+4+j] << 4          (q4_dot4.h:5-6)
// so the 32-bit word 8t+r of a tile body holds row r's columns 8t..8t+3 (low
// nibbles) and 8t+4..8t+7 (high nibbles).
//
// Work decomposition. A workgroup owns a 64-row group (eight 8-row tiles) and
// W <= 16 wavefronts that split the K blocks of that group; every wavefront
// issues the loads of all of its blocks (at most 8 per chunk) before the
// first MFMA, so one launch keeps W x 8 x 1.1 KB of weights in flight per
// workgroup and the weight stream never waits on the activation chain.
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
// in block order within each wavefront; the wavefronts are summed in fixed
// order through LDS, so results are deterministic. With one wavefront per
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
constexpr int kChunk = 8;          // blocks per wavefront held in flight
constexpr int kMaxWaves = 16;
constexpr long kMinus8 = static_cast<long>(0xF8F8F8F8F8F8F8F8ull);  // int8 -8 x 8

__device__ __forceinline__ long unpack_word(uint32_t w) {
  const uint32_t lo = w & 0x0f0f0f0fu;
  const uint32_t hi = (w >> 4) & 0x0f0f0f0fu;
  return static_cast<long>((static_cast<uint64_t>(hi) << 32) | lo);
}

template <bool ARGMAX, bool DOTS>
__global__ __launch_bounds__(1024) void gemm_kernel(GemmArgs a) {
  Q35_DYNAMIC_SHARED(float, smem);
  const int W = static_cast<int>(blockDim.x) >> 6;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int G = lane >> 4, c = lane & 15, h = c & 1, T = c >> 1;
  const int nb = a.nb, ntiles = a.rows >> 3;
  const int groups = (ntiles + 7) >> 3;
  float *act_scale = smem;                  // [nb][16] scales of the token tile
  float *red = smem + nb * 16;              // [W][a.red_tokens][64] wave partials
  unsigned long long *best = reinterpret_cast<unsigned long long *>(red + W * a.red_tokens * 64);  // [16]

  const int per = a.exact ? nb : (nb + W - 1) / W;
  const int b0 = min(nb, wave * per), b1 = min(nb, b0 + per);
  const int token_tiles = (a.tokens + 15) >> 4;
  const uint8_t *wbase = reinterpret_cast<const uint8_t *>(a.w);

  // a wavefront with an empty block range (never produced by gemm_shape, kept
  // safe) reads block 0 and contributes nothing
  const bool has_blocks = b0 < b1;
  const int bl = has_blocks ? b1 - 1 : 0;

  for (int tt = 0; tt < token_tiles; ++tt) {
    const uint64_t *acodes = a.codes + static_cast<size_t>(tt) * nb * 64 + lane;
    bool staged = false;
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

      for (int cb = has_blocks ? b0 : 0; cb < (has_blocks ? b1 : 1); cb += kChunk) {
        // all loads of the chunk first (indices clamped into the wave's
        // range, so no load is predicated), then the MFMAs
        q35_u32x4 q[kChunk];
        q35_u32x2 d[kChunk];
        long act[kChunk];
#pragma unroll
        for (int i = 0; i < kChunk; ++i) {
          const size_t b = static_cast<size_t>(min(cb + i, bl));
          q[i] = Q35_LOAD_NT(reinterpret_cast<const q35_u32x4 *>(qrow + b * 144));
          d[i] = Q35_LOAD_NT(reinterpret_cast<const q35_u32x2 *>(drow + b * 144));
          act[i] = static_cast<long>(acodes[b * 64]);
        }
        if (!staged) {
          // the activation scales of this token tile, staged while the first
          // chunk's weights are in flight (every wavefront reaches this point
          // once per token tile: its first chunk of its first group)
          staged = true;
          __syncthreads();
          for (int i = threadIdx.x; i < nb * 16; i += blockDim.x)
            act_scale[i] = a.params[static_cast<size_t>(tt) * nb * 16 + i].scale;
          if (ARGMAX && threadIdx.x < 16) best[threadIdx.x] = 0ull;
          __syncthreads();
        }
#pragma unroll
        for (int i = 0; i < kChunk; ++i) {
          // a padded slot past the wave's range re-reads its last block; a
          // zero row scale makes its contribution exactly +0 (acc is never -0)
          const bool valid = has_blocks && cb + i < b1;
          const int b = valid ? cb + i : bl;
          if (!valid) d[i] = q35_u32x2{0u, 0u};
          const v4i zero = {0, 0, 0, 0};
          const v4i corr = Q35_MFMA_I32_16X16X32_I8(act[i], kMinus8, zero, 0, 0, 0);
          v4i D[4];
          D[0] = Q35_MFMA_I32_16X16X32_I8(act[i], unpack_word(q[i][0]), corr, 0, 0, 0);
          D[1] = Q35_MFMA_I32_16X16X32_I8(act[i], unpack_word(q[i][1]), corr, 0, 0, 0);
          D[2] = Q35_MFMA_I32_16X16X32_I8(act[i], unpack_word(q[i][2]), corr, 0, 0, 0);
          D[3] = Q35_MFMA_I32_16X16X32_I8(act[i], unpack_word(q[i][3]), corr, 0, 0, 0);
          const float *sp = act_scale + b * 16 + 4 * G;
          const float sa[4] = {sp[0], sp[1], sp[2], sp[3]};
          const float dw[4] = {half_bits_to_float(static_cast<uint16_t>(d[i][0] & 0xffffu)),
                               half_bits_to_float(static_cast<uint16_t>(d[i][0] >> 16)),
                               half_bits_to_float(static_cast<uint16_t>(d[i][1] & 0xffffu)),
                               half_bits_to_float(static_cast<uint16_t>(d[i][1] >> 16))};
#pragma unroll
          for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int j = 0; j < 4; ++j)
              acc[r][j] = fmaf(static_cast<float>(D[r][j]), dw[r] * sa[j], acc[r][j]);
          if constexpr (DOTS) {
            if (!valid) continue;
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

      // Fixed-order sum of the wavefronts' partials, then the epilogue. The
      // token range is reduced in passes of red_tokens tokens (16 or 8) to
      // bound LDS.
      for (int t0 = 0; t0 < 16; t0 += a.red_tokens) {
        if (4 * G >= t0 && 4 * G < t0 + a.red_tokens) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            float *dst = red + (static_cast<size_t>(wave) * a.red_tokens + (4 * G + j - t0)) * 64 + 4 * c;
#pragma unroll
            for (int r = 0; r < 4; ++r) dst[r] = acc[r][j];
          }
        }
        __syncthreads();
        for (int e = threadIdx.x; e < a.red_tokens * 64; e += blockDim.x) {
          const int t = e >> 6, r = e & 63;
          float s = red[static_cast<size_t>(t) * 64 + r];
          for (int w = 1; w < W; ++w) s += red[(static_cast<size_t>(w) * a.red_tokens + t) * 64 + r];
          const int tok = tt * 16 + t0 + t, row = g * kRowsPerGroup + r;
          if constexpr (!ARGMAX) {
            if (tok < a.tokens && row < a.rows && a.out != nullptr) {
              const size_t o = static_cast<size_t>(tok) * a.stride + row;
              a.out[o] = a.residual != nullptr ? a.residual[o] + s : s;
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
            if (lane == 0 && key > best[t0 + t]) best[t0 + t] = key;
          }
        }
        __syncthreads();
      }
    }
    if (ARGMAX) {
      __syncthreads();
      if (threadIdx.x < 16) {
        const int tok = tt * 16 + threadIdx.x;
        if (tok < a.tokens) a.cand[static_cast<size_t>(blockIdx.x) * a.cand_stride + tok] = best[threadIdx.x];
      }
    }
  }
}

// One wavefront per token: the best key over all workgroups' candidates.
__global__ __launch_bounds__(64) void argmax_finalize_kernel(const unsigned long long *cand, int ncand,
                                                             int cand_stride, int tokens, int32_t *index,
                                                             float *value) {
  const int tok = blockIdx.x, lane = threadIdx.x;
  if (tok >= tokens) return;
  unsigned long long key = 0ull;
  for (int i = lane; i < ncand; i += 64) {
    const unsigned long long k = cand[static_cast<size_t>(i) * cand_stride + tok];
    key = k > key ? k : key;
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const unsigned long long o = __shfl_xor(key, m, 64);
    key = o > key ? o : key;
  }
  if (lane == 0) {
    if (index != nullptr) index[tok] = static_cast<int32_t>(argmax_key_index(key));
    if (value != nullptr) value[tok] = argmax_key_value(key);
  }
}

struct GemmShape {
  int waves, grid, red_tokens;
  size_t smem;
};

GemmShape gemm_shape(const GemmArgs &a, int cu_count) {
  GemmShape s{};
  const int groups = (a.rows / 8 + 7) / 8;
  s.waves = a.exact ? 1 : std::min(kMaxWaves, std::max(1, (a.nb + kChunk - 1) / kChunk));
  const bool argmax = a.cand != nullptr;
  const int cus = cu_count > 0 ? cu_count : 256;
  s.grid = argmax ? std::min(groups, a.cand_capacity > 0 ? a.cand_capacity : 4 * cus) : groups;
  s.red_tokens = 16;
  auto bytes = [&](int red_tokens) {
    return (static_cast<size_t>(a.nb) * 16 + static_cast<size_t>(s.waves) * red_tokens * 64) * 4 + 16 * 8;
  };
  s.smem = bytes(16);
  if (s.smem > 65536) {
    s.red_tokens = 8;
    s.smem = bytes(8);
  }
  return s;
}

}  // namespace

int gemm_argmax_grid(int rows, int cu_count) {
  const int groups = (rows / 8 + 7) / 8;
  return std::min(groups, 4 * (cu_count > 0 ? cu_count : 256));
}

bool gemm_shape_supported(int rows, int nb, bool exact) {
  if (rows <= 0 || rows % 8 != 0 || nb <= 0) return false;
  GemmArgs a;
  a.rows = rows;
  a.nb = nb;
  a.exact = exact;
  return gemm_shape(a, 256).smem <= 65536;
}

hipError_t launch_gemm(const GemmArgs &a, hipStream_t stream) {
  if (a.tokens <= 0 || a.rows <= 0) return hipSuccess;
  const GemmShape s = gemm_shape(a, a.cu_count);
  if (s.smem > 65536) return hipErrorInvalidValue;
  GemmArgs b = a;
  b.red_tokens = s.red_tokens;
  if (a.cand != nullptr) {
    Q35_LAUNCH((gemm_kernel<true, false>), dim3(s.grid), dim3(64 * s.waves), s.smem, stream, b);
  } else if (a.block_dots != nullptr) {
    Q35_LAUNCH((gemm_kernel<false, true>), dim3(s.grid), dim3(64 * s.waves), s.smem, stream, b);
  } else {
    Q35_LAUNCH((gemm_kernel<false, false>), dim3(s.grid), dim3(64 * s.waves), s.smem, stream, b);
  }
  return hipGetLastError();
}

hipError_t launch_argmax_finalize(const unsigned long long *cand, int ncand, int cand_stride, int tokens,
                                  int32_t *index, float *value, hipStream_t stream) {
  Q35_LAUNCH((argmax_finalize_kernel), dim3(tokens), dim3(64), 0, stream, cand, ncand, cand_stride, tokens,
             index, value);
  return hipGetLastError();
}

}  // namespace q35
