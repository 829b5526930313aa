// Q4-G32-DOT4 grouped GEMV/GEMM on CDNA4 int8 MFMA.
//
// Reads the reference's 144-byte Q4_0BlockX8 DOT4 tiles in place (no repack):
//   qs[32t+4r+j] = u[r][8t+j] | u[r][8t+4+j] << 4          (q4_dot4.h:5-6)
// A wavefront owns 64 output rows (eight 8-row tiles) and one 16-token tile.
// Lane l loads the 16-byte segment m = 2*(l/16) + (l%16)%2 of tile (l%16)/2:
// four 32-bit words = rows 4h..4h+3 of chunk t = l/16, i.e. eight consecutive
// columns each. Word i, unpacked to two int8x4 (low nibbles = columns 8t..8t+3,
// high nibbles = 8t+4..8t+7), is exactly the A operand of
// v_mfma_i32_16x16x32_i8 #i for virtual row l%16 and k-group l/16, so each
// 128-byte tile body is consumed by one coalesced 16-byte load per lane and
// the per-block int32 dot comes out of four MFMAs:
//   D_i[4G+v][tok] = sum_k u*a - 8*sum_a         (C operand = -8*sum_a)
// which is the reference's integer dot (q4_dot4_simd.inl:66-89). Output lane
// (G, tok) holds rows 16G + 4v + i, so the FP32 epilogue
//   acc = fma(float(dot), half(d_row) * s_tok, acc)   (q4_dot4.cpp:53)
// runs per row and token in block order. Waves of a workgroup split the block
// range; the workgroup sums its waves in fixed order, and split-K workgroups
// are summed in split order by the last one to finish, so results are
// deterministic run to run.
#include "q35_device.h"
#include "q35_internal.h"

namespace q35 {
namespace {

typedef Q35_V4I v4i;

constexpr int kGemmThreads = 256;
constexpr int kRowsPerGroup = 64;
constexpr int kRedStride = 68;  // 64 rows + pad (LDS bank spread)

__device__ __forceinline__ long unpack_word(uint32_t w) {
  const uint32_t lo = w & 0x0f0f0f0fu;
  const uint32_t hi = (w >> 4) & 0x0f0f0f0fu;
  return static_cast<long>((static_cast<uint64_t>(hi) << 32) | lo);
}

template <int TT>
__global__ __launch_bounds__(kGemmThreads) void gemm_kernel(GemmArgs a) {
  __shared__ float red[4][16][kRedStride];
  __shared__ unsigned long long best[4][16];
  __shared__ int last_flag;

  const int rg = blockIdx.x, split = blockIdx.y, tg = blockIdx.z;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int c = lane & 15, G = lane >> 4, T = c >> 1, h = c & 1;
  const int ntiles = a.rows >> 3, nb = a.nb;
  const int rt = rg * 8 + T;
  const bool row_ok = rt < ntiles;
  const int ht0 = rg * 8 + 2 * G;
  const bool h0_ok = ht0 < ntiles, h1_ok = ht0 + 1 < ntiles;

  const int S = a.ksplit;
  const int kb0 = (split * nb) / S, kb1 = ((split + 1) * nb) / S;
  // exact mode: one wave runs the whole block range, so each output is the
  // reference's single fma chain over blocks (bit-exact FP32)
  const int per_wave = a.exact ? (kb1 - kb0) : ((kb1 - kb0 + 3) >> 2);
  const int wb0 = a.exact ? (wave == 0 ? kb0 : kb1) : kb0 + wave * per_wave;
  const int wb1 = a.exact ? (wave == 0 ? kb1 : kb1) : min(kb1, wb0 + per_wave);

  const uint8_t *W = reinterpret_cast<const uint8_t *>(a.w);
  const uint8_t *wrow = W + (static_cast<size_t>(rt) * nb) * 144 + 16 + 16 * (2 * G + h);
  const uint8_t *hrow0 = W + (static_cast<size_t>(ht0) * nb) * 144;
  const uint8_t *hrow1 = hrow0 + static_cast<size_t>(nb) * 144;

  float acc[TT][16];
#pragma unroll
  for (int tt = 0; tt < TT; ++tt)
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[tt][j] = 0.0F;

  for (int b = wb0; b < wb1; ++b) {
    uint4 q = make_uint4(0, 0, 0, 0), d0 = make_uint4(0, 0, 0, 0), d1 = make_uint4(0, 0, 0, 0);
    if (row_ok) q = *reinterpret_cast<const uint4 *>(wrow + static_cast<size_t>(b) * 144);
    if (h0_ok) d0 = *reinterpret_cast<const uint4 *>(hrow0 + static_cast<size_t>(b) * 144);
    if (h1_ok) d1 = *reinterpret_cast<const uint4 *>(hrow1 + static_cast<size_t>(b) * 144);
    const long A0 = unpack_word(q.x), A1 = unpack_word(q.y), A2 = unpack_word(q.z),
               A3 = unpack_word(q.w);
    float ds[16];
    {
      const uint32_t hw[8] = {d0.x, d0.y, d0.z, d0.w, d1.x, d1.y, d1.z, d1.w};
#pragma unroll
      for (int j = 0; j < 16; ++j)
        ds[j] = half_bits_to_float(static_cast<uint16_t>(hw[j >> 1] >> (16 * (j & 1))));
    }
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) {
      const size_t ablk = (static_cast<size_t>(tg * TT + tt) * nb + b);
      const long B = static_cast<long>(a.codes[ablk * 64 + lane]);
      const ActParam p = a.params[ablk * 16 + c];
      const v4i C = {p.corr, p.corr, p.corr, p.corr};
      const v4i D0 = Q35_MFMA_I32_16X16X32_I8(A0, B, C, 0, 0, 0);
      const v4i D1 = Q35_MFMA_I32_16X16X32_I8(A1, B, C, 0, 0, 0);
      const v4i D2 = Q35_MFMA_I32_16X16X32_I8(A2, B, C, 0, 0, 0);
      const v4i D3 = Q35_MFMA_I32_16X16X32_I8(A3, B, C, 0, 0, 0);
      const v4i D[4] = {D0, D1, D2, D3};
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int j = 4 * v + i;
          acc[tt][j] = fmaf(static_cast<float>(D[i][v]), ds[j] * p.scale, acc[tt][j]);
        }
      if (a.block_dots != nullptr) {
        const int tok = (tg * TT + tt) * 16 + c;
        if (tok < a.tokens) {
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
              const int row = rg * kRowsPerGroup + 16 * G + 4 * v + i;
              if (row < a.rows)
                a.block_dots[(static_cast<size_t>(tok) * a.rows + row) * nb + b] = D[i][v];
            }
        }
      }
    }
  }

  // Workgroup reduction (waves in fixed order), then store / split-K / argmax.
#pragma unroll
  for (int tt = 0; tt < TT; ++tt) {
#pragma unroll
    for (int j = 0; j < 16; ++j) red[wave][c][16 * G + j] = acc[tt][j];
    __syncthreads();
    const int tok0 = (tg * TT + tt) * 16;
    float sums[4];
    int rows_[4], toks_[4];
#pragma unroll
    for (int e4 = 0; e4 < 4; ++e4) {
      const int e = threadIdx.x + e4 * kGemmThreads;
      const int tk = e >> 6, row = e & 63;
      sums[e4] = ((red[0][tk][row] + red[1][tk][row]) + red[2][tk][row]) + red[3][tk][row];
      rows_[e4] = rg * kRowsPerGroup + row;
      toks_[e4] = tok0 + tk;
    }
    __syncthreads();
    if (a.argmax_keys != nullptr) {
      // Greedy head: penalty then per-token max key over this group's rows.
#pragma unroll
      for (int e4 = 0; e4 < 4; ++e4) {
        const int tk = toks_[e4], row = rows_[e4];
        unsigned long long key = 0ull;
        if (tk < a.tokens && row < a.rows) {
          float val = sums[e4];
          const float pen = a.penalties != nullptr ? a.penalties[tk] : 1.0F;
          if (pen > 1.0F && a.counts != nullptr) {
            const long long crow = a.count_rows != nullptr ? a.count_rows[tk] : tk;
            if (a.counts[crow * a.counts_stride + row] > 0) val = val > 0.0F ? val / pen : val * pen;
          }
          key = argmax_key(val, static_cast<uint32_t>(row));
        }
        // threads of one wave share the token (e>>6 is wave-uniform per e4)
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) {
          const unsigned long long o = __shfl_xor(key, m, 64);
          key = o > key ? o : key;
        }
        if (lane == 0 && key != 0ull && tk < a.tokens) atomicMax(&a.argmax_keys[tk], key);
      }
      continue;
    }
    if (S == 1) {
      // the block-dots parity entry runs without an FP32 output buffer
      if (a.out == nullptr) continue;
#pragma unroll
      for (int e4 = 0; e4 < 4; ++e4) {
        const int tk = toks_[e4], row = rows_[e4];
        if (tk < a.tokens && row < a.rows) {
          const size_t o = static_cast<size_t>(tk) * a.stride + row;
          float val = sums[e4];
          if (a.residual != nullptr) val = a.residual[o] + val;
          a.out[o] = val;
        }
      }
    } else {
#pragma unroll
      for (int e4 = 0; e4 < 4; ++e4) {
        const int tk = toks_[e4], row = rows_[e4];
        if (tk < a.tokens && row < a.rows)
          a.partials[(static_cast<size_t>(split) * a.tokens + tk) * a.rows + row] = sums[e4];
      }
    }
  }
  (void)best;
  if (a.argmax_keys != nullptr || S == 1) return;

  // Split-K: the last workgroup of this (row group, token group) sums all
  // splits in split order.
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned idx = static_cast<unsigned>(tg) * gridDim.x + rg;
    const unsigned prev = atomicAdd(&a.counters[idx], 1u);
    last_flag = (prev == static_cast<unsigned>(S - 1));
    if (last_flag) a.counters[idx] = 0u;
  }
  __syncthreads();
  if (!last_flag) return;
  __threadfence();
  const int tok_begin = tg * TT * 16;
  const int tok_end = min(a.tokens, tok_begin + TT * 16);
  const int row_begin = rg * kRowsPerGroup;
  const int row_end = min(a.rows, row_begin + kRowsPerGroup);
  const int nrow = row_end - row_begin;
  for (int e = threadIdx.x; e < (tok_end - tok_begin) * kRowsPerGroup; e += kGemmThreads) {
    const int tk = tok_begin + e / kRowsPerGroup, row = row_begin + e % kRowsPerGroup;
    if (e % kRowsPerGroup >= nrow) continue;
    float val = 0.0F;
    for (int s = 0; s < S; ++s) {
      val += a.partials[(static_cast<size_t>(s) * a.tokens + tk) * a.rows + row];
    }
    const size_t o = static_cast<size_t>(tk) * a.stride + row;
    if (a.residual != nullptr) val = a.residual[o] + val;
    a.out[o] = val;
  }
}

__global__ void argmax_unpack_kernel(const unsigned long long *keys, int count, int32_t *index,
                                     float *value) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= count) return;
  const unsigned long long k = keys[i];
  if (index != nullptr) index[i] = static_cast<int32_t>(argmax_key_index(k));
  if (value != nullptr) value[i] = argmax_key_value(k);
}

}  // namespace

int gemm_choose_ksplit(int rows, int nb, int cu_count) {
  const int groups = (rows + kRowsPerGroup - 1) / kRowsPerGroup;
  const int target = cu_count > 0 ? cu_count : 256;
  int s = 1;
  // grow the split while the grid underfills the chip and every wave keeps
  // at least two blocks
  while (groups * s < target && nb / (s * 2) >= 8) s *= 2;
  return s;
}

size_t gemm_partial_floats(int rows, int tokens, int ksplit) {
  return ksplit > 1 ? static_cast<size_t>(ksplit) * tokens * rows : 0;
}

size_t gemm_counter_count(int rows, int tokens) {
  const int groups = (rows + kRowsPerGroup - 1) / kRowsPerGroup;
  const int tgroups = (tokens + 63) / 64 * 4;
  return static_cast<size_t>(groups) * tgroups;
}

hipError_t launch_gemm(const GemmArgs &a, hipStream_t stream) {
  if (a.tokens <= 0 || a.rows <= 0) return hipSuccess;
  const int tiles = (a.tokens + 15) / 16;
  const int groups = (a.rows + kRowsPerGroup - 1) / kRowsPerGroup;
  int TT = tiles >= 4 ? 4 : (tiles >= 2 ? 2 : 1);
  if (TT == 2 && tiles == 3) TT = 4;
  const dim3 block(kGemmThreads);
  const dim3 grid(groups, a.ksplit, (tiles + TT - 1) / TT);
  switch (TT) {
    case 1: Q35_LAUNCH((gemm_kernel<1>), grid, block, 0, stream, a); break;
    case 2: Q35_LAUNCH((gemm_kernel<2>), grid, block, 0, stream, a); break;
    default: Q35_LAUNCH((gemm_kernel<4>), grid, block, 0, stream, a); break;
  }
  return hipGetLastError();
}

hipError_t launch_argmax_unpack(const unsigned long long *keys, int count, int32_t *index,
                                float *value, hipStream_t stream) {
  Q35_LAUNCH((argmax_unpack_kernel), (count + 255) / 256, 256, 0, stream, keys, count, index, value);
  return hipGetLastError();
}

}  // namespace q35
