// Q4-G32-DOT4 GEMV for one to four vectors in a single launch: the
// activation blocks are read in their Q8_0 X1 / X4 layout (no layout kernel),
// the int8 block dots run on the VALU dot4 unit, and each output row is the
// reference's single fma chain over the blocks in order, so the results are
// bit-exact (no split-K, no reduce kernel).
#include "q35_device.h"
#include "q35_internal.h"

namespace q35 {

namespace {
constexpr int kMvThreads = 256;
// blocks per chain pass: 4 wavefronts x 8 block lanes x 4 blocks per lane
constexpr int kMvPass = 128;

struct MvArgs {
  const uint8_t *w;    // Q4_0BlockX8 tiles [rows / 8][nb]
  const uint8_t *act;  // X1 blocks [count][nb] (40 B) or X4 blocks [nb] (152 B)
  int nb;
  int count;
  float *out;
  long long stride;  // output row stride (floats) between vectors
};

// One workgroup per 8-row tile group. Lane (r, j) of wavefront w owns row r
// of the group and blocks j + 8 (w + 4 i) of each 128-block pass: it loads the
// row's four body words (columns 8t..8t+7 of each word t) and the row's
// scale, and per vector forms
//   dot = sum_k (u_k - 8) a_k   (sdot4 of the nibbles against the codes,
//                               then -8 times the code sum, all in int32),
//   scale = half(d_r) * s_a      (q4_dot4.cpp:52-54),
// which land in LDS. The first 8 * count lanes then run the row chains
// result = fma(float(dot), scale, result) block by block
// (q4_dot4.cpp:43-56, restated by q35o_dot4_matvec).
template <int NV, bool X4>
__global__ __launch_bounds__(kMvThreads) void dot4_matvec_kernel(MvArgs a) {
  __shared__ q35_f32x2 fs[NV][8][kMvPass + 1];  // +1: the chain lanes' reads hit distinct banks
  const int g = blockIdx.x;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, r = lane & 7, j = lane >> 3;
  const uint8_t *tiles = a.w + static_cast<size_t>(g) * a.nb * 144;
  float res = 0.0F;
  for (int b0 = 0; b0 < a.nb; b0 += kMvPass) {
    const int n = min(kMvPass, a.nb - b0);
    // every load of the pass first (slots past the pass read its last block
    // and are not stored), then the dots
    uint32_t wq[4][4], c[4][NV][8];
    float dw[4], sa[4][NV];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int b = b0 + min(j + 8 * (wave + 4 * i), n - 1);
      const uint8_t *tile = tiles + static_cast<size_t>(b) * 144;
      const uint32_t *q = reinterpret_cast<const uint32_t *>(tile + 16 + 4 * r);
#pragma unroll
      for (int t = 0; t < 4; ++t) wq[i][t] = Q35_LOAD_NT(q + 8 * t);
      dw[i] = half_bits_to_float(reinterpret_cast<const uint16_t *>(tile)[r]);
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        if (X4) {
          // scales[4], sums[4], qs[4][32]: vector v's codes at byte 24 + 32 v
          const uint8_t *blk = a.act + static_cast<size_t>(b) * 152;
          sa[i][v] = reinterpret_cast<const float *>(blk)[v];
          const q35_u32x2 *cp = reinterpret_cast<const q35_u32x2 *>(blk + 24 + 32 * v);
#pragma unroll
          for (int m = 0; m < 4; ++m) {
            const q35_u32x2 x = cp[m];
            c[i][v][2 * m] = x[0];
            c[i][v][2 * m + 1] = x[1];
          }
        } else {
          // scale, sum, qs[32] from byte 6, pad: five aligned 8-byte words
          const q35_u32x2 *bp = reinterpret_cast<const q35_u32x2 *>(a.act + (static_cast<size_t>(v) * a.nb + b) * 40);
          uint32_t d[10];
#pragma unroll
          for (int m = 0; m < 5; ++m) {
            const q35_u32x2 x = bp[m];
            d[2 * m] = x[0];
            d[2 * m + 1] = x[1];
          }
          sa[i][v] = __uint_as_float(d[0]);
#pragma unroll
          for (int m = 0; m < 8; ++m) c[i][v][m] = (d[m + 1] >> 16) | (d[m + 2] << 16);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int bl = j + 8 * (wave + 4 * i);
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        int acc = 0;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          acc = Q35_SDOT4(wq[i][t] & 0x0f0f0f0fu, c[i][v][2 * t], acc);
          acc = Q35_SDOT4((wq[i][t] >> 4) & 0x0f0f0f0fu, c[i][v][2 * t + 1], acc);
        }
#pragma unroll
        for (int m = 0; m < 8; ++m) acc = Q35_SDOT4(0xF8F8F8F8u, c[i][v][m], acc);
        if (bl < n) fs[v][r][bl] = q35_f32x2{static_cast<float>(acc), dw[i] * sa[i][v]};
      }
    }
    lds_barrier();
    if (tid < 8 * NV) {
      const int rr = tid & 7, v = tid >> 3;
      for (int bl = 0; bl < n; ++bl) {
        const q35_f32x2 p = fs[v][rr][bl];
        res = fmaf(p[0], p[1], res);
      }
    }
    lds_barrier();
  }
  if (tid < 8 * a.count) a.out[(tid >> 3) * a.stride + g * 8 + (tid & 7)] = res;
}
}  // namespace

hipError_t launch_dot4_matvec(const q35_q4_0_block_x8 *w, const void *act, bool x4, int count, int rows, int nb,
                              float *out, long long stride, hipStream_t stream) {
  if (count < 1 || count > kMatvecMaxVectors || (x4 && count != 4) || rows <= 0 || rows % 8 != 0 || nb <= 0)
    return hipErrorInvalidValue;
  MvArgs a;
  a.w = reinterpret_cast<const uint8_t *>(w);
  a.act = static_cast<const uint8_t *>(act);
  a.nb = nb;
  a.count = count;
  a.out = out;
  a.stride = stride;
  const dim3 grid(rows / 8), block(kMvThreads);
  if (x4) {
    Q35_LAUNCH((dot4_matvec_kernel<4, true>), grid, block, 0, stream, a);
  } else {
    switch (count) {
      case 1: Q35_LAUNCH((dot4_matvec_kernel<1, false>), grid, block, 0, stream, a); break;
      case 2: Q35_LAUNCH((dot4_matvec_kernel<2, false>), grid, block, 0, stream, a); break;
      case 3: Q35_LAUNCH((dot4_matvec_kernel<3, false>), grid, block, 0, stream, a); break;
      default: Q35_LAUNCH((dot4_matvec_kernel<4, false>), grid, block, 0, stream, a); break;
    }
  }
  return hipGetLastError();
}

}  // namespace q35
