// Activation preparation for the Q4-G32-DOT4 projections: the producer
// (plain rows, SiLU(gate) * up over split GEMM partials, or residual update +
// RMSNorm) followed by the randomized-sign Hadamard-128 rotation and per-32
// int8 quantization (h128_quantize_lanes).
//
// Reference semantics (bit-exact given the same FP32 input):
//   signs + FWHT stage order 1,2,...,64     src/cpu/q4_h128.cpp:35-61
//   absmax/127, unrounded 1/scale, round half away from zero, clamp +-127,
//   stored scale = binary16(scale) * 1/sqrt(128)   q4_0.cpp:212-235, q4_h128.cpp:319-321
// prep_kernel: 32 lanes per (token, 128-column block), two blocks per
// one-wavefront workgroup. rms_prep_kernel: one workgroup per token (the row's
// sum of squares is shared through LDS), 32 lanes per block (16 with the Q8
// gate tail).
#include "q35_quant.h"

namespace q35 {
namespace {

constexpr int kPrepThreads = 256;

// Four consecutive source values of token t from column c0 (c0 % 4 == 0);
// the split partial rows are summed per column in split order.
template <int SRC, int MS>
__device__ __forceinline__ void load_source4(const PrepArgs &a, int t, int c0, float v[4]) {
  if constexpr (SRC == kPrepPlain) {
    const q35_f32x4 x = *reinterpret_cast<const q35_f32x4 *>(a.x + static_cast<size_t>(t) * a.x_stride + c0);
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = x[e];
  } else {
    const SplitRows &s = a.gate_up;
    const float *q = s.p + static_cast<long long>(t) * s.width + c0;
    q35_f32x4 g[MS], u[MS];
#pragma unroll
    for (int i = 0; i < MS; ++i) {
      const long long off = static_cast<long long>(min(i, s.splits - 1)) * s.split_stride;
      g[i] = *reinterpret_cast<const q35_f32x4 *>(q + off);
      u[i] = *reinterpret_cast<const q35_f32x4 *>(q + off + a.K);
    }
    q35_f32x4 gs = g[0], us = u[0];
#pragma unroll
    for (int i = 1; i < MS; ++i) {
      gs = i < s.splits ? gs + g[i] : gs;
      us = i < s.splits ? us + u[i] : us;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = silu_times(gs[e], us[e]);
  }
}

// kPrepLanes (32) lanes per (token, 128-column block) item, two items per
// wavefront; MS bounds the source's K splits.
constexpr int kPrepLanes = 32;
template <int SRC, int MS>
__global__ __launch_bounds__(kPrepThreads) void prep_kernel(PrepArgs a) {
  constexpr int V = 128 / kPrepLanes;
  const int K = a.K, nb = K >> 5, nblk = K >> 7;
  const int items = a.tokens * nblk;
  const int item0 = static_cast<int>((blockIdx.x * blockDim.x + threadIdx.x) / kPrepLanes);
  const bool active = item0 < items;
  const int item = active ? item0 : items - 1;  // idle rows redo a valid item and store nothing
  const int t = item / nblk, blk = item - t * nblk;
  float v[V];
  const int c0 = blk * 128 + V * (threadIdx.x & (kPrepLanes - 1));
  load_source4<SRC, MS>(a, t, c0, v);
  if (a.y_out != nullptr && active)
#pragma unroll
    for (int e = 0; e < V; ++e) a.y_out[static_cast<size_t>(t) * K + c0 + e] = v[e];
  QuantOut o;
  o.codes = a.codes;
  o.scales = a.scales;
  o.x4 = a.x4;
  o.x1 = a.x1;
  h128_quantize_lanes<kPrepLanes>(v, t, blk, nb, a.h128, a.seed, o, active);
}

// Residual update + RMSNorm + preparation, one workgroup (256 threads) per
// token. Thread i owns the float4 columns 4i + 1024k; the residual and the
// split partial rows of a column batch are loaded before the ordered sum.
constexpr int kRmsThreads = 256;
constexpr int kRmsMaxK = 4096;

// GATES: the Q8 gate rows of the in projection are computed here as well
// (run_q8_gate_tail, weights.inl:1015-1034): the normalized row's
// identity-basis codes go to LDS, each thread takes whole (row, block) int8
// dots, and one thread per gate row runs the block chain
// acc = fma(float(dot), mscale * vscale, acc) in block order.
// EMBED: the rows are gathered from the embedding (MS == 0).
template <int MS, bool GATES, bool EMBED>  // MS: bound on the added rows' K splits (0: nothing to add)
__global__ __launch_bounds__(kRmsThreads) void rms_prep_kernel(RmsPrepArgs a) {
  static_assert(!EMBED || MS == 0, "the embedding gather adds no rows");
  __shared__ float y[kRmsMaxK];
  __shared__ float gsq[kRmsMaxK / 16];  // sums of squares per 16-column group
  __shared__ float total_sq;
  __shared__ __align__(16) int8_t gq[GATES ? kRmsMaxK : 8];
  __shared__ float gsc[GATES ? kRmsMaxK / 32 : 1];
  __shared__ float gdot[GATES ? kMaxGateItems : 1];
  __shared__ float gmul[GATES ? kMaxGateItems : 1];
  // L lanes per 128-column item (V columns each): 32, or 16 with the gate
  // tail, whose identity-basis codes take eight columns per lane
  constexpr int L = GATES ? 16 : 32, V = 128 / L, kItemsPerPass = kRmsThreads / L;
  const int t = blockIdx.x, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int K = a.K, n4 = K >> 2;
  const int nblk = K >> 7, j = tid & (L - 1);
  // (1 + w) of this thread's first quantization item, loaded together with
  // the row so that no load waits behind the barrier
  float w1[V];
  {
    const int blk = min(tid / L, nblk - 1);
    const q35_f32x4 *wp = reinterpret_cast<const q35_f32x4 *>(a.weight + blk * 128 + V * j);
#pragma unroll
    for (int h = 0; h < V / 4; ++h) {
      const q35_f32x4 x = wp[h];
#pragma unroll
      for (int e = 0; e < 4; ++e) w1[4 * h + e] = x[e] + 1.0F;
    }
  }
  // the residual row of output row t (a gathered row set: the head rows)
  const size_t xr = a.rows != nullptr ? static_cast<size_t>(a.rows[t]) : static_cast<size_t>(t);
  const q35_f32x4 *xin = reinterpret_cast<const q35_f32x4 *>(a.x_in + xr * K);
  int token = 0;
  if constexpr (EMBED) token = a.token_ids[t];
  // columns 4i..4i+3 of the row (i = tid + kRmsThreads * it): the input
  // (the residual row, or the token's embedding run) and the split rows to add
  auto load = [&](int i, q35_f32x4 &v, q35_f32x4 x[MS > 0 ? MS : 1]) {
    if constexpr (EMBED) {
      // one 4-byte run of the tile's DOT4 codes (the same nibble half) and
      // the row's binary16 scale, x = half(d) * (u - 8) as embed_kernel forms it
      const int k = 4 * i, b = k >> 5, kk = k & 31, rt = token >> 3, row = token & 7;
      const uint8_t *tile;
      uint16_t dh;
      if (a.embed_g16) {
        tile = reinterpret_cast<const uint8_t *>(a.embed) + (static_cast<size_t>(rt) * (K >> 5) + b) * 160;
        dh = *reinterpret_cast<const uint16_t *>(tile + 2 * (8 * (kk >> 4) + row));
        tile += 32;
      } else {
        tile = reinterpret_cast<const uint8_t *>(a.embed) + (static_cast<size_t>(rt) * (K >> 5) + b) * 144;
        dh = *reinterpret_cast<const uint16_t *>(tile + 2 * row);
        tile += 16;
      }
      const uint32_t q4 = *reinterpret_cast<const uint32_t *>(tile + 32 * (kk >> 3) + 4 * row);
      const int sh = 4 * ((kk & 7) >> 2);
      const float d = half_bits_to_float(dh);
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = d * static_cast<float>(static_cast<int>((q4 >> (8 * e + sh)) & 15u) - 8);
    } else {
      v = xin[i];
    }
    if constexpr (MS > 0) {
      // every split, all loads in flight together
      const float *pp = a.add.p + xr * a.add.width + 4 * i;
#pragma unroll
      for (int u = 0; u < MS; ++u)
        x[u] = *reinterpret_cast<const q35_f32x4 *>(pp + static_cast<long long>(min(u, a.add.splits - 1)) *
                                                             a.add.split_stride);
    }
  };
  auto use = [&](int i, q35_f32x4 v, const q35_f32x4 x[MS > 0 ? MS : 1]) {
    if constexpr (MS > 0) {
      q35_f32x4 sum = x[0];
#pragma unroll
      for (int u = 1; u < MS; ++u)
        if (u < a.add.splits) sum += x[u];
      v += sum;
    }
    if constexpr (EMBED || MS > 0) reinterpret_cast<q35_f32x4 *>(a.x_out + xr * K)[i] = v;
    *reinterpret_cast<q35_f32x4 *>(&y[4 * i]) = v;
    // K % 128 == 0: the four lanes of a group run the same iterations
    const float gs = sq_group16_quad(v);
    if ((tid & 3) == 0) gsq[i >> 2] = gs;
  };
  if constexpr (MS <= 4) {
    // every iteration's loads first (rows up to kRmsMaxK wide), then the sums:
    // one round trip for the whole row
    constexpr int kIters = kRmsMaxK / 4 / kRmsThreads;
    q35_f32x4 v[kIters], x[kIters][MS > 0 ? MS : 1];
#pragma unroll
    for (int it = 0; it < kIters; ++it) {
      if (it * kRmsThreads >= n4) break;  // uniform
      load(min(tid + it * kRmsThreads, n4 - 1), v[it], x[it]);
    }
#pragma unroll
    for (int it = 0; it < kIters; ++it) {
      const int i = tid + it * kRmsThreads;
      if (it * kRmsThreads >= n4) break;  // uniform
      // past the row: whole runs of 32 threads (n4 is a multiple of 32), so
      // the four lanes of a group agree
      if (i < n4) use(i, v[it], x[it]);
    }
  } else {
    for (int i = tid; i < n4; i += kRmsThreads) {
      q35_f32x4 v, x[MS > 0 ? MS : 1];
      load(i, v, x);
      use(i, v, x);
    }
  }
  if constexpr (EMBED) {
    if (tid == 0 && a.counts != nullptr && a.count_input != nullptr && a.count_input[t])
      a.counts[static_cast<long long>(a.slots[t]) * a.counts_stride + token] += 1;
  }
  // only LDS is shared: the x_out stores stay in flight
  lds_barrier();
  if (wave == 0) {
    const float t = norm_total_groups(gsq, K >> 4);
    if (lane == 0) total_sq = t;
  }
  lds_barrier();
  const float total = total_sq;
  const float rms_inv = 1.0F / sqrtf(total / static_cast<float>(K) + a.eps);
  QuantOut o;
  o.codes = a.codes;
  o.scales = a.scales;
  for (int blk0 = 0; blk0 < nblk; blk0 += kItemsPerPass) {
    if (blk0 + wave * (64 / L) >= nblk) break;  // wave-uniform: all of its items idle
    const int want = blk0 + tid / L;
    const bool active = want < nblk;
    const int blk = active ? want : nblk - 1;
    const int c0 = blk * 128 + V * j;
    if (blk0 > 0) {  // wider rows: a further item per thread
#pragma unroll
      for (int e = 0; e < V; ++e) w1[e] = a.weight[c0 + e] + 1.0F;
    }
    float v[V];
#pragma unroll
    for (int e = 0; e < V; ++e) v[e] = y[c0 + e] * rms_inv * w1[e];
    if (a.normed_out != nullptr && active)
#pragma unroll
      for (int e = 0; e < V; ++e) a.normed_out[static_cast<size_t>(t) * K + c0 + e] = v[e];
    if constexpr (GATES) {
      uint64_t word;
      int sum;
      float stored;
      q8_block_codes8(v, word, sum, stored);
      if (active) {
        *reinterpret_cast<uint64_t *>(&gq[c0]) = word;
        if ((j & 3) == 0) gsc[c0 >> 5] = stored;
      }
    }
    h128_quantize_lanes<L>(v, t, blk, K >> 5, a.h128, a.seed, o, active);
  }
  if constexpr (GATES) {
    __syncthreads();
    const int nb = K >> 5, items = a.gate_rows * nb;
    for (int i = tid; i < items; i += kRmsThreads) {
      const int r = i / nb, b = i - r * nb;
      const q35_u32x4 *wp = reinterpret_cast<const q35_u32x4 *>(a.gate_codes + static_cast<size_t>(r) * K + 32 * b);
      const q35_u32x4 wa = wp[0], wb = wp[1];
      const uint32_t *cp = reinterpret_cast<const uint32_t *>(&gq[32 * b]);
      int dot = 0;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const uint32_t wu = u < 4 ? wa[u] : wb[u - 4], cu = cp[u];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          dot += static_cast<int>(static_cast<int8_t>(wu >> (8 * e))) * static_cast<int>(static_cast<int8_t>(cu >> (8 * e)));
      }
      gdot[i] = static_cast<float>(dot);
      gmul[i] = a.gate_scales[i] * gsc[b];  // mscale * vscale, [row][block] as the scales are stored
    }
    __syncthreads();
    // the serial chains read LDS only
    for (int r = tid; r < a.gate_rows; r += kRmsThreads) {
      float acc = 0.0F;
#pragma unroll 8
      for (int b = 0; b < nb; ++b) acc = fmaf(gdot[r * nb + b], gmul[r * nb + b], acc);
      a.gates[static_cast<size_t>(t) * a.gate_rows + r] = acc;
    }
  }
}

// X4 (reference prefill layout) -> A16.
__global__ void x4_to_a16_kernel(const q35_q8_0_block_x4 *x4, int tokens, int nb, uint64_t *codes,
                                 float *scales) {
  const int b = blockIdx.x, tile = blockIdx.y, lane = threadIdx.x;
  const int tok = tile * 16 + (lane & 15), g = lane >> 4;
  uint64_t word = 0;
  float p = 0.0F;
  if (tok < tokens) {
    const q35_q8_0_block_x4 &src = x4[static_cast<size_t>(tok >> 2) * nb + b];
    const uint8_t *q = reinterpret_cast<const uint8_t *>(src.qs) + (tok & 3) * 32 + g * 8;
    for (int i = 0; i < 8; ++i) word |= static_cast<uint64_t>(q[i]) << (8 * i);
    p = src.scales[tok & 3];
  }
  codes[(static_cast<size_t>(tile) * nb + b) * 64 + lane] = word;
  if (g == 0) scales[(static_cast<size_t>(tile) * nb + b) * 16 + (lane & 15)] = p;
}

// X1 rows [token][nb] (independently prepared vectors) -> A16.
__global__ void x1_to_a16_kernel(const q35_q8_0_block_x1 *x1, int tokens, int nb, uint64_t *codes,
                                 float *scales) {
  const int b = blockIdx.x, tile = blockIdx.y, lane = threadIdx.x;
  const int tok = tile * 16 + (lane & 15), g = lane >> 4;
  uint64_t word = 0;
  float p = 0.0F;
  if (tok < tokens) {
    const q35_q8_0_block_x1 &src = x1[static_cast<size_t>(tok) * nb + b];
    const uint8_t *q = reinterpret_cast<const uint8_t *>(src.qs) + g * 8;
    for (int i = 0; i < 8; ++i) word |= static_cast<uint64_t>(q[i]) << (8 * i);
    p = src.scales[0];
  }
  codes[(static_cast<size_t>(tile) * nb + b) * 64 + lane] = word;
  if (g == 0) scales[(static_cast<size_t>(tile) * nb + b) * 16 + (lane & 15)] = p;
}

}  // namespace

hipError_t launch_prep(const PrepArgs &a, hipStream_t stream) {
  if (a.tokens <= 0) return hipSuccess;
  // one wavefront (two items) per workgroup: the split partials a SiLU
  // preparation reads spread over many compute units (one unit keeps only a
  // few tens of KiB in flight), and each lane's rotation chain is short
  constexpr int kThreads = 64, kItems = kThreads / kPrepLanes;
  const int items = a.tokens * (a.K >> 7);
  const dim3 grid((items + kItems - 1) / kItems), block(kThreads);
  if (a.source == kPrepSiluMul) {
    switch (split_bound(a.gate_up.splits)) {
      case 1: Q35_LAUNCH((prep_kernel<kPrepSiluMul, 1>), grid, block, 0, stream, a); break;
      case 4: Q35_LAUNCH((prep_kernel<kPrepSiluMul, 4>), grid, block, 0, stream, a); break;
      case 8: Q35_LAUNCH((prep_kernel<kPrepSiluMul, 8>), grid, block, 0, stream, a); break;
      default: return hipErrorInvalidValue;
    }
  } else {
    Q35_LAUNCH((prep_kernel<kPrepPlain, 1>), grid, block, 0, stream, a);
  }
  return hipGetLastError();
}

hipError_t launch_rms_prep(const RmsPrepArgs &a, hipStream_t stream) {
  if (a.tokens <= 0) return hipSuccess;
  if (a.K % 128 != 0 || a.K > kRmsMaxK || (a.add.p != nullptr && a.x_out == nullptr)) return hipErrorInvalidValue;
  const bool gates = a.gate_rows > 0;
  if (gates && (a.gate_rows > kMaxGateRows || a.gate_rows * (a.K / 32) > kMaxGateItems || a.gate_codes == nullptr ||
                a.gate_scales == nullptr || a.gates == nullptr))
    return hipErrorInvalidValue;
  const dim3 grid(a.tokens), block(kRmsThreads);
  if (a.embed != nullptr) {
    if (a.add.p != nullptr || a.x_out == nullptr || a.token_ids == nullptr) return hipErrorInvalidValue;
    if (gates)
      Q35_LAUNCH((rms_prep_kernel<0, true, true>), grid, block, 0, stream, a);
    else
      Q35_LAUNCH((rms_prep_kernel<0, false, true>), grid, block, 0, stream, a);
    return hipGetLastError();
  }
#define Q35_RMS(MS)                                                                     \
  if (gates) {                                                                          \
    Q35_LAUNCH((rms_prep_kernel<MS, true, false>), grid, block, 0, stream, a);          \
  } else {                                                                              \
    Q35_LAUNCH((rms_prep_kernel<MS, false, false>), grid, block, 0, stream, a);         \
  }
  switch (a.add.p == nullptr ? 0 : split_bound(a.add.splits)) {
    case 0: Q35_RMS(0) break;
    case 1: Q35_RMS(1) break;
    case 4: Q35_RMS(4) break;
    case 8: Q35_RMS(8) break;
    case 16: Q35_RMS(16) break;
    case 32: Q35_RMS(32) break;
    default: return hipErrorInvalidValue;
  }
#undef Q35_RMS
  return hipGetLastError();
}

hipError_t launch_x4_to_a16(const q35_q8_0_block_x4 *x4, int tokens, int nb, uint64_t *codes,
                            float *scales, hipStream_t stream) {
  const dim3 grid(nb, (tokens + 15) / 16);
  Q35_LAUNCH((x4_to_a16_kernel), grid, 64, 0, stream, x4, tokens, nb, codes, scales);
  return hipGetLastError();
}

hipError_t launch_x1_to_a16(const q35_q8_0_block_x1 *x1, int tokens, int nb, uint64_t *codes,
                            float *scales, hipStream_t stream) {
  Q35_LAUNCH((x1_to_a16_kernel), dim3(nb, (tokens + 15) / 16), 64, 0, stream, x1, tokens, nb, codes, scales);
  return hipGetLastError();
}

}  // namespace q35
