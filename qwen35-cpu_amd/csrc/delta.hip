// GatedDeltaNet decode update on CDNA4.
//
// One workgroup (256 or 512 threads) per (value head, request). The head's fp32
// state tile [value_row][key_col] = 128 x 128 (64 KiB) makes exactly one HBM
// round trip; its loads are issued right after the head's few small inputs
// (conv ring, projections, weights), so the 64 KiB are in flight while those
// are combined.
// Sixteen lanes share a value row: lane o = t % 16 owns the two float4 at
// columns 4o + 64m (m = 0, 1), and thread t owns rows t/16 + (threads/16) j.
// A row's dot products are summed per lane in column order and then across
// its 16 lanes with a four-step DPP butterfly (row_sum16) -- delta_row below,
// shared with the prefill chunk scan so both give the same bits -- and one
// load instruction covers 4 rows x 256 contiguous bytes per wavefront.
//
// Per value row (src/cpu/delta_net.cpp:63-98), in the reference's order:
//   S *= alpha;  sk = S.k;  delta = (v - sk) * beta;  S += delta * k;  o = S.q
// The fused variant also runs the rest of run_linear_attention_step
// (src/runtime/layers.inl:96-207) for its head: causal conv1d + SiLU over the
// q/k/v channels (activation.cpp:164-222), L2 normalisation of q
// (x 1/sqrt(d_k)) and k, beta = sigmoid(b), alpha = exp(softplus(a + dt_bias)
// * -exp(A_log)), and the gated RMSNorm (offset 0) times SiLU(z) -- and then
// prepares the head's 128 outputs, which are exactly H128 block `head` of the
// out projection's input, as int8 A16 activations for the DOT4 GEMM. GQA
// (v_heads > k_heads) maps value head vh to key head vh / (v_heads / k_heads),
// as the reference repeats q/k (layers.inl:130-144).
//
// The conv history is a ring of 4 (= conv kernel) slots indexed by
// position % 4 (slot p % 4 receives the input of position p; positions
// p-3 .. p-1 are read), so no workgroup ever reads a slot another one writes
// in the same step.
#include "q35_quant.h"

namespace q35 {
namespace {

constexpr int kDeltaThreads = 256;
constexpr int kDim = 128;
constexpr int kConvKernel = 4;  // linear_conv_kernel_dim of every Qwen3.5 size
constexpr int kRowLanes = 16;                                    // lanes per value row
// decode: THREADS (256 or 512) per (value head, request), kDim * 16 /
// THREADS value rows per thread (rows rowg + THREADS/16 * j). 512 threads
// let two wavefronts per SIMD overlap the row updates when the grid leaves
// most of the GPU idle (256 workgroups at 16 requests); with many
// workgroups (64 requests of the 4B shape: 2048) 256 threads keep more
// (head, request) tiles resident per compute unit and measure faster.

// The delta rule on one value row held by 16 lanes (this lane: columns
// 4o + 64m, m = 0, 1), in the reference's order (delta_net.cpp:63-98):
//   S *= alpha;  sk = S.k;  delta = (v - sk) * beta;  S += delta * k;  o = S.q
// Each dot product is summed over the lane's 8 columns in order, then over
// the row's 16 lanes (row_sum16). Every lane of the row returns o.
__device__ __forceinline__ float delta_row(q35_f32x4 st[2], const q35_f32x4 kc[2], const q35_f32x4 qc[2], float v,
                                           float alpha, float beta) {
  float d = 0.0F;
#pragma unroll
  for (int m = 0; m < 2; ++m) {
    st[m] *= alpha;
#pragma unroll
    for (int e = 0; e < 4; ++e) d += st[m][e] * kc[m][e];
  }
  d = row_sum16(d);
  const float delta = (v - d) * beta;
  float o = 0.0F;
#pragma unroll
  for (int m = 0; m < 2; ++m)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      st[m][e] += delta * kc[m][e];
      o += st[m][e] * qc[m][e];
    }
  o = row_sum16(o);
  return o;
}

// FUSED: the linear-attention step around the update; MS: compile-time bound
// on the in-projection's K splits (so every input load is straight-line).
template <bool FUSED, int MS, int THREADS>
__global__ __launch_bounds__(THREADS) void delta_kernel(DeltaArgs a) {
  constexpr int kDecodeRowStride = THREADS / kRowLanes;
  constexpr int kDecodeRows = kDim / kDecodeRowStride;
  __shared__ float sq[kDim], sk[kDim], sv[kDim], so[kDim];
  __shared__ float red[8];
  __shared__ float s_alpha, s_beta;
  const int vh = blockIdx.x;
  const int r = a.row_list != nullptr ? a.row_list[blockIdx.y] : static_cast<int>(blockIdx.y);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int per = a.v_heads / a.k_heads;
  const int kh = vh / per;
  const int col = tid & (kRowLanes - 1), rowg = tid >> 4;  // rows rowg + (THREADS / 16) j
  // the input phase runs on 256 threads' worth of channels; with 512
  // threads, threads 256..511 repeat threads 0..255 (the same loads and the
  // same values stored)
  const int itid = tid & (kDeltaThreads - 1);

  // state tile pointers (the loads are issued after this head's small inputs,
  // so those arrive first: on gfx9 loads retire in issue order)
  // (the fused step addresses slot-strided state only, so its loads stay
  // global-address-space loads rather than FLAT ones that would also hold
  // every LDS wait)
  float *state_r;
  long long write_offset = 0;  // floats from the loaded state to the stored one
  if constexpr (FUSED) {
    const int parity = a.state_copy_stride > 0 ? (a.positions[r] & 1) : 0;
    state_r = a.state_base + static_cast<long long>(a.slots[r]) * a.state_slot_stride + parity * a.state_copy_stride;
    write_offset = a.state_copy_stride > 0 ? (1 - 2 * parity) * a.state_copy_stride : 0;
  } else {
    state_r = a.state_base != nullptr ? a.state_base + static_cast<long long>(a.slots[r]) * a.state_slot_stride
                                      : a.states[r];
  }
  q35_f32x4 *S = reinterpret_cast<q35_f32x4 *>(state_r + static_cast<size_t>(vh) * kDim * kDim) + rowg * (kDim / 4) + col;
  q35_f32x4 *W = reinterpret_cast<q35_f32x4 *>(reinterpret_cast<float *>(S) + write_offset);
  q35_f32x4 st[kDecodeRows][2];
  auto load_state = [&]() {
#pragma unroll
    for (int j = 0; j < kDecodeRows; ++j)
#pragma unroll
      for (int m = 0; m < 2; ++m) st[j][m] = Q35_LOAD_NT(S + j * kDecodeRowStride * (kDim / 4) + 16 * m);
  };

  // ---- 2. q, k, v, gates of this head: every load first (the conv ring is
  // written only after all reads), then the math
  const int q_dim = a.k_heads * kDim, v_dim = a.v_heads * kDim;
  const int channels = 2 * q_dim + v_dim;
  // output gate and gated-norm weights of columns 2(lane), 2(lane)+1 (wave 0)
  float z[2] = {0.0F, 0.0F};
  float nw[2] = {0.0F, 0.0F};
  if constexpr (FUSED) {
    float *conv = a.conv_base + static_cast<long long>(a.slots[r]) * a.conv_slot_stride;
    constexpr int K = kConvKernel;
    const int pos = a.positions[r];
    // threads 0..127: q channel, 128..255: k channel of key head kh; threads
    // 0..127 also own the v channel of value head vh
    const int i = itid & (kDim - 1);
    const bool is_k = itid >= kDim, has_v = itid < kDim;
    const int chq = (is_k ? q_dim : 0) + kh * kDim + i;
    const int chv = has_v ? 2 * q_dim + vh * kDim + itid : chq;
    // raw (split) loads of every small input first, then the state tile,
    // then the reductions
    float xq_s[MS], xv_s[MS], b_s[MS], a_s[MS];
    q35_f32x2 z_s[MS];
    a.proj.template load<MS>(r, chq, xq_s);
    a.proj.template load<MS>(r, chv, xv_s);
    {
      const float *zq = a.proj.p + static_cast<long long>(r) * a.proj.width + channels + vh * kDim + 2 * lane;
#pragma unroll
      for (int u = 0; u < MS; ++u)
        z_s[u] = *reinterpret_cast<const q35_f32x2 *>(zq + static_cast<long long>(min(u, a.proj.splits - 1)) *
                                                               a.proj.split_stride);
    }
    // with separate gate rows the projection row is [qkv | z] only
    // b and a of this head: projection columns, or (Q8 gate tail) the
    // separate gate rows [batch][2 v_heads] read as one split -- one view, so
    // the loads are issued here, before the state, under no branch (a load
    // under a branch holds its join until every load in flight returns)
    SplitRows ba = a.proj;
    int cb = channels + v_dim + vh, ca = channels + v_dim + a.v_heads + vh;
    if (a.gates != nullptr) {
      ba.p = a.gates;
      ba.splits = 1;
      ba.split_stride = 0;
      ba.width = 2 * a.v_heads;
      cb = vh;
      ca = a.v_heads + vh;
    }
    ba.template load<MS>(r, cb, b_s);
    ba.template load<MS>(r, ca, a_s);
    float hq[K - 1], hv[K - 1], wq[K], wv[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
      wq[k] = a.conv_w[static_cast<size_t>(k) * channels + chq];
      wv[k] = a.conv_w[static_cast<size_t>(k) * channels + chv];
    }
#pragma unroll
    for (int k = 0; k < K - 1; ++k) {
      const int slot = (pos + 1 + k) & (K - 1);  // position pos - (K-1) + k
      hq[k] = conv[static_cast<size_t>(slot) * channels + chq];
      hv[k] = conv[static_cast<size_t>(slot) * channels + chv];
    }
    // (every thread loads these; wave 0 / thread 0 use them)
#pragma unroll
    for (int e = 0; e < 2; ++e) nw[e] = a.norm_w[2 * lane + e];
    const float dtb = a.dt_bias[vh];
    const float sa_ = a.ssm_a[vh];
    load_state();
    const float xq = a.proj.template reduce<MS>(xq_s);
    const float xv = a.proj.template reduce<MS>(xv_s);
    {
      q35_f32x2 zz = z_s[0];
#pragma unroll
      for (int u = 1; u < MS; ++u) zz = u < a.proj.splits ? zz + z_s[u] : zz;
      z[0] = zz[0];
      z[1] = zz[1];
    }
    const float bval = ba.template reduce<MS>(b_s);
    const float aval = ba.template reduce<MS>(a_s);
    // causal conv1d + SiLU (activation.cpp:164-222: x * w[K-1] first, then
    // the history oldest first)
    float yq = xq * wq[K - 1], yv = xv * wv[K - 1];
#pragma unroll
    for (int k = 0; k < K - 1; ++k) {
      yq += hq[k] * wq[k];
      yv += hv[k] * wv[k];
    }
    yq = silu_times(yq, 1.0F);
    yv = silu_times(yv, 1.0F);
    // this position's inputs into the ring
    conv[static_cast<size_t>(pos & (K - 1)) * channels + chq] = xq;
    if (has_v) conv[static_cast<size_t>(pos & (K - 1)) * channels + chv] = xv;
    if (tid == 0) {
      s_beta = sigmoid_stable(bval);
      const float pre = softplus_stable(aval + dtb);
      s_alpha = expf(pre * sa_);
    }
    // L2 norms of q (waves 0-1) and k (waves 2-3) over 128 values
    const float ss = wave_sum(yq * yq);
    if (lane == 0) red[wave] = ss;
    if (has_v) sv[itid] = yv;
    lds_barrier();
    const float tot = is_k ? red[2] + red[3] : red[0] + red[1];
    const float scale = is_k ? 1.0F : 1.0F / sqrtf(static_cast<float>(kDim));
    const float mul = scale / sqrtf(tot + 1.0e-6F);
    if (is_k)
      sk[i] = yq * mul;
    else
      sq[i] = yq * mul;
  } else {
    load_state();
    const size_t qk = (static_cast<size_t>(r) * a.v_heads + vh) * kDim;
    if (tid < kDim) {
      sq[tid] = a.q[qk + tid];
      sk[tid] = a.k[qk + tid];
      sv[tid] = a.v[qk + tid];
    }
    if (tid == 0) {
      s_alpha = a.alpha[static_cast<size_t>(r) * a.v_heads + vh];
      s_beta = a.beta[static_cast<size_t>(r) * a.v_heads + vh];
    }
  }
  lds_barrier();

  // ---- 3. delta rule on the eight rows of this thread
  const float alpha = s_alpha, beta = s_beta;
  q35_f32x4 kc[2], qc[2];
#pragma unroll
  for (int m = 0; m < 2; ++m) {
    kc[m] = *reinterpret_cast<const q35_f32x4 *>(sk + 4 * col + 64 * m);
    qc[m] = *reinterpret_cast<const q35_f32x4 *>(sq + 4 * col + 64 * m);
  }
#pragma unroll
  for (int j = 0; j < kDecodeRows; ++j) {
    const int row = rowg + kDecodeRowStride * j;
    const float o = delta_row(st[j], kc, qc, sv[row], alpha, beta);
    if (col == 0) so[row] = o;
  }
  // the outputs are shared through LDS before the state goes back; waves
  // 1-3 store their rows at once, wave 0 after the epilogue (a later load
  // would wait for earlier stores: vmcnt counts both)
  lds_barrier();
  auto store_state = [&]() {
#pragma unroll
    for (int j = 0; j < kDecodeRows; ++j)
#pragma unroll
      for (int m = 0; m < 2; ++m) Q35_STORE_NT(st[j][m], W + j * kDecodeRowStride * (kDim / 4) + 16 * m);
  };
  if (wave != 0) {
    store_state();
    return;
  }

  // ---- 4. outputs: wave 0
  const int j = lane & 15;
  if constexpr (FUSED) {
    // gated RMSNorm (offset 0) over the head, then * SiLU(z)  (layers.inl:198-207).
    // The sum of squares in 16-lane order (lane j: columns 8j .. 8j+7 in
    // order, then the row butterfly; the four rows compute the same), as the
    // prefill chunk kernel forms it; then lane l finishes columns 2l, 2l+1
    // and the 64 lanes prepare the head's H128 block.
    float ss = 0.0F;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float x = so[8 * j + e];
      ss += x * x;
    }
    ss = row_sum16(ss);
    const float inv = 1.0F / sqrtf(ss / static_cast<float>(kDim) + a.eps);
    float y[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) y[e] = silu_times(z[e], so[2 * lane + e] * inv * (nw[e] + 0.0F));
    if (a.out != nullptr)
      *reinterpret_cast<q35_f32x2 *>(a.out + static_cast<size_t>(r) * v_dim + vh * kDim + 2 * lane) = q35_f32x2{y[0], y[1]};
    if (a.codes != nullptr) {
      QuantOut qo;
      qo.codes = a.codes;
      qo.scales = a.scales;
      h128_quantize_lanes<64>(y, r, vh, v_dim / 32, true, a.seed, qo, true);
    }
  } else if (lane < 16) {
    const size_t o = (static_cast<size_t>(r) * a.v_heads + vh) * kDim + 8 * j;
#pragma unroll
    for (int e = 0; e < 8; ++e) a.out[o + e] = so[8 * j + e];
  }
  store_state();
}

// Chunked prefill (prefill.inl:599-791 runs a prompt in chunks; the
// recurrence itself is delta_net.cpp:63-98 per token). The rows form
// segments (row_seg, seg_row0, seg_count): each segment is consecutive
// positions of ONE request -- a prompt chunk, or a single decode row -- and
// the in-projection rows arrive already summed (one split). Without segment
// arrays the `batch` rows are one segment.
// Only the state recurrence is sequential, so a chunk runs as three kernels:
//   1. delta_chunk_inputs_kernel, one workgroup per (value head, kInTokens
//      tokens):
//      causal conv + SiLU, L2 norms, beta and alpha of every token at once
//      (the conv history of a token is the ring for positions before the
//      chunk and the chunk's own rows after it);
//   2. delta_scan_kernel, one wavefront per 16 value rows of a head: the rows
//      are independent recurrences, so each wavefront walks the chunk's tokens
//      with its rows' state in registers (one load, one store per chunk) and
//      no workgroup barrier;
//   3. delta_chunk_out_kernel, one 16-lane row per (value head, token): gated
//      RMSNorm * SiLU(z) and the A16 preparation of the out projection's
//      input, plus the ring update with the chunk's last K-1 inputs.
// Each step is delta_kernel<true>'s arithmetic in the same order (the same
// lanes own the same columns of a row), so a chunk leaves the state, ring and
// outputs that token-by-token decoding of the same positions produces, bit
// for bit. Scan entries are [token][value head][kDeltaScanStride] floats:
// q (normalised, x 1/sqrt(d_k)) | k (normalised) | v | alpha | beta; the raw
// head outputs follow at scan + batch * v_heads * kDeltaScanStride.
constexpr int kInTokens = 8;  // tokens per workgroup of delta_chunk_inputs_kernel

__global__ __launch_bounds__(kDeltaThreads) void delta_chunk_inputs_kernel(DeltaArgs a, int rows) {
  __shared__ float red[kInTokens][4];
  constexpr int K = kConvKernel;
  const int vh = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int per = a.v_heads / a.k_heads;
  const int kh = vh / per;
  const int q_dim = a.k_heads * kDim, v_dim = a.v_heads * kDim;
  const int channels = 2 * q_dim + v_dim;
  const int i = tid & (kDim - 1);
  const bool is_k = tid >= kDim, has_v = tid < kDim;
  const int chq = (is_k ? q_dim : 0) + kh * kDim + i;
  const int chv = has_v ? 2 * q_dim + vh * kDim + tid : chq;
  const int y0 = blockIdx.y * kInTokens;
  const int nt = min(kInTokens, rows - y0);  // tokens of this workgroup (uniform, >= 1)
  // the head's conv weights and gate constants, once for the workgroup's tokens
  float wq[K], wv[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    wq[k] = a.conv_w[static_cast<size_t>(k) * channels + chq];
    wv[k] = a.conv_w[static_cast<size_t>(k) * channels + chv];
  }
  const float dtb = a.dt_bias[vh];
  const float sa_ = a.ssm_a[vh];
  // every token's loads first (their index chains and inputs do not depend on
  // one another, so they are in flight together), then the arithmetic. Lane
  // t < nt of wave 0 computes token t's gates (beta, alpha): every lane loads
  // the b and a inputs of token min(lane, nt - 1), so no load sits under a
  // branch, and the nt gate computations run side by side instead of one
  // after another on one lane
  const int gy = y0 + min(lane, nt - 1);
  const int gr = a.chunk_rows != nullptr ? a.chunk_rows[gy] : gy;
  const float *grow = a.proj.p + static_cast<long long>(gr) * a.proj.width;
  const float gb = a.gates != nullptr ? a.gates[static_cast<size_t>(gr) * 2 * a.v_heads + vh] : grow[channels + v_dim + vh];
  const float ga = a.gates != nullptr ? a.gates[static_cast<size_t>(gr) * 2 * a.v_heads + a.v_heads + vh]
                                      : grow[channels + v_dim + a.v_heads + vh];
  int rr[kInTokens];
  float xq[kInTokens], xv[kInTokens];
  float hq[kInTokens][K - 1], hv[kInTokens][K - 1];
#pragma unroll
  for (int t = 0; t < kInTokens; ++t) {
    if (t >= nt) break;  // uniform
    const int y = y0 + t;
    const int r = a.chunk_rows != nullptr ? a.chunk_rows[y] : y;
    rr[t] = r;
    // the row's segment: rows seg_row0 .. are consecutive positions of its slot
    const int r0 = a.row_seg != nullptr ? a.seg_row0[a.row_seg[r]] : 0;
    const int slot = a.slots[r0], pos0 = a.positions[r0], pos = pos0 + (r - r0);
    const float *conv = a.conv_base + static_cast<long long>(slot) * a.conv_slot_stride;
    const float *row = a.proj.p + static_cast<long long>(r) * a.proj.width;
    xq[t] = row[chq];
    xv[t] = row[chv];
#pragma unroll
    for (int k = 0; k < K - 1; ++k) {
      const int p = pos - (K - 1) + k;  // oldest first
      if (p >= pos0) {
        const float *hrow = a.proj.p + static_cast<long long>(r0 + p - pos0) * a.proj.width;
        hq[t][k] = hrow[chq];
        hv[t][k] = hrow[chv];
      } else {
        hq[t][k] = conv[static_cast<size_t>(p & (K - 1)) * channels + chq];
        hv[t][k] = conv[static_cast<size_t>(p & (K - 1)) * channels + chv];
      }
    }
  }
  float yq[kInTokens];
#pragma unroll
  for (int t = 0; t < kInTokens; ++t) {
    if (t >= nt) break;
    float q = xq[t] * wq[K - 1], v = xv[t] * wv[K - 1];
#pragma unroll
    for (int k = 0; k < K - 1; ++k) {
      q += hq[t][k] * wq[k];
      v += hv[t][k] * wv[k];
    }
    q = silu_times(q, 1.0F);
    v = silu_times(v, 1.0F);
    yq[t] = q;
    float *e = a.scan + (static_cast<size_t>(rr[t]) * a.v_heads + vh) * kDeltaScanStride;
    const float ss = wave_sum(q * q);
    if (lane == 0) red[t][wave] = ss;
    if (has_v) e[2 * kDim + tid] = v;
  }
  if (tid < nt) {
    float *e = a.scan + (static_cast<size_t>(gr) * a.v_heads + vh) * kDeltaScanStride;
    e[3 * kDim + 1] = sigmoid_stable(gb);
    const float pre = softplus_stable(ga + dtb);
    e[3 * kDim] = expf(pre * sa_);
  }
  lds_barrier();
  const float scale = is_k ? 1.0F : 1.0F / sqrtf(static_cast<float>(kDim));
#pragma unroll
  for (int t = 0; t < kInTokens; ++t) {
    if (t >= nt) break;
    const float tot = is_k ? red[t][2] + red[t][3] : red[t][0] + red[t][1];
    const float mul = scale / sqrtf(tot + 1.0e-6F);
    float *e = a.scan + (static_cast<size_t>(rr[t]) * a.v_heads + vh) * kDeltaScanStride;
    e[(is_k ? kDim : 0) + i] = yq[t] * mul;
  }
}

// One wavefront per 4 value rows (grid: row blocks x value heads x
// segments): the 16 lanes of row 4 * blockIdx.x + lane / 16 hold it as
// delta_kernel does (columns 4o + 64m) and run delta_row per token, so the
// chain of a token is 8 columns long and the scan has a wavefront per SIMD at
// the 4B shapes. Tokens go in blocks of kScanBlock: the block's inputs (q and
// k, the 4 rows' values, alpha and beta) sit in LDS, and the next block's are
// loaded into registers meanwhile and stored after the block, so a token's
// step waits on LDS only, never on memory.
constexpr int kDeltaScanRows = 64 / kRowLanes;
constexpr int kScanBlock = 16;

__global__ __launch_bounds__(64) void delta_scan_kernel(DeltaArgs a) {
  __shared__ q35_f32x4 qk_lds[2][kScanBlock][2 * kDim / 4];
  __shared__ float v_lds[2][kScanBlock][kDeltaScanRows];
  __shared__ float ab_lds[2][kScanBlock][2];
  const int lane = threadIdx.x;
  // workgroup i runs on XCD i % 8: with v_heads % 8 == 0 the row blocks of a
  // head share one XCD, whose L2 then serves the head's q and k to all of
  // them (spread over the XCDs, each XCD would fetch the token stream again)
  int vh = blockIdx.y, rb = blockIdx.x;
  if ((a.v_heads & 7) == 0) {
    const int p = static_cast<int>(blockIdx.x + gridDim.x * blockIdx.y), k = p >> 3;
    vh = (k / static_cast<int>(gridDim.x)) * 8 + (p & 7);
    rb = k % static_cast<int>(gridDim.x);
  }
  const int col = lane & (kRowLanes - 1), row = kDeltaScanRows * rb + (lane >> 4);
  // segment seg: rows r0 .. r0 + count - 1 of one slot, in order; the
  // longest segments are dispatched first, so a prompt chunk's row groups
  // start ahead of a packed step's one-token segments
  const int seg = a.seg_order != nullptr ? a.seg_order[blockIdx.z] : static_cast<int>(blockIdx.z);
  const int r0 = a.row_seg != nullptr ? a.seg_row0[seg] : 0;
  const int count = a.row_seg != nullptr ? a.seg_count[seg] : a.batch;
  const int slot = a.slots[r0], pos0 = a.positions[r0];
  const int rpar = a.state_copy_stride > 0 ? (pos0 & 1) : 0;
  const int wpar = a.state_copy_stride > 0 ? ((pos0 + count) & 1) : 0;
  float *state_slot = a.state_base + static_cast<long long>(slot) * a.state_slot_stride;
  const size_t off = static_cast<size_t>(vh) * kDim * kDim + static_cast<size_t>(row) * kDim + 4 * col;
  const q35_f32x4 *S = reinterpret_cast<const q35_f32x4 *>(state_slot + rpar * a.state_copy_stride + off);
  q35_f32x4 *W = reinterpret_cast<q35_f32x4 *>(state_slot + wpar * a.state_copy_stride + off);
  q35_f32x4 st[2];
#pragma unroll
  for (int m = 0; m < 2; ++m) st[m] = Q35_LOAD_NT(S + 16 * m);
  const size_t tstride = static_cast<size_t>(a.v_heads) * kDeltaScanStride;
  const float *scan = a.scan + static_cast<size_t>(r0) * tstride + static_cast<size_t>(vh) * kDeltaScanStride;
  float *outs = a.scan + static_cast<size_t>(a.batch) * tstride + static_cast<size_t>(r0) * a.v_heads * kDim +
                static_cast<size_t>(vh) * kDim + row;
  // the inputs of tokens t0 .. t0 + kScanBlock - 1 (clamped into the
  // segment): lane l holds q|k floats 4l..4l+3 of every token, the value of
  // row l % 4 of token l / 4, and alpha (l even) or beta (l odd) of token l / 2
  struct Block {
    q35_f32x4 qk[kScanBlock];
    float v, ab;
  };
  const int rbase = kDeltaScanRows * rb;
  auto load = [&](Block &k, int t0) {
#pragma unroll
    for (int i = 0; i < kScanBlock; ++i)
      k.qk[i] = reinterpret_cast<const q35_f32x4 *>(scan + static_cast<size_t>(min(t0 + i, count - 1)) * tstride)[lane];
    k.v = scan[static_cast<size_t>(min(t0 + (lane >> 2), count - 1)) * tstride + 2 * kDim + rbase + (lane & 3)];
    k.ab = scan[static_cast<size_t>(min(t0 + ((lane >> 1) & (kScanBlock - 1)), count - 1)) * tstride + 3 * kDim + (lane & 1)];
  };
  auto store = [&](const Block &k, int buf) {
#pragma unroll
    for (int i = 0; i < kScanBlock; ++i) qk_lds[buf][i][lane] = k.qk[i];
    v_lds[buf][lane >> 2][lane & 3] = k.v;
    if (lane < 2 * kScanBlock) ab_lds[buf][lane >> 1][lane & 1] = k.ab;
  };
  Block blk;
  load(blk, 0);
  store(blk, 0);
  lds_barrier();
  for (int t0 = 0, cur = 0; t0 < count; t0 += kScanBlock, cur ^= 1) {
    const bool more = t0 + kScanBlock < count;
    if (more) load(blk, t0 + kScanBlock);
    // the next block's loads stay issued here, a block ahead of their use
    // (left alone, the compiler sinks them next to the store)
    q35_compiler_fence();
    const int n = min(kScanBlock, count - t0);
    // token i's inputs are read from LDS while token i-1's row update runs
    // (two register sets, alternating), so a step never waits for its own
    // reads; lane `col` keeps the output of token t0 + col of its row and
    // stores it after the block
    struct Tok {
      q35_f32x4 kc[2], qc[2];
      float v, alpha, beta;
    };
    auto read = [&](Tok &x, int i) {
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        x.kc[m] = qk_lds[cur][i][kDim / 4 + col + 16 * m];
        x.qc[m] = qk_lds[cur][i][col + 16 * m];
      }
      x.v = v_lds[cur][i][lane >> 4];
      x.alpha = ab_lds[cur][i][0];
      x.beta = ab_lds[cur][i][1];
    };
    float kept = 0.0F;
    auto step = [&](const Tok &x, int i) {
      const float o = delta_row(st, x.kc, x.qc, x.v, x.alpha, x.beta);
      kept = col == i ? o : kept;
    };
    Tok A, B;
    read(A, 0);
    int i = 0;
    for (; i + 1 < n; i += 2) {
      read(B, i + 1);
      step(A, i);
      read(A, min(i + 2, n - 1));  // past the block's last token: re-read, unused
      step(B, i + 1);
    }
    if (i < n) step(A, i);
    if (col < n) outs[static_cast<size_t>(t0 + col) * a.v_heads * kDim] = kept;
    if (more) store(blk, cur ^ 1);
    lds_barrier();
  }
#pragma unroll
  for (int m = 0; m < 2; ++m) Q35_STORE_NT(st[m], W + 16 * m);
}

// One 16-lane row per (value head, token), kOutTokens tokens of one head per
// workgroup: lane j = lane % 16 holds columns 8j .. 8j+7 of the head's
// outputs, as delta_kernel's epilogue (whose four rows compute the same
// token).
constexpr int kOutTokens = 16;  // tokens per workgroup of delta_chunk_out_kernel

__global__ __launch_bounds__(16 * kOutTokens) void delta_chunk_out_kernel(DeltaArgs a, int rows) {
  constexpr int K = kConvKernel;
  const int vh = blockIdx.x, lane = threadIdx.x & 63;
  const int y = blockIdx.y * kOutTokens + (threadIdx.x >> 4);
  const bool active = y < rows;  // rows past the list compute the last one and store nothing
  const int yy = min(y, rows - 1);
  const int r = a.chunk_rows != nullptr ? a.chunk_rows[yy] : yy;
  const int q_dim = a.k_heads * kDim, v_dim = a.v_heads * kDim;
  const int channels = 2 * q_dim + v_dim;
  const int j = lane & 15;
  const float *prow = a.proj.p + static_cast<long long>(r) * a.proj.width;
  const q35_f32x4 *zp = reinterpret_cast<const q35_f32x4 *>(prow + channels + vh * kDim + 8 * j);
  const q35_f32x4 *op = reinterpret_cast<const q35_f32x4 *>(
      a.scan + static_cast<size_t>(a.batch) * a.v_heads * kDeltaScanStride + (static_cast<size_t>(r) * a.v_heads + vh) * kDim + 8 * j);
  const q35_f32x4 *wp = reinterpret_cast<const q35_f32x4 *>(a.norm_w + 8 * j);
  const q35_f32x4 z0 = zp[0], z1 = zp[1], o0 = op[0], o1 = op[1], w0 = wp[0], w1 = wp[1];
  float yv[8], z[8], nw[8];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    yv[e] = o0[e];
    yv[4 + e] = o1[e];
    z[e] = z0[e];
    z[4 + e] = z1[e];
    nw[e] = w0[e];
    nw[4 + e] = w1[e];
  }
  float yss = 0.0F;
#pragma unroll
  for (int e = 0; e < 8; ++e) yss += yv[e] * yv[e];
  yss = row_sum16(yss);
  const float inv = 1.0F / sqrtf(yss / static_cast<float>(kDim) + a.eps);
#pragma unroll
  for (int e = 0; e < 8; ++e) yv[e] = silu_times(z[e], yv[e] * inv * (nw[e] + 0.0F));
  if (a.out != nullptr && active)
#pragma unroll
    for (int e = 0; e < 8; ++e) a.out[static_cast<size_t>(r) * v_dim + vh * kDim + 8 * j + e] = yv[e];
  if (a.codes != nullptr) {
    QuantOut qo;
    qo.codes = a.codes;
    qo.scales = a.scales;
    h128_quantize_row16(yv, r, vh, v_dim / 32, true, a.seed, qo, active);
  }
  // the segment's last K-1 raw inputs into the ring (slot = position % K);
  // the inputs kernel read the ring before this launch
  const int seg = a.row_seg != nullptr ? a.row_seg[r] : 0;
  const int seg_end = a.row_seg != nullptr ? a.seg_row0[seg] + a.seg_count[seg] : a.batch;
  if (active && r >= seg_end - (K - 1)) {
    const int per = a.v_heads / a.k_heads, kh = vh / per;
    const int r0 = a.row_seg != nullptr ? a.seg_row0[seg] : 0;
    float *ring = a.conv_base + static_cast<long long>(a.slots[r0]) * a.conv_slot_stride +
                  static_cast<size_t>((a.positions[r0] + (r - r0)) & (K - 1)) * channels;
    for (int c = j; c < kDim; c += 16) {
      if (vh % per == 0) {
        ring[kh * kDim + c] = prow[kh * kDim + c];
        ring[q_dim + kh * kDim + c] = prow[q_dim + kh * kDim + c];
      }
      ring[2 * q_dim + vh * kDim + c] = prow[2 * q_dim + vh * kDim + c];
    }
  }
}

}  // namespace

hipError_t launch_delta(const DeltaArgs &a, hipStream_t stream) {
  const int rows = a.row_list != nullptr ? a.row_count : a.batch;
  if (rows <= 0) return hipSuccess;
  if (a.kd != kDim || a.vd != kDim || a.v_heads % a.k_heads != 0) return hipErrorInvalidValue;
  const dim3 grid(a.v_heads, rows);
  // 512 threads while the grid is at most two workgroups per compute unit
  const bool wide = a.v_heads * rows <= 512;
#define Q35_DELTA(F, MS)                                                                   \
  if (wide)                                                                                \
    Q35_LAUNCH((delta_kernel<F, MS, 512>), grid, dim3(512), 0, stream, a);                 \
  else                                                                                     \
    Q35_LAUNCH((delta_kernel<F, MS, 256>), grid, dim3(256), 0, stream, a);
  if (!a.fused) {
    Q35_DELTA(false, 1)
    return hipGetLastError();
  }
  if (a.kernel != kConvKernel) return hipErrorInvalidValue;
  switch (split_bound(a.proj.splits)) {
    case 1: Q35_DELTA(true, 1) break;
    case 4: Q35_DELTA(true, 4) break;
    case 8: Q35_DELTA(true, 8) break;
    default: return hipErrorInvalidValue;
  }
#undef Q35_DELTA
  return hipGetLastError();
}

hipError_t launch_delta_chunk(const DeltaArgs &a, hipStream_t stream) {
  if (a.batch <= 0) return hipSuccess;
  if (!a.fused || a.kd != kDim || a.vd != kDim || a.v_heads % a.k_heads != 0 || a.kernel != kConvKernel ||
      a.state_base == nullptr || a.slots == nullptr || a.positions == nullptr || a.scan == nullptr ||
      a.proj.splits != 1)
    return hipErrorInvalidValue;
  // a packed step's one-row segments run the decode kernel (the same
  // arithmetic), the other segments the three chunk kernels
  const int rows = a.chunk_rows != nullptr ? a.chunk_row_count : a.batch;
  const int scans = a.chunk_rows != nullptr ? a.scan_segments : (a.row_seg != nullptr ? a.segments : 1);
  if (rows > 0) {
    Q35_LAUNCH((delta_chunk_inputs_kernel), dim3(a.v_heads, (rows + kInTokens - 1) / kInTokens), dim3(kDeltaThreads), 0,
               stream, a, rows);
    Q35_LAUNCH((delta_scan_kernel), dim3(kDim / kDeltaScanRows, a.v_heads, scans), dim3(64), 0, stream, a);
    Q35_LAUNCH((delta_chunk_out_kernel), dim3(a.v_heads, (rows + kOutTokens - 1) / kOutTokens), dim3(16 * kOutTokens),
               0, stream, a, rows);
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return a.row_list != nullptr ? launch_delta(a, stream) : hipSuccess;
}

}  // namespace q35
