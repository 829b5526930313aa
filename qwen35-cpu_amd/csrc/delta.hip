// GatedDeltaNet decode update on CDNA4.
//
// One workgroup (256 threads) per (value head, request). The head's fp32
// state tile [value_row][key_col] = 128 x 128 (64 KiB) makes exactly one HBM
// round trip; its loads are issued right after the head's few small inputs
// (conv ring, projections, weights), so the 64 KiB are in flight while those
// are combined.
// Thread t owns rows t/4 and 64 + t/4 and, within each, the eight float4 at
// columns 16m + 4(t%4) (m = 0..7): four lanes share a row, so every row dot
// product finishes with two DPP quad exchanges instead of a shuffle chain,
// and one load instruction covers 16 rows x 64 contiguous bytes.
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

// FUSED: the linear-attention step around the update; MS: compile-time bound
// on the in-projection's K splits (so every input load is straight-line).
template <bool FUSED, int MS>
__global__ __launch_bounds__(kDeltaThreads) void delta_kernel(DeltaArgs a) {
  __shared__ float sq[kDim], sk[kDim], sv[kDim], so[kDim];
  __shared__ float red[8];
  __shared__ float s_alpha, s_beta;
  const int vh = blockIdx.x, r = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int per = a.v_heads / a.k_heads;
  const int kh = vh / per;
  const int quad = tid & 3, rowp = tid >> 2;

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
  q35_f32x4 *S = reinterpret_cast<q35_f32x4 *>(state_r + static_cast<size_t>(vh) * kDim * kDim);
  q35_f32x4 *S0 = S + rowp * (kDim / 4) + quad;         // row rowp
  q35_f32x4 *S1 = S + (rowp + 64) * (kDim / 4) + quad;  // row rowp + 64
  q35_f32x4 *W0 = reinterpret_cast<q35_f32x4 *>(reinterpret_cast<float *>(S0) + write_offset);
  q35_f32x4 *W1 = reinterpret_cast<q35_f32x4 *>(reinterpret_cast<float *>(S1) + write_offset);
  q35_f32x4 st0[8], st1[8];
  auto load_state = [&]() {
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      st0[m] = Q35_LOAD_NT(S0 + 4 * m);
      st1[m] = Q35_LOAD_NT(S1 + 4 * m);
    }
  };

  // ---- 2. q, k, v, gates of this head: every load first (the conv ring is
  // written only after all reads), then the math
  const int q_dim = a.k_heads * kDim, v_dim = a.v_heads * kDim;
  const int channels = 2 * q_dim + v_dim;
  // output gate and gated-norm weights of columns 8(lane%16)..+7 (wave 0)
  float z[8] = {0.0F, 0.0F, 0.0F, 0.0F, 0.0F, 0.0F, 0.0F, 0.0F};
  float nw[8] = {0.0F, 0.0F, 0.0F, 0.0F, 0.0F, 0.0F, 0.0F, 0.0F};
  if constexpr (FUSED) {
    float *conv = a.conv_base + static_cast<long long>(a.slots[r]) * a.conv_slot_stride;
    constexpr int K = kConvKernel;
    const int pos = a.positions[r];
    // threads 0..127: q channel, 128..255: k channel of key head kh; threads
    // 0..127 also own the v channel of value head vh
    const int i = tid & (kDim - 1);
    const bool is_k = tid >= kDim, has_v = tid < kDim;
    const int chq = (is_k ? q_dim : 0) + kh * kDim + i;
    const int chv = has_v ? 2 * q_dim + vh * kDim + tid : chq;
    // raw (split) loads of every small input first, then the state tile,
    // then the reductions
    float xq_s[MS], xv_s[MS], b_s[MS], a_s[MS];
    q35_f32x4 z_s[MS][2];
    a.proj.template load<MS>(r, chq, xq_s);
    a.proj.template load<MS>(r, chv, xv_s);
    a.proj.template load8<MS>(r, channels + vh * kDim + 8 * (lane & 15), z_s);
    a.proj.template load<MS>(r, channels + v_dim + vh, b_s);
    a.proj.template load<MS>(r, channels + v_dim + a.v_heads + vh, a_s);
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
    for (int e = 0; e < 8; ++e) nw[e] = a.norm_w[8 * (lane & 15) + e];
    const float dtb = a.dt_bias[vh];
    const float sa_ = a.ssm_a[vh];
    load_state();
    const float xq = a.proj.template reduce<MS>(xq_s);
    const float xv = a.proj.template reduce<MS>(xv_s);
    a.proj.template reduce8<MS>(z_s, z);
    const float bval = a.proj.template reduce<MS>(b_s);
    const float aval = a.proj.template reduce<MS>(a_s);
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
    if (has_v) sv[tid] = yv;
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

  // ---- 3. delta rule on the two rows of this thread
  const float alpha = s_alpha, beta = s_beta;
  q35_f32x4 kc[8];
#pragma unroll
  for (int m = 0; m < 8; ++m) kc[m] = *reinterpret_cast<const q35_f32x4 *>(sk + 16 * m + 4 * quad);
  float d0 = 0.0F, d1 = 0.0F;
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    st0[m] *= alpha;
    st1[m] *= alpha;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      d0 += st0[m][e] * kc[m][e];
      d1 += st1[m][e] * kc[m][e];
    }
  }
  d0 += q35_quad_xor1(d0);
  d1 += q35_quad_xor1(d1);
  d0 += q35_quad_xor2(d0);
  d1 += q35_quad_xor2(d1);
  const float delta0 = (sv[rowp] - d0) * beta, delta1 = (sv[rowp + 64] - d1) * beta;
  float o0 = 0.0F, o1 = 0.0F;
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    const q35_f32x4 qc = *reinterpret_cast<const q35_f32x4 *>(sq + 16 * m + 4 * quad);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      st0[m][e] += delta0 * kc[m][e];
      st1[m][e] += delta1 * kc[m][e];
      o0 += st0[m][e] * qc[e];
      o1 += st1[m][e] * qc[e];
    }
  }
  o0 += q35_quad_xor1(o0);
  o1 += q35_quad_xor1(o1);
  o0 += q35_quad_xor2(o0);
  o1 += q35_quad_xor2(o1);
  if (quad == 0) {
    so[rowp] = o0;
    so[rowp + 64] = o1;
  }
  // the outputs are shared through LDS before the state goes back; waves
  // 1-3 store their rows at once, wave 0 after the epilogue (a later load
  // would wait for earlier stores: vmcnt counts both)
  lds_barrier();
  auto store_state = [&]() {
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      Q35_STORE_NT(st0[m], W0 + 4 * m);
      Q35_STORE_NT(st1[m], W1 + 4 * m);
    }
  };
  if (wave != 0) {
    store_state();
    return;
  }

  // ---- 4. outputs: wave 0, lane j = lane % 16 holds columns 8j .. 8j+7
  // (the four 16-lane rows compute the same values; row 0 stores)
  const int j = lane & 15;
  const bool writer = lane < 16;
  float y[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) y[e] = so[8 * j + e];
  if constexpr (FUSED) {
    // gated RMSNorm (offset 0) over the head, then * SiLU(z)  (layers.inl:198-207)
    float ss = 0.0F;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += y[e] * y[e];
    ss += q35_row_xor(ss, 1);
    ss += q35_row_xor(ss, 2);
    ss += q35_row_xor(ss, 4);
    ss += q35_row_xor(ss, 8);
    const float inv = 1.0F / sqrtf(ss / static_cast<float>(kDim) + a.eps);
#pragma unroll
    for (int e = 0; e < 8; ++e) y[e] = silu_times(z[e], y[e] * inv * (nw[e] + 0.0F));
    if (a.out != nullptr && writer)
#pragma unroll
      for (int e = 0; e < 8; ++e) a.out[static_cast<size_t>(r) * v_dim + vh * kDim + 8 * j + e] = y[e];
    if (a.codes != nullptr) {
      QuantOut qo;
      qo.codes = a.codes;
      qo.scales = a.scales;
      h128_quantize_row16(y, r, vh, v_dim / 32, true, a.seed, qo, writer);
    }
  } else if (writer) {
    const size_t o = (static_cast<size_t>(r) * a.v_heads + vh) * kDim + 8 * j;
#pragma unroll
    for (int e = 0; e < 8; ++e) a.out[o + e] = y[e];
  }
  store_state();
}

// Chunked prefill scan (prefill.inl:599-791 runs the prompt in chunks; the
// recurrence itself is delta_net.cpp:63-98 per token): one workgroup per value
// head walks the `batch` rows of ONE request -- consecutive positions
// positions[0] .. positions[0] + batch - 1 -- in order. The state tile stays
// in registers for the whole chunk (one load, one store), and the conv
// history slides in registers. Per token the arithmetic is delta_kernel<true>'s
// in the same order, so a chunk leaves the state, ring and outputs that
// token-by-token decoding of the same positions produces, bit for bit.
template <int MS>
__global__ __launch_bounds__(kDeltaThreads) void delta_chunk_kernel(DeltaArgs a) {
  __shared__ float sq[kDim], sk[kDim], sv[kDim], so[kDim];
  __shared__ float red[8];
  __shared__ float s_alpha, s_beta;
  constexpr int K = kConvKernel;
  const int vh = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int per = a.v_heads / a.k_heads;
  const int kh = vh / per;
  const int quad = tid & 3, rowp = tid >> 2;
  const int slot = a.slots[0];
  const int pos0 = a.positions[0], count = a.batch;
  // state copies: read the one for pos0, write the one for pos0 + count
  const int rpar = a.state_copy_stride > 0 ? (pos0 & 1) : 0;
  const int wpar = a.state_copy_stride > 0 ? ((pos0 + count) & 1) : 0;
  float *state_slot = a.state_base + static_cast<long long>(slot) * a.state_slot_stride;
  q35_f32x4 *S = reinterpret_cast<q35_f32x4 *>(state_slot + rpar * a.state_copy_stride +
                                               static_cast<size_t>(vh) * kDim * kDim);
  q35_f32x4 *W = reinterpret_cast<q35_f32x4 *>(state_slot + wpar * a.state_copy_stride +
                                               static_cast<size_t>(vh) * kDim * kDim);
  const int off0 = rowp * (kDim / 4) + quad, off1 = (rowp + 64) * (kDim / 4) + quad;
  q35_f32x4 st0[8], st1[8];
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    st0[m] = Q35_LOAD_NT(S + off0 + 4 * m);
    st1[m] = Q35_LOAD_NT(S + off1 + 4 * m);
  }
  const int q_dim = a.k_heads * kDim, v_dim = a.v_heads * kDim;
  const int channels = 2 * q_dim + v_dim;
  float *conv = a.conv_base + static_cast<long long>(slot) * a.conv_slot_stride;
  const int i = tid & (kDim - 1);
  const bool is_k = tid >= kDim, has_v = tid < kDim;
  const int chq = (is_k ? q_dim : 0) + kh * kDim + i;
  const int chv = has_v ? 2 * q_dim + vh * kDim + tid : chq;
  float hq[K - 1], hv[K - 1], wq[K], wv[K], nw[8];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    wq[k] = a.conv_w[static_cast<size_t>(k) * channels + chq];
    wv[k] = a.conv_w[static_cast<size_t>(k) * channels + chv];
  }
#pragma unroll
  for (int k = 0; k < K - 1; ++k) {
    const int ring = (pos0 + 1 + k) & (K - 1);  // position pos0 - (K-1) + k
    hq[k] = conv[static_cast<size_t>(ring) * channels + chq];
    hv[k] = conv[static_cast<size_t>(ring) * channels + chv];
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) nw[e] = a.norm_w[8 * (lane & 15) + e];
  const float dtb = a.dt_bias[vh];
  const float sa_ = a.ssm_a[vh];
  const int j = lane & 15;
  const bool writer = lane < 16;

  // raw inputs of one token; the next token's are issued as soon as the
  // current ones are summed, so their latency hides behind this token's work
  float xq_s[MS], xv_s[MS], b_s[MS], a_s[MS];
  q35_f32x4 z_s[MS][2];
  auto load_token = [&](int r) {
    a.proj.template load<MS>(r, chq, xq_s);
    a.proj.template load<MS>(r, chv, xv_s);
    a.proj.template load8<MS>(r, channels + vh * kDim + 8 * (lane & 15), z_s);
    a.proj.template load<MS>(r, channels + v_dim + vh, b_s);
    a.proj.template load<MS>(r, channels + v_dim + a.v_heads + vh, a_s);
  };
  load_token(0);
  for (int r = 0; r < count; ++r) {
    // ---- inputs of the token at position pos0 + r
    const float xq = a.proj.template reduce<MS>(xq_s);
    const float xv = a.proj.template reduce<MS>(xv_s);
    float z[8];
    a.proj.template reduce8<MS>(z_s, z);
    const float bval = a.proj.template reduce<MS>(b_s);
    const float aval = a.proj.template reduce<MS>(a_s);
    load_token(min(r + 1, count - 1));
    // causal conv1d + SiLU (activation.cpp:164-222), then slide the history
    float yq = xq * wq[K - 1], yv = xv * wv[K - 1];
#pragma unroll
    for (int k = 0; k < K - 1; ++k) {
      yq += hq[k] * wq[k];
      yv += hv[k] * wv[k];
    }
    yq = silu_times(yq, 1.0F);
    yv = silu_times(yv, 1.0F);
#pragma unroll
    for (int k = 0; k < K - 2; ++k) {
      hq[k] = hq[k + 1];
      hv[k] = hv[k + 1];
    }
    hq[K - 2] = xq;
    hv[K - 2] = xv;
    if (tid == 0) {
      s_beta = sigmoid_stable(bval);
      const float pre = softplus_stable(aval + dtb);
      s_alpha = expf(pre * sa_);
    }
    const float ss = wave_sum(yq * yq);
    if (lane == 0) red[wave] = ss;
    if (has_v) sv[tid] = yv;
    lds_barrier();
    const float tot = is_k ? red[2] + red[3] : red[0] + red[1];
    const float scale = is_k ? 1.0F : 1.0F / sqrtf(static_cast<float>(kDim));
    const float mul = scale / sqrtf(tot + 1.0e-6F);
    if (is_k)
      sk[i] = yq * mul;
    else
      sq[i] = yq * mul;
    lds_barrier();

    // ---- delta rule on this thread's two rows
    const float alpha = s_alpha, beta = s_beta;
    q35_f32x4 kc[8];
#pragma unroll
    for (int m = 0; m < 8; ++m) kc[m] = *reinterpret_cast<const q35_f32x4 *>(sk + 16 * m + 4 * quad);
    float d0 = 0.0F, d1 = 0.0F;
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      st0[m] *= alpha;
      st1[m] *= alpha;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        d0 += st0[m][e] * kc[m][e];
        d1 += st1[m][e] * kc[m][e];
      }
    }
    d0 += q35_quad_xor1(d0);
    d1 += q35_quad_xor1(d1);
    d0 += q35_quad_xor2(d0);
    d1 += q35_quad_xor2(d1);
    const float delta0 = (sv[rowp] - d0) * beta, delta1 = (sv[rowp + 64] - d1) * beta;
    float o0 = 0.0F, o1 = 0.0F;
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      const q35_f32x4 qc = *reinterpret_cast<const q35_f32x4 *>(sq + 16 * m + 4 * quad);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        st0[m][e] += delta0 * kc[m][e];
        st1[m][e] += delta1 * kc[m][e];
        o0 += st0[m][e] * qc[e];
        o1 += st1[m][e] * qc[e];
      }
    }
    o0 += q35_quad_xor1(o0);
    o1 += q35_quad_xor1(o1);
    o0 += q35_quad_xor2(o0);
    o1 += q35_quad_xor2(o1);
    if (quad == 0) {
      so[rowp] = o0;
      so[rowp + 64] = o1;
    }
    lds_barrier();

    // ---- outputs of the token (wave 0): gated RMSNorm * SiLU(z), A16 row r
    if (wave == 0) {
      float y[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) y[e] = so[8 * j + e];
      float yss = 0.0F;
#pragma unroll
      for (int e = 0; e < 8; ++e) yss += y[e] * y[e];
      yss += q35_row_xor(yss, 1);
      yss += q35_row_xor(yss, 2);
      yss += q35_row_xor(yss, 4);
      yss += q35_row_xor(yss, 8);
      const float inv = 1.0F / sqrtf(yss / static_cast<float>(kDim) + a.eps);
#pragma unroll
      for (int e = 0; e < 8; ++e) y[e] = silu_times(z[e], y[e] * inv * (nw[e] + 0.0F));
      if (a.out != nullptr && writer)
#pragma unroll
        for (int e = 0; e < 8; ++e) a.out[static_cast<size_t>(r) * v_dim + vh * kDim + 8 * j + e] = y[e];
      if (a.codes != nullptr) {
        QuantOut qo;
        qo.codes = a.codes;
        qo.scales = a.scales;
        h128_quantize_row16(y, r, vh, v_dim / 32, true, a.seed, qo, writer);
      }
    }
    // the next token rewrites sq, sk, sv, so, red and the gates
    lds_barrier();
  }

  // ---- the chunk's state and the ring's last K-1 inputs go back once
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    Q35_STORE_NT(st0[m], W + off0 + 4 * m);
    Q35_STORE_NT(st1[m], W + off1 + 4 * m);
  }
  const int pos_last = pos0 + count - 1;
#pragma unroll
  for (int k = 0; k < K - 1; ++k) {
    const int ring = (pos_last - (K - 2) + k) & (K - 1);  // position pos_last - (K-2) + k
    conv[static_cast<size_t>(ring) * channels + chq] = hq[k];
    if (has_v) conv[static_cast<size_t>(ring) * channels + chv] = hv[k];
  }
}

}  // namespace

hipError_t launch_delta(const DeltaArgs &a, hipStream_t stream) {
  if (a.batch <= 0) return hipSuccess;
  if (a.kd != kDim || a.vd != kDim || a.v_heads % a.k_heads != 0) return hipErrorInvalidValue;
  const dim3 grid(a.v_heads, a.batch), block(kDeltaThreads);
  if (!a.fused) {
    Q35_LAUNCH((delta_kernel<false, 1>), grid, block, 0, stream, a);
    return hipGetLastError();
  }
  if (a.kernel != kConvKernel) return hipErrorInvalidValue;
  switch (split_bound(a.proj.splits)) {
    case 1: Q35_LAUNCH((delta_kernel<true, 1>), grid, block, 0, stream, a); break;
    case 4: Q35_LAUNCH((delta_kernel<true, 4>), grid, block, 0, stream, a); break;
    case 8: Q35_LAUNCH((delta_kernel<true, 8>), grid, block, 0, stream, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_delta_chunk(const DeltaArgs &a, hipStream_t stream) {
  if (a.batch <= 0) return hipSuccess;
  if (!a.fused || a.kd != kDim || a.vd != kDim || a.v_heads % a.k_heads != 0 || a.kernel != kConvKernel ||
      a.state_base == nullptr || a.slots == nullptr || a.positions == nullptr)
    return hipErrorInvalidValue;
  const dim3 grid(a.v_heads), block(kDeltaThreads);
  switch (split_bound(a.proj.splits)) {
    case 1: Q35_LAUNCH((delta_chunk_kernel<1>), grid, block, 0, stream, a); break;
    case 4: Q35_LAUNCH((delta_chunk_kernel<4>), grid, block, 0, stream, a); break;
    case 8: Q35_LAUNCH((delta_chunk_kernel<8>), grid, block, 0, stream, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace q35
