// GatedDeltaNet decode update on CDNA4.
//
// One workgroup (256 threads) per (request, key head). The head's fp32 state
// tile [value_row][key_col] = 128 x 128 (64 KiB) makes exactly one HBM round
// trip: thread t holds the 16 float4 at flat offsets j*1024 + 4t (rows
// j*8 + t/32, columns 4*(t%32)..+3), so every load/store instruction of the
// workgroup covers 4 KiB contiguously, and each row's dot products reduce over
// the 32 lanes of a half wavefront.
//
// Per value row (src/cpu/delta_net.cpp:63-98):
//   S *= alpha;  sk = S.k;  delta = (v - sk) * beta;  S += delta * k;  o = S.q
// The fused variant also runs the rest of run_linear_attention_step
// (src/runtime/layers.inl:96-207) for its head: causal conv1d + SiLU over the
// q/k/v channels with the (kernel-1)-slot ring (activation.cpp:164-222), L2
// normalisation of q (x 1/sqrt(d_k)) and k, beta = sigmoid(b),
// alpha = exp(softplus(a + dt_bias) * -exp(A_log)), and the gated RMSNorm
// (offset 0) times SiLU(z). GQA heads (v_heads > k_heads) loop over the value
// heads sharing this key head, as the reference repeats q/k (layers.inl:130-144).
#include "q35_device.h"
#include "q35_internal.h"

namespace q35 {
namespace {

constexpr int kDeltaThreads = 256;

template <bool FUSED>
__global__ __launch_bounds__(kDeltaThreads) void delta_kernel(DeltaArgs a) {
  __shared__ float sq[128], sk[128], sv[128], so[128];
  __shared__ float scratch[8];
  __shared__ float s_alpha, s_beta;
  const int kh = blockIdx.x, r = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63;
  const int per = a.v_heads / a.k_heads;
  const int kd = a.kd, vd = a.vd;  // both 128 (checked by the launcher)
  float *state_r = a.state_base != nullptr
                       ? a.state_base + static_cast<long long>(a.slots[r]) * a.state_slot_stride
                       : a.states[r];

  const int q_dim = a.k_heads * kd, v_dim = a.v_heads * vd;
  const int channels = 2 * q_dim + v_dim;
  const float *prow = FUSED ? a.proj + static_cast<size_t>(r) * a.proj_stride : nullptr;
  float *conv = nullptr;
  int ring = 0, hist = a.kernel - 1;
  if constexpr (FUSED) {
    conv = a.conv_base + static_cast<long long>(a.slots[r]) * a.conv_slot_stride;
    ring = a.positions[r] % hist;
  }

  // causal conv1d + SiLU of one channel (batch 1), updating the ring slot
  auto conv_channel = [&](int ch) -> float {
    const float x = prow[ch];
    float sum = x * a.conv_w[static_cast<size_t>(hist) * channels + ch];
    for (int k = 0; k < hist; ++k) {
      const int slot = (ring + k) % hist;
      sum += conv[static_cast<size_t>(slot) * channels + ch] *
             a.conv_w[static_cast<size_t>(k) * channels + ch];
    }
    conv[static_cast<size_t>(ring) * channels + ch] = x;
    return silu_times(sum, 1.0F);
  };

  if constexpr (FUSED) {
    // threads 0..127: q channel, 128..255: k channel of this key head
    const int i = tid & 127;
    const bool is_k = tid >= 128;
    const int ch = (is_k ? q_dim : 0) + kh * kd + i;
    const float y = conv_channel(ch);
    // L2 norm per head over 128 values: each half of the block is two waves
    float ss = group_sum<64>(y * y);
    __syncthreads();
    if (lane == 0) scratch[tid >> 6] = ss;
    __syncthreads();
    ss = is_k ? scratch[2] + scratch[3] : scratch[0] + scratch[1];
    const float scale = is_k ? 1.0F : 1.0F / sqrtf(static_cast<float>(kd));
    const float m = scale / sqrtf(ss + 1.0e-6F);
    if (is_k)
      sk[i] = y * m;
    else
      sq[i] = y * m;
  }

  for (int vi = 0; vi < per; ++vi) {
    const int vh = kh * per + vi;
    if constexpr (FUSED) {
      if (tid < 128) sv[tid] = conv_channel(2 * q_dim + vh * vd + tid);
      if (tid == 0) {
        const float bval = prow[channels + v_dim + vh];
        const float aval = prow[channels + v_dim + a.v_heads + vh];
        s_beta = sigmoid_stable(bval);
        const float pre = softplus_stable(aval + a.dt_bias[vh]);
        s_alpha = expf(pre * a.ssm_a[vh]);
      }
    } else {
      const size_t qk = (static_cast<size_t>(r) * a.v_heads + vh) * kd;
      if (tid < 128) {
        sq[tid] = a.q[qk + tid];
        sk[tid] = a.k[qk + tid];
        sv[tid] = a.v[(static_cast<size_t>(r) * a.v_heads + vh) * vd + tid];
      }
      if (tid == 0) {
        s_alpha = a.alpha[static_cast<size_t>(r) * a.v_heads + vh];
        s_beta = a.beta[static_cast<size_t>(r) * a.v_heads + vh];
      }
    }
    float4 *S = reinterpret_cast<float4 *>(state_r + static_cast<size_t>(vh) * vd * kd);
    float4 st[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) st[j] = S[j * 256 + tid];
    __syncthreads();
    const float alpha = s_alpha, beta = s_beta;
    const int col = 4 * (tid & 31);
    const float4 kc = make_float4(sk[col], sk[col + 1], sk[col + 2], sk[col + 3]);
    const float4 qc = make_float4(sq[col], sq[col + 1], sq[col + 2], sq[col + 3]);
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      float4 s = st[j];
      s.x *= alpha; s.y *= alpha; s.z *= alpha; s.w *= alpha;
      float d = s.x * kc.x + s.y * kc.y + s.z * kc.z + s.w * kc.w;
      d = group_sum<32>(d);
      const int row = j * 8 + (tid >> 5);
      const float delta = (sv[row] - d) * beta;
      s.x += delta * kc.x; s.y += delta * kc.y; s.z += delta * kc.z; s.w += delta * kc.w;
      float e = s.x * qc.x + s.y * qc.y + s.z * qc.z + s.w * qc.w;
      e = group_sum<32>(e);
      st[j] = s;
      if ((tid & 31) == 0) so[row] = e;
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) S[j * 256 + tid] = st[j];
    __syncthreads();
    if constexpr (FUSED) {
      // gated RMSNorm (offset 0) over the head, then * SiLU(z)  (layers.inl:198-207)
      const float o = tid < 128 ? so[tid] : 0.0F;
      const float ss = block_sum<kDeltaThreads / 64>(o * o, scratch);
      if (tid < 128) {
        const float inv = 1.0F / sqrtf(ss / static_cast<float>(vd) + a.eps);
        const float y = o * inv * (a.norm_w[tid] + 0.0F);
        const float z = prow[channels + vh * vd + tid];
        a.out[static_cast<size_t>(r) * v_dim + vh * vd + tid] = silu_times(z, y);
      }
    } else {
      if (tid < 128) a.out[(static_cast<size_t>(r) * a.v_heads + vh) * vd + tid] = so[tid];
    }
    __syncthreads();
  }
}

}  // namespace

hipError_t launch_delta(const DeltaArgs &a, hipStream_t stream) {
  if (a.batch <= 0) return hipSuccess;
  if (a.kd != 128 || a.vd != 128 || a.v_heads % a.k_heads != 0) return hipErrorInvalidValue;
  const dim3 grid(a.k_heads, a.batch), block(kDeltaThreads);
  if (a.fused)
    Q35_LAUNCH((delta_kernel<true>), grid, block, 0, stream, a);
  else
    Q35_LAUNCH((delta_kernel<false>), grid, block, 0, stream, a);
  return hipGetLastError();
}

}  // namespace q35
