// extern "C" wrappers over the reference's own layer composition
// (src/runtime/layers.inl: run_linear_attention_step, prepare_full_attention_row
// + run_full_attention_step), built the way the reference's
// tests/head_runtime_test.cpp builds its runtime tests: this translation unit
// includes src/runtime/cpu_runtime.cpp and is linked with the other reference
// objects (oracle/Makefile, target "ref", oracle/_ref/libq35ref_layers.so).
// Test infrastructure only: it pins the oracle's restated layer steps
// (q35o_linear_attention_row / q35o_full_attention_row) to the reference's;
// never linked into, loaded by or measured as the MI355X product.
//
// Both entries run one row from a given projected row with return_core, so no
// projection weights are involved: the layer holds only the tensors the
// attention block reads. `backend` is the Q8_0Backend of the layer's output
// projection, which selects the kernels of the block (0 = auto_select).
#include "src/runtime/cpu_runtime.cpp"

#include <cstring>
#include <string>
#include <vector>

using namespace qwen35x;

namespace {

RuntimeDims layer_dims(int heads, int kv_heads, int head_dim, int rope_dim, float eps, int kernel, int k_heads,
                       int v_heads, int kdim, int vdim) {
  RuntimeDims d;
  d.n_heads = heads;
  d.n_kv_heads = kv_heads;
  d.head_dim = head_dim;
  d.rope_dim = rope_dim;
  d.rms_eps = eps;
  d.linear_kernel = kernel;
  d.linear_num_k_heads = k_heads;
  d.linear_num_v_heads = v_heads;
  d.linear_head_k_dim = kdim;
  d.linear_head_v_dim = vdim;
  d.linear_q_dim = k_heads * kdim;
  d.linear_v_dim = v_heads * vdim;
  d.linear_conv_channels = 2 * d.linear_q_dim + d.linear_v_dim;
  return d;
}

// A CPU-quantized placeholder, so that the block takes the tensor's backend
// (layers.inl:147-149) instead of auto_select.
void backend_tensor(TensorData &t, int backend) {
  t.q8_0_backend = static_cast<cpu::Q8_0Backend>(backend);
  t.packed_q4_0_blocks.resize(1);
}

}  // namespace

extern "C" {

// run_linear_attention_step (layers.inl:36-217) on one projected row
// [qkv | z | b | a]: conv_state [(kernel-1)][channels] and its ring index,
// recurrent [v_heads][vdim][kdim] are advanced in place; core receives the
// gated-norm output [v_heads * vdim]. conv_kernel_major is [kernel][channels]
// (pack_conv1d_kernel_major's layout). Returns 0, or 1 with the error copied.
int refl_linear_attention_row(int backend, int k_heads, int v_heads, int kdim, int vdim, int kernel, float eps,
                              const float *conv_kernel_major, const float *norm_w, const float *dt_bias,
                              const float *a_log, float *conv_state, std::size_t *ring, float *recurrent,
                              const float *projected, float *core, char *error, std::size_t error_size) {
  const RuntimeDims d = layer_dims(0, 0, 0, 0, eps, kernel, k_heads, v_heads, kdim, vdim);
  const std::size_t ch = static_cast<std::size_t>(d.linear_conv_channels);
  const std::size_t vdim_all = static_cast<std::size_t>(d.linear_v_dim);
  LayerWeights layer;
  layer.is_linear = true;
  layer.linear.conv1d_kernel_major.assign(conv_kernel_major, conv_kernel_major + static_cast<std::size_t>(kernel) * ch);
  layer.linear.norm.data.assign(norm_w, norm_w + vdim);
  layer.linear.dt_bias.data.assign(dt_bias, dt_bias + v_heads);
  // ssm_a = -exp(A_log) in FP32, as the loader forms it (weights.inl:1750-1754)
  for (int h = 0; h < v_heads; ++h) layer.linear.ssm_a.push_back(-std::exp(a_log[h]));
  backend_tensor(layer.linear.out_proj, backend);
  LinearAttentionState state;
  state.conv_state.assign(conv_state, conv_state + static_cast<std::size_t>(kernel - 1) * ch);
  state.recurrent_state.assign(recurrent, recurrent + static_cast<std::size_t>(v_heads) * vdim * kdim);
  state.conv_ring_index = *ring;
  const std::size_t n = ch + vdim_all + 2 * static_cast<std::size_t>(v_heads);
  std::vector<float> x, out;
  std::string err;
  if (!run_linear_attention_step(nullptr, layer, d, state, x, out, err, std::span<const float>(projected, n), true)) {
    std::strncpy(error, err.c_str(), error_size - 1);
    error[error_size - 1] = 0;
    return 1;
  }
  std::memcpy(core, out.data(), vdim_all * sizeof(float));
  std::memcpy(conv_state, state.conv_state.data(), state.conv_state.size() * sizeof(float));
  std::memcpy(recurrent, state.recurrent_state.data(), state.recurrent_state.size() * sizeof(float));
  *ring = state.conv_ring_index;
  return 0;
}

// prepare_full_attention_row + run_full_attention_step (layers.inl:221-395)
// on one projected row [q|gate interleaved per head | k | v] at `position`:
// keys/values [capacity][kv_heads * head_dim] binary16 hold positions
// 0..position-1 and receive row `position`; cosine/sine are the RoPE row of
// `position`; core receives the gated attention output [heads * head_dim].
int refl_full_attention_row(int backend, int heads, int kv_heads, int head_dim, int rope_dim, float eps,
                            const float *q_norm, const float *k_norm, std::uint16_t *keys, std::uint16_t *values,
                            std::size_t capacity, int position, const float *cosine, const float *sine,
                            const float *projected, float *core, char *error, std::size_t error_size) {
  const RuntimeDims d = layer_dims(heads, kv_heads, head_dim, rope_dim, eps, 0, 0, 0, 0, 0);
  const std::size_t kvw = static_cast<std::size_t>(kv_heads) * head_dim;
  LayerWeights layer;
  layer.full.q_norm.data.assign(q_norm, q_norm + head_dim);
  layer.full.k_norm.data.assign(k_norm, k_norm + head_dim);
  backend_tensor(layer.full.o_proj, backend);
  FullAttentionState state;
  state.k_cache_f16.assign(keys, keys + capacity * kvw);
  state.v_cache_f16.assign(values, values + capacity * kvw);
  const std::size_t n = static_cast<std::size_t>(heads + kv_heads) * head_dim * 2;
  std::vector<float> x, out;
  std::string err;
  if (!run_full_attention_step(nullptr, layer, d, state, x, position, cosine, sine, out, err,
                               std::span<const float>(projected, n), true)) {
    std::strncpy(error, err.c_str(), error_size - 1);
    error[error_size - 1] = 0;
    return 1;
  }
  std::memcpy(core, out.data(), static_cast<std::size_t>(heads) * head_dim * sizeof(float));
  const std::size_t at = static_cast<std::size_t>(position) * kvw;
  std::memcpy(keys + at, state.k_cache_f16.data() + at, kvw * sizeof(std::uint16_t));
  std::memcpy(values + at, state.v_cache_f16.data() + at, kvw * sizeof(std::uint16_t));
  return 0;
}

}  // extern "C"
