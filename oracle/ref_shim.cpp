// extern "C" wrappers over the reference CPU engine, compiled together with the
// reference sources (oracle/Makefile, target "ref") into oracle/_ref/. Test
// infrastructure only: used to produce golden vectors and to time the
// reference on the host cores beside the GPU run. Never linked into, loaded by
// or measured as the MI355X product.
//
// Every function forwards to the reference symbol named in its comment; the
// backend argument is the reference's Q8_0Backend enum value
// (include/qwen35x/cpu/q8_0.h:23-31), 0 = auto_select.
#include "qwen35x/cpu/activation.h"
#include "qwen35x/cpu/delta_net.h"
#include "qwen35x/cpu/executor.h"
#include "qwen35x/cpu/full_attention.h"
#include "qwen35x/cpu/q4_0.h"
#include "qwen35x/cpu/q4_dot4.h"
#include "qwen35x/cpu/q4_g16.h"
#include "qwen35x/cpu/q4_h128.h"
#include "qwen35x/cpu/q8_0.h"
#include "qwen35x/compiler/compiler.h"
#include "qwen35x/runtime/cpu_engine.h"
#include "q8_0_internal.h"

#include <chrono>
#include <cstdint>
#include <system_error>
#include <cstring>
#include <string>
#include <vector>

using namespace qwen35x;
using namespace qwen35x::cpu;


namespace {
Q8_0Backend be(int b) { return static_cast<Q8_0Backend>(b); }
}

extern "C" {

// q8_0.h:40-44
int ref_backend_resolve(int b) { return static_cast<int>(q8_0_resolve_backend(be(b))); }
const char *ref_backend_name(int b) { return q8_0_backend_name(be(b)); }

// q8_0.cpp:18 / :57
std::uint16_t ref_float_to_half(float v) { return detail::float_to_half(v); }
float ref_half_to_float(std::uint16_t v) { return detail::half_to_float(v); }

// q4_0.h:109-114 / :101-106
void ref_q8_0_quantize_vector_1(const float *x, void *out, std::size_t blocks, int b) {
  q8_0_quantize_vector_1(x, static_cast<Q8_0BlockX1 *>(out), blocks, be(b));
}
void ref_q8_0_quantize_vectors_4(const float *x, void *out, std::size_t vectors,
                                 std::size_t blocks, int b) {
  q8_0_quantize_vectors_4(x, static_cast<Q8_0BlockX4 *>(out), vectors, blocks, be(b));
}

// q4_h128.h:94-111
int ref_q4_h128_prepare_activation_1(const float *x, void *out, std::size_t cols,
                                     std::uint64_t seed, int b) {
  return q4_h128_prepare_activation_1(x, static_cast<Q8_0BlockX1 *>(out), cols, seed, be(b));
}
int ref_q4_h128_prepare_activations_4(const float *x, void *out, std::size_t vectors,
                                      std::size_t cols, std::uint64_t seed, int b) {
  return q4_h128_prepare_activations_4(x, static_cast<Q8_0BlockX4 *>(out), vectors, cols,
                                       seed, be(b));
}
// q4_h128.h:29-34 (scaled transform, scalar backend)
void ref_q4_h128_transform_block(const float *x, float *y, std::size_t index, std::uint64_t seed) {
  q4_h128_transform_block(x, y, index, seed, Q8_0Backend::scalar);
}
// q4_h128.h:73-78
int ref_q4_h128_quantize_matrix(const float *x, void *out, std::size_t rows, std::size_t cols,
                                std::uint64_t seed) {
  return q4_h128_quantize_matrix(x, static_cast<Q4_0Block *>(out), rows, cols, seed);
}
// q4_h128.h:66-70
void ref_q4_h128_quantize_transformed(const float *x, void *out, std::size_t blocks) {
  q4_h128_quantize_transformed(x, static_cast<Q4_0Block *>(out), blocks);
}

// q4_g16.h:10-25
void ref_q4_g16_dequantize_row(const void *w, std::size_t row, float *out, std::size_t blocks) {
  q4_g16_dequantize_row(static_cast<const Q4G16Tile *>(w), row, out, blocks);
}
void ref_q4_g16_matvec(const void *w, const void *a, float *out, std::size_t rows, std::size_t blocks, int b) {
  q4_g16_matvec(static_cast<const Q4G16Tile *>(w), static_cast<const Q8_0BlockX1 *>(a), out, rows, blocks, be(b));
}
void ref_q4_g16_pack_activations(const void *a, void *out, std::size_t count, std::size_t blocks) {
  q4_g16_pack_activations(static_cast<const Q8_0BlockX1 *>(a), static_cast<Q4G16ActivationTile *>(out), count,
                          blocks);
}
void ref_q4_g16_matmul(const void *w, const void *a, float *out, std::size_t rows, std::size_t count,
                       std::size_t blocks, std::size_t stride, int b) {
  q4_g16_matmul(static_cast<const Q4G16Tile *>(w), static_cast<const Q4G16ActivationTile *>(a), out, rows, count,
                blocks, stride, be(b));
}
// q8_0.h:115-125, matrix scales as run_q8_gate_tail passes them (weights.inl:1030-1032)
void ref_q8_0_matmul(const void *m, const void *v, float *out, std::size_t rows, std::size_t count,
                     std::size_t blocks, std::size_t stride, int b, const float *mscales) {
  q8_0_matmul(static_cast<const Q8_0Block *>(m), static_cast<const Q8_0Block *>(v), out, rows, count, blocks, stride,
              be(b), nullptr, mscales);
}

// q4_dot4.h:7-21
void ref_q4_dot4_pack_rows_8(const void *src, void *dst, std::size_t rows, std::size_t blocks) {
  q4_dot4_pack_rows_8(static_cast<const Q4_0Block *>(src), static_cast<Q4_0BlockX8 *>(dst),
                      rows, blocks);
}
void ref_q4_dot4_unpack_rows_8(const void *src, void *dst, std::size_t rows, std::size_t blocks) {
  q4_dot4_unpack_rows_8(static_cast<const Q4_0BlockX8 *>(src), static_cast<Q4_0Block *>(dst),
                        rows, blocks);
}
void ref_q4_dot4_dequantize_row(const void *m, std::size_t row, float *out, std::size_t blocks) {
  q4_dot4_dequantize_row(static_cast<const Q4_0BlockX8 *>(m), row, out, blocks);
}
void ref_q4_dot4_matvec(const void *m, const void *v, float *out, std::size_t rows,
                        std::size_t blocks, int b) {
  q4_dot4_matvec(static_cast<const Q4_0BlockX8 *>(m), static_cast<const Q8_0BlockX1 *>(v),
                 out, rows, blocks, be(b));
}
void ref_q4_dot4_matmul(const void *m, const void *v, float *out, std::size_t rows,
                        std::size_t count, std::size_t blocks, std::size_t stride, int b) {
  q4_dot4_matmul(static_cast<const Q4_0BlockX8 *>(m), static_cast<const Q8_0BlockX4 *>(v),
                 out, rows, count, blocks, stride, be(b));
}
void ref_q4_dot4_argmax(const void *m, const void *v, const int *counts, float penalty,
                        std::size_t offset, std::size_t rows, std::size_t blocks, int b,
                        float *value, std::uint64_t *index) {
  const auto r = q4_dot4_argmax(static_cast<const Q4_0BlockX8 *>(m),
                                static_cast<const Q8_0BlockX1 *>(v), counts, penalty, offset,
                                rows, blocks, be(b));
  *value = r.value;
  *index = r.index;
}

// delta_net.h:18-31
void ref_gated_delta_net_update_rows(float *state, const float *q, const float *k, const float *v,
                                     const float *alpha, const float *beta, float *out,
                                     std::size_t heads, std::size_t kdim, std::size_t vdim,
                                     std::size_t begin, std::size_t end, int b) {
  gated_delta_net_update_rows(state, q, k, v, alpha, beta, out, heads, kdim, vdim, begin, end,
                              be(b));
}

// full_attention.h:92-112 with AttentionKvRows (full_attention.h:10-20):
// key_rows/value_rows hold one FP16 [kv_heads*head_dim] row pointer per token.
void ref_causal_attention_decode_gqa_pairs(
    const float *q, const float *gates, const std::uint16_t *const *key_rows,
    const std::uint16_t *const *value_rows, float *scores, float *out, std::size_t context_stride,
    std::size_t query_width, std::size_t kv_width, int sequence_length, int heads, int kv_heads,
    int head_dim, float scale, std::size_t pair_begin, std::size_t pair_end, int b) {
  const AttentionKvRows pages{key_rows, value_rows};
  causal_attention_decode_gqa_pairs(q, gates, nullptr, nullptr, nullptr, nullptr, scores, out,
                                    context_stride, query_width, kv_width, sequence_length, heads,
                                    kv_heads, head_dim, scale, pair_begin, pair_end, be(b), &pages);
}
// full_attention.h:22-26
void ref_attention_cache_store_f16(const float *x, std::uint16_t *out, std::size_t n, int b) {
  attention_cache_store_f16(x, out, n, be(b));
}

// activation.h:9-77
void ref_add_f32(const float *a, const float *c, float *out, std::size_t n, int b) {
  add_f32(a, c, out, n, be(b));
}
void ref_rope_f32(float *x, std::size_t heads, std::size_t head_dim, std::size_t rope_dim,
                  const float *cosine, const float *sine, int b) {
  rope_f32(x, heads, head_dim, rope_dim, cosine, sine, be(b));
}
void ref_causal_conv1d_silu_f32(float *state, std::size_t ring, const float *input,
                                std::size_t input_stride, const float *weights, float *out,
                                std::size_t batch, std::size_t channels, std::size_t kernel,
                                int b) {
  causal_conv1d_silu_f32(state, ring, input, input_stride, weights, out, batch, channels, kernel, 0,
                         channels, be(b));
}
void ref_rms_norm_f32(const float *x, const float *w, float *out, std::size_t rows,
                      std::size_t width, float eps, float offset, int b) {
  rms_norm_f32(x, w, out, rows, width, eps, offset, be(b));
}
void ref_l2_normalize_f32(float *x, std::size_t rows, std::size_t width, float eps, float scale,
                          int b) {
  l2_normalize_f32(x, rows, width, eps, scale, be(b));
}
void ref_silu_mul_f32(const float *g, const float *u, float *out, std::size_t n, int b) {
  silu_mul_f32(g, u, out, n, be(b));
}

// Optional logit probes for the next ref_engine_greedy call with logits
// capture: the raw logits at `count` fixed vocabulary indices of every (row,
// step) go to values[row][step][count]. Cleared by passing count 0.
static const std::int32_t *g_probe_index = nullptr;
static std::size_t g_probe_count = 0;
static float *g_probe_values = nullptr;
void ref_engine_set_probe(const std::int32_t *index, std::size_t count, float *values) {
  g_probe_index = index;
  g_probe_count = count;
  g_probe_values = values;
}

// Greedy decode through the reference engine (cpu_engine.h:173-215), the way
// src/cpu_engine_bench_main.cpp:241-301 drives it: every request is prefilled
// with advance(), then advance_batch() runs until all requests complete.
// prompts is [batch][prompt_len]. out_tokens is [batch][new_tokens]. When
// top_values/top_index are non-null, a logits callback records the 8 largest
// raw logits of every (row, step) into [batch][new_tokens][8] (the callback
// makes the engine take its full-logits path, cpu_engine.inl:307-321).
// backend is the Q8_0Backend of every kernel (q8_0.h:23-31; 0 = auto_select).
// forced, when non-null, is [batch][new_tokens]: the rows' forced_output_tokens
// (cpu_engine.h:108; every output is forced and logits are still reported),
// which teacher-forces a fixed token sequence through the decode path.
// Returns 0 on success; the error text is copied into error[error_size].
int ref_engine_greedy(const char *model_dir, const char *artifact, int threads, int backend,
                      const std::int32_t *prompts, std::size_t prompt_len, std::size_t batch,
                      std::size_t new_tokens, float penalty, const std::int32_t *forced,
                      std::int32_t *out_tokens,
                      float *top_values, std::int32_t *top_index, double *decode_ms,
                      char *error, std::size_t error_size) {
  std::string err;
  auto fail = [&](const std::string &message) {
    if (error && error_size) {
      std::strncpy(error, message.c_str(), error_size - 1);
      error[error_size - 1] = 0;
    }
    return 1;
  };
  auto profile = ProfileLoader::load_from_hf_directory(model_dir, err);
  if (!profile) return fail(err);
  CpuLoadOptions options;
  options.model_dir = model_dir;
  options.cpu_q4_h128_path = artifact;
  options.cpu_q8_backend = be(backend);  // options.h:17; 0 = auto_select
  auto model = CpuModel::load(*profile, options, err);
  if (!model) return fail(err);
  CpuEngineConfig config;
  config.threads = threads;
  config.max_resident_requests = batch;
  config.max_context = prompt_len + new_tokens + 8;
  auto engine = CpuEngine::create(model, config, err);
  if (!engine) return fail(err);
  struct Capture {
    float *values;
    std::int32_t *index;
    std::size_t new_tokens, row;
  };
  std::vector<Capture> captures(batch);
  auto callback = [](void *opaque, std::size_t step, std::int32_t, const float *logits,
                     std::size_t count, std::string &) -> bool {
    auto &c = *static_cast<Capture *>(opaque);
    float best[8];
    std::int32_t at[8];
    for (int i = 0; i < 8; ++i) best[i] = -3.0e38F, at[i] = -1;
    for (std::size_t t = 0; t < count; ++t) {
      if (!(logits[t] > best[7])) continue;
      int p = 7;
      while (p > 0 && logits[t] > best[p - 1]) {
        best[p] = best[p - 1];
        at[p] = at[p - 1];
        --p;
      }
      best[p] = logits[t];
      at[p] = static_cast<std::int32_t>(t);
    }
    std::memcpy(c.values + (c.row * c.new_tokens + step) * 8, best, sizeof(best));
    if (g_probe_count != 0) {
      float *dst = g_probe_values + (c.row * c.new_tokens + step) * g_probe_count;
      for (std::size_t i = 0; i < g_probe_count; ++i) dst[i] = logits[g_probe_index[i]];
    }
    std::memcpy(c.index + (c.row * c.new_tokens + step) * 8, at, sizeof(at));
    return true;
  };
  std::vector<CpuRequestId> ids;
  for (std::size_t r = 0; r < batch; ++r) {
    CpuRequestSpec spec;
    spec.prompt_tokens.assign(prompts + r * prompt_len, prompts + (r + 1) * prompt_len);
    spec.max_new_tokens = new_tokens;
    spec.sampling.temperature = 0.0F;
    spec.sampling.repetition_penalty = penalty;
    if (forced != nullptr)
      spec.forced_output_tokens.assign(forced + r * new_tokens, forced + (r + 1) * new_tokens);
    if (top_values && top_index) {
      captures[r] = Capture{top_values, top_index, new_tokens, r};
      spec.logits_callback = callback;
      spec.logits_callback_context = &captures[r];
    }
    const auto id = engine->submit(std::move(spec), err);
    if (!id) return fail(err);
    ids.push_back(id);
    CpuRequestResult state;
    do {
      if (!engine->advance(id, err) || !engine->result(id, state)) return fail(err);
    } while (state.status == CpuRequestStatus::prefill);
  }
  std::vector<CpuRequestId> active = ids;
  const auto start = std::chrono::steady_clock::now();
  while (!active.empty()) {
    if (!engine->advance_batch(active, err)) return fail(err);
    std::vector<CpuRequestId> next;
    for (auto id : active) {
      CpuRequestResult state;
      engine->result(id, state);
      if (state.status == CpuRequestStatus::decode) next.push_back(id);
    }
    active.swap(next);
  }
  if (decode_ms)
    *decode_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - start)
                     .count();
  for (std::size_t r = 0; r < batch; ++r) {
    CpuRequestResult state;
    engine->result(ids[r], state);
    if (state.output_tokens.size() != new_tokens) return fail("short output");
    std::memcpy(out_tokens + r * new_tokens, state.output_tokens.data(),
                new_tokens * sizeof(std::int32_t));
  }
  return 0;
}

// Sampled decode of one request through the reference engine: the request's
// SamplingOptions (options.h:10-13, seed >= 0 seeds its mt19937,
// cpu_engine.inl:379-381), a logits callback (cpu_engine.h:119-121) copying
// every raw logits row into logits[new_tokens][vocab], and the sampled tokens
// into out_tokens[new_tokens] (sample_token_from_logits, layers.inl:491-600,
// through select, cpu_engine.inl:441-487). Returns 0, or 1 with the error.
int ref_engine_sample(const char *model_dir, const char *artifact, int threads, const std::int32_t *prompt,
                      std::size_t prompt_len, std::size_t new_tokens, float temperature, float top_p, int top_k,
                      float penalty, std::int64_t seed, std::int32_t *out_tokens, float *logits, std::size_t vocab,
                      char *error, std::size_t error_size) {
  std::string err;
  auto fail = [&](const std::string &message) {
    if (error && error_size) {
      std::strncpy(error, message.c_str(), error_size - 1);
      error[error_size - 1] = 0;
    }
    return 1;
  };
  auto profile = ProfileLoader::load_from_hf_directory(model_dir, err);
  if (!profile) return fail(err);
  CpuLoadOptions options;
  options.model_dir = model_dir;
  options.cpu_q4_h128_path = artifact;
  auto model = CpuModel::load(*profile, options, err);
  if (!model) return fail(err);
  CpuEngineConfig config;
  config.threads = threads;
  config.max_resident_requests = 1;
  config.max_context = prompt_len + new_tokens + 8;
  auto engine = CpuEngine::create(model, config, err);
  if (!engine) return fail(err);
  struct Capture {
    float *logits;
    std::size_t vocab;
  } capture{logits, vocab};
  auto callback = [](void *opaque, std::size_t step, std::int32_t, const float *row, std::size_t count,
                     std::string &) -> bool {
    auto &c = *static_cast<Capture *>(opaque);
    if (count != c.vocab) return false;
    std::memcpy(c.logits + step * c.vocab, row, count * sizeof(float));
    return true;
  };
  CpuRequestSpec spec;
  spec.prompt_tokens.assign(prompt, prompt + prompt_len);
  spec.max_new_tokens = new_tokens;
  spec.sampling.temperature = temperature;
  spec.sampling.top_p = top_p;
  spec.sampling.top_k = top_k;
  spec.sampling.repetition_penalty = penalty;
  spec.sampling.seed = seed;
  spec.logits_callback = callback;
  spec.logits_callback_context = &capture;
  const auto id = engine->submit(std::move(spec), err);
  if (!id) return fail(err);
  CpuRequestResult state;
  do {
    if (!engine->advance(id, err) || !engine->result(id, state)) return fail(err);
  } while (state.status == CpuRequestStatus::prefill || state.status == CpuRequestStatus::decode);
  if (state.status != CpuRequestStatus::complete || state.output_tokens.size() != new_tokens)
    return fail("incomplete sampled output: " + state.error);
  std::memcpy(out_tokens, state.output_tokens.data(), new_tokens * sizeof(std::int32_t));
  return 0;
}

// ---- configs 1-3 on all cores: the reference's kernels under its own
// CpuExecutor (executor.h:40-77), partitioned as the engine partitions them:
// 8-row DOT4 tiles for the projections (matmul_2d_quantized_batch,
// weights.inl:1297-1502), requests for the DeltaNet update (state_batch,
// cpu_engine_state_batch.inl), requests x query-head pairs for attention.
void *ref_executor_create(std::size_t threads) {
  CpuExecutorConfig c;
  c.thread_count = threads;
  c.min_parallel_rows = 1;
  std::error_code ec;
  auto e = CpuExecutor::create(c, ec);
  return ec ? nullptr : e.release();
}
void ref_executor_destroy(void *e) { delete static_cast<CpuExecutor *>(e); }
std::size_t ref_executor_threads(void *e) { return static_cast<CpuExecutor *>(e)->thread_count(); }

// q4_dot4_matvec (count 1, X1 vector) or q4_dot4_matmul (X4 vectors,
// token-major output of stride `rows`) over the tiles of `rows` rows.
int ref_par_q4_dot4(void *exec, const void *m, const void *v, float *out, std::size_t rows, std::size_t count,
                    std::size_t blocks, int b) {
  struct Job {
    const Q4_0BlockX8 *m;
    const void *v;
    float *out;
    std::size_t rows, count, blocks;
    Q8_0Backend b;
  } job{static_cast<const Q4_0BlockX8 *>(m), v, out, rows, count, blocks, be(b)};
  auto task = [](void *ctx, std::size_t t0, std::size_t t1) noexcept {
    const auto &j = *static_cast<const Job *>(ctx);
    const Q4_0BlockX8 *tile = j.m + t0 * j.blocks;
    if (j.count == 1)
      q4_dot4_matvec(tile, static_cast<const Q8_0BlockX1 *>(j.v), j.out + 8 * t0, 8 * (t1 - t0), j.blocks, j.b);
    else
      q4_dot4_matmul(tile, static_cast<const Q8_0BlockX4 *>(j.v), j.out + 8 * t0, 8 * (t1 - t0), j.count, j.blocks,
                     j.rows, j.b);
  };
  return static_cast<CpuExecutor *>(exec)->parallel_for_rows(rows / 8, task, &job) == CpuExecutorStatus::ok ? 0 : 1;
}

// gated_delta_net_update_rows over every value row of each request; the
// request's state is states[r], its q/k [heads][kdim], v/out [heads][vdim],
// alpha/beta [heads] at offset r.
int ref_par_delta(void *exec, float *const *states, const float *q, const float *k, const float *v,
                  const float *alpha, const float *beta, float *out, std::size_t batch, std::size_t heads,
                  std::size_t kdim, std::size_t vdim, int b) {
  struct Job {
    float *const *states;
    const float *q, *k, *v, *alpha, *beta;
    float *out;
    std::size_t heads, kdim, vdim;
    Q8_0Backend b;
  } job{states, q, k, v, alpha, beta, out, heads, kdim, vdim, be(b)};
  auto task = [](void *ctx, std::size_t r0, std::size_t r1) noexcept {
    const auto &j = *static_cast<const Job *>(ctx);
    for (std::size_t r = r0; r < r1; ++r)
      gated_delta_net_update_rows(j.states[r], j.q + r * j.heads * j.kdim, j.k + r * j.heads * j.kdim,
                                  j.v + r * j.heads * j.vdim, j.alpha + r * j.heads, j.beta + r * j.heads,
                                  j.out + r * j.heads * j.vdim, j.heads, j.kdim, j.vdim, 0, j.heads * j.vdim, j.b);
  };
  return static_cast<CpuExecutor *>(exec)->parallel_for_rows(batch, task, &job) == CpuExecutorStatus::ok ? 0 : 1;
}

// causal_attention_decode_gqa_pairs per (request, query-head pair): request
// r's q/gates/out rows at r * heads * head_dim, its K/V row pointers
// key_rows[r] / value_rows[r], context lens[r]; scores is
// [batch * pairs][context_stride * heads] (one private buffer per item).
int ref_par_attention(void *exec, const float *q, const float *gates, const std::uint16_t *const *const *key_rows,
                      const std::uint16_t *const *const *value_rows, const int *lens, float *scores, float *out,
                      std::size_t batch, std::size_t context_stride, int heads, int kv_heads, int head_dim,
                      float scale, int b) {
  struct Job {
    const float *q, *gates;
    const std::uint16_t *const *const *keys, *const *const *values;
    const int *lens;
    float *scores, *out;
    std::size_t stride, pairs;
    int heads, kv_heads, head_dim;
    float scale;
    Q8_0Backend b;
  } job{q, gates, key_rows, value_rows, lens, scores, out, context_stride, static_cast<std::size_t>(heads) / 2,
        heads, kv_heads, head_dim, scale, be(b)};
  auto task = [](void *ctx, std::size_t i0, std::size_t i1) noexcept {
    const auto &j = *static_cast<const Job *>(ctx);
    const std::size_t width = static_cast<std::size_t>(j.heads) * j.head_dim;
    for (std::size_t i = i0; i < i1; ++i) {
      const std::size_t r = i / j.pairs, p = i % j.pairs;
      const AttentionKvRows pages{j.keys[r], j.values[r]};
      causal_attention_decode_gqa_pairs(j.q + r * width, j.gates + r * width, nullptr, nullptr, nullptr, nullptr,
                                        j.scores + i * j.stride * j.heads, j.out + r * width, j.stride, width,
                                        static_cast<std::size_t>(j.kv_heads) * j.head_dim, j.lens[r], j.heads,
                                        j.kv_heads, j.head_dim, j.scale, p, p + 1, j.b, &pages);
    }
  };
  return static_cast<CpuExecutor *>(exec)->parallel_for_rows(batch * job.pairs, task, &job) == CpuExecutorStatus::ok
             ? 0 : 1;
}

// Config 5 on the reference engine, which cannot put decode rows and a
// prompt chunk in one step (cpu_engine_scheduler.inl:64-80): `rows` requests
// with decode_len-token prompts are prefilled (untimed); one advance_batch of
// all of them is timed (max_decode_batch_size = rows); then a
// prefill_len-token prompt is prefilled through advance() with
// prefill_chunk_size = chunk, timed, calls counted. Greedy, no penalty.
int ref_engine_mixed(const char *model_dir, const char *artifact, int threads, const std::int32_t *decode_prompts,
                     std::size_t decode_len, std::size_t rows, const std::int32_t *prompt, std::size_t prefill_len,
                     std::size_t chunk, double *decode_ms, double *prefill_ms, std::size_t *prefill_calls,
                     char *error, std::size_t error_size) {
  std::string err;
  auto fail = [&](const std::string &message) {
    if (error && error_size) {
      std::strncpy(error, message.c_str(), error_size - 1);
      error[error_size - 1] = 0;
    }
    return 1;
  };
  auto profile = ProfileLoader::load_from_hf_directory(model_dir, err);
  if (!profile) return fail(err);
  CpuLoadOptions options;
  options.model_dir = model_dir;
  options.cpu_q4_h128_path = artifact;
  auto model = CpuModel::load(*profile, options, err);
  if (!model) return fail(err);
  CpuEngineConfig config;
  config.threads = threads;
  config.max_resident_requests = rows + 1;
  config.max_decode_batch_size = rows;
  config.prefill_chunk_size = chunk;
  config.max_context = std::max(decode_len, prefill_len) + 8;
  auto engine = CpuEngine::create(model, config, err);
  if (!engine) return fail(err);
  auto submit = [&](const std::int32_t *tokens, std::size_t n, std::size_t new_tokens) -> CpuRequestId {
    CpuRequestSpec spec;
    spec.prompt_tokens.assign(tokens, tokens + n);
    spec.max_new_tokens = new_tokens;
    spec.sampling.temperature = 0.0F;
    spec.sampling.repetition_penalty = 1.0F;
    return engine->submit(std::move(spec), err);
  };
  std::vector<CpuRequestId> ids;
  for (std::size_t r = 0; r < rows; ++r) {
    const auto id = submit(decode_prompts + r * decode_len, decode_len, 2);
    if (!id) return fail(err);
    CpuRequestResult state;
    do {
      if (!engine->advance(id, err) || !engine->result(id, state)) return fail(err);
    } while (state.status == CpuRequestStatus::prefill);
    ids.push_back(id);
  }
  auto t0 = std::chrono::steady_clock::now();
  if (!engine->advance_batch(ids, err)) return fail(err);
  *decode_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
  const auto id = submit(prompt, prefill_len, 1);
  if (!id) return fail(err);
  std::size_t calls = 0;
  CpuRequestResult state;
  t0 = std::chrono::steady_clock::now();
  do {
    if (!engine->advance(id, err) || !engine->result(id, state)) return fail(err);
    ++calls;
  } while (state.status == CpuRequestStatus::prefill);
  *prefill_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
  *prefill_calls = calls;
  return 0;
}

}  // extern "C"
