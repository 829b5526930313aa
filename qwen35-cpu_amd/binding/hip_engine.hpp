// Reference-side binding: the public interface of qwen35x::CpuModel and
// qwen35x::CpuEngine (include/qwen35x/runtime/cpu_engine.h:11-26, 173-215) on
// the MI355X backend's C ABI (include/q35_hip.h). Header-only C++20; include it
// from code built against the reference's include/ directory and link
// libq35hip.so. The request, result, config and stats types are the
// reference's own, so a caller swaps qwen35x::CpuModel / CpuEngine for
// qwen35x::hip::HipModel / HipEngine and keeps the rest of its code.
//
// Both engine modes are the reference's: direct mode (advance /
// advance_batch) and, with CpuEngineConfig::max_queued_requests > 0, serving
// mode (step / read_output, max_buffered_tokens, automatic prefixes through
// CpuRequestSpec::register_prefix_tokens and trust_namespace).
//
// Differences, each reported as an error rather than ignored:
// - CpuPrefix has a private constructor, so prefixes are HipPrefix handles
//   (register_prefix / find_prefix return them; submit takes one beside the
//   spec) instead of CpuRequestSpec::prefix;
// - drafting (draft_mode, mtp_max_tokens > 1) and the CPU executor knobs
//   (threads, spin counts, KV bit widths) have no counterpart.
#pragma once

#include "q35_hip.h"
#include "qwen35x/runtime/cpu_engine.h"

#include <algorithm>
#include <cstdint>
#include <map>
#include <memory>
#include <span>
#include <string>
#include <utility>
#include <vector>

namespace qwen35x::hip {

// CpuModel::load (cpu_engine.h:14-17): the Q35H128 artifact named by
// CpuLoadOptions::cpu_q4_h128_path, uploaded to one GPU as it is.
class HipModel final {
 public:
  static std::shared_ptr<const HipModel> load(const ModelProfile &profile, const CpuLoadOptions &options,
                                              std::string &error, int device = 0) {
    const TextModelConfig &t = profile.text;
    const auto &schedule = profile.fingerprint.attention_schedule;
    if (options.cpu_q4_h128_path.empty()) {
      error = "HIP backend: cpu_q4_h128_path must name a Q35H128 artifact.";
      return nullptr;
    }
    if (schedule.size() != static_cast<std::size_t>(t.num_hidden_layers)) {
      error = "HIP backend: the profile's attention schedule does not cover every layer.";
      return nullptr;
    }
    q35_model_dims d{};
    d.n_layers = t.num_hidden_layers;
    d.hidden = t.hidden_size;
    d.intermediate = t.intermediate_size;
    d.vocab = t.vocab_size;
    d.n_heads = t.num_attention_heads;
    d.n_kv_heads = t.num_key_value_heads;
    d.head_dim = t.head_dim;
    // rotary width as the reference derives it (weights.inl:1580-1583)
    d.rope_dim = static_cast<int32_t>(static_cast<float>(t.head_dim) * t.partial_rotary_factor);
    if (d.rope_dim % 2 != 0) d.rope_dim -= 1;
    d.rope_theta = t.rope_theta;
    d.rms_eps = t.rms_norm_eps;
    d.lin_kernel = t.linear_conv_kernel_dim;
    d.lin_k_heads = t.linear_num_key_heads;
    d.lin_v_heads = t.linear_num_value_heads;
    d.lin_k_dim = t.linear_key_head_dim;
    d.lin_v_dim = t.linear_value_head_dim;
    d.sign_seed = 0;  // the artifact header's
    std::vector<uint8_t> linear(schedule.size());
    for (std::size_t i = 0; i < schedule.size(); ++i) linear[i] = schedule[i] == AttentionBlock::linear ? 1 : 0;
    std::shared_ptr<HipModel> m(new HipModel());
    if (q35_context_create(device, nullptr, &m->ctx_) != Q35_OK) {
      error = "HIP backend: no usable GPU.";
      return nullptr;
    }
    if (q35_model_load_artifact(m->ctx_, options.cpu_q4_h128_path.c_str(), &d, linear.data(), &m->model_) != Q35_OK) {
      error = std::string("HIP backend: ") + q35_context_last_error(m->ctx_);
      return nullptr;
    }
    return m;
  }
  ~HipModel() {
    if (model_ != nullptr) q35_model_destroy(model_);
    if (ctx_ != nullptr) q35_context_destroy(ctx_);
  }
  HipModel(const HipModel &) = delete;
  HipModel &operator=(const HipModel &) = delete;
  q35_model *handle() const noexcept { return model_; }
  const char *last_error() const noexcept { return q35_context_last_error(ctx_); }

 private:
  HipModel() = default;
  q35_context *ctx_ = nullptr;
  q35_model *model_ = nullptr;
};

namespace detail {
// Owns the backend engine; prefix handles share it, so the engine outlives
// every handle that pins one of its snapshots.
struct EngineHandle {
  std::shared_ptr<const HipModel> model;
  q35_engine *engine = nullptr;
  ~EngineHandle() {
    if (engine != nullptr) q35_engine_destroy(engine);
  }
};

// One request's callbacks and constraint, in the C ABI's form. Lives until
// the request is released, as CpuRequestSpec's callback contexts must.
struct RequestGlue {
  ReferenceLogitsCallback logits = nullptr;
  void *logits_context = nullptr;
  ReferenceLogitsCallback selected = nullptr;
  void *selected_context = nullptr;
  std::shared_ptr<CpuSamplingConstraint> constraint;
  q35_sampling_constraint c_constraint{};
  std::size_t max_new_tokens = 0;
  std::string error;  // the first error a callback or the constraint reported
};

inline int logits_trampoline(void *context, std::size_t index, int32_t forced, const float *logits,
                             std::size_t count) {
  auto *g = static_cast<RequestGlue *>(context);
  return g->logits(g->logits_context, index, forced, logits, count, g->error) ? 1 : 0;
}
inline int selected_trampoline(void *context, std::size_t index, int32_t forced, const float *logits,
                               std::size_t count) {
  auto *g = static_cast<RequestGlue *>(context);
  return g->selected(g->selected_context, index, forced, logits, count, g->error) ? 1 : 0;
}
inline int constraint_apply(void *context, float *logits, std::size_t count) {
  auto *g = static_cast<RequestGlue *>(context);
  return g->constraint->apply(logits, count, g->error) ? 1 : 0;
}
inline int constraint_accept(void *context, int32_t token) {
  auto *g = static_cast<RequestGlue *>(context);
  return g->constraint->accept(token, g->error) ? 1 : 0;
}

inline CpuRequestStatus to_status(int32_t s) {
  switch (s) {
    case Q35_REQ_PREFILL: return CpuRequestStatus::prefill;
    case Q35_REQ_DECODE: return CpuRequestStatus::decode;
    case Q35_REQ_COMPLETE: return CpuRequestStatus::complete;
    case Q35_REQ_CANCELLED: return CpuRequestStatus::cancelled;
    case Q35_REQ_QUEUED: return CpuRequestStatus::queued;
    default: return CpuRequestStatus::failed;
  }
}
}  // namespace detail

// A cached prefix snapshot (CpuPrefix's role): pins it until destroyed.
class HipPrefix final {
 public:
  ~HipPrefix() {
    if (id_ != 0) q35_engine_release_prefix(owner_->engine, id_);
  }
  HipPrefix(const HipPrefix &) = delete;
  HipPrefix &operator=(const HipPrefix &) = delete;
  std::size_t token_count() const noexcept { return tokens_; }
  uint64_t id() const noexcept { return id_; }

 private:
  friend class HipEngine;
  HipPrefix(std::shared_ptr<detail::EngineHandle> owner, uint64_t id, std::size_t tokens)
      : owner_(std::move(owner)), id_(id), tokens_(tokens) {}
  std::shared_ptr<detail::EngineHandle> owner_;
  uint64_t id_ = 0;
  std::size_t tokens_ = 0;
};

// CpuEngine (cpu_engine.h:173-215) on the MI355X backend.
class HipEngine final {
 public:
  static std::unique_ptr<HipEngine> create(std::shared_ptr<const HipModel> model, const CpuEngineConfig &config,
                                           std::string &error, bool packed_steps = false) {
    if (model == nullptr) {
      error = "HIP backend: no model.";
      return nullptr;
    }
    if (config.mtp_max_tokens > 1) {
      error = "HIP backend: MTP drafting is not supported.";
      return nullptr;
    }
    if (config.max_queued_requests > static_cast<std::size_t>(INT32_MAX) ||
        config.max_buffered_tokens > static_cast<std::size_t>(INT32_MAX)) {
      error = "Invalid CPU engine configuration.";
      return nullptr;
    }
    q35_engine_config c{};
    c.max_resident_requests = static_cast<int32_t>(config.max_resident_requests);
    c.max_context = static_cast<int32_t>(config.max_context);
    c.max_decode_batch_size = static_cast<int32_t>(config.max_decode_batch_size);
    c.prefill_chunk_size = static_cast<int32_t>(config.prefill_chunk_size);  // 0: the backend's default
    c.page_tokens = 16;
    c.use_graphs = 1;
    c.max_prefix_bytes = config.max_prefix_bytes;
    c.max_prefill_requests = static_cast<int32_t>(config.max_prefill_requests);
    c.packed_steps = packed_steps ? 1 : 0;
    c.max_queued_requests = static_cast<int32_t>(config.max_queued_requests);
    c.max_buffered_tokens = static_cast<int32_t>(config.max_buffered_tokens);
    auto owner = std::make_shared<detail::EngineHandle>();
    owner->model = std::move(model);
    if (q35_engine_create(owner->model->handle(), &c, &owner->engine) != Q35_OK) {
      error = std::string("HIP backend: ") + owner->model->last_error();
      return nullptr;
    }
    return std::unique_ptr<HipEngine>(new HipEngine(std::move(owner)));
  }

  HipEngine(const HipEngine &) = delete;
  HipEngine &operator=(const HipEngine &) = delete;

  // CpuEngine::submit; `prefix` takes the place of CpuRequestSpec::prefix.
  CpuRequestId submit(CpuRequestSpec spec, std::string &error, std::shared_ptr<const HipPrefix> prefix = nullptr) {
    if (spec.prefix != nullptr || spec.draft_mode != CpuDraftMode::off) {
      error = "HIP backend: use a HipPrefix handle; drafting is not supported.";
      return 0;
    }
    auto glue = std::make_unique<detail::RequestGlue>();
    glue->logits = spec.logits_callback;
    glue->logits_context = spec.logits_callback_context;
    glue->selected = spec.selected_logits_callback;
    glue->selected_context = spec.selected_logits_callback_context;
    glue->constraint = spec.sampling_constraint;
    glue->max_new_tokens = spec.max_new_tokens;
    std::vector<int32_t> stops;
    std::vector<std::size_t> stop_lengths;
    for (const auto &s : spec.stop_token_sequences) {
      stops.insert(stops.end(), s.begin(), s.end());
      stop_lengths.push_back(s.size());
    }
    q35_request_spec r{};
    r.prompt_tokens = spec.prompt_tokens.data();
    r.prompt_count = spec.prompt_tokens.size();
    r.max_new_tokens = spec.max_new_tokens;
    r.temperature = spec.sampling.temperature;
    r.top_p = spec.sampling.top_p;
    r.top_k = spec.sampling.top_k;
    r.repetition_penalty = spec.sampling.repetition_penalty;
    r.seed = spec.sampling.seed;
    r.stop_token_ids = spec.stop_token_ids.data();
    r.stop_count = spec.stop_token_ids.size();
    r.stop_sequences = stops.data();
    r.stop_sequence_lengths = stop_lengths.data();
    r.stop_sequence_count = stop_lengths.size();
    r.forced_output_tokens = spec.forced_output_tokens.data();
    r.forced_count = spec.forced_output_tokens.size();
    if (glue->logits != nullptr) {
      r.logits_callback = detail::logits_trampoline;
      r.logits_callback_context = glue.get();
    }
    if (glue->selected != nullptr) {
      r.selected_logits_callback = detail::selected_trampoline;
      r.selected_logits_callback_context = glue.get();
    }
    r.selected_logit_tokens = spec.selected_logit_tokens.data();
    r.selected_logit_count = spec.selected_logit_tokens.size();
    if (glue->constraint != nullptr) {
      glue->c_constraint = q35_sampling_constraint{glue.get(), detail::constraint_apply, detail::constraint_accept};
      r.sampling_constraint = &glue->c_constraint;
    }
    r.prefix = prefix != nullptr ? prefix->id() : 0;
    r.register_prefix_tokens = spec.register_prefix_tokens;
    r.trust_namespace = spec.trust_namespace.c_str();
    uint64_t id = 0;
    if (q35_engine_submit_spec(owner_->engine, &r, &id) != Q35_OK) {
      error = q35_engine_last_error(owner_->engine);
      return 0;
    }
    glue_[id] = std::move(glue);
    return id;
  }

  // CpuEngine::register_prefix / find_prefix (cpu_engine.h:181-193).
  std::shared_ptr<const HipPrefix> register_prefix(std::span<const std::int32_t> tokens, std::string trust_namespace,
                                                   std::string &error) {
    uint64_t h = 0;
    if (q35_engine_register_prefix(owner_->engine, tokens.data(), tokens.size(), trust_namespace.c_str(), &h) !=
        Q35_OK) {
      error = q35_engine_last_error(owner_->engine);
      return nullptr;
    }
    return std::shared_ptr<const HipPrefix>(new HipPrefix(owner_, h, tokens.size()));
  }
  std::shared_ptr<const HipPrefix> find_prefix(std::span<const std::int32_t> tokens,
                                               const std::string &trust_namespace) {
    uint64_t h = 0;
    std::size_t n = 0;
    if (q35_engine_find_prefix(owner_->engine, tokens.data(), tokens.size(), trust_namespace.c_str(), &h, &n) !=
            Q35_OK ||
        h == 0)
      return nullptr;
    return std::shared_ptr<const HipPrefix>(new HipPrefix(owner_, h, n));
  }

  bool advance(CpuRequestId id, std::string &error) { return check(q35_engine_advance(owner_->engine, id), error); }
  bool advance_batch(std::span<const CpuRequestId> ids, std::string &error) {
    const std::vector<uint64_t> v(ids.begin(), ids.end());
    return check(q35_engine_advance_batch(owner_->engine, v.data(), v.size()), error);
  }
  bool step(bool &progressed, std::string &error) {
    int32_t p = 0;
    const bool ok = check(q35_engine_step(owner_->engine, &p), error);
    progressed = p != 0;
    return ok;
  }
  // CpuEngine::read_output (cpu_engine.h:197-201): appends to `output`.
  bool read_output(CpuRequestId id, std::size_t max_tokens, std::vector<std::int32_t> &output, std::string &error) {
    // at most every output token of the request is unread
    std::size_t total = 0;
    if (q35_engine_result(owner_->engine, id, nullptr, nullptr, 0, &total) == Q35_OK)
      max_tokens = std::min(max_tokens, total);
    const std::size_t at = output.size();
    std::size_t n = 0;
    output.resize(at + max_tokens);
    const bool ok = check(q35_engine_read_output(owner_->engine, id, max_tokens, output.data() + at, &n), error);
    output.resize(at + (ok ? n : 0));
    return ok;
  }

  CpuEngineStats stats() const {
    CpuEngineStats out{};
    q35_engine_stats s{};
    q35_prefix_stats p{};
    if (q35_engine_get_stats(owner_->engine, &s) == Q35_OK) {
      out.batch_ticks = s.batch_ticks;
      out.batch_rows = s.batch_rows;
      out.projection_batches = s.projection_batches;
      out.lm_head_batches = s.lm_head_batches;
      out.greedy_lm_head_batches = s.greedy_lm_head_batches;
      out.state_batches = s.state_batches;
      out.shared_prefill_ticks = s.shared_prefill_ticks;
      out.shared_prefill_requests = s.shared_prefill_requests;
      out.queued_requests = s.queued_requests;
      out.resident_requests = s.resident_requests;
      out.physical_kv_bytes = s.physical_kv_bytes;
    }
    if (q35_engine_prefix_stats(owner_->engine, &p) == Q35_OK) {
      out.prefix_builds = p.prefix_builds;
      out.prefix_build_fallbacks = p.prefix_build_fallbacks;
      out.prefix_hits = p.prefix_hits;
      out.prefix_cached_tokens = p.prefix_cached_tokens;
      out.prefix_evictions = p.prefix_evictions;
      out.prefix_entries = p.prefix_entries;
      out.prefix_bytes = p.prefix_bytes;
    }
    return out;
  }

  bool cancel(CpuRequestId id) { return q35_engine_cancel(owner_->engine, id) == Q35_OK; }
  bool release(CpuRequestId id) {
    const bool ok = q35_engine_release(owner_->engine, id) == Q35_OK;
    if (ok) glue_.erase(id);
    return ok;
  }

  bool result(CpuRequestId id, CpuRequestResult &out) const {
    q35_request_result r{};
    std::size_t n = 0;
    if (q35_engine_result(owner_->engine, id, &r, nullptr, 0, &n) != Q35_OK) return false;
    out = CpuRequestResult{};
    out.output_tokens.resize(n);
    if (n != 0 && q35_engine_result(owner_->engine, id, &r, out.output_tokens.data(), n, &n) != Q35_OK) return false;
    out.status = detail::to_status(r.status);
    out.generated_tokens = r.generated_tokens;
    out.committed_tokens = r.committed_tokens;
    out.prefill_tokens = r.prefill_tokens;
    out.decode_forwards = r.decode_forwards;
    out.cached_prefix_tokens = r.cached_prefix_tokens;
    out.prefix_restore_ms = r.prefix_restore_ms;
    out.prefill_ms = r.prefill_ms;
    out.decode_ms = r.decode_ms;
    out.queue_ms = r.queue_ms;
    out.prefix_written_tokens = r.prefix_written_tokens;
    if (out.status == CpuRequestStatus::failed) {
      const auto g = glue_.find(id);
      out.error = g != glue_.end() && !g->second->error.empty() ? g->second->error : last_error_;
    }
    return true;
  }

 private:
  explicit HipEngine(std::shared_ptr<detail::EngineHandle> owner) : owner_(std::move(owner)) {}
  bool check(int status, std::string &error) {
    if (status == Q35_OK) return true;
    error = last_error_ = q35_engine_last_error(owner_->engine);
    return false;
  }
  std::shared_ptr<detail::EngineHandle> owner_;
  std::map<CpuRequestId, std::unique_ptr<detail::RequestGlue>> glue_;
  std::string last_error_;
};

}  // namespace qwen35x::hip
