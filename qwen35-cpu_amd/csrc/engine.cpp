// q35_engine: the request-level mirror of qwen35x::CpuEngine
// (include/qwen35x/runtime/cpu_engine.h:173-215) for greedy requests, driving
// the device runtime one step at a time.
//   submit          cpu_engine.inl:832-930 (validation, admission)
//   advance         one prefill chunk or one decode row (cpu_engine.inl:668-790)
//   advance_batch   one decode row per distinct active request; validation
//                   leaves requests untouched; a failed forward fails every
//                   row and is never retried (cpu_engine.inl:939-1017)
//   step            serving scheduler (serving mode, max_queued_requests > 0):
//                   retire, admit up to max_prefill_requests, alternate decode
//                   batches with prefill chunks, rotate for fairness, skip
//                   rows whose unread output is full
//                   (cpu_engine_scheduler.inl:2-105) -- or, with packed_steps,
//                   run the decode batch and the prompt chunks of up to
//                   max_prefill_requests requests in one packed step
//   read_output     confirmed tokens, stop-sequence prefixes held back
//                   (cpu_engine_scheduler.inl:107-127)
//   automatic prefixes  register_prefix_tokens in serving mode: built once by
//                   the first request, published when its prefill reaches
//                   the boundary, attached by the requests that waited for it
//                   (cpu_engine_singleflight.inl)
//   register_prefix / find_prefix   cpu_engine_prefix.inl:11-96: a state
//                   snapshot plus the prefix's KV pages, shared by the
//                   requests that attach it (CpuRequestSpec::prefix)
// Request state lives on the device: a slot (DeltaNet state, conv ring,
// penalty counts) and a list of KV pages that grows as positions advance.
// Pages shared with a prefix are copied before the first write into them
// (KvPagesF16::append on a shared tail, kv_pages.h:52-60).
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>
#include <map>
#include <memory>
#include <new>
#include <numeric>
#include <random>
#include <set>
#include <string>
#include <vector>

#include "runtime.h"

namespace {

struct Request {
  uint64_t id = 0;
  std::vector<int32_t> prompt;
  size_t max_new = 0;
  float penalty = 1.0F;
  // SamplingOptions (options.h:10-13); temperature <= 1e-6 is greedy
  float temperature = 0.0F, top_p = 1.0F;
  int32_t top_k = 0;
  std::mt19937 rng;
  std::vector<int32_t> forced;  // forced_output_tokens
  q35_logits_callback callback = nullptr;
  void *callback_context = nullptr;
  const q35_sampling_constraint *constraint = nullptr;
  std::vector<int32_t> selected;  // selected readout token IDs
  q35_logits_callback selected_callback = nullptr;
  void *selected_context = nullptr;
  std::vector<int32_t> stops;
  std::vector<std::vector<int32_t>> stop_sequences;
  int status = Q35_REQ_QUEUED;
  int slot = -1;
  std::vector<int32_t> pages;
  size_t committed = 0;  // tokens whose state is in the slot / KV
  int32_t pending = -1;  // next decode input (last generated token)
  std::vector<int32_t> output;
  size_t consumed = 0;  // output tokens handed out by read_output
  q35_request_result result{};
  bool resident = false;
  uint64_t prefix = 0;  // attached prefix, pinned until the request retires
  size_t register_prefix = 0;  // automatic prefix boundary (0 = none)
  std::string ns;              // trust namespace
  bool has_ns = false;
  std::chrono::steady_clock::time_point arrival;
};

// A cached prefix (CpuPrefix): snapshot, the pages of its tokens (one
// reference each) and the pins of handles and attached requests.
struct Prefix {
  uint64_t id = 0;
  std::vector<int32_t> tokens;
  std::string ns;
  q35_state_snapshot *snap = nullptr;
  std::vector<int32_t> pages;
  size_t bytes = 0;
  int pins = 0;
};

double ms_since(std::chrono::steady_clock::time_point t) {
  return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t).count();
}

}  // namespace

struct q35_engine {
  q35_model *model = nullptr;
  q35_runtime *rt = nullptr;
  q35_engine_config cfg{};
  int32_t max_queued = 0;
  std::map<uint64_t, Request> reqs;
  uint64_t next_id = 1;
  std::string error;
  bool prefer_decode = true, scheduling = false;
  uint64_t last_prefill = 0, last_decode = 0;
  // prefix cache in least-recently-used order (back = most recent)
  std::vector<std::unique_ptr<Prefix>> prefixes;
  uint64_t next_prefix = 1;
  size_t max_prefix_bytes = 0, prefix_bytes = 0;
  q35_prefix_stats prefix_stats{};
  q35_engine_stats stats{};
  bool serving() const { return cfg.max_queued_requests > 0; }
};

namespace {

int fail(q35_engine *e, int status, const std::string &msg) {
  e->error = msg;
  return status;
}

bool terminal(const Request &r) {
  return r.status == Q35_REQ_COMPLETE || r.status == Q35_REQ_CANCELLED || r.status == Q35_REQ_FAILED;
}

Prefix *find_prefix_id(q35_engine *e, uint64_t id) {
  for (auto &p : e->prefixes)
    if (p->id == id) return p.get();
  return nullptr;
}

// Moves a prefix to the most recently used end.
void touch_prefix(q35_engine *e, Prefix *p) {
  auto it = std::find_if(e->prefixes.begin(), e->prefixes.end(), [&](const auto &q) { return q.get() == p; });
  if (it != e->prefixes.end()) std::rotate(it, it + 1, e->prefixes.end());
}

void destroy_prefix(q35_engine *e, Prefix &p) {
  for (int32_t page : p.pages) (void)q35_page_release(e->rt, page);
  p.pages.clear();
  q35_state_snapshot_destroy(p.snap);
  p.snap = nullptr;
}

// prefix_room (cpu_engine.inl:112-131): evict unpinned prefixes, least
// recently used first, until `bytes` fit.
bool prefix_room(q35_engine *e, size_t bytes) {
  if (bytes > e->max_prefix_bytes) return false;
  for (auto it = e->prefixes.begin(); e->prefix_bytes > e->max_prefix_bytes - bytes && it != e->prefixes.end();) {
    if ((*it)->pins == 0) {
      e->prefix_bytes -= (*it)->bytes;
      destroy_prefix(e, **it);
      ++e->prefix_stats.prefix_evictions;
      it = e->prefixes.erase(it);
    } else {
      ++it;
    }
  }
  return e->prefix_bytes <= e->max_prefix_bytes - bytes;
}

void unpin_prefix(q35_engine *e, uint64_t id) {
  Prefix *p = find_prefix_id(e, id);
  if (p != nullptr && p->pins > 0) --p->pins;
}

// Frees a request's device state: KV pages, slot, the attached prefix pin.
void free_resident(q35_engine *e, Request &r) {
  if (!r.resident) return;
  for (int32_t p : r.pages) (void)q35_page_release(e->rt, p);
  r.pages.clear();
  if (r.slot >= 0) (void)q35_slot_free(e->rt, r.slot);
  r.slot = -1;
  r.resident = false;
  if (r.prefix != 0) unpin_prefix(e, r.prefix);
  r.prefix = 0;
}

// retire (cpu_engine.inl:432-440): in serving mode a terminal request gives
// its device state back at once; in direct mode it keeps it until release.
void retire(q35_engine *e, Request &r) {
  if (!e->serving() || !r.resident || !terminal(r)) return;
  free_resident(e, r);
}

int activate(q35_engine *e, Request &r) {
  int32_t slot = -1;
  const int st = q35_slot_alloc(e->rt, r.prompt.data(), r.prompt.size(), &slot);
  if (st != Q35_OK) return fail(e, st, e->model->ctx->error.c_str());
  r.slot = slot;
  r.resident = true;
  r.status = Q35_REQ_PREFILL;
  if (r.prefix != 0) {
    // initialize with spec.prefix (cpu_engine.inl:386-407): restore the
    // state, share the prefix's pages
    const auto t0 = std::chrono::steady_clock::now();
    Prefix *p = find_prefix_id(e, r.prefix);
    int rs = p == nullptr ? Q35_ERR_STATE : q35_state_snapshot_restore(e->rt, p->snap, slot);
    if (rs != Q35_OK) {
      r.status = Q35_REQ_FAILED;
      (void)q35_slot_free(e->rt, slot);
      r.slot = -1;
      r.resident = false;
      return fail(e, rs, "Invalid prefix snapshot.");
    }
    for (int32_t page : p->pages) (void)q35_page_retain(e->rt, page);
    r.pages = p->pages;
    r.committed = p->tokens.size();
    r.result.cached_prefix_tokens = p->tokens.size();
    r.result.committed_tokens = r.committed;
    r.result.prefix_restore_ms = ms_since(t0);
    ++e->prefix_stats.prefix_hits;
    e->prefix_stats.prefix_cached_tokens += p->tokens.size();
    touch_prefix(e, p);
  }
  return Q35_OK;
}

// Copy-on-write of the page that receives position `pos` when it is shared
// (a prefix's partly filled tail page).
int own_page(q35_engine *e, Request &r, size_t pos) {
  const size_t idx = pos / static_cast<size_t>(e->cfg.page_tokens);
  if (idx >= r.pages.size() || q35_page_refcount(e->rt, r.pages[idx]) <= 1) return Q35_OK;
  int32_t fresh = -1;
  int st = q35_page_alloc(e->rt, &fresh);
  if (st != Q35_OK) return fail(e, st, "KV page pool exhausted");
  st = q35_page_copy(e->rt, r.pages[idx], fresh, static_cast<int32_t>(pos % e->cfg.page_tokens));
  if (st != Q35_OK) {
    (void)q35_page_release(e->rt, fresh);
    return fail(e, st, "KV page copy failed");
  }
  (void)q35_page_release(e->rt, r.pages[idx]);
  r.pages[idx] = fresh;
  return Q35_OK;
}

// Make sure a page covers `position` (KvPagesF16::append allocates the next page).
int ensure_page(q35_engine *e, Request &r, size_t position) {
  const size_t need = position / static_cast<size_t>(e->cfg.page_tokens) + 1;
  while (r.pages.size() < need) {
    int32_t p = -1;
    const int st = q35_page_alloc(e->rt, &p);
    if (st != Q35_OK) return fail(e, st, "KV page pool exhausted");
    r.pages.push_back(p);
  }
  return Q35_OK;
}

// The fused greedy head serves a request (cpu_engine.inl:307-313, 676-678).
bool is_greedy(const Request &r) {
  return r.temperature <= 1e-6F && r.forced.empty() && r.callback == nullptr && r.constraint == nullptr &&
         r.selected.empty();
}

// Device candidate settings of a request: greedy argmax (k = 1, scale 1) at
// temperature ~0, top_k candidates when 1 <= top_k <= 64, else one
// placeholder candidate while the host samples from the raw logits.
q35_row_sampling row_sampling(const Request &r) {
  q35_row_sampling s{1, 1.0F};
  if (r.temperature > 1e-6F) {
    s.inv_temperature = 1.0F / r.temperature;
    if (r.top_k >= 1 && r.top_k <= Q35_MAX_CANDIDATES) s.top_k = r.top_k;
  }
  return s;
}
bool needs_raw_logits(const Request &r) {
  return r.callback != nullptr || r.constraint != nullptr || !r.selected.empty() ||
         (r.temperature > 1e-6F && (r.top_k <= 0 || r.top_k > Q35_MAX_CANDIDATES) && r.forced.empty());
}

// sample_token_from_logits (layers.inl:570-615) from the descending candidate
// list: softmax, nucleus cut, one draw of uniform_real_distribution<float>.
int32_t sample_candidates(const q35_candidate *c, int k, float top_p, std::mt19937 &rng) {
  int n = 0;
  while (n < k && c[n].token >= 0) ++n;
  if (n == 0) return -1;
  float max_logit = -INFINITY;
  for (int i = 0; i < n; ++i) max_logit = std::max(max_logit, c[i].value);
  std::vector<float> probs(n);
  float denom = 0.0F;
  for (int i = 0; i < n; ++i) {
    probs[i] = std::exp(c[i].value - max_logit);
    denom += probs[i];
  }
  if (!(denom > 0.0F)) return c[0].token;
  for (float &p : probs) p /= denom;
  size_t keep = probs.size();
  if (top_p < 1.0F) {
    float cumulative = 0.0F;
    keep = 0;
    for (; keep < probs.size(); ++keep) {
      cumulative += probs[keep];
      if (cumulative >= top_p) {
        ++keep;
        break;
      }
    }
    keep = std::max<size_t>(1, std::min(keep, probs.size()));
  }
  probs.resize(keep);
  float renorm = 0.0F;
  for (float p : probs) renorm += p;
  if (!(renorm > 0.0F)) return c[0].token;
  for (float &p : probs) p /= renorm;
  std::uniform_real_distribution<float> dist(0.0F, 1.0F);
  const float draw = dist(rng);
  float cumulative = 0.0F;
  for (size_t i = 0; i < probs.size(); ++i) {
    cumulative += probs[i];
    if (draw <= cumulative || i + 1 == probs.size()) return c[i].token;
  }
  return c[probs.size() - 1].token;
}

// sample_token_from_logits (layers.inl:491-600) on the full raw logits row,
// for samplers that see every token (top_k 0 or above the device list).
int32_t sample_full(const float *raw, int vocab, const std::vector<int32_t> &counts, Request &r) {
  std::vector<float> logits(raw, raw + vocab);
  if (r.penalty > 1.0F)
    for (int i = 0; i < vocab; ++i)
      if (counts[i] > 0) logits[i] = logits[i] > 0.0F ? logits[i] / r.penalty : logits[i] * r.penalty;
  const float inv_temp = 1.0F / r.temperature;
  for (float &v : logits) v *= inv_temp;
  std::vector<int> ids(vocab);
  std::iota(ids.begin(), ids.end(), 0);
  auto greater = [&](int a, int b) { return logits[a] > logits[b]; };
  if (r.top_k > 0 && r.top_k < vocab) {
    std::nth_element(ids.begin(), ids.begin() + r.top_k, ids.end(), greater);
    ids.resize(r.top_k);
  }
  std::sort(ids.begin(), ids.end(), greater);
  std::vector<q35_candidate> c(ids.size());
  for (size_t i = 0; i < ids.size(); ++i) c[i] = {logits[ids[i]], ids[i]};
  return sample_candidates(c.data(), static_cast<int>(c.size()), r.top_p, r.rng);
}

// The token of one row (select, cpu_engine.inl:441-465): the logits callback
// on the raw logits, then the forced token, the greedy candidate, a draw from
// the device candidates, or a draw over the full row.
int choose_token(q35_engine *e, Request &r, const q35_candidate *cands, const float *raw, int32_t &token) {
  const int vocab = e->model->d.vocab;
  const size_t index = r.output.size();
  if (!r.selected.empty()) {
    // selected readout: the head rows of the given tokens, which are the
    // same single-chain dots as the full row (layers.inl:414-455)
    std::vector<float> values(r.selected.size());
    for (size_t i = 0; i < values.size(); ++i) values[i] = raw[r.selected[i]];
    if (!r.selected_callback(r.selected_context, index, r.forced[index], values.data(), values.size()))
      return fail(e, Q35_ERR_STATE, "Selected logits callback failed.");
  }
  if (r.callback != nullptr &&
      !r.callback(r.callback_context, index, r.forced.empty() ? -1 : r.forced[index], raw, static_cast<size_t>(vocab)))
    return fail(e, Q35_ERR_STATE, "Logits callback failed.");
  if (r.constraint != nullptr) {
    // the constraint masks a copy of the raw row; the token is then chosen
    // from the whole masked row (sample_token_from_logits, layers.inl:491-600)
    std::vector<float> masked(raw, raw + vocab);
    if (!r.constraint->apply(r.constraint->context, masked.data(), masked.size()))
      return fail(e, Q35_ERR_STATE, "Sampling constraint rejected the logits.");
    std::vector<int32_t> counts(vocab);
    const int st = q35_slot_counts(e->rt, r.slot, counts.data(), counts.size());
    if (st != Q35_OK) return fail(e, st, e->model->ctx->error.c_str());
    if (r.temperature <= 1e-6F) {
      // argmax after the repetition penalty, lowest index on ties (layers.inl:519-541)
      float best = -INFINITY;
      token = -1;
      for (int i = 0; i < vocab; ++i) {
        float v = masked[i];
        if (r.penalty > 1.0F && counts[i] > 0) v = v > 0.0F ? v / r.penalty : v * r.penalty;
        if (token < 0 || v > best) {
          best = v;
          token = i;
        }
      }
      if (!(best > -INFINITY)) return fail(e, Q35_ERR_STATE, "Sampling constraint left no finite candidate.");
    } else {
      token = sample_full(masked.data(), vocab, counts, r);
    }
    if (token < 0 || token >= vocab) return fail(e, Q35_ERR_STATE, "Invalid sampled token.");
    if (!r.constraint->accept(r.constraint->context, token))
      return fail(e, Q35_ERR_STATE, "Sampling constraint rejected the token.");
    return Q35_OK;
  }
  if (!r.forced.empty()) {
    token = r.forced[index];
  } else if (r.temperature <= 1e-6F) {
    token = cands[0].token;  // argmax with the penalty (layers.inl:519-541)
  } else if (r.top_k >= 1 && r.top_k <= Q35_MAX_CANDIDATES) {
    token = sample_candidates(cands, r.top_k, r.top_p, r.rng);
  } else {
    std::vector<int32_t> counts(vocab);
    const int st = q35_slot_counts(e->rt, r.slot, counts.data(), counts.size());
    if (st != Q35_OK) return fail(e, st, e->model->ctx->error.c_str());
    token = sample_full(raw, vocab, counts, r);
  }
  if (token < 0 || token >= vocab) return fail(e, Q35_ERR_STATE, "Invalid sampled token.");
  return Q35_OK;
}

// select() (cpu_engine.inl:441-487): append, stop ids and stop sequences
// (trimmed from the output), completion.
void select_token(Request &r, int32_t token) {
  ++r.result.generated_tokens;
  r.output.push_back(token);
  r.pending = token;
  size_t trim = std::find(r.stops.begin(), r.stops.end(), token) != r.stops.end() ? 1 : 0;
  for (const auto &stop : r.stop_sequences)
    if (!stop.empty() && stop.size() <= r.output.size() &&
        std::equal(stop.begin(), stop.end(), r.output.end() - static_cast<std::ptrdiff_t>(stop.size())))
      trim = std::max(trim, stop.size());
  if (trim) {
    r.output.resize(r.output.size() - trim);
    r.status = Q35_REQ_COMPLETE;
  } else {
    r.status = r.output.size() == r.max_new ? Q35_REQ_COMPLETE : Q35_REQ_DECODE;
  }
}

// The counters of one forward through every layer (cpu_engine.inl:201-325):
// four projections and one state batch per layer, then the head.
void count_forward(q35_engine *e, bool greedy_head) {
  const uint64_t layers = static_cast<uint64_t>(e->model->d.n_layers);
  e->stats.projection_batches += 4 * layers + (greedy_head ? 1 : 0);
  e->stats.state_batches += layers;
  e->stats.lm_head_batches += 1;
  e->stats.greedy_lm_head_batches += greedy_head ? 1 : 0;
}

// One device step over `rows`: each row feeds `inputs[i]` at position
// rows[i]->committed. count_input marks generated tokens. With `sample` the
// head keeps the logits and returns each row's candidates (and the raw logits
// when a row needs them); the tokens are chosen afterwards by choose_token.
int run_step(q35_engine *e, const std::vector<Request *> &rows, const std::vector<int32_t> &inputs,
             const std::vector<uint8_t> &count_input, std::vector<int32_t> &out, bool sample,
             std::vector<q35_candidate> *cands, std::vector<float> *raw) {
  const int B = static_cast<int>(rows.size());
  const int max_pages = (e->cfg.max_context + e->cfg.page_tokens - 1) / e->cfg.page_tokens;
  std::vector<int32_t> slots(B), positions(B), table(static_cast<size_t>(B) * max_pages, 0);
  std::vector<float> pen(B);
  for (int b = 0; b < B; ++b) {
    Request &r = *rows[b];
    int st = own_page(e, r, r.committed);
    if (st == Q35_OK) st = ensure_page(e, r, r.committed);
    if (st != Q35_OK) return st;
    slots[b] = r.slot;
    positions[b] = static_cast<int32_t>(r.committed);
    pen[b] = r.penalty;
    std::copy(r.pages.begin(), r.pages.end(), table.begin() + static_cast<size_t>(b) * max_pages);
  }
  q35_step_desc d{};
  d.batch = B;
  d.slots = slots.data();
  d.positions = positions.data();
  d.tokens = inputs.data();
  d.count_input = count_input.data();
  d.penalties = pen.data();
  d.page_table = table.data();
  d.max_pages = max_pages;
  out.assign(B, -1);
  int st;
  if (!sample) {
    st = q35_runtime_step(e->rt, &d, out.data(), nullptr);
  } else {
    std::vector<q35_row_sampling> rs(B);
    bool need_raw = false;
    for (int b = 0; b < B; ++b) {
      rs[b] = row_sampling(*rows[b]);
      need_raw = need_raw || needs_raw_logits(*rows[b]);
    }
    cands->assign(static_cast<size_t>(B) * Q35_MAX_CANDIDATES, q35_candidate{});
    raw->assign(need_raw ? static_cast<size_t>(B) * e->model->d.vocab : 0, 0.0F);
    st = q35_runtime_step_candidates(e->rt, &d, rs.data(), cands->data(), need_raw ? raw->data() : nullptr);
  }
  if (st != Q35_OK) return fail(e, st, e->model->ctx->error.c_str());
  for (auto *r : rows) ++r->committed;
  count_forward(e, !sample);
  return Q35_OK;
}

// The first token after a prompt (or a complete prefix hit) of a request the
// fused greedy head does not serve: candidates from the final hidden row.
int choose_after_prompt(q35_engine *e, Request &r, const float *hidden, int32_t &token) {
  const q35_row_sampling rs = row_sampling(r);
  std::vector<q35_candidate> cands(Q35_MAX_CANDIDATES);
  std::vector<float> raw(needs_raw_logits(r) ? e->model->d.vocab : 0);
  const int st = q35_runtime_head_candidates(e->rt, r.slot, hidden, r.penalty, &rs, cands.data(),
                                             raw.empty() ? nullptr : raw.data());
  if (st != Q35_OK) return fail(e, st, e->model->ctx->error.c_str());
  return choose_token(e, r, cands.data(), raw.empty() ? nullptr : raw.data(), token);
}

void fail_rows(const std::vector<Request *> &rows) {
  for (auto *r : rows) r->status = Q35_REQ_FAILED;
}

// Impl::confirmed (cpu_engine.inl:419-428): output tokens that can no longer
// turn into a stop sequence (all of them once the request is terminal).
size_t confirmed(const Request &r) {
  if (terminal(r)) return r.output.size();
  size_t held = 0;
  for (const auto &stop : r.stop_sequences)
    for (size_t n = 1; n < stop.size() && n <= r.output.size(); ++n)
      if (std::equal(stop.begin(), stop.begin() + static_cast<std::ptrdiff_t>(n),
                     r.output.end() - static_cast<std::ptrdiff_t>(n)))
        held = std::max(held, n);
  return r.output.size() - held;
}

// Impl::output_ready (cpu_engine.inl:429-431)
bool output_ready(const q35_engine *e, const Request &r) {
  return r.output.size() - r.consumed < static_cast<size_t>(e->cfg.max_buffered_tokens);
}

// Impl::short_readout (cpu_engine.inl:628-631): a selected readout with at
// most 128 prompt tokens left; the reference shares prefill steps only
// between these.
bool short_readout(const Request &r) {
  const size_t remaining = r.prompt.size() - r.committed;
  return !r.selected.empty() && remaining > 0 && remaining <= 128;
}

// The prompt tokens one advance() or prompt segment prefills
// (cpu_engine.inl:728-741): the canonical chunk (prefill_chunk_size, or 64
// for prompts of at most 128 tokens and 128 otherwise), capped at an
// automatic prefix boundary still ahead.
size_t advance_chunk(const q35_engine *e, const Request &r) {
  const size_t chunk = e->cfg.prefill_chunk_size > 0 ? static_cast<size_t>(e->cfg.prefill_chunk_size)
                                                      : (r.prompt.size() <= 128 ? 64 : 128);
  size_t count = q35_prefill_chunk_token_count(r.committed, r.prompt.size() - r.committed, chunk);
  if (r.register_prefix > r.committed) count = std::min(count, r.register_prefix - r.committed);
  return count;
}

// Device bytes of a prefix of n tokens: one recurrent state copy, the conv
// ring and the final hidden row, plus the K and V rows of its pages.
size_t prefix_size(const q35_engine *e, size_t n) {
  const q35_model_dims &d = e->model->d;
  const size_t pages = (n + e->cfg.page_tokens - 1) / e->cfg.page_tokens;
  return (static_cast<size_t>(e->rt->rec_copy_stride) + e->rt->conv_slot_stride + d.hidden) * 4 +
         pages * e->cfg.page_tokens * static_cast<size_t>(d.n_kv_heads) * d.head_dim * 2 * 2 * e->model->n_full;
}

// A prefix of the first n tokens of slot `slot` (state after n positions,
// `hidden` the final normalized row of position n - 1): the snapshot plus a
// reference to each page holding those positions. Pinned once for the
// caller. Returns nullptr when the snapshot cannot be made.
Prefix *capture_prefix(q35_engine *e, int32_t slot, const std::vector<int32_t> &tokens, const std::string &ns,
                       const std::vector<int32_t> &pages, const float *hidden, size_t bytes) {
  q35_state_snapshot *snap = nullptr;
  if (q35_state_snapshot_create(e->rt, slot, static_cast<int32_t>(tokens.size()), hidden, &snap) != Q35_OK)
    return nullptr;
  auto p = std::make_unique<Prefix>();
  p->id = e->next_prefix++;
  p->tokens = tokens;
  p->ns = ns;
  p->snap = snap;
  const size_t used = (tokens.size() + e->cfg.page_tokens - 1) / e->cfg.page_tokens;
  p->pages.assign(pages.begin(), pages.begin() + static_cast<std::ptrdiff_t>(std::min(used, pages.size())));
  for (int32_t page : p->pages) (void)q35_page_retain(e->rt, page);
  p->bytes = bytes;
  p->pins = 1;
  e->prefix_bytes += bytes;
  e->prefixes.push_back(std::move(p));
  return e->prefixes.back().get();
}

// same_build (cpu_engine_singleflight.inl:2-10): two requests that would
// build the same automatic prefix.
bool same_build(const Request &a, const Request &b) {
  return a.register_prefix != 0 && a.register_prefix == b.register_prefix && a.ns == b.ns &&
         std::equal(a.prompt.begin(), a.prompt.begin() + static_cast<std::ptrdiff_t>(a.register_prefix),
                    b.prompt.begin());
}

// prefix_admissible (cpu_engine_singleflight.inl:11-30): a request with an
// automatic prefix attaches a published prefix of exactly that boundary, or
// waits while another resident request is still building it.
bool prefix_admissible(q35_engine *e, Request &r) {
  const size_t count = r.register_prefix;
  if (count == 0) return true;
  for (auto &p : e->prefixes)
    if (p->tokens.size() == count && p->ns == r.ns && std::equal(p->tokens.begin(), p->tokens.end(), r.prompt.begin())) {
      if (r.prefix != p->id) {
        if (r.prefix != 0) unpin_prefix(e, r.prefix);
        r.prefix = p->id;
        ++p->pins;
      }
      touch_prefix(e, p.get());
      return true;
    }
  for (auto &kv : e->reqs) {
    const Request &o = kv.second;
    if (&o != &r && o.resident && !terminal(o) && o.committed < count && same_build(r, o)) return false;
  }
  return true;
}

// publish_prefix (cpu_engine_singleflight.inl:85-110): after the request's
// prefill reached its boundary, its state and pages become a prefix the
// request itself holds; when it cannot be stored, the request and those of
// the same build go on as ordinary cold requests.
void publish_prefix(q35_engine *e, Request &r, const float *hidden) {
  const size_t count = r.register_prefix;
  // the restored state is already private: the attached prefix may go
  if (r.prefix != 0) unpin_prefix(e, r.prefix);
  r.prefix = 0;
  const size_t bytes = prefix_size(e, count);
  Prefix *p = nullptr;
  if (hidden != nullptr && prefix_room(e, bytes)) {
    const std::vector<int32_t> tokens(r.prompt.begin(), r.prompt.begin() + static_cast<std::ptrdiff_t>(count));
    p = capture_prefix(e, r.slot, tokens, r.ns, r.pages, hidden, bytes);
  }
  if (p != nullptr) {
    r.prefix = p->id;
    ++e->prefix_stats.prefix_builds;
    r.result.prefix_written_tokens = count - r.result.cached_prefix_tokens;
    return;
  }
  ++e->prefix_stats.prefix_build_fallbacks;
  for (auto &kv : e->reqs)
    if (&kv.second != &r && same_build(r, kv.second)) kv.second.register_prefix = 0;
  r.register_prefix = 0;
}

}  // namespace

// detail::prefill_chunk_token_count (src/runtime/prefill_chunk.h:10-17)
extern "C" size_t q35_prefill_chunk_token_count(size_t position, size_t remaining, size_t chunk) {
  constexpr size_t kRowAttentionLimit = 128;  // prefill_attention_row_limit
  if (remaining == 0 || chunk == 0) return 0;
  size_t count = std::min(chunk - position % chunk, remaining);
  if (position < kRowAttentionLimit) count = std::min(count, kRowAttentionLimit - position);
  return count;
}

extern "C" int q35_engine_create(q35_model *m, const q35_engine_config *cfg, q35_engine **out) {
  if (m == nullptr || cfg == nullptr || out == nullptr) return Q35_ERR_INVALID;
  *out = nullptr;
  // CpuEngine::create validation (cpu_engine.inl:795-806)
  if (cfg->max_resident_requests <= 0 || cfg->max_context <= 0 || cfg->max_decode_batch_size <= 0 ||
      cfg->max_decode_batch_size > q35::kMaxTokens || cfg->page_tokens <= 0 || cfg->prefill_chunk_size < 0 ||
      cfg->prefill_chunk_size > q35::kMaxStepRows || cfg->max_prefill_requests < 0 ||
      cfg->max_prefill_requests > q35::kMaxPrefillSegments || cfg->max_queued_requests < 0 ||
      (cfg->max_queued_requests > 0 && cfg->max_buffered_tokens <= 0))
    return set_error(m->ctx, Q35_ERR_INVALID, "Invalid CPU engine configuration.");
  auto *e = new (std::nothrow) q35_engine();
  if (e == nullptr) return Q35_ERR_OOM;
  e->model = m;
  e->cfg = *cfg;
  if (e->cfg.max_prefill_requests == 0) e->cfg.max_prefill_requests = 1;
  e->max_prefix_bytes = cfg->max_prefix_bytes ? static_cast<size_t>(cfg->max_prefix_bytes) : size_t(256) << 20;
  q35_runtime_config rc{};
  // one slot beyond the resident requests for register_prefix builds
  rc.max_slots = cfg->max_resident_requests + 1;
  rc.max_batch = std::max(cfg->max_decode_batch_size, 1);
  rc.max_context = cfg->max_context;
  rc.page_tokens = cfg->page_tokens;
  rc.use_graphs = cfg->use_graphs;
  // rows of the largest step: the prompt chunks of a shared prefill, plus
  // the decode batch when the two are packed together
  // (prefill_chunk_size 0: chunks of at most 128 prompt tokens)
  const long long chunk = e->cfg.prefill_chunk_size > 0 ? e->cfg.prefill_chunk_size : 128;
  const long long step_rows = static_cast<long long>(e->cfg.max_prefill_requests) * chunk +
                              (e->cfg.packed_steps ? rc.max_batch : 0);
  if (step_rows > q35::kMaxStepRows) {
    delete e;
    return set_error(m->ctx, Q35_ERR_INVALID,
                     "max_prefill_requests * prefill_chunk_size (+ max_decode_batch_size with packed_steps) exceeds " +
                         std::to_string(q35::kMaxStepRows) + " rows per step");
  }
  rc.max_step_rows = static_cast<int32_t>(step_rows);
  const int st = q35_runtime_create(m, &rc, &e->rt);
  if (st != Q35_OK) {
    delete e;
    return st;
  }
  *out = e;
  return Q35_OK;
}

extern "C" void q35_engine_destroy(q35_engine *e) {
  if (e == nullptr) return;
  for (auto &p : e->prefixes) destroy_prefix(e, *p);
  e->prefixes.clear();
  q35_runtime_destroy(e->rt);
  delete e;
}

extern "C" const char *q35_engine_last_error(const q35_engine *e) {
  return e ? e->error.c_str() : "null engine";
}

extern "C" int q35_engine_submit(q35_engine *e, const int32_t *prompt, size_t n, size_t max_new,
                                 float penalty, const int32_t *stops, size_t n_stops, uint64_t *out_id) {
  return q35_engine_submit_prefixed(e, prompt, n, max_new, penalty, stops, n_stops, 0, out_id);
}

extern "C" int q35_engine_submit_prefixed(q35_engine *e, const int32_t *prompt, size_t n, size_t max_new,
                                          float penalty, const int32_t *stops, size_t n_stops, uint64_t prefix,
                                          uint64_t *out_id) {
  q35_request_spec spec{};
  spec.prompt_tokens = prompt;
  spec.prompt_count = n;
  spec.max_new_tokens = max_new;
  spec.temperature = 0.0F;  // greedy
  spec.top_p = 1.0F;
  spec.repetition_penalty = penalty;
  spec.seed = 0;
  spec.stop_token_ids = stops;
  spec.stop_count = n_stops;
  spec.prefix = prefix;
  return q35_engine_submit_spec(e, &spec, out_id);
}

extern "C" int q35_engine_submit_spec(q35_engine *e, const q35_request_spec *spec, uint64_t *out_id) {
  if (e == nullptr || out_id == nullptr || spec == nullptr) return Q35_ERR_INVALID;
  *out_id = 0;
  e->error.clear();
  const int vocab = e->model->d.vocab;
  const size_t ctx = static_cast<size_t>(e->cfg.max_context);
  const int32_t *prompt = spec->prompt_tokens;
  const size_t n = spec->prompt_count, max_new = spec->max_new_tokens;
  const float penalty = spec->repetition_penalty;
  const uint64_t prefix = spec->prefix;
  auto valid_token = [&](int32_t t) { return t >= 0 && t < vocab; };
  // record limit: resident plus queued requests, terminal results included
  // until release (cpu_engine.inl:836)
  const size_t records = static_cast<size_t>(e->cfg.max_resident_requests) + e->cfg.max_queued_requests;
  if (prompt == nullptr || n == 0 || max_new == 0 || n > ctx || max_new - 1 > ctx - n || e->reqs.size() >= records ||
      (spec->forced_count != 0 && (spec->forced_output_tokens == nullptr || spec->forced_count != max_new)) ||
      !std::isfinite(spec->temperature) || spec->temperature < 0 || !std::isfinite(spec->top_p) ||
      spec->top_p <= 0 || spec->top_p > 1 || spec->top_k < 0 || !std::isfinite(penalty) || penalty < 1 ||
      (spec->stop_count && spec->stop_token_ids == nullptr) ||
      (spec->stop_sequence_count && (spec->stop_sequences == nullptr || spec->stop_sequence_lengths == nullptr)))
    return fail(e, Q35_ERR_INVALID, "Invalid request or resident/context limit reached.");
  if (!std::all_of(prompt, prompt + n, valid_token) ||
      !std::all_of(spec->forced_output_tokens, spec->forced_output_tokens + spec->forced_count, valid_token))
    return fail(e, Q35_ERR_INVALID, "Invalid request token.");
  const bool selected = spec->selected_logit_count != 0 || spec->selected_logits_callback != nullptr;
  if (spec->sampling_constraint != nullptr &&
      (selected || spec->forced_count != 0 || spec->sampling_constraint->apply == nullptr ||
       spec->sampling_constraint->accept == nullptr))
    return fail(e, Q35_ERR_INVALID, "Sampling constraints cannot be combined with forced or selected readout.");
  if (selected &&
      (spec->selected_logit_count == 0 || spec->selected_logit_tokens == nullptr ||
       spec->selected_logits_callback == nullptr || spec->logits_callback != nullptr || max_new != 1 ||
       spec->forced_count != 1 || e->model->embed_g16 ||
       !std::all_of(spec->selected_logit_tokens, spec->selected_logit_tokens + spec->selected_logit_count,
                    valid_token)))
    return fail(e, Q35_ERR_INVALID,
                "Selected readout requires a Q4 DOT4 head, valid token IDs, its own callback and one forced token.");
  if (e->serving()) {
    // bounded queue; a stop sequence must fit the output buffer (cpu_engine.inl:877-886)
    size_t queued = 0;
    for (auto &kv : e->reqs) queued += kv.second.status == Q35_REQ_QUEUED;
    bool long_stop = false;
    for (size_t i = 0; i < spec->stop_sequence_count; ++i)
      long_stop = long_stop || spec->stop_sequence_lengths[i] > static_cast<size_t>(e->cfg.max_buffered_tokens);
    if (queued >= static_cast<size_t>(e->cfg.max_queued_requests) || long_stop)
      return fail(e, Q35_ERR_INVALID, "Queue full or stop sequence exceeds output buffer capacity.");
  }
  const bool has_ns = spec->trust_namespace != nullptr;
  const std::string ns = has_ns ? spec->trust_namespace : "";
  Prefix *pre = nullptr;
  if (prefix != 0) {
    // the attached prefix must be a prefix of the prompt, of the request's
    // namespace when it names one (cpu_engine.inl:895-910)
    pre = find_prefix_id(e, prefix);
    if (pre == nullptr || pre->tokens.size() > n || !std::equal(pre->tokens.begin(), pre->tokens.end(), prompt) ||
        (has_ns && pre->ns != ns))
      return fail(e, Q35_ERR_INVALID, "Prefix model, configuration, draft kind, namespace or token identity mismatch.");
  }
  // automatic prefix builds (cpu_engine.inl:887-892)
  const size_t reg = spec->register_prefix_tokens;
  if (reg != 0 && (!e->serving() || (pre != nullptr && pre->tokens.size() >= reg) || ns.empty() || reg > n))
    return fail(e, Q35_ERR_INVALID, "Automatic prefix builds require serving mode, a namespace and a valid prefix length.");
  Request r;
  r.prompt.assign(prompt, prompt + n);
  r.max_new = max_new;
  r.penalty = penalty;
  r.temperature = spec->temperature;
  r.top_p = spec->top_p;
  r.top_k = spec->top_k;
  r.rng.seed(spec->seed < 0 ? std::random_device{}() : static_cast<std::uint32_t>(spec->seed));
  r.forced.assign(spec->forced_output_tokens, spec->forced_output_tokens + spec->forced_count);
  r.callback = spec->logits_callback;
  r.callback_context = spec->logits_callback_context;
  r.constraint = spec->sampling_constraint;
  if (selected) r.selected.assign(spec->selected_logit_tokens, spec->selected_logit_tokens + spec->selected_logit_count);
  r.selected_callback = spec->selected_logits_callback;
  r.selected_context = spec->selected_logits_callback_context;
  if (spec->stop_count) r.stops.assign(spec->stop_token_ids, spec->stop_token_ids + spec->stop_count);
  for (size_t i = 0, at = 0; i < spec->stop_sequence_count; at += spec->stop_sequence_lengths[i++])
    r.stop_sequences.emplace_back(spec->stop_sequences + at, spec->stop_sequences + at + spec->stop_sequence_lengths[i]);
  r.status = Q35_REQ_QUEUED;
  r.register_prefix = reg;
  r.ns = pre != nullptr && !has_ns ? pre->ns : ns;
  r.has_ns = has_ns;
  r.arrival = std::chrono::steady_clock::now();
  if (pre != nullptr) {
    r.prefix = prefix;
    ++pre->pins;
  }
  // direct mode activates at once; serving mode queues without device state
  // until step admits it (cpu_engine.inl:918-921)
  if (!e->serving()) {
    const int st = activate(e, r);
    if (st != Q35_OK) {
      if (r.prefix != 0) unpin_prefix(e, r.prefix);
      return st;
    }
  }
  // IDs are monotonic and never reused; a rejected submit takes none
  r.id = e->next_id++;
  *out_id = r.id;
  e->reqs.emplace(r.id, std::move(r));
  return Q35_OK;
}

// Prefill one request for up to `limit` prompt tokens (one advance() chunk,
// cpu_engine.inl:668-790) in device chunks of at most max_decode_batch_size
// positions each (q35_runtime_prefill). The chunk that consumes the last
// prompt token yields the first generated token.
static int prefill_chunks(q35_engine *e, Request &r, size_t limit) {
  const auto t0 = std::chrono::steady_clock::now();
  const size_t rows = static_cast<size_t>(std::max(e->rt->max_rows, 1));
  const int max_pages = (e->cfg.max_context + e->cfg.page_tokens - 1) / e->cfg.page_tokens;
  std::vector<int32_t> table(max_pages, 0);
  if (r.committed == r.prompt.size() && r.status == Q35_REQ_PREFILL) {
    // complete prefix hit: the request's own greedy head on the prefix's
    // final hidden row (cpu_engine.inl:711-726)
    Prefix *p = find_prefix_id(e, r.prefix);
    std::vector<float> hidden(e->model->d.hidden);
    int32_t out = -1;
    int st = p == nullptr ? Q35_ERR_STATE : q35_state_snapshot_hidden(p->snap, hidden.data(), hidden.size());
    if (st == Q35_OK)
      st = is_greedy(r) ? q35_runtime_head(e->rt, r.slot, hidden.data(), r.penalty, &out)
                        : choose_after_prompt(e, r, hidden.data(), out);
    if (st != Q35_OK) {
      r.status = Q35_REQ_FAILED;
      return fail(e, st, e->error.empty() ? "Prefix head selection failed." : e->error);
    }
    select_token(r, out);
    r.result.prefill_ms += ms_since(t0);
    return Q35_OK;
  }
  size_t done = 0;
  while (done < limit && r.committed < r.prompt.size()) {
    size_t n = std::min({rows, limit - done, r.prompt.size() - r.committed});
    // an automatic prefix boundary ends a device chunk, so its state can be
    // captured (cpu_engine.inl:737-741)
    const bool building = r.register_prefix > r.committed;
    if (building) n = std::min(n, r.register_prefix - r.committed);
    int st = own_page(e, r, r.committed);
    if (st == Q35_OK) st = ensure_page(e, r, r.committed + n - 1);
    if (st != Q35_OK) {
      r.status = Q35_REQ_FAILED;
      return st;
    }
    std::copy(r.pages.begin(), r.pages.end(), table.begin());
    int32_t out = -1;
    st = q35_runtime_prefill(e->rt, r.slot, static_cast<int32_t>(r.committed), r.prompt.data() + r.committed,
                             static_cast<int32_t>(n), table.data(), max_pages, r.penalty, &out);
    if (st != Q35_OK) {
      r.status = Q35_REQ_FAILED;
      return fail(e, st, e->model->ctx->error.c_str());
    }
    count_forward(e, true);
    r.committed += n;
    r.result.prefill_tokens += n;
    done += n;
    if (building && r.committed == r.register_prefix) {
      std::vector<float> hidden(e->model->d.hidden);
      const bool have = q35_runtime_last_hidden(e->rt, hidden.data(), hidden.size()) == Q35_OK;
      publish_prefix(e, r, have ? hidden.data() : nullptr);
    }
    if (r.committed == r.prompt.size()) {
      if (!is_greedy(r)) {
        std::vector<float> hidden(e->model->d.hidden);
        st = q35_runtime_last_hidden(e->rt, hidden.data(), hidden.size());
        if (st == Q35_OK) st = choose_after_prompt(e, r, hidden.data(), out);
        if (st != Q35_OK) {
          r.status = Q35_REQ_FAILED;
          return e->error.empty() ? fail(e, st, e->model->ctx->error.c_str()) : st;
        }
      }
      select_token(r, out);
    }
  }
  r.result.prefill_ms += ms_since(t0);
  r.result.committed_tokens = r.committed;
  return Q35_OK;
}

extern "C" int q35_engine_advance(q35_engine *e, uint64_t id) {
  if (e == nullptr) return Q35_ERR_INVALID;
  e->error.clear();
  if (e->serving() && !e->scheduling) return fail(e, Q35_ERR_STATE, "Serving mode must be driven through step.");
  auto it = e->reqs.find(id);
  if (it == e->reqs.end()) return fail(e, Q35_ERR_STATE, "Unknown request ID.");
  Request &r = it->second;
  if (r.status == Q35_REQ_PREFILL) return prefill_chunks(e, r, advance_chunk(e, r));
  if (r.status != Q35_REQ_DECODE) return fail(e, Q35_ERR_STATE, "Request is not active.");
  return q35_engine_advance_batch(e, &id, 1);
}

extern "C" int q35_engine_advance_batch(q35_engine *e, const uint64_t *ids, size_t count) {
  if (e == nullptr) return Q35_ERR_INVALID;
  e->error.clear();
  if (e->serving() && !e->scheduling) return fail(e, Q35_ERR_STATE, "Serving mode must be driven through step.");
  if (count == 0) return Q35_OK;
  if (ids == nullptr || count > static_cast<size_t>(e->cfg.max_decode_batch_size))
    return fail(e, Q35_ERR_INVALID, "Decode batch exceeds max_decode_batch_size.");
  std::vector<Request *> rows;
  for (size_t i = 0; i < count; ++i) {
    auto it = e->reqs.find(ids[i]);
    if (it == e->reqs.end() || it->second.status != Q35_REQ_DECODE ||
        std::find(rows.begin(), rows.end(), &it->second) != rows.end())
      return fail(e, Q35_ERR_INVALID, "Decode batch requires distinct active decode requests.");
    rows.push_back(&it->second);
  }
  const auto t0 = std::chrono::steady_clock::now();
  std::vector<int32_t> in, out;
  std::vector<uint8_t> cnt;
  for (auto *r : rows) {
    in.push_back(r->pending);
    cnt.push_back(1);
  }
  // the fused greedy head only when every row is greedy (cpu_engine.inl:307-313)
  const bool sample = !std::all_of(rows.begin(), rows.end(), [](const Request *r) { return is_greedy(*r); });
  std::vector<q35_candidate> cands;
  std::vector<float> raw;
  const int st = run_step(e, rows, in, cnt, out, sample, &cands, &raw);
  if (st != Q35_OK) {
    // A failed forward may have updated state: never retry it.
    fail_rows(rows);
    return st;
  }
  ++e->stats.batch_ticks;
  e->stats.batch_rows += rows.size();
  const double ms = ms_since(t0);
  const int vocab = e->model->d.vocab;
  int result = Q35_OK;
  std::string first_error;
  for (size_t i = 0; i < rows.size(); ++i) {
    Request *r = rows[i];
    ++r->result.decode_forwards;
    r->result.decode_ms += ms / rows.size();
    r->result.committed_tokens = r->committed;
    if (sample) {
      const int cs = choose_token(e, *r, cands.data() + i * Q35_MAX_CANDIDATES,
                                  raw.empty() ? nullptr : raw.data() + i * static_cast<size_t>(vocab), out[i]);
      if (cs != Q35_OK) {
        // this row fails; the others keep their tokens (cpu_engine.inl:1006-1013)
        r->status = Q35_REQ_FAILED;
        if (result == Q35_OK) first_error = e->error;
        result = cs;
        continue;
      }
    }
    select_token(*r, out[i]);
  }
  if (result != Q35_OK) e->error = first_error;
  return result;
}

// Extension without a reference counterpart: prefill several requests to the
// end of their prompts in one call (the reference prefills one chunk of one
// request per advance()).
extern "C" int q35_engine_prefill_batch(q35_engine *e, const uint64_t *ids, size_t count) {
  if (e == nullptr || (count && ids == nullptr)) return Q35_ERR_INVALID;
  e->error.clear();
  if (e->serving()) return fail(e, Q35_ERR_STATE, "Serving mode must be driven through step.");
  if (count > static_cast<size_t>(e->cfg.max_decode_batch_size))
    return fail(e, Q35_ERR_INVALID, "Prefill batch exceeds max_decode_batch_size.");
  std::vector<Request *> rows;
  for (size_t i = 0; i < count; ++i) {
    auto it = e->reqs.find(ids[i]);
    if (it == e->reqs.end() || it->second.status != Q35_REQ_PREFILL ||
        std::find(rows.begin(), rows.end(), &it->second) != rows.end())
      return fail(e, Q35_ERR_INVALID, "Prefill batch requires distinct prefilling requests.");
    rows.push_back(&it->second);
  }
  for (auto *r : rows) {
    const int st = prefill_chunks(e, *r, r->prompt.size());
    if (st != Q35_OK) return st;
  }
  return Q35_OK;
}

// One packed step (q35_runtime_step_segments): a decode row of every request
// in `decode` and the next prompt chunk of every request in `prefill`. Every
// request's rows get exactly what its advance_batch / advance call would give
// it; a failed step fails every request in it (state may have moved, so it is
// never retried).
static int packed_step(q35_engine *e, const std::vector<Request *> &decode, const std::vector<Request *> &prefill) {
  const auto t0 = std::chrono::steady_clock::now();
  const int max_pages = (e->cfg.max_context + e->cfg.page_tokens - 1) / e->cfg.page_tokens;
  const size_t nd = decode.size(), n = nd + prefill.size();
  std::vector<Request *> all(decode);
  all.insert(all.end(), prefill.begin(), prefill.end());
  std::vector<int32_t> table(n * static_cast<size_t>(max_pages), 0), inputs(nd);
  std::vector<q35_segment> segs(n);
  std::vector<size_t> counts(n, 1);
  // segments that end at an automatic prefix boundary: their head row
  // carries the final hidden row the prefix keeps (its token is not used
  // unless the prompt ends there too)
  std::vector<uint8_t> publish(n, 0), ends(n, 0);
  bool sample = false;
  for (size_t i = 0; i < n; ++i) {
    Request &r = *all[i];
    const bool dec = i < nd;
    if (!dec) {
      counts[i] = advance_chunk(e, r);
      publish[i] = r.register_prefix > r.committed && r.committed + counts[i] == r.register_prefix;
      ends[i] = r.committed + counts[i] == r.prompt.size();
    }
    int st = own_page(e, r, r.committed);
    if (st == Q35_OK) st = ensure_page(e, r, r.committed + counts[i] - 1);
    if (st != Q35_OK) {
      fail_rows(all);
      return st;
    }
    std::copy(r.pages.begin(), r.pages.end(), table.begin() + i * max_pages);
    q35_segment &g = segs[i];
    g.slot = r.slot;
    g.pos0 = static_cast<int32_t>(r.committed);
    g.count = static_cast<int32_t>(counts[i]);
    if (dec) inputs[i] = r.pending;
    g.tokens = dec ? &inputs[i] : r.prompt.data() + r.committed;
    g.page_table = table.data() + i * max_pages;
    g.max_pages = max_pages;
    g.penalty = r.penalty;
    g.count_input = dec ? 1 : 0;
    g.want_token = dec || ends[i] || publish[i];
    if ((dec || ends[i]) && !is_greedy(r)) sample = true;
  }
  std::vector<int32_t> out(n, -1);
  std::vector<q35_row_sampling> rs;
  std::vector<q35_candidate> cands;
  std::vector<float> raw;
  if (sample) {
    bool need_raw = false;
    for (auto *r : all) {
      rs.push_back(row_sampling(*r));
      need_raw = need_raw || needs_raw_logits(*r);
    }
    cands.assign(n * Q35_MAX_CANDIDATES, q35_candidate{});
    raw.assign(need_raw ? n * static_cast<size_t>(e->model->d.vocab) : 0, 0.0F);
  }
  const int st = q35_runtime_step_segments(e->rt, segs.data(), static_cast<int32_t>(n), sample ? rs.data() : nullptr,
                                           out.data(), sample ? cands.data() : nullptr,
                                           raw.empty() ? nullptr : raw.data());
  if (st != Q35_OK) {
    fail_rows(all);
    return fail(e, st, e->model->ctx->error.c_str());
  }
  // hidden rows of the head rows (want_token segments in order), for the
  // prefixes published by this step
  const size_t H = static_cast<size_t>(e->model->d.hidden);
  std::vector<float> hidden;
  std::vector<size_t> head_of(n, 0);
  if (std::find(publish.begin(), publish.end(), 1) != publish.end()) {
    size_t heads = 0;
    for (size_t i = 0; i < n; ++i)
      if (segs[i].want_token) head_of[i] = heads++;
    hidden.assign(heads * H, 0.0F);
    if (q35_runtime_last_hidden(e->rt, hidden.data(), hidden.size()) != Q35_OK) hidden.clear();
  }
  count_forward(e, !sample);
  if (nd > 0) {
    ++e->stats.batch_ticks;
    e->stats.batch_rows += nd;
  }
  if (prefill.size() > 1) {
    ++e->stats.shared_prefill_ticks;
    e->stats.shared_prefill_requests += prefill.size();
  }
  if (nd > 0 && !prefill.empty()) {
    ++e->stats.packed_ticks;
    e->stats.packed_rows += nd + std::accumulate(counts.begin() + nd, counts.end(), size_t{0});
  }
  const double ms = ms_since(t0) / n;
  const int vocab = e->model->d.vocab;
  int result = Q35_OK;
  std::string first_error;
  for (size_t i = 0; i < n; ++i) {
    Request &r = *all[i];
    const bool dec = i < nd;
    r.committed += counts[i];
    if (dec) {
      ++r.result.decode_forwards;
      r.result.decode_ms += ms;
    } else {
      r.result.prefill_tokens += counts[i];
      r.result.prefill_ms += ms;
    }
    r.result.committed_tokens = r.committed;
    if (publish[i]) publish_prefix(e, r, hidden.empty() ? nullptr : hidden.data() + head_of[i] * H);
    if (!segs[i].want_token || (!dec && !ends[i])) continue;
    int32_t token = out[i];
    if (sample) {
      const int cs = choose_token(e, r, cands.data() + i * Q35_MAX_CANDIDATES,
                                  raw.empty() ? nullptr : raw.data() + i * static_cast<size_t>(vocab), token);
      if (cs != Q35_OK) {
        // this request fails; the others keep their tokens (cpu_engine.inl:1006-1013)
        r.status = Q35_REQ_FAILED;
        if (result == Q35_OK) first_error = e->error;
        result = cs;
        continue;
      }
    }
    select_token(r, token);
  }
  if (result != Q35_OK) e->error = first_error;
  return result;
}

extern "C" int q35_engine_step(q35_engine *e, int32_t *progressed) {
  if (e == nullptr || progressed == nullptr) return Q35_ERR_INVALID;
  *progressed = 0;
  e->error.clear();
  if (!e->serving() || e->scheduling)
    return fail(e, Q35_ERR_STATE, "step requires serving mode and a non-reentrant owner.");
  e->scheduling = true;
  struct Guard {
    bool &v;
    ~Guard() { v = false; }
  } guard{e->scheduling};
  size_t resident = 0;
  std::vector<uint64_t> queued;  // in ID order (the map is ordered)
  for (auto &kv : e->reqs) {
    retire(e, kv.second);
    resident += kv.second.resident;
    if (kv.second.status == Q35_REQ_QUEUED) queued.push_back(kv.first);
  }
  // admission: up to max_prefill_requests queued requests while resident
  // room lasts, skipping those waiting on another request's prefix build
  size_t admitted = 0;
  for (uint64_t id : queued) {
    if (resident >= static_cast<size_t>(e->cfg.max_resident_requests) ||
        admitted >= static_cast<size_t>(e->cfg.max_prefill_requests))
      break;
    Request &r = e->reqs.at(id);
    if (!prefix_admissible(e, r)) continue;
    ++admitted;
    ++resident;
    r.result.queue_ms = ms_since(r.arrival);
    *progressed = 1;
    const int st = activate(e, r);
    if (st != Q35_OK) {
      r.status = Q35_REQ_FAILED;
      retire(e, r);
      return st;
    }
  }
  // rows whose unread output is below max_buffered_tokens
  std::vector<uint64_t> prefill, decode;
  for (auto &kv : e->reqs) {
    if (!output_ready(e, kv.second)) continue;
    if (kv.second.status == Q35_REQ_PREFILL) prefill.push_back(kv.first);
    if (kv.second.status == Q35_REQ_DECODE) decode.push_back(kv.first);
  }
  auto rotate = [](std::vector<uint64_t> &ids, uint64_t last) {
    std::rotate(ids.begin(), std::upper_bound(ids.begin(), ids.end(), last), ids.end());
  };
  rotate(prefill, e->last_prefill);
  rotate(decode, e->last_decode);
  if (prefill.empty() && decode.empty()) return Q35_OK;
  *progressed = 1;
  if (e->cfg.packed_steps) {
    // packed steps (no reference counterpart): the decode batch and the
    // prompt chunks of up to max_prefill_requests requests in one step (a
    // complete prefix hit goes through advance(): its first token comes
    // from the prefix)
    auto chunkable = [&](uint64_t id) {
      const Request &r = e->reqs.at(id);
      return r.committed < r.prompt.size();
    };
    std::vector<uint64_t> shared;
    for (auto id : prefill) {
      if (shared.size() == static_cast<size_t>(e->cfg.max_prefill_requests)) break;
      if (chunkable(id)) shared.push_back(id);
    }
    if (!shared.empty() && (shared.size() > 1 || !decode.empty()) && chunkable(prefill.front())) {
      std::vector<Request *> drows, prows;
      decode.resize(std::min(decode.size(), static_cast<size_t>(e->cfg.max_decode_batch_size)));
      for (auto id : decode) drows.push_back(&e->reqs.at(id));
      if (!decode.empty()) e->last_decode = decode.back();
      for (auto id : shared) prows.push_back(&e->reqs.at(id));
      e->last_prefill = shared.back();
      e->prefer_decode = drows.empty();
      const int st = packed_step(e, drows, prows);
      for (auto *r : drows) retire(e, *r);
      for (auto *r : prows) retire(e, *r);
      return st;
    }
  }
  // the reference's alternation (cpu_engine_scheduler.inl:64-104)
  const bool do_decode = !decode.empty() && (prefill.empty() || e->prefer_decode);
  std::vector<uint64_t> work;
  if (do_decode) {
    decode.resize(std::min(decode.size(), static_cast<size_t>(e->cfg.max_decode_batch_size)));
    work = decode;
    e->last_decode = work.back();
  } else {
    work.push_back(prefill.front());
    // several requests share a prefill step only as short selected readouts
    if (e->cfg.max_prefill_requests > 1 && short_readout(e->reqs.at(work.front())))
      for (size_t i = 1; i < prefill.size(); ++i) {
        if (work.size() == static_cast<size_t>(e->cfg.max_prefill_requests)) break;
        if (short_readout(e->reqs.at(prefill[i]))) work.push_back(prefill[i]);
      }
    e->last_prefill = work.back();
  }
  e->prefer_decode = !do_decode;
  int st;
  if (do_decode) {
    st = q35_engine_advance_batch(e, work.data(), work.size());
  } else if (work.size() == 1) {
    st = q35_engine_advance(e, work.front());
  } else {
    // shared prefill: a failed step fails every request in it
    std::vector<Request *> prows;
    for (auto id : work) prows.push_back(&e->reqs.at(id));
    st = packed_step(e, {}, prows);
  }
  for (auto id : work) retire(e, e->reqs.at(id));
  return st;
}

extern "C" int q35_engine_read_output(q35_engine *e, uint64_t id, size_t max_tokens, int32_t *out, size_t *count) {
  if (e == nullptr || count == nullptr || (max_tokens != 0 && out == nullptr)) return Q35_ERR_INVALID;
  *count = 0;
  e->error.clear();
  if (!e->serving()) return fail(e, Q35_ERR_STATE, "read_output requires serving mode.");
  auto it = e->reqs.find(id);
  if (it == e->reqs.end()) return fail(e, Q35_ERR_STATE, "Unknown request ID.");
  Request &r = it->second;
  const size_t n = std::min(max_tokens, confirmed(r) - r.consumed);
  std::copy(r.output.begin() + static_cast<std::ptrdiff_t>(r.consumed),
            r.output.begin() + static_cast<std::ptrdiff_t>(r.consumed + n), out);
  r.consumed += n;
  *count = n;
  return Q35_OK;
}

extern "C" int q35_engine_result(q35_engine *e, uint64_t id, q35_request_result *out, int32_t *tokens,
                                 size_t capacity, size_t *count) {
  if (e == nullptr) return Q35_ERR_INVALID;
  auto it = e->reqs.find(id);
  if (it == e->reqs.end()) return fail(e, Q35_ERR_STATE, "Unknown request ID.");
  const Request &r = it->second;
  if (out != nullptr) {
    *out = r.result;
    out->status = r.status;
    out->committed_tokens = r.committed;
  }
  if (count != nullptr) *count = r.output.size();
  if (tokens != nullptr) std::memcpy(tokens, r.output.data(), std::min(capacity, r.output.size()) * 4);
  return Q35_OK;
}

extern "C" q35_runtime *q35_engine_runtime(q35_engine *e) { return e ? e->rt : nullptr; }

extern "C" int q35_engine_get_stats(const q35_engine *e, q35_engine_stats *out) {
  if (e == nullptr || out == nullptr) return Q35_ERR_INVALID;
  *out = e->stats;
  out->queued_requests = out->resident_requests = 0;
  std::set<int32_t> pages;
  for (const auto &kv : e->reqs) {
    out->queued_requests += kv.second.status == Q35_REQ_QUEUED;
    out->resident_requests += kv.second.resident;
    pages.insert(kv.second.pages.begin(), kv.second.pages.end());
  }
  for (const auto &p : e->prefixes) pages.insert(p->pages.begin(), p->pages.end());
  const q35_model_dims &d = e->model->d;
  // K and V rows of every full-attention layer, FP16
  const uint64_t page_bytes = static_cast<uint64_t>(e->cfg.page_tokens) * d.n_kv_heads * d.head_dim * 2 * 2 *
                              static_cast<uint64_t>(e->model->n_full);
  out->physical_kv_bytes = pages.size() * page_bytes;
  return Q35_OK;
}

extern "C" int q35_engine_cancel(q35_engine *e, uint64_t id) {
  if (e == nullptr) return Q35_ERR_INVALID;
  auto it = e->reqs.find(id);
  if (it == e->reqs.end()) return Q35_ERR_STATE;
  Request &r = it->second;
  if (!terminal(r)) r.status = Q35_REQ_CANCELLED;
  retire(e, r);
  return Q35_OK;
}

extern "C" int q35_engine_release(q35_engine *e, uint64_t id) {
  if (e == nullptr) return Q35_ERR_INVALID;
  auto it = e->reqs.find(id);
  if (it == e->reqs.end()) return Q35_ERR_STATE;
  Request &r = it->second;
  free_resident(e, r);
  if (r.prefix != 0) unpin_prefix(e, r.prefix);  // a queued request never became resident
  e->reqs.erase(it);
  return Q35_OK;
}

// ---------------------------------------------------------------- prefixes

extern "C" int q35_engine_register_prefix(q35_engine *e, const int32_t *tokens, size_t n, const char *ns,
                                          uint64_t *out) {
  if (e == nullptr || out == nullptr) return Q35_ERR_INVALID;
  *out = 0;
  e->error.clear();
  const int vocab = e->model->d.vocab;
  if (tokens == nullptr || n == 0 || n > static_cast<size_t>(e->cfg.max_context) || ns == nullptr || ns[0] == 0 ||
      !std::all_of(tokens, tokens + n, [&](int32_t t) { return t >= 0 && t < vocab; }))
    return fail(e, Q35_ERR_INVALID, "Invalid registered prefix tokens or trust namespace.");
  for (auto &p : e->prefixes)
    if (p->ns == ns && p->tokens.size() == n && std::equal(tokens, tokens + n, p->tokens.begin())) {
      ++p->pins;
      touch_prefix(e, p.get());
      *out = p->id;
      return Q35_OK;
    }
  // snapshot (one state copy and the conv ring) plus the prefix's KV rows
  const q35_model_dims &d = e->model->d;
  const size_t pages = (n + e->cfg.page_tokens - 1) / e->cfg.page_tokens;
  const size_t bytes = (static_cast<size_t>(e->rt->rec_copy_stride) + e->rt->conv_slot_stride + d.hidden) * 4 +
                       pages * e->cfg.page_tokens * static_cast<size_t>(d.n_kv_heads) * d.head_dim * 2 * 2 *
                           e->model->n_full;
  if (!prefix_room(e, bytes)) return fail(e, Q35_ERR_OOM, "Prefix store is full; active handles pin its snapshots.");
  // build: prefill the tokens on a private slot (cpu_engine_prefix.inl:56-94)
  Request tmp;
  tmp.prompt.assign(tokens, tokens + n);
  tmp.max_new = 1;
  int st = activate(e, tmp);
  if (st != Q35_OK) return st;
  st = prefill_chunks(e, tmp, n);
  std::vector<float> hidden(d.hidden);
  if (st == Q35_OK) st = q35_runtime_last_hidden(e->rt, hidden.data(), hidden.size());
  q35_state_snapshot *snap = nullptr;
  if (st == Q35_OK) st = q35_state_snapshot_create(e->rt, tmp.slot, static_cast<int32_t>(n), hidden.data(), &snap);
  (void)q35_slot_free(e->rt, tmp.slot);
  if (st != Q35_OK) {
    for (int32_t p : tmp.pages) (void)q35_page_release(e->rt, p);
    ++e->prefix_stats.prefix_build_fallbacks;
    return fail(e, st, e->error.empty() ? "Could not build the prefix." : e->error);
  }
  auto p = std::make_unique<Prefix>();
  p->id = e->next_prefix++;
  p->tokens = tmp.prompt;
  p->ns = ns;
  p->snap = snap;
  p->pages = std::move(tmp.pages);
  p->bytes = bytes;
  p->pins = 1;
  *out = p->id;
  e->prefix_bytes += bytes;
  ++e->prefix_stats.prefix_builds;
  e->prefixes.push_back(std::move(p));
  return Q35_OK;
}

extern "C" int q35_engine_find_prefix(q35_engine *e, const int32_t *tokens, size_t n, const char *ns,
                                      uint64_t *out, size_t *out_tokens) {
  if (e == nullptr || out == nullptr || (n && tokens == nullptr) || ns == nullptr) return Q35_ERR_INVALID;
  *out = 0;
  if (out_tokens) *out_tokens = 0;
  Prefix *best = nullptr;
  for (auto &p : e->prefixes)
    if (p->ns == ns && p->tokens.size() <= n && (best == nullptr || p->tokens.size() > best->tokens.size()) &&
        std::equal(p->tokens.begin(), p->tokens.end(), tokens))
      best = p.get();
  if (best == nullptr) return Q35_OK;
  ++best->pins;
  touch_prefix(e, best);
  *out = best->id;
  if (out_tokens) *out_tokens = best->tokens.size();
  return Q35_OK;
}

extern "C" int q35_engine_release_prefix(q35_engine *e, uint64_t id) {
  if (e == nullptr) return Q35_ERR_INVALID;
  Prefix *p = find_prefix_id(e, id);
  if (p == nullptr || p->pins <= 0) return fail(e, Q35_ERR_STATE, "Unknown or unpinned prefix.");
  --p->pins;
  return Q35_OK;
}

extern "C" int q35_engine_prefix_stats(const q35_engine *e, q35_prefix_stats *out) {
  if (e == nullptr || out == nullptr) return Q35_ERR_INVALID;
  *out = e->prefix_stats;
  out->prefix_entries = e->prefixes.size();
  out->prefix_bytes = e->prefix_bytes;
  return Q35_OK;
}
