// A serving loop on the reference-side binding (hip_engine.hpp), driven the
// way the reference's server drives CpuEngine (src/server.cpp:255-300): build
// a ModelProfile, HipModel::load, HipEngine::create in serving mode, submit
// every request, then step() and read_output() each active request after
// every step until all are terminal, releasing each as it finishes.
//
// Built by __graft_entry__.build() against the reference's public headers
// (the profile, options and engine types are the reference's own) and run by
// tests/test_gpu_reference_binding.py on the GPU.
//
// Usage: serve_binding <artifact> <requests file> key=value ...
//   keys: layers hidden intermediate heads kv_heads head_dim lin_k_heads
//   lin_v_heads lin_k_dim lin_v_dim conv vocab interval (full attention
//   every `interval` layers), resident queued batch prefill_requests
//   buffered max_new register (automatic prefix tokens, 0 = none) ns
//   read (tokens per read_output call)
// The requests file holds one prompt per line (token IDs separated by
// spaces). Output: one line per request, "request <i> <status> <tokens...>",
// then "stats builds=<n> hits=<n> steps=<n>".
#include "hip_engine.hpp"

#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <map>
#include <sstream>
#include <string>
#include <vector>

namespace {

const char *status_name(qwen35x::CpuRequestStatus s) {
  using S = qwen35x::CpuRequestStatus;
  switch (s) {
    case S::prefill: return "prefill";
    case S::decode: return "decode";
    case S::complete: return "complete";
    case S::cancelled: return "cancelled";
    case S::failed: return "failed";
    case S::queued: return "queued";
  }
  return "?";
}

}  // namespace

int main(int argc, char **argv) {
  using namespace qwen35x;
  if (argc < 3) {
    std::fprintf(stderr, "usage: serve_binding <artifact> <requests> key=value ...\n");
    return 2;
  }
  std::map<std::string, std::string> kv;
  for (int i = 3; i < argc; ++i) {
    const std::string a = argv[i];
    const auto eq = a.find('=');
    if (eq == std::string::npos) return std::fprintf(stderr, "bad argument %s\n", argv[i]), 2;
    kv[a.substr(0, eq)] = a.substr(eq + 1);
  }
  auto num = [&](const char *k, long long dflt) { return kv.count(k) ? std::atoll(kv[k].c_str()) : dflt; };

  // the profile profile_loader.cpp builds for a Qwen3.5 text model
  ModelProfile profile;
  TextModelConfig &t = profile.text;
  t.num_hidden_layers = static_cast<int>(num("layers", 24));
  t.hidden_size = static_cast<int>(num("hidden", 1024));
  t.intermediate_size = static_cast<int>(num("intermediate", 3584));
  t.num_attention_heads = static_cast<int>(num("heads", 8));
  t.num_key_value_heads = static_cast<int>(num("kv_heads", 2));
  t.head_dim = static_cast<int>(num("head_dim", 256));
  t.linear_conv_kernel_dim = static_cast<int>(num("conv", 4));
  t.linear_num_key_heads = static_cast<int>(num("lin_k_heads", 16));
  t.linear_num_value_heads = static_cast<int>(num("lin_v_heads", 16));
  t.linear_key_head_dim = static_cast<int>(num("lin_k_dim", 128));
  t.linear_value_head_dim = static_cast<int>(num("lin_v_dim", 128));
  t.vocab_size = static_cast<int>(num("vocab", 248320));
  t.full_attention_interval = static_cast<int>(num("interval", 4));
  profile.fingerprint.num_hidden_layers = t.num_hidden_layers;
  for (int i = 0; i < t.num_hidden_layers; ++i)
    profile.fingerprint.attention_schedule.push_back((i + 1) % t.full_attention_interval == 0 ? AttentionBlock::full
                                                                                               : AttentionBlock::linear);
  CpuLoadOptions load;
  load.cpu_q4_h128_path = argv[1];

  std::vector<std::vector<std::int32_t>> prompts;
  {
    std::ifstream in(argv[2]);
    std::string line;
    while (std::getline(in, line)) {
      std::istringstream ls(line);
      std::vector<std::int32_t> p;
      for (long long v; ls >> v;) p.push_back(static_cast<std::int32_t>(v));
      if (!p.empty()) prompts.push_back(std::move(p));
    }
  }
  std::string error;
  auto model = hip::HipModel::load(profile, load, error);
  if (!model) return std::fprintf(stderr, "load: %s\n", error.c_str()), 1;
  CpuEngineConfig config;
  config.max_resident_requests = static_cast<std::size_t>(num("resident", 4));
  config.max_queued_requests = static_cast<std::size_t>(num("queued", 16));
  config.max_decode_batch_size = static_cast<std::size_t>(num("batch", 4));
  config.max_prefill_requests = static_cast<std::size_t>(num("prefill_requests", 1));
  config.max_buffered_tokens = static_cast<std::size_t>(num("buffered", 256));
  config.max_context = static_cast<std::size_t>(num("context", 1024));
  auto engine = hip::HipEngine::create(model, config, error);
  if (!engine) return std::fprintf(stderr, "create: %s\n", error.c_str()), 1;

  struct Active {
    CpuRequestId id;
    std::size_t index;
    std::vector<std::int32_t> output;
  };
  std::vector<Active> active;
  const std::size_t register_tokens = static_cast<std::size_t>(num("register", 0));
  for (std::size_t i = 0; i < prompts.size(); ++i) {
    CpuRequestSpec spec;
    spec.prompt_tokens = prompts[i];
    spec.max_new_tokens = static_cast<std::size_t>(num("max_new", 8));
    spec.sampling.temperature = 0.0F;
    spec.sampling.repetition_penalty = 1.0F;
    spec.trust_namespace = kv.count("ns") ? kv["ns"] : "bench";
    if (register_tokens != 0 && prompts[i].size() >= register_tokens) spec.register_prefix_tokens = register_tokens;
    const CpuRequestId id = engine->submit(std::move(spec), error);
    if (!id) return std::fprintf(stderr, "submit %zu: %s\n", i, error.c_str()), 1;
    active.push_back({id, i, {}});
  }
  std::vector<std::string> lines(prompts.size());
  const std::size_t read_limit = static_cast<std::size_t>(num("read", 5));
  long long steps = 0;
  while (!active.empty()) {
    bool progressed = false;
    if (!engine->step(progressed, error)) return std::fprintf(stderr, "step: %s\n", error.c_str()), 1;
    ++steps;
    for (auto it = active.begin(); it != active.end();) {
      CpuRequestResult result;
      if (!engine->read_output(it->id, read_limit, it->output, error) || !engine->result(it->id, result))
        return std::fprintf(stderr, "read_output: %s\n", error.c_str()), 1;
      const bool terminal = result.status == CpuRequestStatus::complete ||
                            result.status == CpuRequestStatus::cancelled || result.status == CpuRequestStatus::failed;
      if (terminal && it->output.size() == result.output_tokens.size()) {
        std::string s = "request " + std::to_string(it->index) + " " + status_name(result.status);
        for (auto tok : it->output) s += " " + std::to_string(tok);
        s += " cached=" + std::to_string(result.cached_prefix_tokens);
        lines[it->index] = s;
        engine->release(it->id);
        it = active.erase(it);
      } else {
        ++it;
      }
    }
    if (!progressed && steps > 100000) return std::fprintf(stderr, "no progress\n"), 1;
  }
  for (const auto &l : lines) std::printf("%s\n", l.c_str());
  const CpuEngineStats st = engine->stats();
  std::printf("stats builds=%llu hits=%llu steps=%lld\n", static_cast<unsigned long long>(st.prefix_builds),
              static_cast<unsigned long long>(st.prefix_hits), steps);
  return 0;
}
