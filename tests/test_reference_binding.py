"""The reference-side C++ binding (qwen35-cpu_amd/binding/hip_engine.hpp)
compiles against the reference's own public headers
(include/qwen35x/runtime/cpu_engine.h, options.h) and links against
libq35hip.so: every CpuEngine method it mirrors is called with the
reference's request, result, config and stats types. Compile and link only
(no GPU); skipped where the reference tree or the library is absent. The
binding runs in tests/test_gpu_reference_binding.py."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_INCLUDE = "/root/reference/include"
LIB = os.path.join(ROOT, "qwen35-cpu_amd", "libq35hip.so")

USE = r'''
#include "hip_engine.hpp"
#include <cstdio>

namespace {
struct Mask final : qwen35x::CpuSamplingConstraint {
  bool apply(float *logits, std::size_t count, std::string &) override {
    for (std::size_t i = 1; i < count; i += 2) logits[i] = -1e30f;
    return true;
  }
  bool accept(std::int32_t, std::string &) override { return true; }
};
bool on_logits(void *, std::size_t, std::int32_t, const float *, std::size_t, std::string &) { return true; }
}  // namespace

int run(const char *artifact) {
  using namespace qwen35x;
  ModelProfile profile;
  profile.text.num_hidden_layers = 24;
  profile.fingerprint.attention_schedule.assign(24, AttentionBlock::linear);
  CpuLoadOptions load;
  load.cpu_q4_h128_path = artifact;
  std::string error;
  auto model = hip::HipModel::load(profile, load, error);
  if (!model) return std::fprintf(stderr, "%s\n", error.c_str()), 1;
  CpuEngineConfig config;
  config.max_decode_batch_size = 16;
  auto engine = hip::HipEngine::create(model, config, error);
  if (!engine) return 1;
  CpuRequestSpec spec;
  spec.prompt_tokens = {1, 2, 3};
  spec.sampling.temperature = 0.0f;
  spec.logits_callback = on_logits;
  spec.sampling_constraint = std::make_shared<Mask>();
  spec.trust_namespace = "ns";
  auto prefix = engine->register_prefix(std::span<const std::int32_t>(spec.prompt_tokens), "ns", error);
  const CpuRequestId id = engine->submit(spec, error, prefix);
  bool progressed = false;
  engine->step(progressed, error);
  engine->advance(id, error);
  const CpuRequestId ids[1] = {id};
  engine->advance_batch(std::span<const CpuRequestId>(ids), error);
  CpuRequestResult result;
  engine->result(id, result);
  std::vector<std::int32_t> read;
  engine->read_output(id, 4, read, error);
  const CpuEngineStats stats = engine->stats();
  auto found = engine->find_prefix(std::span<const std::int32_t>(spec.prompt_tokens), "ns");
  engine->cancel(id);
  engine->release(id);
  return static_cast<int>(stats.batch_ticks + result.output_tokens.size() + (found ? 1 : 0));
}

int main(int argc, char **argv) { return argc > 1 ? run(argv[1]) : 0; }
'''


@pytest.mark.skipif(not os.path.isdir(REF_INCLUDE), reason="the reference tree is not present")
@pytest.mark.skipif(shutil.which("g++") is None, reason="no g++")
def test_binding_compiles_against_reference_headers(tmp_path):
    src = tmp_path / "use_binding.cpp"
    src.write_text(USE)
    args = ["g++", "-std=c++20", "-Wall", "-Werror", "-I" + REF_INCLUDE, "-I" + os.path.join(ROOT, "include"),
            "-I" + os.path.join(ROOT, "qwen35-cpu_amd", "binding"), str(src)]
    if os.path.exists(LIB):
        args += ["-o", str(tmp_path / "use_binding"), "-L" + os.path.dirname(LIB), "-lq35hip",
                 "-Wl,--allow-shlib-undefined"]
    else:
        args += ["-c", "-o", str(tmp_path / "use_binding.o")]
    r = subprocess.run(args, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-4000:]
