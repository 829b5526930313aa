// Host-side objects behind the C ABI: model weights in HBM, per-request
// device state, the paged KV pool and the captured decode step.
#pragma once

#include <array>
#include <map>
#include <set>
#include <string>
#include <utility>
#include <vector>

#include "q35_internal.h"

struct q35_context : q35::Context {};

namespace q35 {

struct LayerDev {
  bool linear = false;
  const q35_q4_0_block_x8 *in_proj = nullptr, *out_proj = nullptr, *gate_up = nullptr,
                          *down = nullptr;
  int in_rows = 0, out_cols = 0;
  const float *input_norm = nullptr, *post_norm = nullptr;
  const float *conv_w = nullptr, *lin_norm = nullptr, *dt_bias = nullptr, *ssm_a = nullptr;
  const float *q_norm = nullptr, *k_norm = nullptr;
  // Q8 gate rows (linear_attn.in_proj_ba): int8 codes [gate_rows][hidden],
  // F32 block scales [gate_rows][hidden / 32]; in_proj then holds [qkv | z]
  int gate_rows = 0;
  const int8_t *gate_codes = nullptr;
  const float *gate_scales = nullptr;
};

// Shape of one packed step: `rows` rows in `segments` segments (each a run
// of consecutive positions of one request; a decode row is a segment of one),
// `heads` rows that get a token (the last row of their segment), `tiles`
// attention query tiles, and the chunks of the longest context (rounded up
// to a power of two) the attention grid covers.
struct StepShape {
  int rows = 0, segments = 0, heads = 0, tiles = 0, grid_splits = 1;
  int attn_rows = 0;           // rows of one-row segments (the decode attention kernel in a packed step)
  bool single = true;          // every segment is one row (the decode kernels)
  bool heads_identity = true;  // head h is row h
  std::array<int, 8> key(bool want_logits) const {
    return {rows, segments, heads, tiles, grid_splits, (single ? 1 : 0) | (heads_identity ? 2 : 0),
            want_logits ? 1 : 0, attn_rows};
  }
};
constexpr int kMaxPrefillSegments = 16;  // prefill segments per packed step

}  // namespace q35

struct q35_model {
  q35::Context *ctx = nullptr;
  q35_model_dims d{};
  std::vector<uint8_t> is_linear;
  const q35_q4_0_block_x8 *embed = nullptr;
  bool embed_g16 = false;  // embed holds Q4G16Tile tiles (160 bytes per 8 x 32)
  const float *final_norm = nullptr;
  std::vector<q35::LayerDev> layers;
  std::vector<void *> allocations;
  std::set<std::string> uploaded;
  std::set<std::string> required;
  bool finalized = false;
  size_t weight_bytes = 0;  // packed projection + head bytes in HBM
  int n_linear = 0, n_full = 0;
  std::vector<int> linear_index, full_index;  // per layer
};

struct q35_runtime {
  q35_model *model = nullptr;
  q35::Context *ctx = nullptr;
  q35_runtime_config cfg{};
  int max_pages_per_row = 0;
  int max_rows = 0;      // rows per packed step (>= cfg.max_batch)
  int max_segments = 0;  // segments (and head rows) per packed step
  int split_tokens = q35::kAttnChunkTokens, max_splits = 1;
  // slot state
  float *recurrent = nullptr;  // [slots][2 copies][n_lin][vh][vd][kd]
  float *conv = nullptr;       // [slots][n_lin][kernel-1][channels]
  int32_t *counts = nullptr;   // [slots][vocab]
  long long rec_slot_stride = 0, rec_copy_stride = 0, conv_slot_stride = 0;
  std::vector<uint8_t> slot_used;
  // KV pool [n_full][pages][page_tokens][kvh][hd]
  uint16_t *k_pool = nullptr, *v_pool = nullptr;
  size_t layer_pool_elems = 0;
  std::vector<int> page_ref;
  std::vector<int> free_pages;
  float *rope_cos = nullptr, *rope_sin = nullptr;
  // work buffers
  float *x[2] = {nullptr, nullptr};  // residual stream, ping-pong
  float *sq_groups = nullptr;         // [16][hidden / 16] group sums of squares of the residual rows
  float *proj = nullptr, *q_rot = nullptr, *gates = nullptr;
  float *q8_gates = nullptr;      // Q8 gate rows of the in projection [rows][kMaxGateRows]
  float *rows_final = nullptr;  // chunked steps of split GEMMs: summed in-projection rows [rows][proj_width]
  float *delta_scan = nullptr;  // prefill: DeltaNet chunk scan entries and raw outputs
  unsigned long long *sample_scratch = nullptr;  // sampling: the slices' surviving keys
  q35_candidate *candidates = nullptr;           // sampling: [max_batch][kMaxCandidates]
  float *part_o = nullptr, *part_ml = nullptr, *logits = nullptr;
  float *prompt_o = nullptr, *prompt_ml = nullptr;  // prompt rows' merged attention partials
  float *hidden_out = nullptr;
  uint64_t *codes = nullptr;
  float *scales = nullptr;
  // greedy head: per-workgroup best keys [cand_rows][kMaxTokens]
  unsigned long long *cand = nullptr;
  int cand_rows = 0;
  int32_t *tokens_out_dev = nullptr;  // device address of tokens_out_host (pinned, mapped)
  // step metadata (pinned host + device copy)
  size_t meta_bytes = 0;
  unsigned char *meta_host = nullptr, *meta_dev = nullptr;
  int32_t *tokens_out_host = nullptr;
  size_t proj_width = 0, core_width = 0;
  q35::StepShape shape;  // of the step last packed
  std::map<std::array<int, 8>, hipGraphExec_t> graphs;
  int last_batch = 0;
  std::vector<void *> allocations;
  // kernel-level timing: event pairs reused across steps, the (class, bytes)
  // of each bracketed launch of the step in flight, and per-class totals
  bool profiling = false;
  std::vector<std::pair<hipEvent_t, hipEvent_t>> prof_events;
  struct ProfLaunch {
    int cls;       // kernel class
    double bytes;  // algorithmic bytes (on the first kernel of a logical launch)
    bool counted;  // first kernel of a logical launch
  };
  std::vector<ProfLaunch> prof_pending;
  // decode steps of one token tile run the fused projections (fused.hip)
  bool fuse_decode = true;
  // stage trace (test hook): (layer, point) -> device copy and its size
  bool tracing = false;
  std::map<std::pair<int, int>, std::pair<void *, size_t>> trace;
  double prof_ms[Q35_KERNEL_CLASSES] = {};
  double prof_bytes[Q35_KERNEL_CLASSES] = {};
  uint64_t prof_launches[Q35_KERNEL_CLASSES] = {};
  // step timing: one event pair around each step's launch (graphs still
  // replayed) and the accumulated GPU time
  bool step_timing = false;
  hipEvent_t step_events[2] = {nullptr, nullptr};
  double step_gpu_ms = 0.0;
  uint64_t step_count = 0;
};

namespace q35 {
// Enqueues one packed step whose metadata is in rt->meta_host (the host copy
// is part of the enqueued work, so the step can be captured as a graph).
int runtime_enqueue_step(q35_runtime *rt, const StepShape &shape, bool want_logits);
// Algorithmic HBM bytes of one GEMM launch: packed weights, A16 codes and
// scales of every token, FP32 outputs (and the residual read when fused).
double gemm_algorithmic_bytes(int rows, int nb, int tokens, bool stores, bool residual);
}
