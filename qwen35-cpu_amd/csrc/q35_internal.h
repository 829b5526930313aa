// Internal declarations shared by the HIP kernels and the host runtime of the
// MI355X decode backend. Not part of the public ABI (include/q35_hip.h).
#pragma once

#include "q35_hip_api.h"

#include <cstddef>
#include <cstdint>
#include <string>

#include "q35_hip.h"

namespace q35 {

// ---------------------------------------------------------------- context
struct Context {
  int device = 0;
  hipStream_t stream = nullptr;
  bool own_stream = false;
  int cu_count = 0;
  std::string arch;
  std::string error;
  hipEvent_t t0 = nullptr, t1 = nullptr;
};

int set_error(Context *ctx, int status, const std::string &message);
int hip_error(Context *ctx, hipError_t e, const char *what);

#define Q35_HIP_TRY(ctx, expr)                                   \
  do {                                                           \
    hipError_t q35_e_ = (expr);                                  \
    if (q35_e_ != hipSuccess) return ::q35::hip_error((ctx), q35_e_, #expr); \
  } while (0)

// ------------------------------------------------------------- block types
static_assert(sizeof(q35_q4_0_block_x8) == 144, "Q4_0BlockX8 is 144 bytes");
static_assert(sizeof(q35_q8_0_block_x4) == 152, "Q8_0BlockX4 is 152 bytes");
static_assert(sizeof(q35_q8_0_block_x1) == 40, "Q8_0BlockX1 is 40 bytes");
static_assert(offsetof(q35_q8_0_block_x4, qs) == 24, "Q8_0BlockX4 layout");
static_assert(offsetof(q35_q8_0_block_x1, qs) == 6, "Q8_0BlockX1 layout");

// Prepared activations in the layout the MFMA GEMM consumes ("A16"): for each
// 16-token tile and 32-column block, 64 lanes x 8 bytes where lane l carries
// token (l % 16) and columns 8*(l/16) .. 8*(l/16)+7 of the block; plus one
// FP32 scale per (tile, block, token): the binary16-rounded activation scale
// with the H128 1/sqrt(128) folded in exactly as the reference does. The int8
// code sums the reference keeps beside each block (the offset-binary
// correction of q4_dot4_simd.inl:89) are re-derived by the GEMM with an MFMA.
constexpr float kH128InvSqrt = 0.08838834764831844055F;  // q4_h128.h:24
constexpr int kMaxTokens = 64;                            // rows per split GEMM launch
constexpr int kMaxStepRows = 8192;                        // rows per packed step (runtime bound)

// ------------------------------------------------------------ launchers
// All launchers enqueue on `stream` and return hipSuccess or the launch error.

// Rows of a GEMM output that may still be split along K: the consumer adds
// the `splits` partial rows in split order (deterministic).
struct SplitRows {
  const float *p = nullptr;   // [splits][tokens][width]
  int splits = 1;
  long long split_stride = 0; // tokens * width
  int width = 0;              // floats per token row
  // Loads for splits <= MS (checked by the launchers): MS loads, index
  // clamped, issued together; reduce*() then sums the first `splits` in split
  // order with selects (no branch, so loads issued after the load call are
  // not held back by a wait).
  template <int MS>
  __device__ __forceinline__ void load(int t, int col, float x[MS]) const {
    const float *q = p + static_cast<long long>(t) * width + col;
#pragma unroll
    for (int u = 0; u < MS; ++u) x[u] = q[static_cast<long long>(min(u, splits - 1)) * split_stride];
  }
  template <int MS>
  __device__ __forceinline__ float reduce(const float x[MS]) const {
    float v = x[0];
#pragma unroll
    for (int u = 1; u < MS; ++u) v = u < splits ? v + x[u] : v;
    return v;
  }
  template <int MS>
  __device__ __forceinline__ float sum(int t, int col) const {
    float x[MS];
    load<MS>(t, col, x);
    return reduce<MS>(x);
  }
  // Eight consecutive values (col % 4 == 0, width % 4 == 0).
  template <int MS>
  __device__ __forceinline__ void load8(int t, int col, q35_f32x4 x[MS][2]) const {
    const float *q = p + static_cast<long long>(t) * width + col;
#pragma unroll
    for (int u = 0; u < MS; ++u) {
      const q35_f32x4 *r = reinterpret_cast<const q35_f32x4 *>(q + static_cast<long long>(min(u, splits - 1)) * split_stride);
      x[u][0] = r[0];
      x[u][1] = r[1];
    }
  }
  template <int MS>
  __device__ __forceinline__ void reduce8(const q35_f32x4 x[MS][2], float out[8]) const {
    q35_f32x4 lo = x[0][0], hi = x[0][1];
#pragma unroll
    for (int u = 1; u < MS; ++u) {
      lo = u < splits ? lo + x[u][0] : lo;
      hi = u < splits ? hi + x[u][1] : hi;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      out[e] = lo[e];
      out[4 + e] = hi[e];
    }
  }
  template <int MS>
  __device__ __forceinline__ void sum8(int t, int col, float out[8]) const {
    q35_f32x4 x[MS][2];
    load8<MS>(t, col, x);
    reduce8<MS>(x, out);
  }
};

// Smallest supported compile-time split bound >= splits (0 when too many).
inline int split_bound(int splits) {
  return splits <= 1 ? 1 : splits <= 4 ? 4 : splits <= 8 ? 8 : splits <= 16 ? 16 : splits <= 32 ? 32 : 0;
}

// Activation preparation source modes (one wavefront per token and 128-column block).
enum PrepSource : int {
  kPrepPlain = 0,      // y = x
  kPrepSiluMul = 2,    // y = silu(gate) * up, gate/up = halves of a split 2K-wide row
};

struct PrepArgs {
  int source = kPrepPlain;
  const float *x = nullptr;      // plain: [tokens][x_stride]
  int x_stride = 0;
  SplitRows gate_up;             // silu: [splits][tokens][2K]
  // output
  int tokens = 0, K = 0;
  bool h128 = true;
  uint64_t seed = 0;
  uint64_t *codes = nullptr;       // A16 layout
  float *scales = nullptr;
  q35_q8_0_block_x4 *x4 = nullptr; // reference X4 layout (optional)
  q35_q8_0_block_x1 *x1 = nullptr; // reference X1 layout (optional)
  float *y_out = nullptr;          // optional FP32 source rows [tokens][K] (before the rotation)
};
hipError_t launch_prep(const PrepArgs &a, hipStream_t stream);

// Residual update + RMSNorm(1 + w) + activation preparation, one workgroup per
// token: x_out = x_in + sum of the split partial rows (when given),
// y = rms_norm(x_out) (prefill.inl:3-14), then H128 (or identity) int8
// quantization into A16; normed_out optionally keeps y.
struct RmsPrepArgs {
  const float *x_in = nullptr;   // [tokens][K]
  SplitRows add;                 // optional split partial rows to add (add.p == nullptr: none)
  float *x_out = nullptr;        // new residual rows (required when add.p != nullptr)
  const float *weight = nullptr; // RMSNorm weight [K]
  float eps = 1e-6F;
  int tokens = 0, K = 0;
  bool h128 = true;
  uint64_t seed = 0;
  uint64_t *codes = nullptr;
  float *scales = nullptr;
  float *normed_out = nullptr;   // optional [tokens][K]
  // optional: residual row of each output row (x_in, add and x_out rows are
  // rows[t]; codes, normed_out and gates stay at t)
  const int32_t *rows = nullptr;
  // optional Q8 gate rows (run_q8_gate_tail, weights.inl:1015-1034): the
  // normalized row quantized in the identity basis, then gate_rows Q8 rows
  // (codes [gate_rows][K], F32 block scales [gate_rows][K/32]) written as
  // gates[token][gate_rows]
  const int8_t *gate_codes = nullptr;
  const float *gate_scales = nullptr;
  int gate_rows = 0;
  float *gates = nullptr;
  // optional embedding gather in place of x_in (no rows to add): row t is
  // the dequantized embedding row of token_ids[t], written to x_out as the
  // residual stream, and the penalty counts of rows with count_input[t] set
  // count the token (dequantize_embedding_row, gguf_matrix.inl:21-26)
  const q35_q4_0_block_x8 *embed = nullptr;
  bool embed_g16 = false;  // Q4G16Tile (160-byte) tiles
  const int32_t *token_ids = nullptr;
  int32_t *counts = nullptr;
  long long counts_stride = 0;
  const int32_t *slots = nullptr;
  const uint8_t *count_input = nullptr;
};
constexpr int kMaxGateRows = 64;
constexpr int kMaxGateItems = 6144;  // gate rows x K/32 blocks staged in LDS (4B: 64 x 80)
hipError_t launch_rms_prep(const RmsPrepArgs &a, hipStream_t stream);


// Converts reference X4 blocks into the A16 layout (kernel-level matmul entry).
hipError_t launch_x4_to_a16(const q35_q8_0_block_x4 *x4, int tokens, int nb, uint64_t *codes,
                            float *scales, hipStream_t stream);
hipError_t launch_x1_to_a16(const q35_q8_0_block_x1 *x1, int tokens, int nb, uint64_t *codes,
                            float *scales, hipStream_t stream);

struct GemmArgs {
  const q35_q4_0_block_x8 *w = nullptr;
  int rows = 0, nb = 0;            // rows % 8 == 0
  const uint64_t *codes = nullptr; // A16 [token_tile][nb][64]
  const float *scales = nullptr;   // [token_tile][nb][16]
  int tokens = 0;                  // valid tokens
  float *out = nullptr;            // [tokens][stride] (single split)
  int stride = 0;
  const float *residual = nullptr; // optional, added in the epilogue, [tokens][stride]
  float *partials = nullptr;       // [split][tokens][rows] when the plan splits K
  int32_t *block_dots = nullptr;   // parity hook: [tokens][rows][nb]
  bool exact = false;              // one wavefront per row group runs all blocks
  // greedy head mode: per-workgroup best (penalised value, lowest index) keys
  unsigned long long *cand = nullptr;  // [grid][cand_stride]
  int cand_stride = 0;
  const int32_t *counts = nullptr;  // [rows of counts][counts_stride]
  const int32_t *count_rows = nullptr; // optional per-token row index into counts
  long long counts_stride = 0;
  const float *penalties = nullptr;
  int cu_count = 0;
  int force_ks = 0, force_split = 0;  // plan overrides (0 = automatic)
  int max_split = 0;                  // bound on the K splits (0 = 32)
  int group_rows = 0;                 // split path: rows per wavefront, 16 or 32 (0 = by shape)
  // tall single-split matrix (the vocabulary head): the streaming kernel
  // with activations staged in LDS; implied by `cand`
  bool head = false;
  int force_gpw = 0;  // head: 64-row groups per wavefront (0 = automatic)
  bool g16 = false;   // head: `w` holds Q4G16Tile (160-byte) tiles
};
// Launch plan of one GEMM: blocks per wavefront chunk, wavefronts per
// workgroup, K splits across workgroups, workgroups along the rows, LDS bytes.
struct GemmPlan {
  int ks, waves, split, grid;
  size_t smem;
};
// max_split bounds the K splits (a consumer that sums at most that many
// split partials); one wavefront then walks several chunks.
GemmPlan gemm_plan(int rows, int nb, bool exact, bool argmax, int cu_count, int force_ks, int force_split,
                   int max_split = 32);
// Candidate rows per token that the greedy head launch for this shape writes
// (and argmax_finalize must read).
int gemm_argmax_cands(int rows, int nb, int tokens, int cu_count, int force_gpw = 0, bool g16 = false);
// Upper bound of gemm_argmax_cands over every nb <= 4096/32 and tokens <= 64
// (the size of a candidate buffer).
int gemm_argmax_cand_capacity(int rows, int cu_count);
// Floats of partial sums a split launch writes (0 when it does not split).
size_t gemm_partial_floats(int rows, int nb, int tokens, int cu_count);
hipError_t launch_gemm(const GemmArgs &a, hipStream_t stream);
// Decode projections of one token tile (at most 16 rows) with a neighbour
// folded in (fused.hip); both give the bits of the split launch + consumer.
// gemm_norm: the RMSNorm(1 + w) + H128 preparation of complete residual rows
// as the prologue of the split projection (plan as launch_gemm with
// max_split); outputs as launch_gemm's (partials, or out for one split),
// described for the consumer in *out_rows.
struct NormGemmArgs {
  GemmArgs g;                     // w, rows, nb, tokens, partials or out/stride, cu_count
  int max_split = 32;
  const float *x = nullptr;       // [tokens][nb * 32] complete residual rows
  const float *weight = nullptr;  // RMSNorm weight, applied as (1 + w)
  float eps = 1e-6F;
  uint64_t seed = 0;
  const float *sq_groups = nullptr;  // [tokens][nb * 2] group sums of squares (gemm_resid)
  uint64_t *codes_out = nullptr;  // optional copy of the prepared A16 activations (token tile 0)
  float *scales_out = nullptr;
  float *normed_out = nullptr;    // optional normalized rows [tokens][nb * 32]
};
bool gemm_norm_fits(int rows, int nb, int tokens, int cu_count, int max_split);
hipError_t launch_gemm_norm(const NormGemmArgs &a, SplitRows *out_rows, hipStream_t stream);
// gemm_resid: x_out = residual + the projection of the A16 activations in
// g.codes/g.scales (every K split of the default plan, summed in split
// order); proj_out optionally keeps the projection rows. Rows are
// [tokens][rows]. It also leaves each token's sums of squares of x_out per
// 16-column group, which the next gemm_norm reads (the norm tree of
// norm_total_groups).
struct ResidGemmArgs {
  GemmArgs g;                     // w, rows, nb, codes, scales, tokens, cu_count
  const float *residual = nullptr;
  float *x_out = nullptr;
  float *proj_out = nullptr;
  float *sq_groups = nullptr;     // [tokens][rows / 16] sums of squares of x_out per 16-column group
  int splits = 0;                 // set by the launcher
};
bool gemm_resid_fits(int rows, int nb, int tokens, int cu_count);
hipError_t launch_gemm_resid(const ResidGemmArgs &a, hipStream_t stream);
// Dense GEMM for many tokens (any count): writes the finished rows to
// a.out [tokens][stride] with the bits the split launch of the same shape
// and consumer bound (a.max_split) gives after its consumer's ordered sum;
// no partials. K splits it reproduces:
int gemm_dense_splits(int rows, int nb, int cu_count, int max_split);
hipError_t launch_gemm_dense(const GemmArgs &a, hipStream_t stream);
// Single-launch GEMV of 1..kMatvecMaxVectors vectors in X1 blocks ([count][nb])
// or one X4 group (count 4): each output is the block-order fma chain, so the
// rows are bit-exact; out[v * stride + row]. rows % 8 == 0.
constexpr int kMatvecMaxVectors = 4;
hipError_t launch_dot4_matvec(const q35_q4_0_block_x8 *w, const void *act, bool x4, int count, int rows, int nb,
                              float *out, long long stride, hipStream_t stream);
// Whether the dense GEMM fills the GPU for `rows` x `tokens` (at least two
// two-tile units per CU, and at least as many tokens as one split launch
// takes); the split launches give the same bits, so the step picks by speed
// alone. At 64 tokens of the 4B shapes that is the gate_up projection only
// (the 64-row decode step 7.47 -> 7.26 ms); the in / qkv projections run
// faster split.
bool gemm_dense_fits(int rows, int tokens, int cu_count);
// Tokens per launch of the kernel-level dense path.
constexpr int kDenseChunk = 4096;

// The kernel-level DOT4 GEMM (runtime.cpp): argument checks, the scratch
// bytes of `chunk` tokens per launch, and the run itself over caller scratch.
int dot4_matmul_check(Context *ctx, const q35_q4_0_block_x8 *m, const q35_q8_0_block_x4 *x4,
                      const q35_q8_0_block_x1 *x1, const void *out, const int32_t *dots, const int32_t *index,
                      size_t rows, size_t vectors, size_t blocks, size_t stride);
// `chunk` tokens per launch: above kMaxTokens the dense GEMM runs (plain
// outputs only), which needs no partials.
size_t dot4_matmul_scratch_bytes(int rows, int nb, int chunk, bool argmax, int cu_count);
int dot4_matmul_run(Context *ctx, const q35_q4_0_block_x8 *m, const q35_q8_0_block_x4 *x4,
                    const q35_q8_0_block_x1 *x1, float *out, int32_t *dots, size_t rows, size_t vectors,
                    size_t blocks, size_t stride, bool exact, int32_t *index, float *value, const int32_t *counts,
                    const float *penalties, void *scratch, size_t chunk);
// Resolves, once per device, the address of the file-scope scratch array of
// the allocation-free entry point (noalloc.hip); called by context creation
// with the context's device current.
int static_scratch_init(Context *ctx);
hipError_t launch_split_reduce(const SplitRows &src, int tokens, float *out, int stride, const float *residual,
                               hipStream_t stream);
hipError_t launch_argmax_finalize(const unsigned long long *cand, int ncand, int cand_stride, int tokens,
                                  int32_t *index, float *value, hipStream_t stream);

// DeltaNet
struct DeltaArgs {
  bool fused = true;          // fused linear-attention step (conv, norms, gates, gated norm)
  float *const *states = nullptr;  // [batch] -> [v_heads][vd][kd]
  float *state_base = nullptr;     // alternative: slot-strided base
  const int32_t *slots = nullptr;  // [batch] slot of each row (with state_base)
  long long state_slot_stride = 0; // floats between slots
  // fused mode: > 0 selects double-buffered state -- the row at position p
  // reads the copy at (p & 1) * stride and writes the other one, so the
  // update never stores over the lines it just loaded (such stores leave
  // dirty lines in the last-level cache that a later streaming kernel pays
  // to write back); 0 updates in place
  long long state_copy_stride = 0;
  int batch = 0, k_heads = 0, v_heads = 0, kd = 0, vd = 0;
  // raw mode inputs
  const float *q = nullptr, *k = nullptr, *v = nullptr, *alpha = nullptr, *beta = nullptr;
  float *out = nullptr;            // raw: [batch][v_heads][vd]; fused: core [batch][v_heads*vd]
  // fused mode inputs
  SplitRows proj;                  // [splits][batch][in_rows] = [qkv | z | b | a]
  const float *gates = nullptr;    // when set: b and a rows as [batch][2 v_heads] (Q8 gate tail), proj = [qkv | z]
  float *conv_base = nullptr;      // slot-strided conv ring [kernel][channels], slot = position % kernel
  long long conv_slot_stride = 0;
  const int32_t *positions = nullptr;
  const float *conv_w = nullptr;   // kernel-major [kernel][channels]
  int kernel = 4;
  const float *dt_bias = nullptr, *ssm_a = nullptr, *norm_w = nullptr;
  float eps = 1e-6F;
  // fused mode: the gated outputs prepared as A16 activations of the out
  // projection (H128 block = value head); `out` (FP32) is optional then
  uint64_t *codes = nullptr;
  float *scales = nullptr;
  uint64_t seed = 0;
  // chunked prefill: per-token scan entries, then the raw head outputs
  // (delta_chunk_scan_floats(batch, v_heads) floats)
  float *scan = nullptr;
  // chunked prefill segments (NULL: the batch is one segment): segment of
  // each row, first row and row count of each segment
  const int32_t *row_seg = nullptr, *seg_row0 = nullptr, *seg_count = nullptr;
  int segments = 0;
  const int32_t *seg_order = nullptr;  // segments longest first (the scan's dispatch order; NULL: in order)
  // packed steps: the rows of segments of two or more rows (the chunk
  // kernels; NULL: every row) and how many leading seg_order entries such
  // segments are; the rows of one-row segments, which run delta_kernel
  const int32_t *chunk_rows = nullptr;
  int chunk_row_count = 0, scan_segments = 0;
  const int32_t *row_list = nullptr;  // delta_kernel's rows (NULL: rows 0 .. batch-1)
  int row_count = 0;
};
hipError_t launch_delta(const DeltaArgs &a, hipStream_t stream);
// Chunked prefill: each segment's rows are consecutive positions of ONE
// request (without segment arrays: the whole batch, slots[0], positions[0] + r)
// with the in-projection rows summed (one split); the state recurrence is
// scanned in order per segment, everything else runs per token.
constexpr int kDeltaScanStride = 3 * 128 + 4;  // q | k | v | alpha | beta | pad
inline size_t delta_chunk_scan_floats(int batch, int v_heads) {
  return static_cast<size_t>(batch) * v_heads * (kDeltaScanStride + 128);
}
hipError_t launch_delta_chunk(const DeltaArgs &a, hipStream_t stream);

// Sampling candidates: per row, the top_k (<= kMaxCandidates) penalized,
// temperature-scaled logits, descending (ties: lower token first).
constexpr int kMaxCandidates = 64;
struct SampleArgs {
  const float *logits = nullptr;      // [rows][logits_stride]
  long long logits_stride = 0;
  int rows = 0, vocab = 0;
  const int32_t *counts = nullptr;    // penalty counts [count_rows[r]][vocab] (optional)
  const int32_t *count_rows = nullptr;
  const float *penalties = nullptr;   // [rows] (optional: 1)
  const float *inv_temperature = nullptr;  // [rows] (optional: 1)
  const int32_t *top_k = nullptr;     // [rows], 1..kMaxCandidates (optional: 1)
  q35_candidate *out = nullptr;       // [rows][kMaxCandidates]
};
size_t sample_scratch_bytes(int rows);
hipError_t launch_sample_candidates(const SampleArgs &a, unsigned long long *scratch, hipStream_t stream);

// Full attention
struct AttnPrepArgs {
  SplitRows proj;               // [splits][batch][in_rows] = [q|gate interleaved per head | k | v]
  int batch = 0, heads = 0, kv_heads = 0, head_dim = 0, rope_dim = 0;
  const float *q_norm = nullptr, *k_norm = nullptr;
  float eps = 1e-6F;
  const float *rope_cos = nullptr, *rope_sin = nullptr;  // [max_context][rope_dim/2]
  const int32_t *positions = nullptr;
  const int32_t *page_table = nullptr;  // [segment][max_pages]
  const int32_t *row_seg = nullptr;     // segment (page-table row) of each row; NULL: the row itself
  int max_pages = 0, page_tokens = 0;
  uint16_t *k_pool = nullptr, *v_pool = nullptr;  // this layer's pool base
  float *q_out = nullptr, *gate_out = nullptr;    // [batch][heads][head_dim]
};
hipError_t launch_attn_prep(const AttnPrepArgs &a, hipStream_t stream);

struct AttnArgs {
  const float *q = nullptr;       // [batch][heads][head_dim]
  const uint16_t *k_pool = nullptr, *v_pool = nullptr;
  const int32_t *page_table = nullptr;
  int max_pages = 0, page_tokens = 0;
  const int32_t *seq_lens = nullptr;     // either seq_lens or positions(+1)
  const int32_t *positions = nullptr;
  int batch = 0, heads = 0, kv_heads = 0, head_dim = 0;
  float scale = 0.0625F;
  int split_tokens = 64, max_splits = 1;  // split_tokens must be kAttnChunkTokens
  int grid_splits = 0;            // chunks launched per row (>= the longest context's; 0: max_splits)
  // chunk partials of the decode kernel's rows, by the row's ordinal in the
  // launch (its index in row_list, or the row itself): [ordinal][heads][max_splits][..]
  float *part_o = nullptr;        // [decode rows][heads][max_splits][head_dim]
  float *part_ml = nullptr;       // [decode rows][heads][max_splits][2] (max, sum)
  // the one merged partial of each prompt row of a tiled launch, by row
  float *prompt_o = nullptr;      // [rows][heads][head_dim]
  float *prompt_ml = nullptr;     // [rows][heads][2]
  const int32_t *row_seg = nullptr;  // page-table row of each row (NULL: the row itself)
  // query tiles of a packed step or prompt chunk (NULL: one workgroup per
  // row and chunk): tile z covers rows tile_row0[z] .. + tile_rows[z] - 1,
  // consecutive positions of one segment of two or more rows, whose chunks
  // one workgroup merges itself (one partial per row); the rows of one-row
  // segments are listed in row_list and run as decode rows
  const int32_t *tile_row0 = nullptr, *tile_rows = nullptr;
  int tiles = 0;
  const int32_t *row_list = nullptr;  // rows of the decode kernel (NULL: rows 0 .. batch-1)
  int row_count = 0;
  // tiled launches: the rows of the segments of two or more rows, whose one
  // merged partial attention_finish_kernel completes
  const int32_t *prompt_rows = nullptr;
  int prompt_row_count = 0;
};
constexpr int kAttnTileRows = 16;  // query rows per tile
hipError_t launch_attention(const AttnArgs &a, hipStream_t stream);
// Merge of the chunk partials + sigmoid gate: FP32 rows into `out` and/or the
// o projection's A16 activations into codes/scales (either may be null).
// split_tokens must be kAttnChunkTokens.
constexpr int kAttnChunkTokens = 64;
hipError_t launch_attention_merge(const AttnArgs &a, const float *gates, float *out, uint64_t *codes,
                                  float *scales, uint64_t seed, hipStream_t stream);

// Elementwise / small ops (kernel-level entries and the step)
hipError_t launch_rms_norm(const float *x, const float *w, float *y, int rows, int width,
                           float eps, float offset, hipStream_t stream);
hipError_t launch_l2_normalize(float *x, int rows, int width, float eps, float scale,
                               hipStream_t stream);
hipError_t launch_conv1d_silu(float *state, int ring, const float *input, long long stride, const float *w,
                              float *out, int batch, int channels, int kernel, int begin, int end, hipStream_t stream);
hipError_t launch_silu_mul(const float *g, const float *u, float *out, long long n,
                           hipStream_t stream);
hipError_t launch_rope(float *x, int heads, int head_dim, int rope_dim, const float *c,
                       const float *s, hipStream_t stream);
hipError_t launch_store_f16(const float *x, uint16_t *y, long long n, hipStream_t stream);
// Embedding gather of the tied identity-basis head (gguf_matrix.inl:21-26) plus
// the penalty-count increment of the step's input tokens.
hipError_t launch_embed(const q35_q4_0_block_x8 *embed, int nb, const int32_t *tokens,
                        int batch, float *x, int hidden, int32_t *counts, long long counts_stride,
                        const int32_t *slots, const uint8_t *count_input, hipStream_t stream, bool g16 = false);

}  // namespace q35
