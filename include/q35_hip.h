/* q35_hip.h -- C ABI of the MI355X (gfx950) batched-decode backend for the
 * qwen35-cpu engine.
 *
 * The reference engine runs its decode step in CpuEngine::Impl::forward_batch
 * (src/runtime/cpu_engine.inl:201-325) through free functions on raw
 * caller-owned buffers (the headers in include/qwen35x/cpu/). This header is the seam a
 * HIP backend plugs into: plain C, POD arguments, integer status codes, no
 * exceptions, no torch or HIP types in any signature. Every kernel-level entry
 * point takes DEVICE pointers and enqueues on the context's stream; the
 * *_sync helpers and q35_context_synchronize() wait for completion.
 *
 * Each declaration names the reference interface it replaces (file:line,
 * paths relative to the reference checkout).
 *
 * Threading: one owner thread per context, like the reference engine contract
 * (docs/cpu-engine-api.md:3-6). Calls on one context must not overlap.
 */
#ifndef Q35_HIP_H
#define Q35_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- status */
enum {
  Q35_OK = 0,
  Q35_ERR_INVALID = 1,     /* bad argument or geometry (state untouched)      */
  Q35_ERR_HIP = 2,         /* a HIP runtime call failed                       */
  Q35_ERR_OOM = 3,         /* device or host allocation failed                */
  Q35_ERR_STATE = 4,       /* wrong object state (unknown slot/request, ...)  */
  Q35_ERR_UNSUPPORTED = 5, /* shape outside what the kernels implement        */
  Q35_ERR_IO = 6           /* artifact read/write failure                     */
};

/* ------------------------------------------------------------ block types
 * Byte-compatible mirrors of the reference block layouts, include/qwen35x/cpu/q4_0.h:36-70.
 * Q4_0BlockX8 DOT4 encoding (q4_dot4.h:5-6): qs[32t+4r+j] = u[r][8t+j] | u[r][8t+4+j] << 4,
 * value = (u - 8) * half(d[r]); matrices are ordered [row/8][block]. */
typedef struct { uint16_t d[8]; uint8_t qs[128]; } q35_q4_0_block_x8;                  /* 144 B */
typedef struct { float scales[4]; int16_t sums[4]; int8_t qs[128]; } q35_q8_0_block_x4; /* 152 B */
typedef struct { float scales[1]; int16_t sums[1]; int8_t qs[32]; int16_t pad; } q35_q8_0_block_x1; /* 40 B */

typedef struct q35_context q35_context;

/* ------------------------------------------------------------- context
 * Replaces the executor (include/qwen35x/cpu/executor.h:45-123): the GPU grid
 * and one HIP stream take its role. stream == NULL creates a private stream;
 * otherwise the given hipStream_t is used and not destroyed. */
int q35_context_create(int device, void *stream, q35_context **out);
void q35_context_destroy(q35_context *ctx);
int q35_context_synchronize(q35_context *ctx);
void *q35_context_stream(q35_context *ctx);
const char *q35_context_last_error(const q35_context *ctx);
const char *q35_status_string(int status);
/* Device properties as read at create time: CU count, gcnArch name. */
int q35_context_device_info(const q35_context *ctx, int *cu_count, char *arch, size_t arch_size);

/* Plain device memory plumbing for callers without their own allocator. */
int q35_device_alloc(q35_context *ctx, size_t bytes, void **out);
int q35_device_free(q35_context *ctx, void *ptr);
int q35_memcpy_h2d(q35_context *ctx, void *dst, const void *src, size_t bytes); /* synchronous */
int q35_memcpy_d2h(q35_context *ctx, void *dst, const void *src, size_t bytes); /* synchronous */
int q35_memcpy_d2d(q35_context *ctx, void *dst, const void *src, size_t bytes); /* async */
int q35_memset_device(q35_context *ctx, void *dst, int value, size_t bytes);    /* async */
/* HIP-event timing on the context stream: begin() records, end() records,
 * waits, and returns the elapsed milliseconds. */
int q35_timer_begin(q35_context *ctx);
int q35_timer_end(q35_context *ctx, double *elapsed_ms);

/* -------------------------------------------------- activation preparation */
/* q8_0_quantize_vector_1, include/qwen35x/cpu/q4_0.h:109-114 (identity basis) */
int q35_q8_0_quantize_vector_1(q35_context *ctx, const float *input, q35_q8_0_block_x1 *output,
                               size_t blocks_per_vector);
/* q8_0_quantize_vectors_4, q4_0.h:101-106; vector_count % 4 == 0 */
int q35_q8_0_quantize_vectors_4(q35_context *ctx, const float *input, q35_q8_0_block_x4 *output,
                                size_t vector_count, size_t blocks_per_vector);
/* q4_h128_prepare_activation_1, include/qwen35x/cpu/q4_h128.h:94-99 */
int q35_q4_h128_prepare_activation_1(q35_context *ctx, const float *input,
                                     q35_q8_0_block_x1 *output, size_t column_count,
                                     uint64_t sign_seed);
/* q4_h128_prepare_activations_4, q4_h128.h:105-111; vector_count % 4 == 0 */
int q35_q4_h128_prepare_activations_4(q35_context *ctx, const float *input,
                                      q35_q8_0_block_x4 *output, size_t vector_count,
                                      size_t column_count, uint64_t sign_seed);

/* ------------------------------------------------------- Q4-G32-DOT4 GEMV/GEMM */
/* q4_dot4_matvec, include/qwen35x/cpu/q4_dot4.h:10-11; rows % 8 == 0 */
int q35_q4_dot4_matvec(q35_context *ctx, const q35_q4_0_block_x8 *matrix,
                       const q35_q8_0_block_x1 *vector, float *output, size_t rows,
                       size_t blocks);
/* q4_dot4_matmul, q4_dot4.h:12-13; rows % 8 == 0, vectors % 4 == 0, output
 * token-major with row stride `stride` (>= rows). */
int q35_q4_dot4_matmul(q35_context *ctx, const q35_q4_0_block_x8 *matrix,
                       const q35_q8_0_block_x4 *vectors, float *output, size_t rows,
                       size_t vectors_count, size_t blocks, size_t stride);
/* q4_dot4_matmul_x1, q4_dot4.h:15-18: `count` independently prepared X1 rows
 * ([count][blocks]) with matmul's output layout (row stride `stride`). */
int q35_q4_dot4_matmul_x1(q35_context *ctx, const q35_q4_0_block_x8 *matrix,
                          const q35_q8_0_block_x1 *vectors, float *output, size_t rows,
                          size_t count, size_t blocks, size_t stride);
/* q4_dot4_has_x1_tile, q4_dot4.h:14: whether matmul_x1 has a tiled path for
 * `count` rows (every count >= 1 runs the MFMA tiles here). */
int q35_q4_dot4_has_x1_tile(size_t count);
/* Same contraction with one wavefront per 64-row group running the whole block
 * range, so every output is the reference's single fma chain over blocks
 * (q4_dot4.cpp:43-56): bit-exact FP32. No reference counterpart; slower. */
int q35_q4_dot4_matmul_exact(q35_context *ctx, const q35_q4_0_block_x8 *matrix,
                             const q35_q8_0_block_x4 *vectors, float *output, size_t rows,
                             size_t vectors_count, size_t blocks, size_t stride);
/* No reference counterpart: for callers that cannot allocate device memory
 * (code under stream capture, serving loops or harnesses that forbid
 * hipMalloc). Same arguments, contraction and output bits as
 * q35_q4_dot4_matmul, but the activation layout and split partials live in a
 * 16 MiB file-scope device array per GPU (held until the process ends) instead
 * of context scratch; calls no allocating routine. Returns
 * Q35_ERR_UNSUPPORTED when a 16-token chunk of the shape does not fit the
 * array. Calls that overlap on one GPU race on the array. */
int q35_q4_dot4_matmul_noalloc(q35_context *ctx, const q35_q4_0_block_x8 *matrix,
                               const q35_q8_0_block_x4 *vectors, float *output, size_t rows,
                               size_t vectors_count, size_t blocks, size_t stride);
/* Integer parity hook (no reference counterpart): the exact int32 per-block dot
 * sum_k (u-8)*a that the matmul kernel forms before its FP32 scaling, written
 * as [vectors][rows][blocks]. Runs the same device code as q35_q4_dot4_matmul. */
int q35_q4_dot4_block_dots(q35_context *ctx, const q35_q4_0_block_x8 *matrix,
                           const q35_q8_0_block_x4 *vectors, int32_t *output, size_t rows,
                           size_t vectors_count, size_t blocks);
/* Batched greedy head: q4_dot4_argmax (q4_dot4.h:19-21) for `vectors_count`
 * rows sharing each weight tile, as greedy_batch_rows does
 * (src/runtime/cpu_engine_greedy.inl:12-63): per-row repetition penalty
 * (v > 0 ? v/p : v*p when counts[row][token] > 0 and p > 1), lowest index on
 * ties. counts is [vectors][rows] int32 or NULL; penalties is [vectors] or NULL.
 * Writes out_index[vectors] and out_value[vectors] (device pointers). */
int q35_q4_dot4_argmax_batch(q35_context *ctx, const q35_q4_0_block_x8 *matrix,
                             const q35_q8_0_block_x4 *vectors, const int32_t *counts,
                             const float *penalties, size_t rows, size_t vectors_count,
                             size_t blocks, int32_t *out_index, float *out_value);

/* --------------------------------------------------------------- DeltaNet */
/* gated_delta_net_update_rows, include/qwen35x/cpu/delta_net.h:18-31.
 * state [head][value_dim][key_dim]; q,k [head][key_dim]; v,out [head][value_dim]. */
int q35_gated_delta_net_update_rows(q35_context *ctx, float *state, const float *q,
                                    const float *k, const float *v, const float *alpha,
                                    const float *beta, float *output, size_t head_count,
                                    size_t key_dim, size_t value_dim, size_t row_begin,
                                    size_t row_end);
/* Batched form used by the step: `batch` requests, each with its own state at
 * states[r] (device array of device pointers). q,k [batch][head][key_dim],
 * v,output [batch][head][value_dim], alpha,beta [batch][head]. key_dim must be 128. */
int q35_gated_delta_net_update_batch(q35_context *ctx, float *const *states, const float *q,
                                     const float *k, const float *v, const float *alpha,
                                     const float *beta, float *output, size_t batch,
                                     size_t head_count, size_t key_dim, size_t value_dim);

/* ------------------------------------------------------ paged attention */
/* causal_attention_decode_gqa_pairs with AttentionKvRows
 * (include/qwen35x/cpu/full_attention.h:10-20,92-112), batched over requests
 * and walking page tables instead of per-token row pointers.
 * K/V pools are FP16 [page][page_tokens][kv_heads][head_dim]; page_table is
 * [batch][max_pages] int32 page ids; seq_lens[batch] (>= 1) tokens to attend.
 * q, gates, output are [batch][heads][head_dim]. head_dim must be 256 and
 * page_tokens a power of two (Q35_ERR_UNSUPPORTED otherwise). */
int q35_attention_decode_paged(q35_context *ctx, const float *q, const float *gates,
                               const uint16_t *k_pool, const uint16_t *v_pool,
                               const int32_t *page_table, size_t max_pages,
                               const int32_t *seq_lens, size_t page_tokens, float *output,
                               size_t batch, int heads, int kv_heads, int head_dim, float scale);
/* attention_cache_store_f16, full_attention.h:22-26 (RNE, quiet NaN) */
int q35_attention_cache_store_f16(q35_context *ctx, const float *input, uint16_t *output,
                                  size_t count);

/* ------------------------------------------------------ activation ops */
/* rms_norm_f32, include/qwen35x/cpu/activation.h:45-55 */
int q35_rms_norm_f32(q35_context *ctx, const float *input, const float *weight, float *output,
                     size_t rows, size_t width, float eps, float weight_offset);
/* l2_normalize_f32, activation.h:57-63 (in place) */
int q35_l2_normalize_f32(q35_context *ctx, float *values, size_t rows, size_t width, float eps,
                         float output_scale);
/* causal_conv1d_silu_f32, activation.h:29-43: batch_size tokens in order
 * (input row t at input + t * input_stride, output [batch][channel_count]),
 * each advancing the ring of kernel_size - 1 channel-major slots whose oldest
 * slot is ring_index; kernel-major weights; channels [channel_begin,
 * channel_end) only. */
int q35_causal_conv1d_silu_f32(q35_context *ctx, float *state, size_t ring_index, const float *input,
                               size_t input_stride, const float *kernel_major_weights, float *output,
                               size_t batch_size, size_t channel_count, size_t kernel_size,
                               size_t channel_begin, size_t channel_end);
/* silu_mul_f32, activation.h:71-77 */
int q35_silu_mul_f32(q35_context *ctx, const float *gate, const float *up, float *output,
                     size_t count);
/* rope_f32, activation.h:16-27 */
int q35_rope_f32(q35_context *ctx, float *values, size_t head_count, size_t head_dim,
                 size_t rope_dim, const float *cosine, const float *sine);

/* =================================================================== model
 * Shapes of a Qwen3.5 hybrid text model (RuntimeDims, src/runtime/weights.inl:336-357). */
typedef struct {
  int32_t n_layers, hidden, intermediate, vocab;
  int32_t n_heads, n_kv_heads, head_dim, rope_dim;
  float rope_theta, rms_eps;
  int32_t lin_kernel, lin_k_heads, lin_v_heads, lin_k_dim, lin_v_dim;
  uint64_t sign_seed;
} q35_model_dims;

/* Tensor encodings of the Q35H128 artifact (include/qwen35x/weights/q4_h128_artifact.h:13-29). */
enum {
  Q35_ENC_F32 = 0,
  Q35_ENC_Q4_0_DOT4 = 5,
  Q35_ENC_Q4_H128_DOT4 = 6,
  Q35_ENC_Q8_0 = 7,          /* row-major Q8_0Block: Q8 gate rows (linear_attn.in_proj_ba) */
  Q35_ENC_Q4_G16_DOT4 = 8    /* Q4G16Tile, identity basis: the tied embedding / head */
};

typedef struct q35_model q35_model;

/* Model upload. CpuModel::load + load_model_weights_from_q4_h128
 * (src/runtime/cpu_engine.inl:32-69, weights.inl:1624-1816): tensors are
 * addressed by their HF names and given as the artifact bytes as-is (DOT4
 * tiles, FP32 vectors). layer_is_linear[n_layers] is the attention schedule. */
int q35_model_create(q35_context *ctx, const q35_model_dims *dims,
                     const uint8_t *layer_is_linear, q35_model **out);
int q35_model_upload_tensor(q35_model *model, const char *name, int encoding,
                            const uint64_t *shape, size_t rank, const void *host_bytes,
                            size_t byte_count);
int q35_model_finalize(q35_model *model); /* checks every required tensor is present */
void q35_model_destroy(q35_model *model);
/* Reads a Q35H128 v1 artifact (src/weights/q4_h128_artifact.cpp) and uploads it.
 * The header's layers, hidden, intermediate and vocab must match dims;
 * dims->sign_seed must equal the header's H128 sign seed, or be 0 to take it. */
int q35_model_load_artifact(q35_context *ctx, const char *artifact_path,
                            const q35_model_dims *dims, const uint8_t *layer_is_linear,
                            q35_model **out);
/* Dims of the named reference shapes: 0 = 0.8B, 1 = 2B, 2 = 4B
 * (text_architecture, src/compiler/profile_loader.cpp:439-462). */
int q35_model_dims_preset(int which, q35_model_dims *dims, uint8_t *layer_is_linear,
                          size_t layer_capacity);
/* Random-init artifact in the Q35H128 v1 format: linear weights ~N(0, std)
 * pushed through the reference's H128 + Q4 packing math (q4_h128.cpp:195-252,
 * q4_dot4.cpp:5-18), identity-basis tied head, norms 0 (Qwen 1+w form), linear
 * attention norm 1, seeded A_log/dt_bias/conv weights. Host-only. */
int q35_write_random_artifact(const char *path, const q35_model_dims *dims,
                              const uint8_t *layer_is_linear, uint64_t seed, float weight_std);
/* q35_write_random_artifact with the optional encodings of the reference
 * packer (q4_h128_convert_main.cpp --head-g16 / --q8-gates): the tied head as
 * q4_g16_cpu_dot4 (encoding 8, identity basis, scale group 16) and each linear
 * layer's b, a rows as a separate q8_0 tensor linear_attn.in_proj_ba.weight
 * (encoding 7) with in_proj_all holding [qkv | z]. Host-only. */
enum { Q35_ARTIFACT_HEAD_G16 = 1u, Q35_ARTIFACT_Q8_GATES = 2u };
int q35_write_random_artifact_ex(const char *path, const q35_model_dims *dims, const uint8_t *layer_is_linear,
                                 uint64_t seed, float weight_std, uint32_t flags);
/* The FP32 rows [row0, row0+rows) x cols that the generator draws for tensor
 * `name` before packing (no reference counterpart; lets tests run the same
 * rows through the reference packer). */
int q35_random_weight_rows(const char *name, uint64_t seed, uint64_t row0, uint64_t rows,
                           uint64_t cols, float weight_std, float *out);

/* ================================================================= runtime
 * Device state for decode: request slots (DeltaNet state, conv ring, token
 * counts), a paged FP16 KV pool, work buffers and captured step graphs. */
typedef struct {
  int32_t max_slots;      /* resident requests (CpuEngineConfig::max_resident_requests) */
  int32_t max_batch;      /* rows per step (<= 64)                                      */
  int32_t max_context;    /* tokens per request (CpuEngineConfig::max_context)          */
  int32_t page_tokens;    /* tokens per KV page (a power of two)                        */
  int32_t total_pages;    /* KV pool capacity in pages; 0 = max_slots*ceil(ctx/page)    */
  int32_t use_graphs;     /* capture each step shape as a hipGraph and replay it        */
  int32_t max_step_rows;  /* rows of a packed step: decode rows plus prefill positions  */
                          /* (<= 8192; 0 = max_batch). Prefill chunks and packed steps  */
                          /* above 64 rows run the dense projection GEMM.               */
} q35_runtime_config;

/* One sampling candidate: a penalized, temperature-scaled logit and its token. */
typedef struct {
  float value;
  int32_t token;
} q35_candidate;
#define Q35_MAX_CANDIDATES 64

typedef struct q35_runtime q35_runtime;

int q35_runtime_create(q35_model *model, const q35_runtime_config *config, q35_runtime **out);
void q35_runtime_destroy(q35_runtime *rt);

/* Slot lifecycle: CpuEngine::Impl::initialize / retire (cpu_engine.inl:327-383,
 * 432-440). Allocation zeroes the slot's DeltaNet and conv state and sets its
 * token counts from the prompt (cpu_engine.inl:376-378). */
int q35_slot_alloc(q35_runtime *rt, const int32_t *prompt_tokens, size_t prompt_count,
                   int32_t *out_slot);
int q35_slot_free(q35_runtime *rt, int32_t slot);

/* KV page pool honouring KvPagesF16 (include/qwen35x/cpu/kv_pages.h:12-100):
 * pages are reference counted; q35_page_copy is the copy-on-write step used
 * when appending to a shared tail page. One page id covers every full
 * attention layer. */
int q35_page_alloc(q35_runtime *rt, int32_t *out_page);
int q35_page_retain(q35_runtime *rt, int32_t page);
int q35_page_release(q35_runtime *rt, int32_t page);
int q35_page_copy(q35_runtime *rt, int32_t src_page, int32_t dst_page, int32_t tokens);
int q35_page_refcount(q35_runtime *rt, int32_t page);
int q35_runtime_free_pages(q35_runtime *rt);

/* One decode step for `batch` rows -- the body of forward_batch
 * (cpu_engine.inl:201-325) followed by greedy_batch (cpu_engine_greedy.inl:65-128).
 * All arrays are HOST memory and are packed into device metadata once per step.
 *   slots[b]      request slot of row b (distinct)
 *   positions[b]  tokens already committed for the row (the input token is
 *                 written to KV position positions[b])
 *   tokens[b]     input token
 *   count_input[b] 1 when the input token must be added to the row's penalty
 *                 counts before the head (a generated token), 0 for prompt
 *                 tokens (already counted at slot allocation)
 *   penalties[b]  repetition penalty (1 = none)
 *   page_table    [batch][max_pages] page ids covering positions 0..positions[b]
 * out_tokens[b] receives the greedy token; out_logits, when non-NULL, receives
 * the raw logits [batch][vocab] (the full-logits path, cpu_engine.inl:321). */
typedef struct {
  int32_t batch;
  const int32_t *slots;
  const int32_t *positions;
  const int32_t *tokens;
  const uint8_t *count_input;
  const float *penalties;
  const int32_t *page_table;
  int32_t max_pages;
} q35_step_desc;
int q35_runtime_step(q35_runtime *rt, const q35_step_desc *desc, int32_t *out_tokens,
                     float *out_logits);
/* Chunked prefill of one request (a packed step of one segment): prompt
 * tokens tokens[0..count) at positions
 * pos0 .. pos0 + count - 1 run through every layer in one pass -- the prefill
 * chunk of CpuEngine::advance (cpu_engine.inl:668-790; run_forward_cpu_q8_batch,
 * prefill.inl:599-791). The DeltaNet recurrence scans the chunk in order and
 * attention is causal over the request's KV pages plus the chunk, so the
 * resulting state equals count single-token steps. count <= max(max_batch,
 * max_step_rows);
 * page_table[max_pages] covers positions 0 .. pos0 + count - 1. The prompt
 * tokens must already be counted (q35_slot_alloc does). out_token (optional)
 * receives the greedy token after the chunk's last position: the first
 * generated token when the chunk ends the prompt. */
int q35_runtime_prefill(q35_runtime *rt, int32_t slot, int32_t pos0, const int32_t *tokens,
                        int32_t count, const int32_t *page_table, int32_t max_pages, float penalty,
                        int32_t *out_token);
struct q35_row_sampling_s; /* q35_row_sampling, below */
/* One segment of a packed step: `count` consecutive positions pos0 .. of one
 * request -- a prompt chunk (prefill.inl:683-696 packs such segments of
 * several requests into one projection), or one decode row (count 1).
 *   tokens       [count] input tokens
 *   page_table   [max_pages] page ids covering positions 0 .. pos0 + count - 1
 *   count_input  1: the tokens join the slot's penalty counts before the head
 *                (generated tokens fed back), 0: prompt tokens (already counted)
 *   want_token   1: run the head on the segment's last position */
typedef struct {
  int32_t slot;
  int32_t pos0;
  int32_t count;
  const int32_t *tokens;
  const int32_t *page_table;
  int32_t max_pages;
  float penalty;
  uint8_t count_input;
  uint8_t want_token;
} q35_segment;
/* One packed step over `count` segments on distinct slots (at most max_batch
 * + 16 segments and max_step_rows rows in total): decode rows and prompt
 * chunks of several requests in one pass through every layer, e.g. config 5's
 * 64 decode rows plus a prefill chunk. Each segment's state, KV rows and
 * token equal what separate q35_runtime_step / q35_runtime_prefill calls give
 * for it, bit for bit. With `sampling` NULL, out_tokens[s] receives the greedy
 * token of each segment with want_token (-1 for the others). With `sampling`
 * ([count], read for want_token segments) the head writes logits and
 * out_candidates [count][Q35_MAX_CANDIDATES] (and raw_logits
 * [count][vocab], optional) receive them per segment; out_tokens is then -1. */
int q35_runtime_step_segments(q35_runtime *rt, const q35_segment *segments, int32_t count,
                              const struct q35_row_sampling_s *sampling, int32_t *out_tokens,
                              q35_candidate *out_candidates, float *raw_logits);
/* Sampled decoding (sample_token_from_logits, layers.inl:491-600). Per row:
 * top_k candidates (1..Q35_MAX_CANDIDATES; 1 with inv_temperature 1 is the
 * greedy argmax) of the logits after the repetition penalty
 * (apply_repetition_penalty_inplace, layers.inl:471-489) and the scaling
 * v *= inv_temperature (layers.inl:546-549), in descending order, ties to the
 * lower token (layers.inl:552-568). The host finishes softmax, top_p and the
 * draw in the reference's order. */
typedef struct q35_row_sampling_s {
  int32_t top_k;
  float inv_temperature;  /* 1 / SamplingOptions::temperature */
} q35_row_sampling;
/* One decode step (as q35_runtime_step) whose head writes the raw logits on
 * the device; out_candidates [batch][Q35_MAX_CANDIDATES] receives each row's
 * candidate list (unused entries: token -1, value -inf). raw_logits (HOST,
 * [batch][vocab], optional) receives the raw logits, for logits callbacks
 * and for samplers that need every token (top_k 0). */
int q35_runtime_step_candidates(q35_runtime *rt, const q35_step_desc *desc, const q35_row_sampling *sampling,
                                q35_candidate *out_candidates, float *raw_logits);
/* The same for one final normalized hidden row (HOST [hidden]) with a slot's
 * counts: the first token after a prefill (q35_runtime_last_hidden row 0) or
 * a complete prefix hit. out_candidates [Q35_MAX_CANDIDATES], raw_logits
 * [vocab] (optional). */
int q35_runtime_head_candidates(q35_runtime *rt, int32_t slot, const float *hidden, float penalty,
                                const q35_row_sampling *sampling, q35_candidate *out_candidates,
                                float *raw_logits);
/* A slot's penalty counts (HOST int32 [vocab]): the prompt tokens plus every
 * token fed back with count_input (CpuEngine's Sequence::counts). */
int q35_slot_counts(q35_runtime *rt, int32_t slot, int32_t *out, size_t count);
/* Copies the final normalized hidden rows of the last step ([batch][hidden]);
 * after q35_runtime_prefill, row 0 is the chunk's last position. */
int q35_runtime_last_hidden(q35_runtime *rt, float *out, size_t count);
/* Greedy head of one final normalized hidden row with a slot's penalty counts:
 * greedy_q4_token (weights.inl:1217-1295), the head a complete prefix hit runs
 * on the prefix's stored hidden row (cpu_engine.inl:711-726). hidden is HOST
 * memory [hidden]; the row is prepared exactly as the step's final norm
 * prepares it, so the token equals the one a full prefill would select. */
int q35_runtime_head(q35_runtime *rt, int32_t slot, const float *hidden, float penalty,
                     int32_t *out_token);

/* Hybrid prefix snapshot: CpuPrefix (cpu_engine.h:32-45), captured by
 * CpuEngine::register_prefix (cpu_engine_prefix.inl:31-96) and restored by
 * initialize (cpu_engine.inl:386-407). It copies, in device memory, a slot's
 * DeltaNet state and conv ring after `tokens` positions and keeps the final
 * normalized hidden row of position tokens - 1 (host memory, optional). KV
 * pages are not copied: the owner retains the pages that cover the prefix
 * (q35_page_retain) and shares them; the first append to a shared, partly
 * filled page copies it (q35_page_copy). Destroy snapshots before their runtime. */
typedef struct q35_state_snapshot q35_state_snapshot;
int q35_state_snapshot_create(q35_runtime *rt, int32_t slot, int32_t tokens, const float *hidden,
                              q35_state_snapshot **out);
int q35_state_snapshot_restore(q35_runtime *rt, const q35_state_snapshot *snap, int32_t slot);
int32_t q35_state_snapshot_tokens(const q35_state_snapshot *snap);
size_t q35_state_snapshot_bytes(const q35_state_snapshot *snap);
int q35_state_snapshot_hidden(const q35_state_snapshot *snap, float *out, size_t count);
void q35_state_snapshot_destroy(q35_state_snapshot *snap);

/* Kernel-level timing, no reference counterpart (the reference reports only
 * request-level prefill_ms/decode_ms, cpu_engine.h:147). While enabled,
 * steps launch eagerly (no graph replay) and every kernel launch is bracketed
 * by a pair of HIP events on the runtime's stream; elapsed times, launch
 * counts and the launches' algorithmic HBM bytes accumulate per kernel class
 * until q35_runtime_profile_reset. */
enum { Q35_KERNEL_EMBED = 0, Q35_KERNEL_PREP = 1, Q35_KERNEL_GEMM = 2, Q35_KERNEL_DELTA = 3,
       Q35_KERNEL_ATTN_PREP = 4, Q35_KERNEL_ATTENTION = 5, Q35_KERNEL_ARGMAX = 6,
       Q35_KERNEL_HEAD = 7, /* the vocabulary head's Q4 GEMV (greedy or full logits) */
       Q35_KERNEL_CLASSES = 8 };
int q35_runtime_set_profiling(q35_runtime *rt, int enable);
int q35_runtime_profile_reset(q35_runtime *rt);
int q35_runtime_profile_read(q35_runtime *rt, int kernel_class, double *total_ms,
                             uint64_t *launches, double *algorithmic_bytes);

/* Step timing, no reference counterpart (the reference reports request-level
 * prefill_ms/decode_ms only, cpu_engine.h:147). While enabled, each step's
 * launch -- the graph replay, or the eager launches when graphs are off -- is
 * bracketed by a pair of HIP events on the runtime's stream; their elapsed
 * time and a step count accumulate until the next q35_runtime_set_step_timing.
 * Unlike q35_runtime_set_profiling it leaves the graphs in place, so it gives
 * the GPU time of the path the engine runs; a caller's wall time per step
 * minus it is the step's host share. Each timed step waits for its end event
 * before returning (it does anyway). */
int q35_runtime_set_step_timing(q35_runtime *rt, int enable);
int q35_runtime_step_timing_read(q35_runtime *rt, double *gpu_ms, uint64_t *steps);

/* Stage trace of the decode step (no reference counterpart: a test hook for
 * stage-wise parity). While enabled, q35_runtime_step launches eagerly and,
 * for every layer, keeps a device copy of each stage's input and output --
 * the buffers the next kernel reads, plus the FP32 values a fused kernel
 * quantizes -- so that a checker can restart every stage from the GPU's own
 * input. Copies are addressed by (layer, point); the final norm's points use
 * layer = n_layers. Shapes ([batch] rows unless noted):
 *   X_IN      residual entering the layer [hidden]      NORMED_IN  input RMSNorm [hidden]
 *   CODES_*   A16 codes [tiles][hidden-or-K / 32][64] u64, SCALES_* [tiles][K / 32][16] f32
 *             (tiles = ceil(batch / 16); lane l of a block: token l % 16, columns 8(l / 16)..+7)
 *   GATES     Q8 gate rows [gate_rows]                  PROJ_IN    in projection rows [in_rows]
 *   STATE_*   linear: recurrent state read / written [v_heads][v_dim][k_dim]
 *   CONV_*    linear: conv ring [kernel][channels] before / after (slot = position % kernel)
 *   CORE      linear: gated-norm output [v_dim]; full: gated attention output [heads * head_dim]
 *   Q_ROT, ATTN_GATE  full: [heads][head_dim]           K_POOL, V_POOL  full: the layer's pools
 *   PROJ_OUT  out projection rows [hidden]              X_MID      residual after the attention block
 *   NORMED_POST [hidden]   GATE_UP [2 * intermediate]   SILU [intermediate]   DOWN [hidden]
 *   X_FINAL, HIDDEN (layer n_layers) final residual and final normalized rows [hidden] */
enum {
  Q35_TRACE_X_IN = 0, Q35_TRACE_NORMED_IN, Q35_TRACE_CODES_IN, Q35_TRACE_SCALES_IN, Q35_TRACE_GATES,
  Q35_TRACE_PROJ_IN, Q35_TRACE_STATE_BEFORE, Q35_TRACE_STATE_AFTER, Q35_TRACE_CONV_BEFORE,
  Q35_TRACE_CONV_AFTER, Q35_TRACE_CORE, Q35_TRACE_CODES_CORE, Q35_TRACE_SCALES_CORE, Q35_TRACE_Q_ROT,
  Q35_TRACE_ATTN_GATE, Q35_TRACE_K_POOL, Q35_TRACE_V_POOL, Q35_TRACE_PROJ_OUT, Q35_TRACE_X_MID,
  Q35_TRACE_NORMED_POST, Q35_TRACE_CODES_POST, Q35_TRACE_SCALES_POST, Q35_TRACE_GATE_UP, Q35_TRACE_SILU,
  Q35_TRACE_CODES_DOWN, Q35_TRACE_SCALES_DOWN, Q35_TRACE_DOWN, Q35_TRACE_X_FINAL, Q35_TRACE_HIDDEN,
  Q35_TRACE_CODES_HEAD, Q35_TRACE_SCALES_HEAD, Q35_TRACE_POINTS
};
int q35_runtime_set_trace(q35_runtime *rt, int enable);

/* Fused decode projections (no reference counterpart: a test and measurement
 * switch, on by default). Steps of at most 16 rows fold each residual +
 * RMSNorm + H128 preparation into the prologue of the projection that
 * consumes it, and finish the out / o and down projections with the residual
 * added (6 kernels per linear layer instead of 8). Disabled, the same steps
 * run the general split path; both give identical bits. */
int q35_runtime_set_fused(q35_runtime *rt, int enable);
/* Copies the traced bytes of (layer, point) of the last step into `out`
 * (at most `capacity` bytes); *bytes receives the traced size (0: none). */
int q35_runtime_trace_read(q35_runtime *rt, int layer, int point, void *out, size_t capacity, size_t *bytes);

/* ================================================================= engine
 * C mirror of qwen35x::CpuEngine (include/qwen35x/runtime/cpu_engine.h:173-215)
 * for greedy requests, built on the runtime above. IDs are monotonic and never
 * reused; one owner calls serially; a failed batch marks every row failed
 * (cpu_engine.inl:970-977). */
typedef struct q35_engine q35_engine;
enum { Q35_REQ_PREFILL = 0, Q35_REQ_DECODE = 1, Q35_REQ_COMPLETE = 2, Q35_REQ_CANCELLED = 3,
       Q35_REQ_FAILED = 4, Q35_REQ_QUEUED = 5 };
typedef struct {
  int32_t max_resident_requests;
  int32_t max_context;
  int32_t max_decode_batch_size;
  int32_t prefill_chunk_size;  /* prompt tokens per advance() of a prefilling request */
  int32_t page_tokens;
  int32_t use_graphs;
  uint64_t max_prefix_bytes;   /* CpuEngineConfig::max_prefix_bytes; 0 = 256 MiB */
  int32_t max_prefill_requests; /* CpuEngineConfig::max_prefill_requests: prompt chunks of up to this
                                   many requests share one step (1..16; 0 = 1) */
  int32_t packed_steps;         /* no reference counterpart: 1 = q35_engine_step runs the decode batch
                                   and the prompt chunks of up to max_prefill_requests requests in one
                                   packed step, 0 = the reference scheduler (cpu_engine_scheduler.inl) */
  /* CpuEngineConfig::max_queued_requests (cpu_engine.h:76-79): nonzero
   * enables bounded serving mode, driven through q35_engine_step and
   * q35_engine_read_output; submit then queues without device state, and
   * advance / advance_batch are refused outside step. The record limit is
   * max_resident_requests + max_queued_requests, terminal results included
   * until release. 0 = direct mode (submit activates at once; step and
   * read_output are refused). */
  int32_t max_queued_requests;
  /* CpuEngineConfig::max_buffered_tokens: in serving mode a request whose
   * unread output reaches this many tokens is not scheduled until
   * read_output drains it (cpu_engine.inl:429-431). Must be > 0 in serving
   * mode. */
  int32_t max_buffered_tokens;
} q35_engine_config;
/* CpuEngineStats (cpu_engine.h:151-168) for the counters this engine keeps;
 * packed_ticks / packed_rows (steps that carried decode rows and prompt
 * chunks together) have no reference counterpart. */
typedef struct {
  uint64_t batch_ticks, batch_rows;            /* advance_batch calls, their rows */
  uint64_t projection_batches;                 /* projection GEMM launches (plus greedy heads) */
  uint64_t lm_head_batches, greedy_lm_head_batches;
  uint64_t state_batches;                      /* per-layer DeltaNet / attention batches */
  uint64_t shared_prefill_ticks, shared_prefill_requests;
  uint64_t packed_ticks, packed_rows;
  uint64_t queued_requests, resident_requests;
  uint64_t physical_kv_bytes;                  /* KV pages held by requests and prefixes */
} q35_engine_stats;
typedef struct {
  int32_t status;
  uint64_t generated_tokens, committed_tokens, prefill_tokens, decode_forwards;
  double prefill_ms, decode_ms;
  uint64_t cached_prefix_tokens;  /* prompt tokens restored from a prefix snapshot */
  double prefix_restore_ms;
  double queue_ms;                /* submit to admission (serving mode) */
  uint64_t prefix_written_tokens; /* newly computed tokens published in an automatic prefix */
} q35_request_result;

/* ReferenceLogitsCallback (options.h:20) in C: called synchronously with a
 * row's raw logits before penalties and sampling; index is the output token
 * index, forced_token the forced output token or -1. Returns nonzero to go on;
 * zero fails the request. It must not call back into the engine. */
typedef int (*q35_logits_callback)(void *context, size_t index, int32_t forced_token, const float *logits,
                                   size_t count);
/* CpuSamplingConstraint (cpu_engine.h:84-94) in C, owned by the caller and
 * alive until the request ends; called by the engine owner only. apply masks
 * disallowed logits of a row in place (count = vocab; it must leave a finite
 * candidate), accept advances after the token is chosen; each returns nonzero
 * to go on, zero to fail the request. */
typedef struct {
  void *context;
  int (*apply)(void *context, float *logits, size_t count);
  int (*accept)(void *context, int32_t token);
} q35_sampling_constraint;
/* CpuRequestSpec (cpu_engine.h:105-133) without drafting. Sampling follows
 * SamplingOptions (options.h:10-13): temperature <= 1e-6 is greedy; seed < 0
 * seeds the request's mt19937 from random_device (cpu_engine.inl:379-381).
 * stop_sequences holds stop_sequence_count sequences back to back, of the
 * given lengths. select() order (cpu_engine.inl:441-465): selected readout
 * callback, logits callback, constraint apply, forced / greedy / sampled
 * token, constraint accept. A selected readout (values at the given token
 * IDs, duplicates included) needs its own callback, no logits callback,
 * max_new_tokens 1 and one forced token; a constraint cannot be combined
 * with forced or selected readout (cpu_engine.inl:866-875). */
typedef struct {
  const int32_t *prompt_tokens;
  size_t prompt_count;
  size_t max_new_tokens;
  float temperature, top_p;
  int32_t top_k;
  float repetition_penalty;
  int64_t seed;
  const int32_t *stop_token_ids;
  size_t stop_count;
  const int32_t *stop_sequences;
  const size_t *stop_sequence_lengths;
  size_t stop_sequence_count;
  const int32_t *forced_output_tokens; /* empty, or exactly max_new_tokens tokens */
  size_t forced_count;
  q35_logits_callback logits_callback;
  void *logits_callback_context;
  uint64_t prefix;                     /* 0 = none (q35_engine_register_prefix) */
  const q35_sampling_constraint *sampling_constraint; /* NULL = none */
  const int32_t *selected_logit_tokens;
  size_t selected_logit_count;
  q35_logits_callback selected_logits_callback;
  void *selected_logits_callback_context;
  /* CpuRequestSpec::register_prefix_tokens / trust_namespace
   * (cpu_engine.h:126-129, cpu_engine_singleflight.inl): serving mode only;
   * the first register_prefix_tokens prompt tokens are built once and
   * published as a prefix of trust_namespace when the request's prefill
   * reaches them; a queued request of the same build waits for it and then
   * attaches it. 0 = none. trust_namespace (NUL-terminated, may be NULL =
   * unnamed) must equal the namespace of an attached prefix when given. */
  uint64_t register_prefix_tokens;
  const char *trust_namespace;
} q35_request_spec;

int q35_engine_create(q35_model *model, const q35_engine_config *config, q35_engine **out);
void q35_engine_destroy(q35_engine *engine);
int q35_engine_submit(q35_engine *engine, const int32_t *prompt_tokens, size_t prompt_count,
                      size_t max_new_tokens, float repetition_penalty,
                      const int32_t *stop_token_ids, size_t stop_count, uint64_t *out_id);
/* CpuEngine::submit (cpu_engine.inl:832-930) with a full request spec. */
int q35_engine_submit_spec(q35_engine *engine, const q35_request_spec *spec, uint64_t *out_id);
int q35_engine_advance(q35_engine *engine, uint64_t id);
int q35_engine_advance_batch(q35_engine *engine, const uint64_t *ids, size_t count);
/* CpuEngine::step (cpu_engine_scheduler.inl:2-105): serving mode only.
 * Retires terminal requests, admits up to max_prefill_requests queued
 * requests (in ID order, skipping those whose automatic prefix another
 * request is still building), then runs one decode batch or prompt chunk,
 * alternating between the two and rotating requests for fairness. Rows whose
 * unread output holds max_buffered_tokens are skipped. *progressed = 1 when
 * any work was admitted or run. */
int q35_engine_step(q35_engine *engine, int32_t *progressed);
/* CpuEngine::read_output (cpu_engine_scheduler.inl:107-127): serving mode
 * only. Copies up to max_tokens confirmed, unread output tokens of a request
 * into out (capacity >= max_tokens) and *count; tokens that may still be the
 * start of a stop sequence are held back until resolved. */
int q35_engine_read_output(q35_engine *engine, uint64_t id, size_t max_tokens, int32_t *out, size_t *count);
/* detail::prefill_chunk_token_count (src/runtime/prefill_chunk.h:10-17): the
 * prompt tokens one advance() prefills from `position` with `remaining` left,
 * for a canonical chunk of `chunk`: up to the chunk boundary, and not past the
 * first 128 positions. Host-only; no device. */
size_t q35_prefill_chunk_token_count(size_t position, size_t remaining, size_t chunk);
/* No reference counterpart: prefill several requests, each to the end of its
 * prompt in chunks of up to prefill_chunk_size positions (the reference
 * prefills one chunk of one request per advance(), cpu_engine.inl:668-790). */
int q35_engine_prefill_batch(q35_engine *engine, const uint64_t *ids, size_t count);
/* CpuEngine::stats (cpu_engine.inl:1017-1043). */
int q35_engine_get_stats(const q35_engine *engine, q35_engine_stats *out);
int q35_engine_result(q35_engine *engine, uint64_t id, q35_request_result *out,
                      int32_t *tokens, size_t token_capacity, size_t *token_count);
int q35_engine_cancel(q35_engine *engine, uint64_t id);
/* The runtime the engine steps (for q35_runtime_set_profiling and friends). */
q35_runtime *q35_engine_runtime(q35_engine *engine);
int q35_engine_release(q35_engine *engine, uint64_t id);
const char *q35_engine_last_error(const q35_engine *engine);

/* Prefix cache: CpuEngine::register_prefix / find_prefix (cpu_engine.h:181-193,
 * cpu_engine_prefix.inl:11-96) and CpuRequestSpec::prefix (cpu_engine.h:124).
 * A prefix is a state snapshot (q35_state_snapshot) plus the KV pages of its
 * tokens, shared by every request that attaches it. Handles are nonzero ids;
 * each handle returned by register/find pins the snapshot until
 * q35_engine_release_prefix. Unpinned snapshots stay cached and are evicted
 * least recently used first when max_prefix_bytes would be exceeded
 * (cpu_engine.inl:112-143). Matching is by exact tokens and trust namespace. */
int q35_engine_register_prefix(q35_engine *engine, const int32_t *tokens, size_t count,
                               const char *trust_namespace, uint64_t *out_prefix);
/* Longest cached prefix of tokens[0..count) in the namespace; *out_prefix = 0
 * (and *out_tokens = 0) when none matches. */
int q35_engine_find_prefix(q35_engine *engine, const int32_t *tokens, size_t count,
                           const char *trust_namespace, uint64_t *out_prefix, size_t *out_tokens);
int q35_engine_release_prefix(q35_engine *engine, uint64_t prefix);
/* submit with CpuRequestSpec::prefix: the prompt must start with the prefix's
 * tokens; the request restores the snapshot instead of prefilling them
 * (cpu_engine.inl:386-407, validation :895-910). prefix 0 = none. */
int q35_engine_submit_prefixed(q35_engine *engine, const int32_t *prompt_tokens, size_t prompt_count,
                               size_t max_new_tokens, float repetition_penalty,
                               const int32_t *stop_token_ids, size_t stop_count, uint64_t prefix,
                               uint64_t *out_id);
/* CpuEngineStats' prefix counters (cpu_engine.h:160-162). */
typedef struct {
  uint64_t prefix_builds, prefix_build_fallbacks, prefix_hits, prefix_cached_tokens, prefix_evictions;
  uint64_t prefix_entries, prefix_bytes;
} q35_prefix_stats;
int q35_engine_prefix_stats(const q35_engine *engine, q35_prefix_stats *out);

#ifdef __cplusplus
}
#endif
#endif /* Q35_HIP_H */
