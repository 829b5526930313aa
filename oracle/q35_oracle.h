/* CPU restatement of the qwen35-cpu batched-decode path, used ONLY as the
 * parity checker by tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg. It is never part of the product path. Each function cites
 * the reference file:line whose scalar semantics it restates (paths relative
 * to the reference checkout). Parity pins are listed in q35_oracle.c. */
#ifndef Q35_ORACLE_H
#define Q35_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Byte-compatible mirrors of the reference block types (q4_0.h:36-70). */
typedef struct { uint16_t d[8]; uint8_t qs[128]; } q35o_q4x8;          /* 144 B */
typedef struct { float scales[4]; int16_t sums[4]; int8_t qs[128]; } q35o_q8x4; /* 152 B */
typedef struct { float scales[1]; int16_t sums[1]; int8_t qs[32]; int16_t pad; } q35o_q8x1; /* 40 B */
typedef struct { uint16_t d; uint8_t qs[16]; } q35o_q4_0;              /* 18 B */
/* Q4G16Tile (q4_g16.h:5-6): per 8-row x 32-column tile, binary16 scales
 * d[half][row] for columns 0-15 and 16-31, then the DOT4 code bytes */
typedef struct { uint16_t d[2][8]; uint8_t qs[128]; } q35o_g16;         /* 160 B */
/* Q8_0Block (q4_0.h:13-16): binary16 scale, 32 signed codes */
typedef struct { uint16_t d; int8_t qs[32]; } q35o_q8_0;                /* 34 B */

uint16_t q35o_float_to_half(float value);
float q35o_half_to_float(uint16_t value);
uint16_t q35o_attention_float_to_half(float value);
void q35o_attention_store_f16(const float *x, uint16_t *out, size_t n);

void q35o_q8_quantize_vector_1(const float *x, q35o_q8x1 *out, size_t blocks);
void q35o_q8_quantize_vectors_4(const float *x, q35o_q8x4 *out, size_t vectors, size_t blocks);

uint64_t q35o_h128_sign_word(size_t block, size_t word, uint64_t seed);
void q35o_h128_transform_unscaled(const float *x, float *y, size_t block, uint64_t seed);
void q35o_h128_transform(const float *x, float *y, size_t block, uint64_t seed);
int q35o_h128_prepare_activation_1(const float *x, q35o_q8x1 *out, size_t cols, uint64_t seed);
int q35o_h128_prepare_activations_4(const float *x, q35o_q8x4 *out, size_t vectors, size_t cols,
                                    uint64_t seed);
void q35o_q4_quantize_transformed(const float *x, q35o_q4_0 *out, size_t blocks);
int q35o_h128_quantize_matrix(const float *x, q35o_q4_0 *out, size_t rows, size_t cols,
                              uint64_t seed);

void q35o_dot4_pack_rows_8(const q35o_q4_0 *src, q35o_q4x8 *dst, size_t rows, size_t blocks);
void q35o_dot4_unpack_rows_8(const q35o_q4x8 *src, q35o_q4_0 *dst, size_t rows, size_t blocks);
void q35o_dot4_dequantize_row(const q35o_q4x8 *m, size_t row, float *out, size_t blocks);
void q35o_dot4_block_dots(const q35o_q4x8 *m, const int8_t *codes, const int16_t *sums,
                          int32_t *out, size_t rows, size_t blocks);
void q35o_dot4_matvec(const q35o_q4x8 *m, const q35o_q8x1 *v, float *out, size_t rows,
                      size_t blocks);
void q35o_dot4_matmul(const q35o_q4x8 *m, const q35o_q8x4 *v, float *out, size_t rows,
                      size_t count, size_t blocks, size_t stride);
void q35o_dot4_argmax(const q35o_q4x8 *m, const q35o_q8x1 *v, const int *counts, float penalty,
                      size_t offset, size_t rows, size_t blocks, float *value, size_t *index);

/* q4_g16.cpp:98-103 */
void q35o_g16_dequantize_row(const q35o_g16 *m, size_t row, float *out, size_t blocks);
/* q4_g16_matmul_wide (q4_g16_evex.cpp:25-49) and q4_g16_matvec_avx2: per
 * block, half 0 then half 1, acc = fma(float(dot_half), half(d) * s, acc);
 * out[t * stride + r] for `count` X1 activation rows */
void q35o_g16_matmul(const q35o_g16 *m, const q35o_q8x1 *v, float *out, size_t rows, size_t count,
                     size_t blocks, size_t stride);
/* q8_0_matmul with matrix scales (q8_0.cpp:160-193, the VNNI path's fma
 * chain): out[t * stride + r] = chain over blocks of fma(float(dot),
 * mscale * vscale, acc) */
void q35o_q8_matmul(const q35o_q8_0 *m, const float *mscales, const q35o_q8x1 *v, float *out, size_t rows,
                    size_t count, size_t blocks, size_t stride);
void q35o_delta_net_update_rows(float *state, const float *q, const float *k, const float *v,
                                const float *alpha, const float *beta, float *out, size_t kdim,
                                size_t vdim, size_t row_begin, size_t row_end);

void q35o_attention_decode(const float *q, const float *gates, const uint16_t *const *key_rows,
                           const uint16_t *const *value_rows, float *scores, float *out,
                           size_t query_width, int sequence_length, int heads, int kv_heads,
                           int head_dim, float scale, size_t row_begin, size_t row_end);

void q35o_rms_norm(const float *x, const float *w, float *y, size_t rows, size_t width, float eps,
                   float offset);
void q35o_l2_normalize(float *x, size_t rows, size_t width, float eps, float scale);
void q35o_conv1d_silu(float *state, size_t ring, const float *input, const float *kernel_major,
                      float *out, size_t channels, size_t kernel);
void q35o_silu_mul(const float *gate, const float *up, float *out, size_t n);
void q35o_rope(float *x, size_t heads, size_t head_dim, size_t rope_dim, const float *cosine,
               const float *sine);
float q35o_sigmoid(float x);
float q35o_softplus(float x);
void q35o_rope_tables(float theta, int rope_dim, size_t positions, float *cosine, float *sine);

/* ---- whole decode step (cpu_engine.inl:201-325) ---- */
typedef struct {
  int n_layers, hidden, intermediate, vocab;
  int n_heads, n_kv_heads, head_dim, rope_dim;
  float rope_theta, rms_eps;
  int lin_kernel, lin_k_heads, lin_v_heads, lin_k_dim, lin_v_dim;
  uint64_t sign_seed;
} q35o_dims;

typedef struct {
  int is_linear;
  const q35o_q4x8 *in_proj;   /* linear: in_proj_all; full: qkv_proj (H128 DOT4) */
  const q35o_q4x8 *out_proj;  /* linear: out_proj; full: o_proj */
  const q35o_q4x8 *gate_up;
  const q35o_q4x8 *down;
  const float *input_norm, *post_norm;
  const float *conv_w;   /* [channels][kernel] as stored (HF layout) */
  const float *lin_norm, *a_log, *dt_bias;
  const float *q_norm, *k_norm;
  /* optional Q8 gate rows of in_proj_all (weights.inl:1015-1034): the last
   * gate_rows outputs come from Q8_0 rows over the identity-basis input */
  int gate_rows;
  const q35o_q8_0 *gate_q8;
  const float *gate_scales; /* [gate_rows][hidden / 32] */
} q35o_layer;

typedef struct {
  const q35o_q4x8 *embed;  /* tied identity-basis head [vocab, hidden] */
  const q35o_g16 *embed_g16;  /* when set: the head and embedding as G16 tiles */
  const float *final_norm;
  const q35o_layer *layers;
} q35o_weights;

typedef struct {
  float **conv_state;    /* per linear layer: [(kernel-1) * channels] */
  size_t *conv_ring;     /* per linear layer */
  float **recurrent;     /* per linear layer: [v_heads][v_dim][k_dim] */
  uint16_t **keys;       /* per full layer: [capacity][kv_heads*head_dim] */
  uint16_t **values;
  int *counts;           /* [vocab] token counts (prompt + generated) */
  size_t position;       /* tokens already committed */
  size_t capacity;
} q35o_state;

/* One decode step for `batch` rows. tokens[r] is the pending input token of row
 * r; states[r] is advanced by one position. Writes the greedy token (with the
 * repetition penalty rule of cpu_engine_greedy.inl:45-57) into out_tokens (the
 * caller adds selected tokens to counts, as select() does) and,
 * when out_logits is non-null, the raw logits [batch][vocab]. Returns 0 or -1
 * when the scratch allocation fails. */
int q35o_forward_batch(const q35o_dims *d, const q35o_weights *w, q35o_state *const *states,
                       const int32_t *tokens, size_t batch, float penalty, int32_t *out_tokens,
                       float *out_logits, float *out_hidden);

/* Stage entry points (stage-wise parity): one row of one layer.
 * linear: run_linear_attention_step (layers.inl:36-217) from the projected
 * row [qkv | z | b | a] (with Q8 gate rows, their two outputs take the
 * place of b and a), the conv state [(kernel-1)][channels] with its ring
 * index (both advanced) and the recurrent state [v_heads][v_dim][k_dim]
 * (updated); core receives the gated-norm output [v_heads * v_dim].
 * full: prepare_full_attention_row + run_full_attention_step
 * (layers.inl:221-395) at `position`; keys/values [position + 1][kv_width]
 * binary16 receive the new row; cosine/sine are the RoPE row of `position`.
 * Both return 0, or -1 when the scratch allocation fails. */
int q35o_linear_attention_row(const q35o_dims *d, const q35o_layer *L, float *conv_state, size_t *ring,
                              float *recurrent, const float *projected, float *core);
int q35o_full_attention_row(const q35o_dims *d, const q35o_layer *L, uint16_t *keys, uint16_t *values,
                            size_t position, const float *cosine, const float *sine, const float *projected,
                            float *core);

#ifdef __cplusplus
}
#endif
#endif
