// Host runtime and C ABI (include/q35_hip.h): context, kernel-level entry
// points, model upload, request slots, KV page pool and the decode step.
#include "runtime.h"

#include "q35_hip_api.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <new>
#include <string>
#include <vector>

namespace q35 {

int set_error(Context *ctx, int status, const std::string &message) {
  if (ctx != nullptr) ctx->error = message;
  return status;
}

int hip_error(Context *ctx, hipError_t e, const char *what) {
  return set_error(ctx, e == hipErrorOutOfMemory ? Q35_ERR_OOM : Q35_ERR_HIP,
                   std::string(what) + ": " + hipGetErrorString(e));
}

namespace {

// Grow-only scratch owned by a context for the kernel-level entry points.
struct Scratch {
  void *ptr = nullptr;
  size_t bytes = 0;
};
std::map<const Context *, Scratch> g_scratch;

int scratch_get(Context *ctx, size_t bytes, void **out) {
  Scratch &s = g_scratch[ctx];
  if (s.bytes < bytes) {
    Q35_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    if (s.ptr != nullptr) Q35_HIP_TRY(ctx, hipFree(s.ptr));
    s.ptr = nullptr;
    s.bytes = 0;
    Q35_HIP_TRY(ctx, hipMalloc(&s.ptr, bytes));
    s.bytes = bytes;
  }
  *out = s.ptr;
  return Q35_OK;
}

size_t align256(size_t n) { return (n + 255) & ~static_cast<size_t>(255); }

int launch_status(Context *ctx, hipError_t e, const char *what) {
  return e == hipSuccess ? Q35_OK : hip_error(ctx, e, what);
}

}  // namespace
}  // namespace q35

using namespace q35;

// ====================================================================== context
extern "C" int q35_context_create(int device, void *stream, q35_context **out) {
  if (out == nullptr) return Q35_ERR_INVALID;
  *out = nullptr;
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count <= device || device < 0)
    return Q35_ERR_HIP;
  auto *ctx = new (std::nothrow) q35_context();
  if (ctx == nullptr) return Q35_ERR_OOM;
  ctx->device = device;
  if (hipSetDevice(device) != hipSuccess) {
    delete ctx;
    return Q35_ERR_HIP;
  }
  hipDeviceProp_t prop{};
  if (hipGetDeviceProperties(&prop, device) == hipSuccess) {
    ctx->cu_count = prop.multiProcessorCount;
    ctx->arch = prop.gcnArchName;
  }
  if (stream != nullptr) {
    ctx->stream = static_cast<hipStream_t>(stream);
  } else {
    if (hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking) != hipSuccess) {
      delete ctx;
      return Q35_ERR_HIP;
    }
    ctx->own_stream = true;
  }
  if (hipEventCreate(&ctx->t0) != hipSuccess || hipEventCreate(&ctx->t1) != hipSuccess) {
    if (ctx->own_stream) (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return Q35_ERR_HIP;
  }
  if (const int st = static_scratch_init(ctx); st != Q35_OK) {
    (void)hipEventDestroy(ctx->t0);
    (void)hipEventDestroy(ctx->t1);
    if (ctx->own_stream) (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return st;
  }
  *out = ctx;
  return Q35_OK;
}

extern "C" void q35_context_destroy(q35_context *ctx) {
  if (ctx == nullptr) return;
  (void)hipSetDevice(ctx->device);
  (void)hipStreamSynchronize(ctx->stream);
  auto it = g_scratch.find(ctx);
  if (it != g_scratch.end()) {
    if (it->second.ptr != nullptr) (void)hipFree(it->second.ptr);
    g_scratch.erase(it);
  }
  (void)hipEventDestroy(ctx->t0);
  (void)hipEventDestroy(ctx->t1);
  if (ctx->own_stream) (void)hipStreamDestroy(ctx->stream);
  delete ctx;
}

extern "C" int q35_context_synchronize(q35_context *ctx) {
  if (ctx == nullptr) return Q35_ERR_INVALID;
  Q35_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
  return Q35_OK;
}

extern "C" void *q35_context_stream(q35_context *ctx) { return ctx ? ctx->stream : nullptr; }

extern "C" const char *q35_context_last_error(const q35_context *ctx) {
  return ctx ? ctx->error.c_str() : "null context";
}

extern "C" const char *q35_status_string(int status) {
  switch (status) {
    case Q35_OK: return "ok";
    case Q35_ERR_INVALID: return "invalid argument";
    case Q35_ERR_HIP: return "HIP runtime error";
    case Q35_ERR_OOM: return "out of memory";
    case Q35_ERR_STATE: return "invalid state";
    case Q35_ERR_UNSUPPORTED: return "unsupported shape";
    case Q35_ERR_IO: return "I/O error";
    default: return "unknown status";
  }
}

extern "C" int q35_context_device_info(const q35_context *ctx, int *cu_count, char *arch,
                                       size_t arch_size) {
  if (ctx == nullptr) return Q35_ERR_INVALID;
  if (cu_count) *cu_count = ctx->cu_count;
  if (arch && arch_size) {
    std::strncpy(arch, ctx->arch.c_str(), arch_size - 1);
    arch[arch_size - 1] = 0;
  }
  return Q35_OK;
}

extern "C" int q35_device_alloc(q35_context *ctx, size_t bytes, void **out) {
  if (ctx == nullptr || out == nullptr) return Q35_ERR_INVALID;
  Q35_HIP_TRY(ctx, hipMalloc(out, bytes ? bytes : 1));
  return Q35_OK;
}
extern "C" int q35_device_free(q35_context *ctx, void *ptr) {
  if (ctx == nullptr) return Q35_ERR_INVALID;
  Q35_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
  Q35_HIP_TRY(ctx, hipFree(ptr));
  return Q35_OK;
}
extern "C" int q35_memcpy_h2d(q35_context *ctx, void *dst, const void *src, size_t bytes) {
  if (ctx == nullptr) return Q35_ERR_INVALID;
  Q35_HIP_TRY(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
  Q35_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
  return Q35_OK;
}
extern "C" int q35_memcpy_d2h(q35_context *ctx, void *dst, const void *src, size_t bytes) {
  if (ctx == nullptr) return Q35_ERR_INVALID;
  Q35_HIP_TRY(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
  Q35_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
  return Q35_OK;
}
extern "C" int q35_memcpy_d2d(q35_context *ctx, void *dst, const void *src, size_t bytes) {
  if (ctx == nullptr) return Q35_ERR_INVALID;
  Q35_HIP_TRY(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, ctx->stream));
  return Q35_OK;
}
extern "C" int q35_memset_device(q35_context *ctx, void *dst, int value, size_t bytes) {
  if (ctx == nullptr) return Q35_ERR_INVALID;
  Q35_HIP_TRY(ctx, hipMemsetAsync(dst, value, bytes, ctx->stream));
  return Q35_OK;
}
extern "C" int q35_timer_begin(q35_context *ctx) {
  if (ctx == nullptr) return Q35_ERR_INVALID;
  Q35_HIP_TRY(ctx, hipEventRecord(ctx->t0, ctx->stream));
  return Q35_OK;
}
extern "C" int q35_timer_end(q35_context *ctx, double *elapsed_ms) {
  if (ctx == nullptr || elapsed_ms == nullptr) return Q35_ERR_INVALID;
  Q35_HIP_TRY(ctx, hipEventRecord(ctx->t1, ctx->stream));
  Q35_HIP_TRY(ctx, hipEventSynchronize(ctx->t1));
  float ms = 0.0F;
  Q35_HIP_TRY(ctx, hipEventElapsedTime(&ms, ctx->t0, ctx->t1));
  *elapsed_ms = ms;
  return Q35_OK;
}

// ======================================================= activation preparation
static int prep_entry(q35_context *ctx, const float *input, q35_q8_0_block_x1 *x1,
                      q35_q8_0_block_x4 *x4, size_t vectors, size_t columns, bool h128,
                      uint64_t seed) {
  if (ctx == nullptr || input == nullptr || (x1 == nullptr && x4 == nullptr))
    return Q35_ERR_INVALID;
  if (columns == 0 || columns % (h128 ? 128 : 32) != 0 || vectors == 0 || vectors > (1u << 20))
    return set_error(ctx, Q35_ERR_INVALID, "invalid activation geometry");
  if (!h128 && columns % 128 != 0)
    return set_error(ctx, Q35_ERR_UNSUPPORTED, "identity preparation needs columns % 128 == 0");
  PrepArgs a;
  a.source = kPrepPlain;
  a.x = input;
  a.x_stride = static_cast<int>(columns);
  a.tokens = static_cast<int>(vectors);
  a.K = static_cast<int>(columns);
  a.h128 = h128;
  a.seed = seed;
  a.x1 = x1;
  a.x4 = x4;
  return launch_status(ctx, launch_prep(a, ctx->stream), "prep kernel");
}

extern "C" int q35_q8_0_quantize_vector_1(q35_context *ctx, const float *input,
                                          q35_q8_0_block_x1 *output, size_t blocks) {
  return prep_entry(ctx, input, output, nullptr, 1, blocks * 32, false, 0);
}
extern "C" int q35_q8_0_quantize_vectors_4(q35_context *ctx, const float *input,
                                           q35_q8_0_block_x4 *output, size_t vectors,
                                           size_t blocks) {
  if (vectors % 4 != 0) return set_error(ctx, Q35_ERR_INVALID, "vector_count % 4 != 0");
  return prep_entry(ctx, input, nullptr, output, vectors, blocks * 32, false, 0);
}
extern "C" int q35_q4_h128_prepare_activation_1(q35_context *ctx, const float *input,
                                                q35_q8_0_block_x1 *output, size_t columns,
                                                uint64_t seed) {
  return prep_entry(ctx, input, output, nullptr, 1, columns, true, seed);
}
extern "C" int q35_q4_h128_prepare_activations_4(q35_context *ctx, const float *input,
                                                 q35_q8_0_block_x4 *output, size_t vectors,
                                                 size_t columns, uint64_t seed) {
  if (vectors % 4 != 0) return set_error(ctx, Q35_ERR_INVALID, "vector_count % 4 != 0");
  return prep_entry(ctx, input, nullptr, output, vectors, columns, true, seed);
}

// ================================================================ DOT4 GEMM
namespace q35 {
int dot4_matmul_check(Context *ctx, const q35_q4_0_block_x8 *m, const q35_q8_0_block_x4 *x4,
                      const q35_q8_0_block_x1 *x1, const void *out, const int32_t *dots, const int32_t *index,
                      size_t rows, size_t vectors, size_t blocks, size_t stride) {
  if (ctx == nullptr || m == nullptr || (x4 == nullptr && x1 == nullptr) ||
      (out == nullptr && dots == nullptr && index == nullptr))
    return Q35_ERR_INVALID;
  if (rows == 0 || rows % 8 != 0 || blocks == 0 || vectors == 0 || rows > (1u << 28) ||
      blocks > (1u << 16) || (out != nullptr && stride < rows))
    return set_error(ctx, Q35_ERR_INVALID, "invalid DOT4 geometry");
  return Q35_OK;
}

size_t dot4_matmul_scratch_bytes(int rows, int nb, int chunk, bool argmax, int cu_count) {
  const size_t tiles = static_cast<size_t>(chunk + 15) / 16;
  const size_t code_bytes = align256(tiles * 64 * static_cast<size_t>(nb) * sizeof(uint64_t));
  const size_t scale_bytes = align256(tiles * 16 * static_cast<size_t>(nb) * sizeof(float));
  const size_t cand_bytes =
      argmax ? align256(static_cast<size_t>(gemm_argmax_cand_capacity(rows, cu_count)) * kMaxTokens * 8) : 0;
  // dense chunks write finished rows: no partials
  const size_t part_bytes = chunk > kMaxTokens ? 0 : align256(gemm_partial_floats(rows, nb, chunk, cu_count) * 4);
  return code_bytes + scale_bytes + cand_bytes + part_bytes;
}

// Runs the GEMM over `vectors` tokens, `chunk` (a multiple of 16; above
// kMaxTokens only for plain outputs, which then run the dense GEMM) at a time, from X4 or X1 activations, with the activation
// layout, candidates and split partials in `scratch` (at least
// dot4_matmul_scratch_bytes). `exact` forces the single-wave fma chain per
// row. With `index` set it runs the greedy head instead (penalty + argmax per
// vector). The K split depends on rows and blocks only, so every chunk size
// gives the same bits.
int dot4_matmul_run(Context *ctx, const q35_q4_0_block_x8 *m, const q35_q8_0_block_x4 *x4,
                    const q35_q8_0_block_x1 *x1, float *out, int32_t *dots, size_t rows, size_t vectors,
                    size_t blocks, size_t stride, bool exact, int32_t *index, float *value, const int32_t *counts,
                    const float *penalties, void *scratch, size_t chunk) {
  const int nb = static_cast<int>(blocks);
  if (out != nullptr && dots == nullptr && index == nullptr && !exact && vectors <= kMatvecMaxVectors) {
    // one to four vectors: the single-launch dot4 GEMV (bit-exact chains)
    const hipError_t e = launch_dot4_matvec(m, x4 != nullptr ? static_cast<const void *>(x4) : x1, x4 != nullptr,
                                            static_cast<int>(vectors), static_cast<int>(rows), nb, out,
                                            static_cast<long long>(stride), ctx->stream);
    if (e != hipSuccess) return hip_error(ctx, e, "dot4 GEMV kernel");
    return Q35_OK;
  }
  const size_t tiles = (chunk + 15) / 16;
  const size_t code_bytes = align256(tiles * 64 * static_cast<size_t>(nb) * sizeof(uint64_t));
  const size_t scale_bytes = align256(tiles * 16 * static_cast<size_t>(nb) * sizeof(float));
  const size_t cand_bytes =
      index != nullptr
          ? align256(static_cast<size_t>(gemm_argmax_cand_capacity(static_cast<int>(rows), ctx->cu_count)) * kMaxTokens * 8)
          : 0;
  char *base = static_cast<char *>(scratch);
  auto *codes = reinterpret_cast<uint64_t *>(base);
  auto *scales = reinterpret_cast<float *>(base + code_bytes);
  auto *cand = reinterpret_cast<unsigned long long *>(base + code_bytes + scale_bytes);
  auto *partials = reinterpret_cast<float *>(base + code_bytes + scale_bytes + cand_bytes);
  for (size_t t0 = 0; t0 < vectors; t0 += chunk) {
    const size_t n = std::min(chunk, vectors - t0);
    hipError_t e;
    if (x4 != nullptr)
      e = launch_x4_to_a16(x4 + (t0 / 4) * blocks, static_cast<int>(n), nb, codes, scales, ctx->stream);
    else
      e = launch_x1_to_a16(x1 + t0 * blocks, static_cast<int>(n), nb, codes, scales, ctx->stream);
    if (e != hipSuccess) return hip_error(ctx, e, "activation layout kernel");
    GemmArgs g;
    g.w = m;
    g.rows = static_cast<int>(rows);
    g.nb = nb;
    g.codes = codes;
    g.scales = scales;
    g.tokens = static_cast<int>(n);
    g.out = out ? out + t0 * stride : nullptr;
    g.stride = static_cast<int>(stride);
    g.partials = partials;
    g.block_dots = dots ? dots + t0 * rows * blocks : nullptr;
    g.exact = exact;
    g.cu_count = ctx->cu_count;
    if (index != nullptr) {
      g.cand = cand;
      g.cand_stride = kMaxTokens;
      g.counts = counts ? counts + t0 * rows : nullptr;
      g.counts_stride = static_cast<long long>(rows);
      g.penalties = penalties ? penalties + t0 : nullptr;
    }
    if (chunk > static_cast<size_t>(kMaxTokens)) {
      // many tokens: the dense GEMM writes the finished rows (same bits)
      e = launch_gemm_dense(g, ctx->stream);
      if (e != hipSuccess) return hip_error(ctx, e, "dense DOT4 GEMM kernel");
      continue;
    }
    e = launch_gemm(g, ctx->stream);
    if (e != hipSuccess) return hip_error(ctx, e, "DOT4 GEMM kernel");
    const GemmPlan plan = gemm_plan(g.rows, nb, exact || dots != nullptr, index != nullptr, ctx->cu_count, 0, 0);
    if (out != nullptr && plan.split > 1) {
      SplitRows src;
      src.p = partials;
      src.splits = plan.split;
      src.split_stride = static_cast<long long>(n) * rows;
      src.width = static_cast<int>(rows);
      e = launch_split_reduce(src, static_cast<int>(n), out + t0 * stride, static_cast<int>(stride), nullptr,
                              ctx->stream);
      if (e != hipSuccess) return hip_error(ctx, e, "split reduce");
    }
    if (index != nullptr) {
      const int ncand = gemm_argmax_cands(g.rows, nb, static_cast<int>(n), ctx->cu_count);
      e = launch_argmax_finalize(cand, ncand, kMaxTokens, static_cast<int>(n), index + t0,
                                 value ? value + t0 : nullptr, ctx->stream);
      if (e != hipSuccess) return hip_error(ctx, e, "argmax finalize");
    }
  }
  return Q35_OK;
}
}  // namespace q35

namespace {
// The kernel-level DOT4 entry points: chunks of kMaxTokens tokens through the
// context's grow-only scratch.
int matmul_entry(q35_context *ctx, const q35_q4_0_block_x8 *m, const q35_q8_0_block_x4 *x4,
                 const q35_q8_0_block_x1 *x1, float *out, int32_t *dots, size_t rows,
                 size_t vectors, size_t blocks, size_t stride, bool exact, int32_t *index,
                 float *value, const int32_t *counts, const float *penalties) {
  int st = dot4_matmul_check(ctx, m, x4, x1, out, dots, index, rows, vectors, blocks, stride);
  if (st != Q35_OK) return st;
  // plain outputs of more than kMaxTokens vectors: dense chunks (a chunk is
  // a multiple of 16, so X4 groups never straddle two)
  const bool dense = out != nullptr && dots == nullptr && index == nullptr && !exact &&
                     vectors > static_cast<size_t>(kMaxTokens);
  const size_t chunk = dense ? std::min<size_t>((vectors + 15) / 16 * 16, kDenseChunk) : kMaxTokens;
  void *scratch = nullptr;
  // one to four plain outputs: the single-launch GEMV, no scratch
  if (out != nullptr && dots == nullptr && index == nullptr && !exact && vectors <= kMatvecMaxVectors)
    return dot4_matmul_run(ctx, m, x4, x1, out, dots, rows, vectors, blocks, stride, exact, index, value, counts,
                           penalties, nullptr, chunk);
  st = scratch_get(ctx,
                   dot4_matmul_scratch_bytes(static_cast<int>(rows), static_cast<int>(blocks), static_cast<int>(chunk),
                                             index != nullptr, ctx->cu_count),
                   &scratch);
  if (st != Q35_OK) return st;
  return dot4_matmul_run(ctx, m, x4, x1, out, dots, rows, vectors, blocks, stride, exact, index, value, counts,
                         penalties, scratch, chunk);
}
}  // namespace

extern "C" int q35_q4_dot4_matvec(q35_context *ctx, const q35_q4_0_block_x8 *matrix,
                                  const q35_q8_0_block_x1 *vector, float *output, size_t rows,
                                  size_t blocks) {
  return matmul_entry(ctx, matrix, nullptr, vector, output, nullptr, rows, 1, blocks, rows, false,
                      nullptr, nullptr, nullptr, nullptr);
}
extern "C" int q35_q4_dot4_matmul_x1(q35_context *ctx, const q35_q4_0_block_x8 *matrix,
                                     const q35_q8_0_block_x1 *vectors, float *output, size_t rows, size_t count,
                                     size_t blocks, size_t stride) {
  return matmul_entry(ctx, matrix, nullptr, vectors, output, nullptr, rows, count, blocks, stride, false,
                      nullptr, nullptr, nullptr, nullptr);
}
extern "C" int q35_q4_dot4_has_x1_tile(size_t count) { return count >= 1 ? 1 : 0; }
extern "C" int q35_q4_dot4_matmul(q35_context *ctx, const q35_q4_0_block_x8 *matrix,
                                  const q35_q8_0_block_x4 *vectors, float *output, size_t rows,
                                  size_t count, size_t blocks, size_t stride) {
  if (count % 4 != 0) return set_error(ctx, Q35_ERR_INVALID, "vector_count % 4 != 0");
  return matmul_entry(ctx, matrix, vectors, nullptr, output, nullptr, rows, count, blocks, stride,
                      false, nullptr, nullptr, nullptr, nullptr);
}
// Bit-exact FP32 variant (no public declaration in the reference; used by the parity tests).
extern "C" int q35_q4_dot4_matmul_exact(q35_context *ctx, const q35_q4_0_block_x8 *matrix,
                                        const q35_q8_0_block_x4 *vectors, float *output,
                                        size_t rows, size_t count, size_t blocks, size_t stride) {
  if (count % 4 != 0) return set_error(ctx, Q35_ERR_INVALID, "vector_count % 4 != 0");
  return matmul_entry(ctx, matrix, vectors, nullptr, output, nullptr, rows, count, blocks, stride,
                      true, nullptr, nullptr, nullptr, nullptr);
}
extern "C" int q35_q4_dot4_block_dots(q35_context *ctx, const q35_q4_0_block_x8 *matrix,
                                      const q35_q8_0_block_x4 *vectors, int32_t *output,
                                      size_t rows, size_t count, size_t blocks) {
  if (count % 4 != 0) return set_error(ctx, Q35_ERR_INVALID, "vector_count % 4 != 0");
  return matmul_entry(ctx, matrix, vectors, nullptr, nullptr, output, rows, count, blocks, rows,
                      true, nullptr, nullptr, nullptr, nullptr);
}
extern "C" int q35_q4_dot4_argmax_batch(q35_context *ctx, const q35_q4_0_block_x8 *matrix,
                                        const q35_q8_0_block_x4 *vectors, const int32_t *counts,
                                        const float *penalties, size_t rows, size_t count,
                                        size_t blocks, int32_t *out_index, float *out_value) {
  if (ctx == nullptr || out_index == nullptr) return Q35_ERR_INVALID;
  if (count % 4 != 0 || count == 0) return set_error(ctx, Q35_ERR_INVALID, "vector_count % 4 != 0");
  return matmul_entry(ctx, matrix, vectors, nullptr, nullptr, nullptr, rows, count, blocks, rows, false,
                      out_index, out_value, counts, penalties);
}

// ================================================================= DeltaNet
namespace q35 {
namespace {
__global__ void delta_rows_kernel(float *state, const float *q, const float *k, const float *v,
                                  const float *alpha, const float *beta, float *out, int kd, int vd,
                                  long long row_begin) {
  const long long row = row_begin + blockIdx.x;
  const int head = static_cast<int>(row / vd), vrow = static_cast<int>(row % vd);
  const int lane = threadIdx.x;
  float *s = state + row * kd;
  const float *kh = k + static_cast<size_t>(head) * kd, *qh = q + static_cast<size_t>(head) * kd;
  const float al = alpha[head];
  float sk = 0.0F;
  for (int c = lane; c < kd; c += 64) {
    const float dec = s[c] * al;
    s[c] = dec;
    sk += dec * kh[c];
  }
  for (int m = 32; m >= 1; m >>= 1) sk += __shfl_xor(sk, m, 64);
  const float delta = (v[static_cast<size_t>(head) * vd + vrow] - sk) * beta[head];
  float sq = 0.0F;
  for (int c = lane; c < kd; c += 64) {
    const float up = s[c] + delta * kh[c];
    s[c] = up;
    sq += up * qh[c];
  }
  for (int m = 32; m >= 1; m >>= 1) sq += __shfl_xor(sq, m, 64);
  if (lane == 0) out[static_cast<size_t>(head) * vd + vrow] = sq;
}
}  // namespace
}  // namespace q35

extern "C" int q35_gated_delta_net_update_rows(q35_context *ctx, float *state, const float *q,
                                               const float *k, const float *v, const float *alpha,
                                               const float *beta, float *output, size_t heads,
                                               size_t kd, size_t vd, size_t row_begin,
                                               size_t row_end) {
  if (ctx == nullptr) return Q35_ERR_INVALID;
  const size_t total = heads * vd;
  // delta_net.cpp:193-200: empty or out-of-range row spans are a no-op
  if (row_begin >= row_end || row_begin >= total) return Q35_OK;
  const size_t end = std::min(row_end, total);
  Q35_LAUNCH((q35::delta_rows_kernel), static_cast<unsigned>(end - row_begin), 64, 0, ctx->stream, 
      state, q, k, v, alpha, beta, output, static_cast<int>(kd), static_cast<int>(vd),
      static_cast<long long>(row_begin));
  return launch_status(ctx, hipGetLastError(), "delta rows kernel");
}

extern "C" int q35_gated_delta_net_update_batch(q35_context *ctx, float *const *states,
                                                const float *q, const float *k, const float *v,
                                                const float *alpha, const float *beta,
                                                float *output, size_t batch, size_t heads,
                                                size_t kd, size_t vd) {
  if (ctx == nullptr || states == nullptr) return Q35_ERR_INVALID;
  if (kd != 128 || vd != 128) return set_error(ctx, Q35_ERR_UNSUPPORTED, "DeltaNet tile needs d_k = d_v = 128");
  DeltaArgs a;
  a.fused = false;
  a.states = states;
  a.batch = static_cast<int>(batch);
  a.k_heads = static_cast<int>(heads);
  a.v_heads = static_cast<int>(heads);
  a.kd = 128;
  a.vd = 128;
  a.q = q;
  a.k = k;
  a.v = v;
  a.alpha = alpha;
  a.beta = beta;
  a.out = output;
  return launch_status(ctx, launch_delta(a, ctx->stream), "DeltaNet kernel");
}

// ================================================================ attention
extern "C" int q35_attention_decode_paged(q35_context *ctx, const float *q, const float *gates,
                                          const uint16_t *k_pool, const uint16_t *v_pool,
                                          const int32_t *page_table, size_t max_pages,
                                          const int32_t *seq_lens, size_t page_tokens,
                                          float *output, size_t batch, int heads, int kv_heads,
                                          int head_dim, float scale) {
  if (ctx == nullptr || q == nullptr || gates == nullptr || output == nullptr) return Q35_ERR_INVALID;
  if (head_dim != 256 || kv_heads <= 0 || heads % kv_heads != 0 || batch == 0 || page_tokens == 0 ||
      (page_tokens & (page_tokens - 1)) != 0 || page_tokens > (1u << 20))
    return set_error(ctx, Q35_ERR_UNSUPPORTED,
                     "attention needs head_dim 256, heads % kv_heads == 0 and a power-of-two page size");
  std::vector<int32_t> lens(batch);
  Q35_HIP_TRY(ctx, hipMemcpyAsync(lens.data(), seq_lens, batch * 4, hipMemcpyDeviceToHost, ctx->stream));
  Q35_HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
  int max_len = 1;
  for (auto l : lens) {
    if (l <= 0 || static_cast<size_t>(l) > max_pages * page_tokens)
      return set_error(ctx, Q35_ERR_INVALID, "sequence length outside the page table");
    max_len = std::max(max_len, l);
  }
  AttnArgs a;
  a.q = q;
  a.k_pool = k_pool;
  a.v_pool = v_pool;
  a.page_table = page_table;
  a.max_pages = static_cast<int>(max_pages);
  a.page_tokens = static_cast<int>(page_tokens);
  a.seq_lens = seq_lens;
  a.batch = static_cast<int>(batch);
  a.heads = heads;
  a.kv_heads = kv_heads;
  a.head_dim = head_dim;
  a.scale = scale;
  a.split_tokens = kAttnChunkTokens;
  a.max_splits = (max_len + kAttnChunkTokens - 1) / kAttnChunkTokens;
  const size_t parts = batch * static_cast<size_t>(heads) * a.max_splits;
  void *scratch = nullptr;
  int st = scratch_get(ctx, align256(parts * 256 * 4) + align256(parts * 2 * 4), &scratch);
  if (st != Q35_OK) return st;
  a.part_o = static_cast<float *>(scratch);
  a.part_ml = reinterpret_cast<float *>(static_cast<char *>(scratch) + align256(parts * 256 * 4));
  hipError_t e = launch_attention(a, ctx->stream);
  if (e != hipSuccess) return hip_error(ctx, e, "attention kernel");
  return launch_status(ctx, launch_attention_merge(a, gates, output, nullptr, nullptr, 0, ctx->stream),
                       "attention merge");
}

extern "C" int q35_attention_cache_store_f16(q35_context *ctx, const float *input, uint16_t *output,
                                             size_t count) {
  if (ctx == nullptr) return Q35_ERR_INVALID;
  return launch_status(ctx, launch_store_f16(input, output, static_cast<long long>(count), ctx->stream),
                       "store f16");
}

// ============================================================ activation ops
extern "C" int q35_rms_norm_f32(q35_context *ctx, const float *input, const float *weight,
                                float *output, size_t rows, size_t width, float eps, float offset) {
  if (ctx == nullptr) return Q35_ERR_INVALID;
  return launch_status(ctx, launch_rms_norm(input, weight, output, static_cast<int>(rows),
                                            static_cast<int>(width), eps, offset, ctx->stream),
                       "rms norm");
}
extern "C" int q35_l2_normalize_f32(q35_context *ctx, float *values, size_t rows, size_t width,
                                    float eps, float scale) {
  if (ctx == nullptr) return Q35_ERR_INVALID;
  return launch_status(ctx, launch_l2_normalize(values, static_cast<int>(rows), static_cast<int>(width),
                                                eps, scale, ctx->stream),
                       "l2 normalize");
}
extern "C" int q35_causal_conv1d_silu_f32(q35_context *ctx, float *state, size_t ring_index, const float *input,
                                          size_t input_stride, const float *kernel_major_weights, float *output,
                                          size_t batch_size, size_t channel_count, size_t kernel_size,
                                          size_t channel_begin, size_t channel_end) {
  if (ctx == nullptr) return Q35_ERR_INVALID;
  // activation.cpp:177-179: an empty kernel or channel range is a no-op
  if (kernel_size == 0 || channel_begin >= channel_end || batch_size == 0) return Q35_OK;
  if (channel_end > channel_count || (kernel_size > 1 && ring_index >= kernel_size - 1) ||
      (batch_size > 1 && input_stride < channel_end))
    return set_error(ctx, Q35_ERR_INVALID, "conv1d: channel range, ring index or input stride out of range");
  return launch_status(ctx, launch_conv1d_silu(state, static_cast<int>(ring_index), input,
                                               static_cast<long long>(input_stride), kernel_major_weights, output,
                                               static_cast<int>(batch_size), static_cast<int>(channel_count),
                                               static_cast<int>(kernel_size), static_cast<int>(channel_begin),
                                               static_cast<int>(channel_end), ctx->stream),
                       "conv1d");
}
extern "C" int q35_silu_mul_f32(q35_context *ctx, const float *gate, const float *up, float *output,
                                size_t count) {
  if (ctx == nullptr) return Q35_ERR_INVALID;
  return launch_status(ctx, launch_silu_mul(gate, up, output, static_cast<long long>(count), ctx->stream),
                       "silu mul");
}
extern "C" int q35_rope_f32(q35_context *ctx, float *values, size_t heads, size_t head_dim,
                            size_t rope_dim, const float *cosine, const float *sine) {
  if (ctx == nullptr) return Q35_ERR_INVALID;
  // activation.cpp:131-133: invalid rotary width is a no-op
  if (rope_dim == 0 || rope_dim > head_dim || (rope_dim & 1u) != 0 || rope_dim > 512) return Q35_OK;
  return launch_status(ctx, launch_rope(values, static_cast<int>(heads), static_cast<int>(head_dim),
                                        static_cast<int>(rope_dim), cosine, sine, ctx->stream),
                       "rope");
}
