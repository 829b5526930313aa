// The allocation-free variant of the kernel-level DOT4 GEMM: the activation
// layout and split-K partials live in a file-scope device array (`scratch`,
// kStaticScratchBytes per device, held until the process ends) instead of the
// context's grow-only buffer, so a caller that must not allocate device memory
// (code under stream capture, a serving loop that forbids hipMalloc) can call
// it. Each device holds its own copy of the array at its own address: context
// creation resolves that address once per device with hipGetSymbolAddress,
// and host code passes only the resolved pointer to kernels and copies.
#include "runtime.h"

#include "q35_hip_api.h"

#include <algorithm>
#include <mutex>
#include <string>

namespace q35 {
namespace {
constexpr size_t kStaticScratchBytes = size_t{16} << 20;
constexpr int kMaxDevices = 64;
}  // namespace
}  // namespace q35

// In host code this name is a host-side stand-in, not a device address: only
// HIP_SYMBOL(scratch) below may name it.
static __device__ __align__(256) unsigned char scratch[q35::kStaticScratchBytes];

namespace q35 {
namespace {
std::mutex g_static_mutex;
void *g_static_ptr[kMaxDevices] = {};

}  // namespace

int static_scratch_init(Context *ctx) {
  if (ctx->device < 0 || ctx->device >= kMaxDevices)
    return set_error(ctx, Q35_ERR_UNSUPPORTED, "device index beyond the static scratch table");
  std::lock_guard<std::mutex> lock(g_static_mutex);
  if (g_static_ptr[ctx->device] != nullptr) return Q35_OK;
  void *ptr = nullptr;
  const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (e != hipSuccess) return hip_error(ctx, e, "hipGetSymbolAddress(static scratch)");
  if (ptr == nullptr) return set_error(ctx, Q35_ERR_HIP, "static scratch resolved to a null address");
  g_static_ptr[ctx->device] = ptr;
  return Q35_OK;
}

}  // namespace q35

using namespace q35;

// The same contraction and bits as q35_q4_dot4_matmul, with no device
// allocation: tokens go through the GEMM in chunks of 64, 48, 32 or 16 (the
// largest whose layout and partials fit the static array; the K split, and so
// every output bit, does not depend on the chunk). Rejects shapes whose
// 16-token chunk does not fit. Calls that overlap on one device race on the
// array.
extern "C" int q35_q4_dot4_matmul_noalloc(q35_context *ctx, const q35_q4_0_block_x8 *matrix,
                                          const q35_q8_0_block_x4 *vectors, float *output, size_t rows,
                                          size_t vectors_count, size_t blocks, size_t stride) {
  int st = dot4_matmul_check(ctx, matrix, vectors, nullptr, output, nullptr, nullptr, rows, vectors_count, blocks,
                             stride);
  if (st != Q35_OK) return st;
  if (output == nullptr) return set_error(ctx, Q35_ERR_INVALID, "output is NULL");
  if (vectors_count % 4 != 0) return set_error(ctx, Q35_ERR_INVALID, "vector_count % 4 != 0");
  void *ptr = nullptr;
  {
    std::lock_guard<std::mutex> lock(g_static_mutex);
    if (ctx->device >= 0 && ctx->device < kMaxDevices) ptr = g_static_ptr[ctx->device];
  }
  if (ptr == nullptr) return set_error(ctx, Q35_ERR_HIP, "static scratch not resolved for this device");
  // one to four vectors run the single-launch GEMV, which needs no scratch
  size_t chunk = vectors_count <= static_cast<size_t>(kMatvecMaxVectors) ? kMaxTokens : 0;
  for (size_t c = kMaxTokens; chunk == 0 && c >= 16; c -= 16) {
    if (dot4_matmul_scratch_bytes(static_cast<int>(rows), static_cast<int>(blocks), static_cast<int>(c), false,
                                  ctx->cu_count) <= kStaticScratchBytes) {
      chunk = c;
      break;
    }
  }
  if (chunk == 0)
    return set_error(ctx, Q35_ERR_UNSUPPORTED,
                     "q35_q4_dot4_matmul_noalloc: " + std::to_string(rows) + " rows x " + std::to_string(blocks) +
                         " blocks need more than the " + std::to_string(kStaticScratchBytes >> 20) +
                         " MiB static scratch for 16 tokens");
  return dot4_matmul_run(ctx, matrix, vectors, nullptr, output, nullptr, rows, vectors_count, blocks, stride, false,
                         nullptr, nullptr, nullptr, nullptr, ptr, chunk);
}
