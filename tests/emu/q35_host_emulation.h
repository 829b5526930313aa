// Test-only host emulation of the HIP subset used by qwen35-cpu_amd/csrc.
// Compiling the unchanged kernel sources with -DQ35_HOST_EMULATION runs every
// kernel on host threads (one std::thread per work-item, blocks of a launch
// in sequence), so AddressSanitizer bounds-checks every device access on the
// CPU. Wavefront operations are emulated with 64-lane barriers:
//   __shfl_xor     exchange through a per-wavefront slot array
//   MFMA i8        v_mfma_i32_16x16x32_i8 operand layout: A lane l = row l%16,
//                  k 8*(l/16)..+7; B lane l = column l%16, same k; D lane l =
//                  rows 4*(l/16)..+3 of column l%16
//   __syncthreads  std::barrier over the block
// Device memory is plain heap memory; streams are synchronous; stream capture
// records launches and copies and graph launch replays them.
#pragma once

#include <algorithm>
#include <atomic>
#include <barrier>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <memory>
#include <thread>
#include <vector>

using std::max;
using std::min;
using std::isnan;

#define __global__
#define __device__
#define __host__
#define __forceinline__ inline
#define __launch_bounds__(...)
#define Q35_WAVES_PER_EU(n)
#define __align__(n) alignas(n)
// Blocks of one launch run one after another, so a function-local static is a
// faithful per-block shared array.
#define __shared__ static

struct dim3 {
  unsigned x, y, z;
  dim3(unsigned a = 1, unsigned b = 1, unsigned c = 1) : x(a), y(b), z(c) {}
};
struct uint2 { unsigned x, y; };
struct uint4 { unsigned x, y, z, w; };
struct float4 { float x, y, z, w; };
inline uint4 make_uint4(unsigned a, unsigned b, unsigned c, unsigned d) { return {a, b, c, d}; }
inline float4 make_float4(float a, float b, float c, float d) { return {a, b, c, d}; }

namespace q35emu {

struct Launch {
  std::barrier<> *block = nullptr;
  std::vector<std::unique_ptr<std::barrier<>>> waves;
  std::vector<std::vector<uint64_t>> slots_a, slots_b, slots_c, slots_d;  // per wave, 64 lanes
  std::vector<float> dynamic_smem;
};

struct ThreadCtx {
  dim3 thread_idx, block_idx, block_dim, grid_dim;
  Launch *launch = nullptr;
  int lane = 0, wave = 0;
};
inline thread_local ThreadCtx t_ctx;

inline void wave_sync() { t_ctx.launch->waves[t_ctx.wave]->arrive_and_wait(); }

// value of `v` in lane `src` of the wavefront (every lane must call it)
inline int readlane(int v, int src) {
  auto &slots = t_ctx.launch->slots_a[t_ctx.wave];
  slots[t_ctx.lane] = static_cast<uint32_t>(v);
  wave_sync();
  const int got = static_cast<int>(static_cast<uint32_t>(slots[src & 63]));
  wave_sync();
  return got;
}

template <typename T>
inline T shfl_xor(T v, int mask) {
  static_assert(sizeof(T) <= 8, "shuffle of at most 8 bytes");
  auto &slots = t_ctx.launch->slots_a[t_ctx.wave];
  uint64_t bits = 0;
  std::memcpy(&bits, &v, sizeof(T));
  slots[t_ctx.lane] = bits;
  wave_sync();
  const uint64_t got = slots[(t_ctx.lane ^ mask) & 63];
  wave_sync();
  T r;
  std::memcpy(&r, &got, sizeof(T));
  return r;
}

// value of `v` in lane `src` of the wavefront (every lane must call it)
template <typename T>
inline T shfl_src(T v, int src) {
  static_assert(sizeof(T) <= 8, "shuffle of at most 8 bytes");
  auto &slots = t_ctx.launch->slots_a[t_ctx.wave];
  uint64_t bits = 0;
  std::memcpy(&bits, &v, sizeof(T));
  slots[t_ctx.lane] = bits;
  wave_sync();
  const uint64_t got = slots[src & 63];
  wave_sync();
  T r;
  std::memcpy(&r, &got, sizeof(T));
  return r;
}

inline std::atomic<bool> g_capturing{false};
inline std::vector<std::function<void()>> *g_capture = nullptr;

template <typename K, typename... Args>
void run_launch(K kernel, dim3 grid, dim3 block, size_t smem, Args... args) {
  const unsigned n = block.x * block.y * block.z;
  Launch L;
  std::barrier<> bar(static_cast<std::ptrdiff_t>(n));
  L.block = &bar;
  const unsigned nw = (n + 63) / 64;
  for (unsigned w = 0; w < nw; ++w)
    L.waves.emplace_back(new std::barrier<>(static_cast<std::ptrdiff_t>(std::min(64u, n - 64 * w))));
  L.slots_a.assign(nw, std::vector<uint64_t>(64));
  L.slots_b.assign(nw, std::vector<uint64_t>(64));
  L.slots_c.assign(nw, std::vector<uint64_t>(64));
  L.slots_d.assign(nw, std::vector<uint64_t>(64));
  L.dynamic_smem.assign(smem / sizeof(float) + 1, 0.0F);
  std::vector<std::thread> pool;
  pool.reserve(n);
  for (unsigned t = 0; t < n; ++t) {
    pool.emplace_back([&, t]() {
      t_ctx.launch = &L;
      t_ctx.block_dim = block;
      t_ctx.grid_dim = grid;
      t_ctx.thread_idx = dim3(t % block.x, (t / block.x) % block.y, t / (block.x * block.y));
      t_ctx.lane = static_cast<int>(t % 64);
      t_ctx.wave = static_cast<int>(t / 64);
      for (unsigned bz = 0; bz < grid.z; ++bz)
        for (unsigned by = 0; by < grid.y; ++by)
          for (unsigned bx = 0; bx < grid.x; ++bx) {
            t_ctx.block_idx = dim3(bx, by, bz);
            kernel(args...);
            bar.arrive_and_wait();
          }
    });
  }
  for (auto &th : pool) th.join();
}

template <typename K, typename... Args>
void launch(K kernel, dim3 grid, dim3 block, size_t smem, Args... args) {
  if (g_capturing.load()) {
    g_capture->push_back([=]() { run_launch(kernel, grid, block, smem, args...); });
    return;
  }
  run_launch(kernel, grid, block, smem, args...);
}

inline uint16_t f2h(float value) {
  uint32_t bits;
  std::memcpy(&bits, &value, 4);
  const uint32_t sign = (bits >> 16) & 0x8000u, mag = bits & 0x7fffffffu;
  if (mag >= 0x7f800000u) return static_cast<uint16_t>(sign | (mag > 0x7f800000u ? 0x7e00u : 0x7c00u));
  if (mag > 0x477fefffu) return static_cast<uint16_t>(sign | 0x7c00u);
  if (mag < 0x38800000u) {
    if (mag < 0x33000001u) return static_cast<uint16_t>(sign);
    const uint32_t e = mag >> 23, mant = (mag & 0x7fffffu) | 0x800000u, shift = 126u - e;
    uint32_t hm = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u), half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (hm & 1u))) ++hm;
    return static_cast<uint16_t>(sign | hm);
  }
  const uint32_t rounded = mag + 0x00000fffu + ((mag >> 13) & 1u);
  return static_cast<uint16_t>(sign | ((rounded - 0x38000000u) >> 13));
}
inline float h2f(uint16_t h) {
  const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu, bits;
  if (e == 0) {
    if (m == 0) {
      bits = sign;
    } else {
      uint32_t ne = 113u;
      while ((m & 0x400u) == 0) { m <<= 1; --ne; }
      bits = sign | (ne << 23) | ((m & 0x3ffu) << 13);
    }
  } else if (e == 0x1fu) {
    bits = sign | 0x7f800000u | (m << 13);
  } else {
    bits = sign | ((e + 112u) << 23) | (m << 13);
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

}  // namespace q35emu

#define threadIdx (::q35emu::t_ctx.thread_idx)
#define blockIdx (::q35emu::t_ctx.block_idx)
#define blockDim (::q35emu::t_ctx.block_dim)
#define gridDim (::q35emu::t_ctx.grid_dim)

inline void __syncthreads() { ::q35emu::t_ctx.launch->block->arrive_and_wait(); }
inline void __threadfence() { std::atomic_thread_fence(std::memory_order_seq_cst); }
template <typename T>
inline T __shfl_xor(T v, int mask, int width = 64) {
  (void)width;
  return ::q35emu::shfl_xor(v, mask);
}
inline unsigned atomicAdd(unsigned *p, unsigned v) { return __atomic_fetch_add(p, v, __ATOMIC_SEQ_CST); }
inline unsigned long long atomicMax(unsigned long long *p, unsigned long long v) {
  unsigned long long cur = __atomic_load_n(p, __ATOMIC_SEQ_CST);
  while (cur < v && !__atomic_compare_exchange_n(p, &cur, v, false, __ATOMIC_SEQ_CST, __ATOMIC_SEQ_CST)) {
  }
  return cur;
}
inline unsigned __float_as_uint(float f) { unsigned u; std::memcpy(&u, &f, 4); return u; }
inline int __builtin_amdgcn_readlane(int v, int src) { return ::q35emu::readlane(v, src); }
// v_perm_b32: byte i of the result is byte sel.byte[i] of the eight bytes
// {s1 (bytes 0-3), s0 (bytes 4-7)}; selector 12 gives 0x00 and 13 and up
// 0xFF; the sign-replicating selectors 8-11 are not used here
inline unsigned __builtin_amdgcn_perm(unsigned s0, unsigned s1, unsigned sel) {
  const unsigned long long both = (static_cast<unsigned long long>(s0) << 32) | s1;
  unsigned r = 0;
  for (int i = 0; i < 4; ++i) {
    const unsigned b = (sel >> (8 * i)) & 0xFFu;
    if (b >= 8 && b <= 11) std::abort();
    const unsigned byte = b < 8 ? static_cast<unsigned>((both >> (8 * b)) & 0xFFu) : (b == 12 ? 0u : 0xFFu);
    r |= byte << (8 * i);
  }
  return r;
}
// value of `v` in lane `src` (per lane) of the wavefront; every lane calls it
template <typename T>
inline T __shfl(T v, int src, int width = 64) {
  (void)width;
  static_assert(sizeof(T) <= 8, "shuffle of at most 8 bytes");
  auto &slots = ::q35emu::t_ctx.launch->slots_a[::q35emu::t_ctx.wave];
  uint64_t bits = 0;
  std::memcpy(&bits, &v, sizeof(T));
  slots[::q35emu::t_ctx.lane] = bits;
  ::q35emu::wave_sync();
  const uint64_t got = slots[src & 63];
  ::q35emu::wave_sync();
  T r;
  std::memcpy(&r, &got, sizeof(T));
  return r;
}
inline int __float_as_int(float f) { int u; std::memcpy(&u, &f, 4); return u; }
inline float __int_as_float(int u) { float f; std::memcpy(&f, &u, 4); return f; }
inline float __uint_as_float(unsigned u) { float f; std::memcpy(&f, &u, 4); return f; }

struct __half { uint16_t bits; };
inline __half __ushort_as_half(uint16_t b) { return __half{b}; }
inline uint16_t __half_as_ushort(__half h) { return h.bits; }
inline float __half2float(__half h) { return ::q35emu::h2f(h.bits); }
inline __half __float2half_rn(float f) { return __half{::q35emu::f2h(f)}; }

#define Q35_V4I int __attribute__((vector_size(16)))
typedef int q35emu_v4i __attribute__((vector_size(16)));
inline q35emu_v4i q35emu_mfma_i8(long a, long b, q35emu_v4i c) {
  auto &ctx = ::q35emu::t_ctx;
  auto &sa = ctx.launch->slots_a[ctx.wave];
  auto &sb = ctx.launch->slots_b[ctx.wave];
  sa[ctx.lane] = static_cast<uint64_t>(a);
  sb[ctx.lane] = static_cast<uint64_t>(b);
  ::q35emu::wave_sync();
  q35emu_v4i d;
  const int col = ctx.lane % 16;
  for (int v = 0; v < 4; ++v) {
    const int row = 4 * (ctx.lane / 16) + v;
    int32_t sum = c[v];
    for (int k = 0; k < 32; ++k) {
      const int8_t av = static_cast<int8_t>(sa[row + 16 * (k / 8)] >> (8 * (k % 8)));
      const int8_t bv = static_cast<int8_t>(sb[col + 16 * (k / 8)] >> (8 * (k % 8)));
      sum += static_cast<int32_t>(av) * static_cast<int32_t>(bv);
    }
    d[v] = sum;
  }
  ::q35emu::wave_sync();
  return d;
}
#define Q35_MFMA_I32_16X16X32_I8(a, b, c, cbsz, abid, blgp) q35emu_mfma_i8(a, b, c)
typedef unsigned int q35_u32x4 __attribute__((vector_size(16)));
typedef unsigned int q35_u32x2 __attribute__((vector_size(8)));
typedef float q35_f32x4 __attribute__((vector_size(16)));
typedef float q35_f32x2 __attribute__((vector_size(8)));
// fp16 MFMA (v_mfma_f32_16x16x32_f16): the i8 operand layout with eight
// binary16 values per lane; each output is C plus the 32 products summed in
// k order in fp32 (the hardware's internal order differs; every use here is
// compared across paths of this same emulation or against a tolerance)
// Buffer resources: the extent is checked on every load (the kernels never
// read past it, so a load that would is a bug, not the hardware's zero read).
inline int q35_uniform(int v) { return v; }
struct q35_buffer {
  const uint8_t *base;
  int extent;
};
inline q35_buffer q35_make_buffer(const void *base, int extent) {
  return q35_buffer{static_cast<const uint8_t *>(base), extent};
}
template <typename T>
inline T q35emu_buffer_load(q35_buffer r, int voff, int soff) {
  const long long off = static_cast<long long>(voff) + soff;
  if (voff < 0 || soff < 0 || off + static_cast<long long>(sizeof(T)) > r.extent) std::abort();
  T v;
  std::memcpy(&v, r.base + off, sizeof(T));
  return v;
}
inline q35_u32x4 q35_buffer_load16(q35_buffer r, int voff, int soff) { return q35emu_buffer_load<q35_u32x4>(r, voff, soff); }
inline q35_u32x2 q35_buffer_load8(q35_buffer r, int voff, int soff) { return q35emu_buffer_load<q35_u32x2>(r, voff, soff); }
inline uint32_t q35_buffer_load4(q35_buffer r, int voff, int soff) { return q35emu_buffer_load<uint32_t>(r, voff, soff); }
typedef uint16_t q35_f16x8 __attribute__((vector_size(16)));
inline q35_f16x8 q35_f16x8_bits(q35_u32x4 raw) {
  q35_f16x8 r;
  std::memcpy(&r, &raw, 16);
  return r;
}
inline void q35_split_f16(const float x[8], q35_f16x8 &hi, q35_f16x8 &lo) {
  for (int i = 0; i < 8; ++i) {
    hi[i] = ::q35emu::f2h(x[i]);
    lo[i] = ::q35emu::f2h(x[i] - ::q35emu::h2f(hi[i]));
  }
}
inline q35_f32x4 q35emu_mfma_f16(q35_f16x8 a, q35_f16x8 b, q35_f32x4 c) {
  auto &ctx = ::q35emu::t_ctx;
  auto &a0 = ctx.launch->slots_a[ctx.wave], &a1 = ctx.launch->slots_b[ctx.wave];
  auto &b0 = ctx.launch->slots_c[ctx.wave], &b1 = ctx.launch->slots_d[ctx.wave];
  uint64_t w[4];
  std::memcpy(w, &a, 16);
  a0[ctx.lane] = w[0];
  a1[ctx.lane] = w[1];
  std::memcpy(w, &b, 16);
  b0[ctx.lane] = w[0];
  b1[ctx.lane] = w[1];
  ::q35emu::wave_sync();
  auto elem = [](const std::vector<uint64_t> &lo, const std::vector<uint64_t> &hi, int lane, int k) {
    const uint64_t word = k < 4 ? lo[lane] : hi[lane];
    return ::q35emu::h2f(static_cast<uint16_t>(word >> (16 * (k % 4))));
  };
  q35_f32x4 d;
  const int col = ctx.lane % 16;
  for (int v = 0; v < 4; ++v) {
    const int row = 4 * (ctx.lane / 16) + v;
    float sum = c[v];
    for (int k = 0; k < 32; ++k)
      sum += elem(a0, a1, row + 16 * (k / 8), k % 8) * elem(b0, b1, col + 16 * (k / 8), k % 8);
    d[v] = sum;
  }
  ::q35emu::wave_sync();
  return d;
}
#define Q35_MFMA_F32_16X16X32_F16(a, b, c) q35emu_mfma_f16(a, b, c)
typedef float q35_f32x16 __attribute__((vector_size(64)));
inline q35_f32x16 q35emu_mfma_outer4(float a, float b, q35_f32x16 c) {
  auto &ctx = ::q35emu::t_ctx;
  auto &as = ctx.launch->slots_a[ctx.wave], &bs = ctx.launch->slots_b[ctx.wave];
  uint32_t ab, bb;
  std::memcpy(&ab, &a, 4);
  std::memcpy(&bb, &b, 4);
  as[ctx.lane] = ab;
  bs[ctx.lane] = bb;
  ::q35emu::wave_sync();
  q35_f32x16 d;
  const int l = ctx.lane;
  for (int blk = 0; blk < 4; ++blk)
    for (int k = 0; k < 4; ++k) {
      float x, y;
      const uint32_t xa = static_cast<uint32_t>(as[16 * blk + 4 * (l / 16) + k]), yb = static_cast<uint32_t>(bs[16 * blk + l % 16]);
      std::memcpy(&x, &xa, 4);
      std::memcpy(&y, &yb, 4);
      d[4 * blk + k] = x * y + c[4 * blk + k];
    }
  ::q35emu::wave_sync();
  return d;
}
#define Q35_MFMA_F32_16X16X1_4B(a, b, c) q35emu_mfma_outer4(a, b, c)
#define Q35_LOAD_NT(ptr) (*(ptr))
inline int q35emu_sdot4(uint32_t a, uint32_t b, int c) {
  for (int i = 0; i < 4; ++i)
    c += static_cast<int>(static_cast<int8_t>(a >> (8 * i))) * static_cast<int>(static_cast<int8_t>(b >> (8 * i)));
  return c;
}
#define Q35_SDOT4(a, b, c) q35emu_sdot4(static_cast<uint32_t>(a), static_cast<uint32_t>(b), (c))
inline void lds_barrier() { __syncthreads(); }
inline void wave_lds_sync() { ::q35emu::wave_sync(); }
inline void q35_compiler_fence() { asm volatile("" ::: "memory"); }
inline void q35_materialize(float &) {}
inline int __lane_id() { return ::q35emu::t_ctx.lane; }
// a product rounded on its own (never contracted into an fma)
inline float __fmul_rn(float a, float b) {
  volatile float p = a * b;
  return p;
}
inline float q35_quad_xor1(float v) { return ::q35emu::shfl_xor(v, 1); }
inline float q35_quad_xor2(float v) { return ::q35emu::shfl_xor(v, 2); }
inline float q35_row_xor(float v, int m) { return ::q35emu::shfl_xor(v, m); }
inline int q35_row_xor_i(int v, int m) { return ::q35emu::shfl_xor(v, m); }
inline float q35_lane_xor(float v, int m) { return ::q35emu::shfl_xor(v, m); }
inline int q35_lane_xor_i(int v, int m) { return ::q35emu::shfl_xor(v, m); }
inline float q35_row_half_mirror(float v) {
  const int l = ::q35emu::t_ctx.lane;
  return ::q35emu::shfl_src(v, (l & ~7) | (7 - (l & 7)));
}
#define Q35_STORE_NT(value, ptr) (*(ptr) = (value))
#define Q35_DYNAMIC_SHARED(type, name) \
  type *name = reinterpret_cast<type *>(::q35emu::t_ctx.launch->dynamic_smem.data())
#define Q35_LAUNCH(kernel, grid, block, smem, stream, ...) \
  ::q35emu::launch(kernel, dim3(grid), dim3(block), static_cast<size_t>(smem), __VA_ARGS__)

// ------------------------------------------------------------- host API
typedef int hipError_t;
enum { hipSuccess = 0, hipErrorInvalidValue = 1, hipErrorOutOfMemory = 2, hipErrorNotSupported = 801 };
enum hipMemcpyKind { hipMemcpyHostToHost, hipMemcpyHostToDevice, hipMemcpyDeviceToHost, hipMemcpyDeviceToDevice };
enum { hipStreamNonBlocking = 1 };
enum hipStreamCaptureMode { hipStreamCaptureModeGlobal, hipStreamCaptureModeThreadLocal };
typedef void *hipStream_t;
typedef struct q35emu_event { std::chrono::steady_clock::time_point t; } *hipEvent_t;
typedef std::vector<std::function<void()>> *hipGraph_t;
typedef std::vector<std::function<void()>> *hipGraphExec_t;
struct hipDeviceProp_t {
  int multiProcessorCount;
  char gcnArchName[256];
};

inline const char *hipGetErrorString(hipError_t e) { return e == 0 ? "no error" : "emulated HIP error"; }
inline hipError_t hipGetLastError() { return hipSuccess; }
inline hipError_t hipGetDeviceCount(int *n) { *n = 1; return hipSuccess; }
inline hipError_t hipSetDevice(int) { return hipSuccess; }
inline hipError_t hipGetDeviceProperties(hipDeviceProp_t *p, int) {
  p->multiProcessorCount = 256;
  std::strcpy(p->gcnArchName, "host-emulation");
  return hipSuccess;
}
inline hipError_t hipStreamCreateWithFlags(hipStream_t *s, unsigned) { *s = new int(0); return hipSuccess; }
inline hipError_t hipStreamDestroy(hipStream_t s) { delete static_cast<int *>(s); return hipSuccess; }
inline hipError_t hipStreamSynchronize(hipStream_t) { return hipSuccess; }
// a __device__ array is a host array here: its symbol address is the array
#define HIP_SYMBOL(x) (&(x))
inline hipError_t hipGetSymbolAddress(void **p, const void *symbol) {
  *p = const_cast<void *>(symbol);
  return hipSuccess;
}
inline hipError_t hipEventCreate(hipEvent_t *e) { *e = new q35emu_event(); return hipSuccess; }
inline hipError_t hipEventDestroy(hipEvent_t e) { delete e; return hipSuccess; }
inline hipError_t hipEventRecord(hipEvent_t e, hipStream_t) { e->t = std::chrono::steady_clock::now(); return hipSuccess; }
inline hipError_t hipEventSynchronize(hipEvent_t) { return hipSuccess; }
inline hipError_t hipEventElapsedTime(float *ms, hipEvent_t a, hipEvent_t b) {
  *ms = std::chrono::duration<float, std::milli>(b->t - a->t).count();
  return hipSuccess;
}
inline hipError_t hipMalloc(void **p, size_t n) { *p = std::malloc(n); return *p ? hipSuccess : hipErrorOutOfMemory; }
template <typename T>
inline hipError_t hipMalloc(T **p, size_t n) { return hipMalloc(reinterpret_cast<void **>(p), n); }
inline hipError_t hipFree(void *p) { std::free(p); return hipSuccess; }
inline hipError_t hipHostMalloc(void **p, size_t n) { return hipMalloc(p, n); }
inline hipError_t hipHostFree(void *p) { return hipFree(p); }
inline hipError_t hipHostGetDevicePointer(void **d, void *h, unsigned) { *d = h; return hipSuccess; }
inline hipError_t hipMallocAsync(void **p, size_t n, hipStream_t) { return hipMalloc(p, n); }
inline hipError_t hipFreeAsync(void *p, hipStream_t) { return hipFree(p); }
inline hipError_t hipMemcpy(void *d, const void *s, size_t n, hipMemcpyKind) { std::memmove(d, s, n); return hipSuccess; }
inline hipError_t hipMemcpyAsync(void *d, const void *s, size_t n, hipMemcpyKind, hipStream_t) {
  if (::q35emu::g_capturing.load()) {
    ::q35emu::g_capture->push_back([=]() { std::memmove(d, s, n); });
    return hipSuccess;
  }
  std::memmove(d, s, n);
  return hipSuccess;
}
inline hipError_t hipMemset(void *d, int v, size_t n) { std::memset(d, v, n); return hipSuccess; }
inline hipError_t hipMemsetAsync(void *d, int v, size_t n, hipStream_t) {
  if (::q35emu::g_capturing.load()) return hipErrorNotSupported;  // never captured by the backend
  std::memset(d, v, n);
  return hipSuccess;
}
inline hipError_t hipStreamBeginCapture(hipStream_t, hipStreamCaptureMode) {
  ::q35emu::g_capture = new std::vector<std::function<void()>>();
  ::q35emu::g_capturing = true;
  return hipSuccess;
}
inline hipError_t hipStreamEndCapture(hipStream_t, hipGraph_t *g) {
  ::q35emu::g_capturing = false;
  *g = ::q35emu::g_capture;
  ::q35emu::g_capture = nullptr;
  return hipSuccess;
}
inline hipError_t hipGraphInstantiate(hipGraphExec_t *e, hipGraph_t g, void *, void *, size_t) {
  *e = new std::vector<std::function<void()>>(*g);
  return hipSuccess;
}
inline hipError_t hipGraphDestroy(hipGraph_t g) { delete g; return hipSuccess; }
inline hipError_t hipGraphExecDestroy(hipGraphExec_t e) { delete e; return hipSuccess; }
inline hipError_t hipGraphLaunch(hipGraphExec_t e, hipStream_t) {
  for (auto &f : *e) f();
  return hipSuccess;
}
