// The HIP API surface used by the backend. The product is always built by
// hipcc for gfx950; Q35_HOST_EMULATION selects the test-only CPU build in
// tests/emu/ (the same kernel sources run on host threads under
// AddressSanitizer to bounds-check every kernel before it runs on a GPU).
#pragma once

#ifdef Q35_HOST_EMULATION
#include "q35_host_emulation.h"
#else
#include <hip/hip_ext.h>
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

namespace q35 {
// Profiling hook of the launch macro: while a profiled step is enqueued it
// returns true with a fresh event pair, which the launch records its own
// dispatch start and end into (hipExtLaunchKernelGGL), so the pair brackets
// the kernel's execution and nothing else. Otherwise it returns false.
bool launch_events(hipEvent_t *start, hipEvent_t *stop);
}  // namespace q35

#define Q35_LAUNCH(kernel, grid, block, smem, stream, ...)                                        \
  do {                                                                                            \
    hipEvent_t q35_ev0_ = nullptr, q35_ev1_ = nullptr;                                            \
    if (::q35::launch_events(&q35_ev0_, &q35_ev1_))                                               \
      hipExtLaunchKernelGGL(kernel, grid, block, smem, stream, q35_ev0_, q35_ev1_, 0, __VA_ARGS__); \
    else                                                                                          \
      hipLaunchKernelGGL(kernel, grid, block, smem, stream, __VA_ARGS__);                         \
  } while (0)
#define Q35_V4I int __attribute__((ext_vector_type(4)))
#define Q35_MFMA_I32_16X16X32_I8(a, b, c, cbsz, abid, blgp) \
  __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, c, cbsz, abid, blgp)
#define Q35_DYNAMIC_SHARED(type, name) extern __shared__ type name[]
// occupancy target of a kernel: at least n wavefronts per SIMD (caps its VGPRs)
#define Q35_WAVES_PER_EU(n) __attribute__((amdgpu_waves_per_eu(n)))
// fp16 MFMA operands: eight binary16 values per lane
typedef _Float16 q35_f16x8 __attribute__((ext_vector_type(8)));
#define Q35_MFMA_F32_16X16X32_F16(a, b, c) __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0)
// four 16x16 fp32 outer products (K = 1): lane 16b + m supplies A_b[m], lane
// 16b + n supplies B_b[n]; element 4b + k of lane l is A_b[4(l/16) + k] x
// B_b[l % 16] (+ c)
typedef float q35_f32x16 __attribute__((ext_vector_type(16)));
#define Q35_MFMA_F32_16X16X1_4B(a, b, c) __builtin_amdgcn_mfma_f32_16x16x1f32(a, b, c, 0, 0, 0)
// four int8 products of a and b (byte-wise, signed) added to c: v_dot4_i32_i8
#define Q35_SDOT4(a, b, c) __builtin_amdgcn_sdot4(static_cast<int>(a), static_cast<int>(b), (c), false)
// Streaming loads of data read once per step (weights, recurrent state, KV):
// marked non-temporal so they do not displace reused lines in L1/L2.
typedef unsigned int q35_u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int q35_u32x2 __attribute__((ext_vector_type(2)));
typedef float q35_f32x4 __attribute__((ext_vector_type(4)));
typedef float q35_f32x2 __attribute__((ext_vector_type(2)));
#define Q35_LOAD_NT(ptr) __builtin_nontemporal_load(ptr)
#define Q35_STORE_NT(value, ptr) __builtin_nontemporal_store(value, ptr)
#endif

#ifndef Q35_HOST_EMULATION
// Exchange with lane l^m inside each 16-lane row, as register-to-register DPP
// moves (no LDS crossbar): m = 1, 2 are quad_perm [1,0,3,2] / [2,3,0,1];
// m = 4 combines row_shl:4 (lanes with bit 2 clear) and row_shr:4 (set);
// m = 8 is row_ror:8 (a rotation by half the row is the exchange l <-> l^8).
__device__ __forceinline__ int q35_row_xor_i(int v, int m) {
  switch (m) {
    case 1: return __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, true);
    case 2: return __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, true);
    case 4: {
      const int up = __builtin_amdgcn_update_dpp(0, v, 0x104, 0xF, 0xF, true);
      const int dn = __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, true);
      return (__lane_id() & 4) ? dn : up;
    }
    default: return __builtin_amdgcn_update_dpp(0, v, 0x128, 0xF, 0xF, true);
  }
}
__device__ __forceinline__ float q35_row_xor(float v, int m) {
  return __int_as_float(q35_row_xor_i(__float_as_int(v), m));
}
// Exchange with lane l^m for m = 1 .. 32: DPP row moves inside a 16-lane row,
// ds_swizzle's xor mode across the two rows of a 32-lane half (m = 16), and
// a bpermute across the halves (m = 32).
__device__ __forceinline__ int q35_lane_xor_i(int v, int m) {
  if (m < 16) return q35_row_xor_i(v, m);
  if (m == 16) return __builtin_amdgcn_ds_swizzle(v, 0x401F);  // and 0x1F, or 0, xor 0x10
  return __shfl_xor(v, 32, 64);
}
__device__ __forceinline__ float q35_lane_xor(float v, int m) {
  return __int_as_float(q35_lane_xor_i(__float_as_int(v), m));
}
// The value of lane 7 - i of this lane's 8-lane half row (row_half_mirror):
// one DPP move to a lane of the other quad of the half.
__device__ __forceinline__ float q35_row_half_mirror(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, true));
}
// Workgroup barrier that orders LDS only: outstanding global loads and
// stores keep flying (__syncthreads is a release fence at workgroup scope and
// waits for them -- on gfx9 the vmcnt counter covers loads and stores).
// Compiler-only fence: no memory access is moved across it (no instruction
// is emitted). Bounds how far the compiler hoists loads out of unrolled loops.
__device__ __forceinline__ void q35_compiler_fence() { asm volatile("" ::: "memory"); }
// Forces `x` to be computed at this point (an empty asm reading and writing
// it), so the compiler cannot sink the arithmetic that produces it past later
// loads and keep their results live meanwhile.
__device__ __forceinline__ void q35_materialize(float &x) { asm volatile("" : "+v"(x)); }
// A wave-uniform value moved into a scalar register (every lane holds the
// same value; the compiler then treats what derives from it as uniform).
__device__ __forceinline__ int q35_uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }
// Raw (stride 0) buffer resource over [base, base + extent) with a
// wave-uniform base: a load takes a per-lane byte offset and a wave-uniform
// one (a scalar register, so per-iteration offsets cost no VALU work); an
// offset at or past the extent reads 0. Word 3 is gfx9's: 32-bit data
// format, no swizzle.
typedef __amdgpu_buffer_rsrc_t q35_buffer;
__device__ __forceinline__ q35_buffer q35_make_buffer(const void *base, int extent) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, extent, 0x00020000);
}
__device__ __forceinline__ q35_u32x4 q35_buffer_load16(q35_buffer r, int voff, int soff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
}
__device__ __forceinline__ q35_u32x2 q35_buffer_load8(q35_buffer r, int voff, int soff) {
  return __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0);
}
__device__ __forceinline__ uint32_t q35_buffer_load4(q35_buffer r, int voff, int soff) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
}

// Orders a wavefront's LDS writes before its later LDS reads by other lanes of
// the same wavefront. The LDS executes one wavefront's instructions in order,
// so this only stops the compiler from moving LDS accesses across it.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
}
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}
// Sixteen bytes of binary16 bits as an fp16 MFMA operand.
__device__ __forceinline__ q35_f16x8 q35_f16x8_bits(q35_u32x4 raw) { return __builtin_bit_cast(q35_f16x8, raw); }
// x = hi + lo with hi = binary16(x) and lo = binary16(x - hi) (round to
// nearest even): 22 significant bits in two fp16 operands, whose products with
// an fp16 value are exact in fp32.
__device__ __forceinline__ void q35_split_f16(const float x[8], q35_f16x8 &hi, q35_f16x8 &lo) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const _Float16 h = static_cast<_Float16>(x[i]);
    hi[i] = h;
    lo[i] = static_cast<_Float16>(x[i] - static_cast<float>(h));
  }
}
__device__ __forceinline__ float q35_quad_xor1(float v) { return q35_row_xor(v, 1); }
__device__ __forceinline__ float q35_quad_xor2(float v) { return q35_row_xor(v, 2); }
#endif
