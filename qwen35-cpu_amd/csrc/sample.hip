// Candidate selection for sampled decoding (sample_token_from_logits,
// src/runtime/layers.inl:491-600): per row, the repetition penalty
// (apply_repetition_penalty_inplace, layers.inl:471-489: a counted token's
// logit v becomes v / p when v > 0, else v * p), the temperature scaling
// v *= 1 / temperature (layers.inl:546-549), and the top_k largest values in
// descending order (layers.inl:552-568). Only these k candidates reach the
// host, which finishes the softmax, the nucleus cut and the draw in the
// reference's order. Greedy rows use k = 1 and scale 1: the argmax with the
// lowest index among equal values (argmax_index, layers.inl:459-469).
//
// Each value becomes a 64-bit key: the float's bits mapped to an unsigned
// order (sign flipped for positives, all bits flipped for negatives) in the
// high word and the inverted token id in the low word, so a descending sort
// orders by value and then by lower token id.
//   stage 1: grid (kSampleSlices, rows): slice s of a row (at most 4096
//            tokens) sorts its keys in LDS and keeps its top kMaxCandidates;
//   stage 2: grid (rows): the slices' survivors (kSampleSlices x
//            kMaxCandidates = 4096 keys) are sorted and the row's top k written.
#include "q35_device.h"
#include "q35_internal.h"

namespace q35 {
namespace {

constexpr int kSortKeys = 4096;
constexpr int kSortThreads = 1024;
constexpr int kSampleSlices = kSortKeys / kMaxCandidates;  // 64

__device__ __forceinline__ unsigned long long candidate_key(float v, int token) {
  const uint32_t u = __float_as_uint(v);
  const uint32_t ordered = (u & 0x80000000u) != 0u ? ~u : (u | 0x80000000u);
  return (static_cast<unsigned long long>(ordered) << 32) | static_cast<uint32_t>(~static_cast<uint32_t>(token));
}

__device__ __forceinline__ float key_value(unsigned long long key) {
  const uint32_t ordered = static_cast<uint32_t>(key >> 32);
  return __uint_as_float((ordered & 0x80000000u) != 0u ? (ordered & 0x7fffffffu) : ~ordered);
}

// Bitonic sort of kSortKeys keys in LDS, descending; every thread of the
// workgroup takes part.
__device__ void sort_desc(unsigned long long *keys) {
  for (int size = 2; size <= kSortKeys; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = threadIdx.x; i < kSortKeys / 2; i += kSortThreads) {
        const int lo = 2 * i - (i & (stride - 1));
        const int hi = lo + stride;
        const bool desc = (lo & size) == 0;
        const unsigned long long a = keys[lo], b = keys[hi];
        if ((a < b) == desc) {
          keys[lo] = b;
          keys[hi] = a;
        }
      }
      __syncthreads();
    }
  }
}

__global__ __launch_bounds__(kSortThreads) void sample_slices_kernel(SampleArgs a, unsigned long long *survivors) {
  __shared__ unsigned long long keys[kSortKeys];
  const int s = blockIdx.x, r = blockIdx.y;
  const int per = (a.vocab + kSampleSlices - 1) / kSampleSlices;
  const int t0 = s * per, t1 = min(a.vocab, t0 + per);
  const float *logits = a.logits + static_cast<size_t>(r) * a.logits_stride;
  const float pen = a.penalties != nullptr ? a.penalties[r] : 1.0F;
  const int32_t *counts =
      a.counts != nullptr ? a.counts + static_cast<long long>(a.count_rows != nullptr ? a.count_rows[r] : r) * a.vocab
                          : nullptr;
  const float scale = a.inv_temperature != nullptr ? a.inv_temperature[r] : 1.0F;
  for (int i = threadIdx.x; i < kSortKeys; i += kSortThreads) {
    const int t = t0 + i;
    unsigned long long key = 0ull;  // below every real key
    if (t < t1) {
      float v = logits[t];
      if (pen > 1.0F && counts != nullptr && counts[t] > 0) v = v > 0.0F ? v / pen : v * pen;
      v *= scale;
      key = candidate_key(v, t);
    }
    keys[i] = key;
  }
  __syncthreads();
  sort_desc(keys);
  unsigned long long *out = survivors + (static_cast<size_t>(r) * kSampleSlices + s) * kMaxCandidates;
  for (int i = threadIdx.x; i < kMaxCandidates; i += kSortThreads) out[i] = keys[i];
}

__global__ __launch_bounds__(kSortThreads) void sample_merge_kernel(SampleArgs a, const unsigned long long *survivors) {
  __shared__ unsigned long long keys[kSortKeys];
  const int r = blockIdx.x;
  const unsigned long long *in = survivors + static_cast<size_t>(r) * kSortKeys;
  for (int i = threadIdx.x; i < kSortKeys; i += kSortThreads) keys[i] = in[i];
  __syncthreads();
  sort_desc(keys);
  const int k = a.top_k != nullptr ? a.top_k[r] : 1;
  q35_candidate *out = a.out + static_cast<size_t>(r) * kMaxCandidates;
  for (int i = threadIdx.x; i < kMaxCandidates; i += kSortThreads) {
    q35_candidate c;
    if (i < k && keys[i] != 0ull) {
      c.value = key_value(keys[i]);
      c.token = static_cast<int32_t>(~static_cast<uint32_t>(keys[i]));
    } else {
      c.value = -INFINITY;
      c.token = -1;
    }
    out[i] = c;
  }
}

}  // namespace

size_t sample_scratch_bytes(int rows) { return static_cast<size_t>(rows) * kSortKeys * sizeof(unsigned long long); }

hipError_t launch_sample_candidates(const SampleArgs &a, unsigned long long *scratch, hipStream_t stream) {
  if (a.rows <= 0) return hipSuccess;
  if (a.vocab <= 0 || a.vocab > kSampleSlices * kSortKeys || a.logits == nullptr || a.out == nullptr ||
      scratch == nullptr)
    return hipErrorInvalidValue;
  Q35_LAUNCH((sample_slices_kernel), dim3(kSampleSlices, a.rows), dim3(kSortThreads), 0, stream, a, scratch);
  Q35_LAUNCH((sample_merge_kernel), dim3(a.rows), dim3(kSortThreads), 0, stream, a, scratch);
  return hipGetLastError();
}

}  // namespace q35
