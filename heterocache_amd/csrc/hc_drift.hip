// Pivot-head drift monitoring, entirely on the device (no host sync).
//
// The reference (heterocache/cache_utils.py:1059-1082) keeps, per pivot, the
// prefill top-K position set; every decode_step calls it takes the top-K set
// of each buffered step, measures |cur ∩ ref| / K, averages over the batch,
// takes the median over the steps and, when it falls below stable_threshold,
// replaces the reference set by the last step's set and retrieves tokens for
// the pivot's satellites.  Here:
//   hc_set_bits        position lists -> per-set bitmasks (optionally only for
//                      sets whose trigger flag is raised);
//   hc_overlap_count   |list ∩ bitmask| per list (bit tests + block reduce);
//   hc_drift_decide    per pivot: batch mean, median over steps, threshold,
//                      trigger flag written to device memory.
// The trigger flag gates the set update and the retrieval gather
// (hc_gather_store's trigger argument), so the decode loop never waits on the
// host.
#include <algorithm>

#include "hc_common.h"
#include "hc_internal.h"

namespace hc {

// Each set's bitmap is split into slices of at most kBitsLds words, one
// workgroup per (slice, set): the workgroup reads the set's whole list (from
// L2 after the first slice), ORs the positions that fall in its slice into
// LDS and writes the slice's words, zeros included, with plain stores.  No
// order is assumed and no global atomics are needed, and a set's time is no
// longer one workgroup's chain of dependent loads: a layer has few sets (its
// pivot leaders), and with one workgroup per set a 64K-position set took
// 30 us.
constexpr int kBitsLds = 8192;       // words per slice at most (262144 positions, 32 KB)
constexpr int kSetBitsSlices = 16;   // slices per set at least
constexpr int kSetBitsBatch = 8;     // loads per thread in flight together

__device__ __forceinline__ void set_bit_in(uint32_t* s_bits, int x, int lo, int hi, int w0) {
  if (x >= lo && x < hi) atomicOr(&s_bits[(x >> 5) - w0], 1u << (x & 31));
}

__global__ __launch_bounds__(1024) void set_bits_kernel(const int32_t* __restrict__ idx, int64_t idx_stride,
                                                        const int32_t* __restrict__ counts, int fixed_count,
                                                        uint32_t* __restrict__ bits, int64_t words, int nbits,
                                                        const int32_t* __restrict__ trigger,
                                                        const int32_t* __restrict__ trig_of, int slice_words,
                                                        const int64_t* __restrict__ row_of) {
  const int j = blockIdx.y;
  if (trigger && trigger[trig_of ? trig_of[j] : j] == 0) return;
  const int64_t w0 = (int64_t)blockIdx.x * slice_words;
  const int nw = (int)min((int64_t)slice_words, words - w0);
  if (nw <= 0) return;
  __shared__ uint32_t s_bits[kBitsLds];
  for (int w = threadIdx.x; w < nw; w += blockDim.x) s_bits[w] = 0u;
  __syncthreads();
  // Positions of this slice: [lo, hi), inside [0, nbits).
  const int lo = (int)min(w0 * 32, (int64_t)nbits);
  const int hi = (int)min((w0 + nw) * 32, (int64_t)nbits);
  const int n = counts ? counts[j] : fixed_count;
  const int32_t* ix = idx + (row_of ? row_of[j] : (int64_t)j) * idx_stride;
  const int wb = (int)w0;
  const int bd = blockDim.x;
  int i_tail = 0;
  if ((reinterpret_cast<uintptr_t>(ix) & 15) == 0) {
    // Four positions per 16-byte load.
    const int n4 = n / 4;
    const int4* ix4 = reinterpret_cast<const int4*>(ix);
    for (int i0 = threadIdx.x; i0 < n4; i0 += bd * kSetBitsBatch) {
      int4 v[kSetBitsBatch];
#pragma unroll
      for (int u = 0; u < kSetBitsBatch; ++u) {
        const int i = i0 + u * bd;
        v[u] = i < n4 ? ix4[i] : make_int4(-1, -1, -1, -1);
      }
#pragma unroll
      for (int u = 0; u < kSetBitsBatch; ++u) {
        set_bit_in(s_bits, v[u].x, lo, hi, wb);
        set_bit_in(s_bits, v[u].y, lo, hi, wb);
        set_bit_in(s_bits, v[u].z, lo, hi, wb);
        set_bit_in(s_bits, v[u].w, lo, hi, wb);
      }
    }
    i_tail = n4 * 4;
  }
  for (int i0 = i_tail + threadIdx.x; i0 < n; i0 += bd * kSetBitsBatch) {
    int t[kSetBitsBatch];
#pragma unroll
    for (int u = 0; u < kSetBitsBatch; ++u) {
      const int i = i0 + u * bd;
      t[u] = i < n ? ix[i] : -1;
    }
#pragma unroll
    for (int u = 0; u < kSetBitsBatch; ++u) set_bit_in(s_bits, t[u], lo, hi, wb);
  }
  __syncthreads();
  uint32_t* b = bits + (int64_t)j * words + w0;
  for (int w = threadIdx.x; w < nw; w += blockDim.x) b[w] = s_bits[w];
}

__global__ __launch_bounds__(1024) void overlap_count_kernel(const int32_t* __restrict__ idx, int64_t idx_stride,
                                                             int count, const uint32_t* __restrict__ bits,
                                                             int64_t words, int nbits,
                                                             const int32_t* __restrict__ ref_of,
                                                             int32_t* __restrict__ out) {
  const int j = blockIdx.x;
  const uint32_t* b = bits + (int64_t)(ref_of ? ref_of[j] : j) * words;
  const int32_t* ix = idx + (int64_t)j * idx_stride;
  __shared__ uint32_t s_bits[kBitsLds];
  const bool lds = words <= kBitsLds;
  if (lds) {
    for (int w = threadIdx.x; w < words; w += blockDim.x) s_bits[w] = b[w];
    __syncthreads();
  }
  const uint32_t* bb = lds ? s_bits : b;
  int c = 0;
  int i = threadIdx.x;
  for (; i + 3 * 1024 < count; i += 4 * 1024) {
    const int t0 = ix[i], t1 = ix[i + 1024], t2 = ix[i + 2048], t3 = ix[i + 3072];
    c += (t0 >= 0 && t0 < nbits) ? (bb[t0 >> 5] >> (t0 & 31)) & 1u : 0;
    c += (t1 >= 0 && t1 < nbits) ? (bb[t1 >> 5] >> (t1 & 31)) & 1u : 0;
    c += (t2 >= 0 && t2 < nbits) ? (bb[t2 >> 5] >> (t2 & 31)) & 1u : 0;
    c += (t3 >= 0 && t3 < nbits) ? (bb[t3 >> 5] >> (t3 & 31)) & 1u : 0;
  }
  for (; i < count; i += 1024) {
    const int t = ix[i];
    if (t >= 0 && t < nbits) c += (bb[t >> 5] >> (t & 31)) & 1u;
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) c += __shfl_xor(c, off, 64);
  __shared__ int s[16];
  if ((threadIdx.x & 63) == 0) s[threadIdx.x >> 6] = c;
  __syncthreads();
  if (threadIdx.x == 0) {
    int tot = 0;
    for (int w = 0; w < 16; ++w) tot += s[w];
    out[j] = tot;
  }
}

// counts: [npiv][batch][steps]; one thread per pivot.
__global__ void drift_decide_kernel(const int32_t* __restrict__ counts, int npiv, int batch, int steps, int K,
                                    double threshold, float* __restrict__ overlap, double* __restrict__ median,
                                    int32_t* __restrict__ trigger) {
  const int p = blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= npiv) return;
  float v[64];
  for (int s = 0; s < steps; ++s) {
    // (count / K) per batch row in float32, then the float32 batch mean.
    float acc = 0.f;
    for (int b = 0; b < batch; ++b) acc += (float)counts[((int64_t)p * batch + b) * steps + s] / (float)K;
    v[s] = acc / (float)batch;
    if (overlap) overlap[(int64_t)p * steps + s] = v[s];
  }
  // Insertion sort of the (<= 64) step values, then the median as
  // statistics.median defines it (mean of the middle pair for even counts).
  for (int i = 1; i < steps; ++i) {
    const float x = v[i];
    int j = i - 1;
    while (j >= 0 && v[j] > x) {
      v[j + 1] = v[j];
      --j;
    }
    v[j + 1] = x;
  }
  const double med = (steps & 1) ? (double)v[steps / 2] : ((double)v[steps / 2 - 1] + (double)v[steps / 2]) / 2.0;
  if (median) median[p] = med;
  trigger[p] = med < threshold ? 1 : 0;
}

}  // namespace hc

using namespace hc;

extern "C" int hc_set_bits(const int32_t* idx, int64_t idx_stride, const int32_t* counts, int fixed_count, int nsets,
                           uint32_t* bits, int64_t words, int nbits, const int32_t* trigger, const int32_t* trig_of,
                           const int64_t* row_of, void* stream) {
  clear_error();
  if (nsets < 0 || nsets > 65535 || words < (nbits + 31) / 32 || nbits < 0)
    return set_error(HC_ERR_INVALID, "hc_set_bits: nsets=%d words=%lld nbits=%d", nsets, (long long)words, nbits);
  if (nsets == 0) return HC_OK;
  if (!idx || !bits) return set_error(HC_ERR_INVALID, "hc_set_bits: null pointer argument");
  if (!counts && fixed_count > idx_stride) return set_error(HC_ERR_INVALID, "hc_set_bits: count exceeds the stride");
  if (words > (int64_t)kBitsLds * 65535) return set_error(HC_ERR_INVALID, "hc_set_bits: %lld words", (long long)words);
  // At least kSetBitsSlices slices, each within the LDS bitmap.
  const int64_t slices = std::max<int64_t>(kSetBitsSlices, (words + kBitsLds - 1) / kBitsLds);
  const int slice_words = (int)((words + slices - 1) / slices);
  const int grid_x = (int)((words + slice_words - 1) / slice_words);
  hipLaunchKernelGGL(set_bits_kernel, dim3(grid_x, nsets), dim3(1024), 0, (hipStream_t)stream, idx, idx_stride, counts,
                     fixed_count, bits, words, nbits, trigger, trig_of, slice_words, row_of);
  return check_launch("hc_set_bits");
}

extern "C" int hc_overlap_count(const int32_t* idx, int64_t idx_stride, int count, int nlists, const uint32_t* bits,
                                int64_t words, int nbits, const int32_t* ref_of, int32_t* out, void* stream) {
  clear_error();
  if (nlists < 0 || nlists > 65535 || count < 0 || count > idx_stride || words < (nbits + 31) / 32)
    return set_error(HC_ERR_INVALID, "hc_overlap_count: nlists=%d count=%d stride=%lld", nlists, count,
                     (long long)idx_stride);
  if (nlists == 0) return HC_OK;
  if (!idx || !bits || !out) return set_error(HC_ERR_INVALID, "hc_overlap_count: null pointer argument");
  hipLaunchKernelGGL(overlap_count_kernel, dim3(nlists), dim3(1024), 0, (hipStream_t)stream, idx, idx_stride, count,
                     bits, words, nbits, ref_of, out);
  return check_launch("hc_overlap_count");
}

extern "C" int hc_drift_decide(const int32_t* counts, int npiv, int batch, int steps, int K, double threshold,
                               float* overlap, double* median, int32_t* trigger, void* stream) {
  clear_error();
  if (npiv < 0 || batch < 1 || steps < 1 || steps > 64 || K < 1)
    return set_error(HC_ERR_INVALID, "hc_drift_decide: npiv=%d batch=%d steps=%d K=%d", npiv, batch, steps, K);
  if (npiv == 0) return HC_OK;
  if (!counts || !trigger) return set_error(HC_ERR_INVALID, "hc_drift_decide: null pointer argument");
  hipLaunchKernelGGL(drift_decide_kernel, dim3((npiv + 63) / 64), dim3(64), 0, (hipStream_t)stream, counts, npiv,
                     batch, steps, K, threshold, overlap, median, trigger);
  return check_launch("hc_drift_decide");
}
