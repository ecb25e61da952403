// Per-head variable-budget top-k, returned in ascending position order.
//
// For job j with budget cap[j] over scores s[0, span):
//   kept = the cap positions ranked first by (score descending, position
//          ascending), sorted ascending;
//   with window > 0 (SnapKV style) the budget is cap - window over
//   [0, span) and positions span .. span+window-1 are appended.
// This is the reference's topk(max_cap) -> mask rank >= cap_h -> sort
// (heterocache/cache_utils.py:831-851), SnapKV's topk(cap - W) + window
// concat (heterocache/kv_cluster.py:187-197) and the drift/retrieval topk
// (heterocache/cache_utils.py:1060-1061, :1090-1093) under the stated tie
// rule: equal scores keep the lower position first.
//
// One 1024-thread workgroup per job:
//  1. radix select, four 8-bit MSB-first passes over order-preserving uint32
//     keys with an LDS histogram, finds the exact key tau of the last kept
//     element and how many elements equal to tau are kept;
//  2. one ordered pass emits every position with key > tau plus the first
//     `need_eq` positions with key == tau, using block-wide exclusive scans,
//     so the output is ascending by construction.
#include "hc_common.h"
#include "hc_internal.h"

namespace hc {

constexpr int kSelThreads = 1024;
constexpr int kSelItems = 4;  // consecutive positions per thread per compaction step

__device__ __forceinline__ uint32_t order_key(float f) {
  uint32_t u = __float_as_uint(f);
  if (u == 0x80000000u) u = 0u;  // -0 ranks equal to +0
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Exclusive scan of one int per thread across the workgroup; returns the
// exclusive prefix and writes the total to *total.
__device__ __forceinline__ int block_exclusive_scan(int v, int* s_wave, int* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(x, off, 64);
    if (lane >= off) x += y;
  }
  if (lane == 63) s_wave[wave] = x;
  __syncthreads();
  if (wave == 0) {
    int w = lane < kSelThreads / 64 ? s_wave[lane] : 0;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int y = __shfl_up(w, off, 64);
      if (lane >= off) w += y;
    }
    if (lane < kSelThreads / 64) s_wave[lane] = w;  // inclusive prefix of wave totals
  }
  __syncthreads();
  const int before = wave > 0 ? s_wave[wave - 1] : 0;
  *total = s_wave[kSelThreads / 64 - 1];
  __syncthreads();
  return before + x - v;
}

__global__ __launch_bounds__(kSelThreads) void select_topk_kernel(const float* __restrict__ scores,
                                                                   int64_t score_stride, int span,
                                                                   const int32_t* __restrict__ caps, int window,
                                                                   int32_t* __restrict__ idx, int64_t idx_stride,
                                                                   int32_t* __restrict__ counts) {
  const int job = blockIdx.x;
  const float* s = scores + (int64_t)job * score_stride;
  int32_t* out = idx + (int64_t)job * idx_stride;
  const int tid = threadIdx.x;
  __shared__ unsigned s_hist[256];
  __shared__ int s_wave[kSelThreads / 64];
  __shared__ unsigned s_digit, s_above;

  // Budget clamped to what the index row can hold; a window (SnapKV) is
  // always kept whole (its reference asserts cap > window).
  const int cap = max(0, (int)min((int64_t)caps[job], idx_stride));
  const int tail = window;
  int body = min(window > 0 ? max(cap - window, 0) : cap, span);
  body = min(body, (int)max((int64_t)0, idx_stride - tail));

  if (body >= span) {
    for (int t = tid; t < span; t += kSelThreads) out[t] = t;
  } else if (body > 0) {
    // 1. radix select of the body-th largest key.
    uint32_t prefix = 0, mask = 0;
    int k_rem = body;
    for (int pass = 0; pass < 4; ++pass) {
      const int shift = 24 - 8 * pass;
      for (int i = tid; i < 256; i += kSelThreads) s_hist[i] = 0;
      __syncthreads();
      for (int t = tid; t < span; t += kSelThreads) {
        const uint32_t u = order_key(s[t]);
        if ((u & mask) == prefix) atomicAdd(&s_hist[(u >> shift) & 255u], 1u);
      }
      __syncthreads();
      if (tid == 0) {
        unsigned above = 0;
        int d = 255;
        for (; d > 0; --d) {
          if (above + s_hist[d] >= (unsigned)k_rem) break;
          above += s_hist[d];
        }
        s_digit = (unsigned)d;
        s_above = above;
      }
      __syncthreads();
      prefix |= s_digit << shift;
      mask |= 255u << shift;
      k_rem -= (int)s_above;
      __syncthreads();
    }
    const uint32_t tau = prefix;
    const int need_eq = k_rem;  // >= 1 elements equal to tau are kept
    // 2. ordered compaction.
    int sel_base = 0, eq_base = 0;
    for (int t0 = 0; t0 < span; t0 += kSelThreads * kSelItems) {
      const int tb = t0 + tid * kSelItems;
      uint32_t keys[kSelItems];
      int n_eq = 0;
#pragma unroll
      for (int i = 0; i < kSelItems; ++i) {
        const int t = tb + i;
        keys[i] = t < span ? order_key(s[t]) : 0u;
        if (t < span) n_eq += keys[i] == tau;
      }
      int tot_eq;
      const int eq_before = eq_base + block_exclusive_scan(n_eq, s_wave, &tot_eq);
      // Positions this thread keeps, given the running count of ties.
      int n_sel = 0;
      {
        int e = eq_before;
#pragma unroll
        for (int i = 0; i < kSelItems; ++i) {
          const int t = tb + i;
          if (t >= span) continue;
          if (keys[i] > tau) ++n_sel;
          else if (keys[i] == tau) { n_sel += (e < need_eq); ++e; }
        }
      }
      int tot_sel;
      int pos = sel_base + block_exclusive_scan(n_sel, s_wave, &tot_sel);
      {
        int e = eq_before;
#pragma unroll
        for (int i = 0; i < kSelItems; ++i) {
          const int t = tb + i;
          if (t >= span) continue;
          bool take = false;
          if (keys[i] > tau) take = true;
          else if (keys[i] == tau) { take = (e < need_eq); ++e; }
          if (take) out[pos++] = t;
        }
      }
      sel_base += tot_sel;
      eq_base += tot_eq;
    }
  }
  // Force-kept window tail.
  for (int i = tid; i < tail; i += kSelThreads) out[body + i] = span + i;
  if (tid == 0 && counts) counts[job] = body + tail;
}

}  // namespace hc

using namespace hc;

extern "C" int hc_select_topk(const float* scores, int64_t score_stride, int njobs, int span, const int32_t* caps,
                              int window, int32_t* idx, int64_t idx_stride, int32_t* counts, void* stream) {
  clear_error();
  if (njobs < 0 || njobs > 65535 || span < 0 || window < 0)
    return set_error(HC_ERR_INVALID, "hc_select_topk: njobs=%d span=%d window=%d", njobs, span, window);
  if (njobs == 0) return HC_OK;
  if (!scores || !caps || !idx) return set_error(HC_ERR_INVALID, "hc_select_topk: null pointer argument");
  if (score_stride < span || idx_stride < window || idx_stride < 1)
    return set_error(HC_ERR_INVALID, "hc_select_topk: strides too small (scores %lld, idx %lld)",
                     (long long)score_stride, (long long)idx_stride);
  hipLaunchKernelGGL(select_topk_kernel, dim3(njobs), dim3(kSelThreads), 0, (hipStream_t)stream, scores,
                     score_stride, span, caps, window, idx, idx_stride, counts);
  return check_launch("hc_select_topk");
}
