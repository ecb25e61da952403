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
// Multi-workgroup radix select: every job is cut into 4096-position chunks,
// one 256-thread workgroup per (chunk, job), six launches per call:
//  1-4. select_hist_kernel(pass p): histogram of the 8-bit digit p (MSB
//       first) of the order-preserving uint32 keys that match the digits
//       already fixed, per wave in LDS, summed into a global per-job
//       histogram.  Each workgroup recovers the fixed digits by replaying
//       the picks on the earlier global histograms (one wave-wide scan each).
//  5.   select_count_kernel: replays all four picks -> the exact key tau of
//       the last kept element and how many elements equal to tau are kept;
//       counts per chunk the keys above tau and equal to tau.
//  6.   select_write_kernel: chunk bases from the per-chunk counts, then an
//       ordered compaction (ballot ranks inside each 64-position row, LDS
//       scan across rows), so the output is ascending by construction.  It
//       also clears the global histograms for the next call and writes the
//       force-kept window tail.
#include <algorithm>

#include "hc_common.h"
#include "hc_internal.h"

namespace hc {

constexpr int kSelThreads = 256;
constexpr int kSelWaves = kSelThreads / 64;
constexpr int kSelChunk = 4096;                      // positions per workgroup
constexpr int kSelRows = kSelChunk / kSelThreads;    // 16 rows of 256 positions
constexpr int kSelBins = 256;
constexpr int kSelMaxChunks = 4096;
constexpr int kSelSub = 1;    // LDS sub-histograms per wave (power of two)

struct SelJob {
  int body;  // positions selected from [0, span)
  int tail;  // window positions appended
};

// Budget clamped to what the index row can hold; a window (SnapKV) is always
// kept whole (its reference asserts cap > window).
__device__ __forceinline__ SelJob sel_job(const int32_t* caps, int job, int span, int window, int64_t idx_stride) {
  const int cap = max(0, (int)min((int64_t)caps[job], idx_stride));
  SelJob j;
  j.tail = window;
  const int body = min(window > 0 ? max(cap - window, 0) : cap, span);
  j.body = min(body, (int)max((int64_t)0, idx_stride - window));
  return j;
}

struct SelState {
  uint32_t prefix, mask;
  int k_rem, ties;
};

// Replay the digit picks of passes [0, npass) from the global histograms.
// Reached by every thread of the workgroup; wave 0 does the scans.
__device__ __forceinline__ SelState sel_replay(const unsigned* __restrict__ ghist, int body, int npass,
                                               int* s_pick) {
  SelState st;
  st.prefix = 0;
  st.mask = 0;
  st.k_rem = body;
  st.ties = 0;
  const int lane = threadIdx.x & 63;
  for (int p = 0; p < npass; ++p) {
    if (threadIdx.x < 64) {
      // Lane l owns bins 255-4l .. 252-4l (descending digit order).
      int c[4], sum = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        c[i] = (int)ghist[p * kSelBins + kSelBins - 1 - 4 * lane - i];
        sum += c[i];
      }
      int incl = sum;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_up(incl, off, 64);
        if (lane >= off) incl += y;
      }
      int above = incl - sum;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (above < st.k_rem && above + c[i] >= st.k_rem) {
          s_pick[0] = kSelBins - 1 - 4 * lane - i;
          s_pick[1] = above;
          s_pick[2] = c[i];
        }
        above += c[i];
      }
    }
    __syncthreads();
    const int shift = 24 - 8 * p;
    st.prefix |= (uint32_t)s_pick[0] << shift;
    st.mask |= 0xFFu << shift;
    st.k_rem -= s_pick[1];
    st.ties = s_pick[2];
    __syncthreads();
  }
  return st;
}

__global__ __launch_bounds__(kSelThreads) void select_hist_kernel(const float* __restrict__ scores,
                                                                  int64_t score_stride, int span,
                                                                  const int32_t* __restrict__ caps, int window,
                                                                  int64_t idx_stride, unsigned* __restrict__ ghist,
                                                                  int pass) {
  const int job = blockIdx.y, chunk = blockIdx.x;
  const SelJob jb = sel_job(caps, job, span, window, idx_stride);
  if (jb.body <= 0 || jb.body >= span) return;
  // kSelSub histograms per wave (lane % kSelSub) spread same-bin atomics.
  __shared__ unsigned s_hist[kSelWaves * kSelSub][kSelBins];
  __shared__ int s_pick[3];
  unsigned* gh = ghist + (int64_t)job * 4 * kSelBins;
  const SelState st = sel_replay(gh, jb.body, pass, s_pick);
  for (int i = threadIdx.x; i < kSelWaves * kSelSub * kSelBins; i += kSelThreads) (&s_hist[0][0])[i] = 0;
  __syncthreads();
  const float* s = scores + (int64_t)job * score_stride;
  const int t0 = chunk * kSelChunk;
  const int shift = 24 - 8 * pass;
  unsigned* wh = s_hist[(threadIdx.x >> 6) * kSelSub + (threadIdx.x & (kSelSub - 1))];
  float v[kSelRows];
#pragma unroll
  for (int r = 0; r < kSelRows; ++r) {
    const int t = t0 + r * kSelThreads + threadIdx.x;
    v[r] = t < span ? s[t] : 0.f;
  }
#pragma unroll
  for (int r = 0; r < kSelRows; ++r) {
    const int t = t0 + r * kSelThreads + threadIdx.x;
    const uint32_t u = order_key(v[r]);
    const bool valid = t < span && (u & st.mask) == st.prefix;
    const uint32_t d = (u >> shift) & 0xFFu;
    // One LDS atomic per position.  (Counting the lanes of a wave that share
    // a digit by one atomic of their first lane, up to six digits a wave by
    // readlane / ballot rounds, was slower on clustered pooled scores:
    // 0.067 against 0.050 ms for 8 rows of 128K, top 49629.)
    if (valid) atomicAdd(&wh[d], 1u);
  }
  __syncthreads();
  for (int b = threadIdx.x; b < kSelBins; b += kSelThreads) {
    unsigned c = 0;
#pragma unroll
    for (int w = 0; w < kSelWaves * kSelSub; ++w) c += s_hist[w][b];
    if (c) atomicAdd(&gh[pass * kSelBins + b], c);
  }
}

// state[job] = {tau, need_eq, all_ties}; cnt[job][chunk] = {#key > tau, #key == tau}.
__global__ __launch_bounds__(kSelThreads) void select_count_kernel(const float* __restrict__ scores,
                                                                   int64_t score_stride, int span,
                                                                   const int32_t* __restrict__ caps, int window,
                                                                   int64_t idx_stride,
                                                                   const unsigned* __restrict__ ghist,
                                                                   int* __restrict__ state, int* __restrict__ cnt,
                                                                   int32_t* __restrict__ counts, int nchunks,
                                                                   int32_t* __restrict__ zero_out, int npass) {
  const int job = blockIdx.y, chunk = blockIdx.x;
  const SelJob jb = sel_job(caps, job, span, window, idx_stride);
  if (chunk == 0 && threadIdx.x == 0 && counts) counts[job] = jb.body + jb.tail;
  if (chunk == 0 && threadIdx.x == 0 && zero_out) zero_out[job] = 0;
  if (jb.body <= 0 || jb.body >= span) return;
  __shared__ int s_pick[3];
  __shared__ int s_red[2][kSelWaves];
  // With npass < 4 the keys' remaining low digits are zero (the caller's
  // contract), so the picked prefix is the key itself.
  const SelState st = sel_replay(ghist + (int64_t)job * 4 * kSelBins, jb.body, npass, s_pick);
  const uint32_t tau = st.prefix;
  if (chunk == 0 && threadIdx.x == 0) {
    int* sp = state + job * 4;
    sp[0] = (int)tau;
    sp[1] = st.k_rem;
    sp[2] = st.ties == st.k_rem ? 1 : 0;
  }
  const float* s = scores + (int64_t)job * score_stride;
  const int t0 = chunk * kSelChunk;
  int n_gt = 0, n_eq = 0;
#pragma unroll
  for (int r = 0; r < kSelRows; ++r) {
    const int t = t0 + r * kSelThreads + threadIdx.x;
    if (t < span) {
      const uint32_t u = order_key(s[t]);
      n_gt += u > tau;
      n_eq += u == tau;
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    n_gt += __shfl_xor(n_gt, off, 64);
    n_eq += __shfl_xor(n_eq, off, 64);
  }
  if ((threadIdx.x & 63) == 0) {
    s_red[0][threadIdx.x >> 6] = n_gt;
    s_red[1][threadIdx.x >> 6] = n_eq;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int a = 0, b = 0;
    for (int w = 0; w < kSelWaves; ++w) {
      a += s_red[0][w];
      b += s_red[1][w];
    }
    cnt[((int64_t)job * nchunks + chunk) * 2 + 0] = a;
    cnt[((int64_t)job * nchunks + chunk) * 2 + 1] = b;
  }
}

__global__ __launch_bounds__(kSelThreads) void select_write_kernel(const float* __restrict__ scores,
                                                                   int64_t score_stride, int span,
                                                                   const int32_t* __restrict__ caps, int window,
                                                                   int32_t* __restrict__ idx, int64_t idx_stride,
                                                                   unsigned* __restrict__ ghist,
                                                                   const int* __restrict__ state,
                                                                   const int* __restrict__ cnt, int nchunks) {
  const int job = blockIdx.y, chunk = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const SelJob jb = sel_job(caps, job, span, window, idx_stride);
  int32_t* out = idx + (int64_t)job * idx_stride;
  const int t0 = chunk * kSelChunk;
  if (chunk == 0) {
    for (int i = tid; i < jb.tail; i += kSelThreads) out[jb.body + i] = span + i;
    for (int i = tid; i < 4 * kSelBins; i += kSelThreads) ghist[(int64_t)job * 4 * kSelBins + i] = 0u;
  }
  if (jb.body <= 0) return;
  if (jb.body >= span) {
    for (int i = tid; i < kSelChunk; i += kSelThreads)
      if (t0 + i < span) out[t0 + i] = t0 + i;
    return;
  }
  __shared__ int s_base[2];
  __shared__ int s_cnt[2][kSelRows][kSelWaves];
  __shared__ int s_off[2][kSelRows][kSelWaves];
  const uint32_t tau = (uint32_t)state[job * 4];
  const int need_eq = state[job * 4 + 1];
  const bool all_ties = state[job * 4 + 2] != 0;
  if (wave == 0) {
    // Kept elements and ties in the chunks before this one: G keys above tau
    // and EQ ties in all, of which the ties taken in position order number
    // min(max(need_eq, 0), EQ) (the chunk-by-chunk sum of
    // max(0, min(e_c, need_eq - ties before c)) telescopes to it).  Summed
    // by the 64 lanes: one thread walking the chunks took a round trip per
    // few chunks, ~8 us for the last chunk of a 128K row.
    int g = 0, e = 0;
    for (int c = lane; c < chunk; c += 64) {
      g += cnt[((int64_t)job * nchunks + c) * 2];
      e += cnt[((int64_t)job * nchunks + c) * 2 + 1];
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      g += __shfl_xor(g, off, 64);
      e += __shfl_xor(e, off, 64);
    }
    if (lane == 0) {
      s_base[0] = g + (all_ties ? e : min(max(need_eq, 0), e));
      s_base[1] = e;
    }
  }
  const float* s = scores + (int64_t)job * score_stride;
  uint32_t keys[kSelRows];
#pragma unroll
  for (int r = 0; r < kSelRows; ++r) {
    const int t = t0 + r * kSelThreads + tid;
    keys[r] = t < span ? order_key(s[t]) : 0u;
  }
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  // Ties: ranks of equal keys in position order (row-major over (row, wave)).
  uint64_t eqm[kSelRows];
#pragma unroll
  for (int r = 0; r < kSelRows; ++r) {
    const int t = t0 + r * kSelThreads + tid;
    eqm[r] = __ballot(t < span && keys[r] == tau);
    if (lane == 0) s_cnt[1][r][wave] = __popcll(eqm[r]);
  }
  __syncthreads();
  if (tid == 0) {
    int e = s_base[1];
    for (int r = 0; r < kSelRows; ++r)
      for (int w = 0; w < kSelWaves; ++w) {
        s_off[1][r][w] = e;
        e += s_cnt[1][r][w];
      }
  }
  __syncthreads();
  uint64_t selm[kSelRows];
#pragma unroll
  for (int r = 0; r < kSelRows; ++r) {
    const int t = t0 + r * kSelThreads + tid;
    bool take = t < span && keys[r] > tau;
    if (t < span && keys[r] == tau) {
      const int rank = s_off[1][r][wave] + __popcll(eqm[r] & below);
      take = all_ties || rank < need_eq;
    }
    selm[r] = __ballot(take);
    if (lane == 0) s_cnt[0][r][wave] = __popcll(selm[r]);
  }
  __syncthreads();
  if (tid == 0) {
    int p = s_base[0];
    for (int r = 0; r < kSelRows; ++r)
      for (int w = 0; w < kSelWaves; ++w) {
        s_off[0][r][w] = p;
        p += s_cnt[0][r][w];
      }
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < kSelRows; ++r) {
    if ((selm[r] >> lane) & 1ull) out[s_off[0][r][wave] + __popcll(selm[r] & below)] = t0 + r * kSelThreads + tid;
  }
}

// 64 bits of a bitmask set starting at a multiple-of-64 position.
__device__ __forceinline__ uint64_t bits64(const uint32_t* __restrict__ b, int64_t words, int pos) {
  const int64_t w = pos >> 5;
  const uint64_t lo = w < words ? b[w] : 0u, hi = w + 1 < words ? b[w + 1] : 0u;
  return lo | (hi << 32);
}

// ---------------------------------------------------------------------------
// Drift selection (hc_drift_select).  The scorer left per step row a
// histogram of the top kKeyDigitBits bits of its scores' keys, so:
//  pick     the bin b* holding the K-th largest key and how many of the bin
//           are still to keep (k);
//  compact  one pass over the scores, chunk by chunk: keys above b* are kept
//           (the chunk's reference-set hits are counted), keys in b* are the
//           chunk's candidates (key, position), written to the chunk's own
//           segment -- no global atomics;
//  resolve  per row, a radix over the candidates' remaining key bits gives
//           the exact threshold tau and how many of its ties to keep, and a
//           radix over the ties' positions the cut pcut (the lowest
//           positions win); kept candidates add their hits;
//  decide   median of the batch-mean overlaps < threshold;
//  bits     triggered sets := keys > tau, or == tau at positions <= pcut.
// ---------------------------------------------------------------------------
enum DriftMode { kDriftNone = 0, kDriftAll = 1, kDriftPartial = 2 };

static size_t align256(size_t x) { return (x + 255) / 256 * 256; }
static int drift_chunks(int span) { return (span + kSelChunk - 1) / kSelChunk; }
// state [njobs][4], thresholds [njobs][4], per-chunk (candidates, hits) [njobs][nchunks][2]
static size_t drift_head_bytes(int njobs, int span) {
  return align256((size_t)njobs * 8 * sizeof(int) + (size_t)njobs * drift_chunks(span) * 2 * sizeof(int));
}
static size_t drift_cand_bytes(int njobs, int span) {
  return (size_t)njobs * drift_chunks(span) * kSelChunk * sizeof(uint2);
}
static size_t drift_hist_bytes(int njobs) { return (size_t)njobs * kKeyDigitBins * sizeof(uint32_t); }

// [head][candidate segments][histograms, used when the caller brings none]
size_t drift_scratch_bytes(int njobs, int span) {
  return drift_head_bytes(njobs, span) + drift_cand_bytes(njobs, span) + drift_hist_bytes(njobs);
}

// First-digit key histograms of the score rows, for callers whose scorer did
// not build them: workgroup (x, row) counts positions [x * kDriftHistSpan,
// +kDriftHistSpan) of the row in LDS and adds its nonzero bins to the row's
// histogram, which drift_zero_kernel cleared.  Each thread loads its 32
// positions (eight 16-byte loads) before counting any, so the loads are in
// flight together, then adds one LDS atomic per position.  Measured on the
// drift check's 165 rows of 128K pooled probabilities: 24 us; one workgroup
// per row, one position per thread and loop step, 66 us; counting lanes of a
// wave that share a digit by one atomic of their first lane (the readlane /
// ballot rounds of select_hist_kernel), 81 us; runs of equal digits among a
// thread's four consecutive positions counted once, 24 us (no gain).
constexpr int kDriftHistThreads = 256;
constexpr int kDriftHistVec = 8;  // 16-byte loads per thread
constexpr int kDriftHistSpan = kDriftHistThreads * 4 * kDriftHistVec;
__global__ __launch_bounds__(256) void drift_zero_kernel(uint32_t* __restrict__ p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) p[i] = 0u;
}

__global__ __launch_bounds__(kDriftHistThreads) void drift_hist_kernel(const float* __restrict__ scores,
                                                                       int64_t score_stride, int span,
                                                                       uint32_t* __restrict__ hist) {
  __shared__ uint32_t h[kKeyDigitBins];
  for (int b = threadIdx.x; b < kKeyDigitBins; b += kDriftHistThreads) h[b] = 0u;
  const float* s = scores + (int64_t)blockIdx.y * score_stride;
  const int t0 = blockIdx.x * kDriftHistSpan;
  const bool vec = (score_stride & 3) == 0;
  f32x4 x[kDriftHistVec];
  if (vec) {
    // Every lane loads 16 bytes, a group past the row's end from the last
    // group that holds a position (inside the row: the stride is a multiple
    // of 4), so no lane branches around the loads and all eight are in
    // flight together.  (With a per-lane branch to scalar loads into the
    // same registers each load waited for the previous one; removing it
    // took the drift check's 165 rows of 128K from 20.8 to 20.4 us: the
    // LDS atomics, not the loads, bound the kernel.)
    const int last = ((span - 1) / 4) * 4;
#pragma unroll
    for (int v = 0; v < kDriftHistVec; ++v) {
      const int t = t0 + (v * kDriftHistThreads + threadIdx.x) * 4;
      x[v] = *reinterpret_cast<const f32x4*>(s + min(t, last));
    }
  } else {
#pragma unroll
    for (int v = 0; v < kDriftHistVec; ++v) {
      const int t = t0 + (v * kDriftHistThreads + threadIdx.x) * 4;
#pragma unroll
      for (int e = 0; e < 4; ++e) x[v][e] = t + e < span ? s[t + e] : 0.f;
    }
  }
  __syncthreads();
#pragma unroll
  for (int v = 0; v < kDriftHistVec; ++v)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int t = t0 + (v * kDriftHistThreads + threadIdx.x) * 4 + e;
      if (t < span) atomicAdd(&h[order_key(x[v][e]) >> kKeyDigitShift], 1u);
    }
  __syncthreads();
  uint32_t* o = hist + (int64_t)blockIdx.y * kKeyDigitBins;
  for (int b = threadIdx.x; b < kKeyDigitBins; b += kDriftHistThreads)
    if (h[b]) atomicAdd(&o[b], h[b]);
}

// Inclusive prefix sum of one value per thread across a workgroup of NT.
template <int NT>
__device__ __forceinline__ int block_inclusive_scan(int v, int* s_tmp) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int u = __shfl_up(v, d, 64);
    if (lane >= d) v += u;
  }
  if (lane == 63) s_tmp[wave] = v;
  __syncthreads();
  int add = 0;
  for (int w = 0; w < wave; ++w) add += s_tmp[w];
  __syncthreads();
  return v + add;
}

// The bin of an NBINS histogram where the count, accumulated in scan order
// (descending bins when desc), reaches k (1 <= k <= total): s_out = {bin,
// k - count before the bin}.  Reached by the whole workgroup.
template <int NT, int NBINS>
__device__ __forceinline__ void block_find_bin(const uint32_t* h, int k, bool desc, int* s_tmp, int* s_out) {
  constexpr int BPT = NBINS / NT;
  static_assert(BPT * NT == NBINS, "bins must split evenly over the threads");
  if (threadIdx.x == 0) {  // stays {0, 0} if the histogram holds fewer than k
    s_out[0] = 0;
    s_out[1] = 0;
  }
  int c[BPT], sum = 0;
#pragma unroll
  for (int i = 0; i < BPT; ++i) {
    const int pos = threadIdx.x * BPT + i;
    c[i] = (int)h[desc ? NBINS - 1 - pos : pos];
    sum += c[i];
  }
  const int incl = block_inclusive_scan<NT>(sum, s_tmp);
  int before = incl - sum;
  if (before < k && incl >= k) {
#pragma unroll
    for (int i = 0; i < BPT; ++i) {
      if (before < k && before + c[i] >= k) {
        const int pos = threadIdx.x * BPT + i;
        s_out[0] = desc ? NBINS - 1 - pos : pos;
        s_out[1] = k - before;
      }
      before += c[i];
    }
  }
  __syncthreads();
}

// state[job] = {b*, k, mode}.
__global__ __launch_bounds__(256) void drift_pick_kernel(const uint32_t* __restrict__ hist,
                                                         const int32_t* __restrict__ caps, int span,
                                                         int* __restrict__ state) {
  const int job = blockIdx.x;
  __shared__ int s_tmp[4], s_out[2];
  const int K = max(0, min((int)caps[job], span));
  int* st = state + job * 4;
  if (K == 0 || K >= span) {
    if (threadIdx.x == 0) {
      st[0] = 0;
      st[1] = 0;
      st[2] = K == 0 ? kDriftNone : kDriftAll;
    }
    return;
  }
  block_find_bin<256, kKeyDigitBins>(hist + (int64_t)job * kKeyDigitBins, K, true, s_tmp, s_out);
  if (threadIdx.x == 0) {
    st[0] = s_out[0];
    st[1] = s_out[1];
    st[2] = kDriftPartial;
  }
}

// One chunk of one step row: its hits of the keys above b* against the row's
// reference set, and its keys in b* as candidates (key, position) in the
// chunk's segment; chunk_info[job][chunk] = {candidates, hits}.
__global__ __launch_bounds__(kSelThreads) void drift_compact_kernel(
    const float* __restrict__ scores, int64_t score_stride, int span, const int* __restrict__ state,
    const uint32_t* __restrict__ bits, int64_t words, int steps, int* __restrict__ chunk_info,
    uint2* __restrict__ cand, int64_t cand_stride) {
  const int job = blockIdx.y, chunk = blockIdx.x, nchunks = gridDim.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int* st = state + job * 4;
  const int mode = st[2];
  if (mode == kDriftNone) return;
  const uint32_t bstar = (uint32_t)st[0];
  const float* s = scores + (int64_t)job * score_stride;
  const uint32_t* ref = bits + (int64_t)(job / steps) * words;
  const int t0 = chunk * kSelChunk;
  uint2* seg = cand + (int64_t)job * cand_stride + t0;
  constexpr int kWords = kSelChunk / 32;
  __shared__ uint32_t s_ref[kWords];
  __shared__ int s_cnt;
  __shared__ int s_sum[kSelWaves];
  if (tid == 0) s_cnt = 0;
  for (int w = tid; w < kWords; w += kSelThreads) {
    const int64_t gw = (int64_t)(t0 >> 5) + w;
    s_ref[w] = gw < words ? ref[gw] : 0u;
  }
  float v[kSelRows];
#pragma unroll
  for (int r = 0; r < kSelRows; ++r) {
    const int t = t0 + r * kSelThreads + tid;
    v[r] = t < span ? s[t] : 0.f;
  }
  __syncthreads();
  // Per row: the wave's hits above b* and its candidate ballot; then one
  // LDS reservation per wave for all rows' candidates.
  // Ballots are wave-uniform (scalar registers); the keys are recomputed
  // from the scores when the candidates are written, and the rows go in two
  // halves, which keeps the kernel near 64 VGPRs without scalar spills.
  constexpr int kHalf = kSelRows / 2;
  int hits = 0;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    int ncand = 0;
    uint64_t mc[kHalf];
#pragma unroll
    for (int i = 0; i < kHalf; ++i) {
      const int r = h * kHalf + i;
      const int wb = r * kSelThreads + 64 * wave;  // chunk-local position of the wave's lane 0
      const bool valid = t0 + wb + lane < span;
      const uint32_t d = order_key(v[r]) >> kKeyDigitShift;
      const uint64_t mh = __ballot(valid && (mode == kDriftAll || d > bstar));
      const uint64_t rb = (uint64_t)s_ref[wb >> 5] | ((uint64_t)s_ref[(wb >> 5) + 1] << 32);
      hits += __popcll(mh & rb);
      mc[i] = __ballot(valid && mode == kDriftPartial && d == bstar);
      ncand += __popcll(mc[i]);
    }
    if (ncand) {
      int base = 0;
      if (lane == 0) base = atomicAdd(&s_cnt, ncand);
      base = __shfl(base, 0, 64);
#pragma unroll
      for (int i = 0; i < kHalf; ++i) {
        const int r = h * kHalf + i;
        const int t = t0 + r * kSelThreads + 64 * wave + lane;
        const uint32_t key = order_key(v[r]);
        if (t < span && mode == kDriftPartial && (key >> kKeyDigitShift) == bstar) {
          // Rank among the row's candidates of this wave: set bits of the
          // (uniform) ballot below this lane.
          const int rank = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mc[i] >> 32),
                                                          __builtin_amdgcn_mbcnt_lo((uint32_t)mc[i], 0u));
          seg[base + rank] = make_uint2(key, (uint32_t)t);
        }
        base += __popcll(mc[i]);
      }
    }
  }
  if (lane == 0) s_sum[wave] = hits;
  __syncthreads();
  if (tid == 0) {
    int tot = 0;
    for (int w = 0; w < kSelWaves; ++w) tot += s_sum[w];
    int* ci = chunk_info + ((int64_t)job * nchunks + chunk) * 2;
    ci[0] = s_cnt;
    ci[1] = tot;
  }
}

constexpr int kResolveThreads = 1024;
constexpr int kResolveRegs = 16;  // candidates per thread kept in registers

// Candidate i of a row whose chunk segments start at s_pref (exclusive
// prefix of the chunk counts, s_pref[nchunks] = total).
__device__ __forceinline__ uint2 cand_at(const uint2* __restrict__ c, const int* s_pref, int nchunks, int i) {
  int lo = 0, hi = nchunks - 1;  // last chunk whose prefix is <= i
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (s_pref[mid] <= i) lo = mid; else hi = mid - 1;
  }
  return c[(int64_t)lo * kSelChunk + (i - s_pref[lo])];
}

// thr[job] = {tau, pcut, mode}: kept = key > tau, or key == tau at a
// position <= pcut; overlap[job] = the chunks' hits + the kept candidates'.
__global__ __launch_bounds__(kResolveThreads) void drift_resolve_kernel(
    const int* __restrict__ state, const int* __restrict__ chunk_info, int nchunks, const uint2* __restrict__ cand,
    int64_t cand_stride, const uint32_t* __restrict__ bits, int64_t words, int steps, int32_t* __restrict__ overlap,
    int* __restrict__ thr) {
  const int job = blockIdx.x, tid = threadIdx.x;
  const int* st = state + job * 4;
  int* th = thr + job * 4;
  const int mode = st[2];
  __shared__ uint32_t h[2048];
  __shared__ int s_pref[kSelMaxChunks + 1];
  __shared__ int s_tmp[kResolveThreads / 64], s_out[2];
  if (mode == kDriftNone) {
    if (tid == 0) {
      th[0] = 0;
      th[1] = -1;
      th[2] = kDriftNone;
      overlap[job] = 0;
    }
    return;
  }
  // Chunk prefix of the candidate counts and the sum of the chunks' hits.
  const int* ci = chunk_info + (int64_t)job * nchunks * 2;
  int n = 0, hits = 0;
  for (int base = 0; base < nchunks; base += kResolveThreads) {
    const int ch = base + tid;
    const int cnt = ch < nchunks ? ci[2 * ch] : 0;
    if (ch < nchunks) hits += ci[2 * ch + 1];
    const int incl = block_inclusive_scan<kResolveThreads>(cnt, s_tmp);
    if (ch < nchunks) s_pref[ch] = n + incl - cnt;
    if (tid == kResolveThreads - 1) s_out[0] = incl;  // the block's total
    __syncthreads();
    n += s_out[0];
    __syncthreads();
  }
  if (tid == 0) s_pref[nchunks] = n;
  const uint2* c = cand + (int64_t)job * cand_stride;
  const uint32_t* ref = bits + (int64_t)(job / steps) * words;
  uint32_t tau = 0;
  int pcut = mode == kDriftAll ? INT_MAX : -1;
  __syncthreads();
  if (mode == kDriftPartial) {
    const uint32_t bstar = (uint32_t)st[0];
    int k = st[1];
    // The first kResolveRegs * kResolveThreads candidates stay in registers
    // for all the passes below; any beyond are re-read each pass.
    uint2 rc[kResolveRegs];
#pragma unroll
    for (int u = 0; u < kResolveRegs; ++u) {
      const int i = tid + u * kResolveThreads;
      rc[u] = i < n ? cand_at(c, s_pref, nchunks, i) : make_uint2(0u, 0u);
    }
    auto visit = [&](auto&& f) {
#pragma unroll
      for (int u = 0; u < kResolveRegs; ++u)
        if (tid + u * kResolveThreads < n) f(rc[u]);
      for (int i = tid + kResolveRegs * kResolveThreads; i < n; i += kResolveThreads) f(cand_at(c, s_pref, nchunks, i));
    };
    // Key bits [19:10], then [9:0] within the chosen bin.
    for (int b = tid; b < 1024; b += kResolveThreads) h[b] = 0u;
    __syncthreads();
    visit([&](uint2 x) { atomicAdd(&h[(x.x >> 10) & 1023u], 1u); });
    __syncthreads();
    block_find_bin<kResolveThreads, 1024>(h, k, true, s_tmp, s_out);
    const uint32_t ba = (uint32_t)s_out[0];
    k = s_out[1];
    for (int b = tid; b < 1024; b += kResolveThreads) h[b] = 0u;
    __syncthreads();
    visit([&](uint2 x) {
      if (((x.x >> 10) & 1023u) == ba) atomicAdd(&h[x.x & 1023u], 1u);
    });
    __syncthreads();
    block_find_bin<kResolveThreads, 1024>(h, k, true, s_tmp, s_out);
    const uint32_t bb = (uint32_t)s_out[0];
    k = s_out[1];
    tau = (bstar << kKeyDigitShift) | (ba << 10) | bb;
    const int n_eq = (int)h[bb];
    __syncthreads();
    pcut = INT_MAX;
    if (k < n_eq) {
      // The k lowest positions among the keys equal to tau: position bits
      // [30:20], [19:10], [9:0], ascending.
      uint32_t pref = 0;  // position bits found so far
      for (int lv = 0; lv < 3; ++lv) {
        const int shift = lv == 0 ? 20 : (lv == 1 ? 10 : 0);
        const int nb = lv == 0 ? 2048 : 1024;
        for (int b = tid; b < nb; b += kResolveThreads) h[b] = 0u;
        __syncthreads();
        visit([&](uint2 x) {
          if (x.x == tau && (lv == 0 || (x.y >> (shift + 10)) == pref))
            atomicAdd(&h[(x.y >> shift) & (uint32_t)(nb - 1)], 1u);
        });
        __syncthreads();
        if (lv == 0)
          block_find_bin<kResolveThreads, 2048>(h, k, false, s_tmp, s_out);
        else
          block_find_bin<kResolveThreads, 1024>(h, k, false, s_tmp, s_out);
        pref = lv == 0 ? (uint32_t)s_out[0] : (pref << 10) | (uint32_t)s_out[0];
        k = s_out[1];
        __syncthreads();
      }
      pcut = (int)pref;
    }
    visit([&](uint2 x) {
      const int pos = (int)x.y;
      if ((x.x > tau || (x.x == tau && pos <= pcut)) && ((ref[pos >> 5] >> (pos & 31)) & 1u)) ++hits;
    });
  }
  if (tid == 0) {
    th[0] = (int)tau;
    th[1] = pcut;
    th[2] = mode;
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) hits += __shfl_xor(hits, off, 64);
  if ((tid & 63) == 0) s_tmp[tid >> 6] = hits;
  __syncthreads();
  if (tid == 0) {
    int tot = 0;
    for (int w = 0; w < kResolveThreads / 64; ++w) tot += s_tmp[w];
    overlap[job] = tot;
  }
}

// Set j := the kept positions of its last step row, for sets whose leader
// triggered (trigger[trig_of[j]] != 0); other sets are left as they are.
// Each workgroup writes its chunk's words (chunk 0 also any words past the
// last chunk), so no set needs clearing first.
__global__ __launch_bounds__(kSelThreads) void drift_bits_kernel(
    const float* __restrict__ scores, int64_t score_stride, int span, const int* __restrict__ thr,
    uint32_t* __restrict__ bits, int64_t words, int steps, const int32_t* __restrict__ trigger,
    const int32_t* __restrict__ trig_of, int nchunks) {
  const int set = blockIdx.y, chunk = blockIdx.x;
  if (trigger[trig_of ? trig_of[set] : set] == 0) return;
  const int job = set * steps + steps - 1;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int* th = thr + job * 4;
  const uint32_t tau = (uint32_t)th[0];
  const int pcut = th[1], mode = th[2];
  const float* s = scores + (int64_t)job * score_stride;
  uint32_t* out = bits + (int64_t)set * words;
  const int t0 = chunk * kSelChunk;
  if (chunk == 0)
    for (int64_t w = (int64_t)nchunks * (kSelChunk / 32) + tid; w < words; w += kSelThreads) out[w] = 0u;
  float v[kSelRows];
#pragma unroll
  for (int r = 0; r < kSelRows; ++r) {
    const int t = t0 + r * kSelThreads + tid;
    v[r] = t < span ? s[t] : 0.f;
  }
#pragma unroll
  for (int r = 0; r < kSelRows; ++r) {
    const int tb = t0 + r * kSelThreads + 64 * wave;
    const int t = tb + lane;
    const uint32_t key = order_key(v[r]);
    const bool keep = t < span && (mode == kDriftAll ||
                                   (mode == kDriftPartial && (key > tau || (key == tau && t <= pcut))));
    const uint64_t m = __ballot(keep);
    if (lane == 0) {
      const int64_t w = tb >> 5;
      if (w < words) out[w] = (uint32_t)m;
      if (w + 1 < words) out[w + 1] = (uint32_t)(m >> 32);
    }
  }
}

// The histograms live in a buffer that must be zero before the first call and
// that every completed call leaves zeroed; state and chunk counts live in a
// per-call scratch buffer that needs no initialisation.
size_t select_hist_bytes(int njobs) { return (size_t)njobs * 4 * kSelBins * sizeof(unsigned); }

size_t select_scratch_bytes(int njobs, int span) {
  const int nchunks = (span + kSelChunk - 1) / kSelChunk;
  return (size_t)njobs * (4 * sizeof(int) + (size_t)nchunks * 2 * sizeof(int));
}

}  // namespace hc

using namespace hc;

extern "C" size_t hc_select_hist_size(int njobs) {
  if (njobs <= 0) return 0;
  return select_hist_bytes(njobs);
}

extern "C" size_t hc_select_scratch_size(int njobs, int span) {
  if (njobs <= 0 || span < 0) return 0;
  return select_scratch_bytes(njobs, span);
}

extern "C" int hc_select_topk(const float* scores, int64_t score_stride, int njobs, int span, const int32_t* caps,
                              int window, int32_t* idx, int64_t idx_stride, int32_t* counts, void* hist,
                              size_t hist_bytes, void* scratch, size_t scratch_bytes, int key_bits, void* stream) {
  clear_error();
  if (njobs < 0 || njobs > 65535 || span < 0 || window < 0)
    return set_error(HC_ERR_INVALID, "hc_select_topk: njobs=%d span=%d window=%d", njobs, span, window);
  if (key_bits < 0 || key_bits > 32)
    return set_error(HC_ERR_INVALID, "hc_select_topk: key_bits=%d (0..32)", key_bits);
  // Radix passes: the 8-bit digits that can differ between the scores' keys.
  const int npass = key_bits == 0 ? 4 : std::max(1, (key_bits + 7) / 8);
  if (njobs == 0) return HC_OK;
  if (!scores || !caps || !idx || !hist || !scratch)
    return set_error(HC_ERR_INVALID, "hc_select_topk: null pointer argument");
  if (score_stride < span || idx_stride < window || idx_stride < 1)
    return set_error(HC_ERR_INVALID, "hc_select_topk: strides too small (scores %lld, idx %lld)",
                     (long long)score_stride, (long long)idx_stride);
  const int nchunks = (span + kSelChunk - 1) / kSelChunk;
  if (nchunks > kSelMaxChunks) return set_error(HC_ERR_INVALID, "hc_select_topk: span %d too long", span);
  if (hist_bytes < select_hist_bytes(njobs) || scratch_bytes < select_scratch_bytes(njobs, span))
    return set_error(HC_ERR_INVALID, "hc_select_topk: histogram or scratch buffer too small");
  unsigned* ghist = reinterpret_cast<unsigned*>(hist);
  int* state = reinterpret_cast<int*>(scratch);
  int* cnt = state + (size_t)njobs * 4;
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid(nchunks > 0 ? nchunks : 1, njobs);
  if (nchunks > 0) {
    for (int pass = 0; pass < npass; ++pass) {
      hipLaunchKernelGGL(select_hist_kernel, grid, dim3(kSelThreads), 0, s, scores, score_stride, span, caps, window,
                         idx_stride, ghist, pass);
      int rc = check_launch("hc_select_topk(hist)");
      if (rc) return rc;
    }
  }
  hipLaunchKernelGGL(select_count_kernel, grid, dim3(kSelThreads), 0, s, scores, score_stride, span, caps, window,
                     idx_stride, ghist, state, cnt, counts, nchunks, (int32_t*)nullptr, npass);
  int rc = check_launch("hc_select_topk(count)");
  if (rc) return rc;
  hipLaunchKernelGGL(select_write_kernel, grid, dim3(kSelThreads), 0, s, scores, score_stride, span, caps, window,
                     idx, idx_stride, ghist, state, cnt, nchunks);
  return check_launch("hc_select_topk(write)");
}

extern "C" size_t hc_drift_scratch_size(int njobs, int span) {
  if (njobs <= 0 || span <= 0) return 0;
  return drift_scratch_bytes(njobs, span);
}

extern "C" int hc_drift_select(const float* scores, int64_t score_stride, int nsets, int steps, int batch, int span,
                               const int32_t* caps, int K, uint32_t* bits, int64_t words, const int32_t* trig_of,
                               int nlead, double threshold, int32_t* overlap, int32_t* trigger, const uint32_t* hist,
                               void* scratch, size_t scratch_bytes, void* stream) {
  clear_error();
  const int64_t njobs64 = (int64_t)nsets * steps;
  if (nsets < 0 || steps < 1 || steps > 64 || batch < 1 || span < 1 || K < 1 || njobs64 > 65535 ||
      (int64_t)nlead * batch != nsets || words < (span + 31) / 32)
    return set_error(HC_ERR_INVALID, "hc_drift_select: nsets=%d steps=%d batch=%d span=%d K=%d nlead=%d words=%lld",
                     nsets, steps, batch, span, K, nlead, (long long)words);
  if (nsets == 0) return HC_OK;
  if (!scores || !caps || !bits || !overlap || !trigger || !scratch)
    return set_error(HC_ERR_INVALID, "hc_drift_select: null pointer argument");
  const int njobs = (int)njobs64;
  if (score_stride < span) return set_error(HC_ERR_INVALID, "hc_drift_select: score stride below the span");
  const int nchunks = drift_chunks(span);
  if (nchunks > kSelMaxChunks) return set_error(HC_ERR_INVALID, "hc_drift_select: span %d too long", span);
  if (scratch_bytes < drift_scratch_bytes(njobs, span))
    return set_error(HC_ERR_INVALID, "hc_drift_select: scratch buffer too small (%zu < %zu bytes)", scratch_bytes,
                     drift_scratch_bytes(njobs, span));
  int* state = reinterpret_cast<int*>(scratch);
  int* thr = state + (size_t)njobs * 4;
  int* chunk_info = thr + (size_t)njobs * 4;
  char* base = reinterpret_cast<char*>(scratch);
  uint2* cand = reinterpret_cast<uint2*>(base + drift_head_bytes(njobs, span));
  const int64_t cand_stride = (int64_t)nchunks * kSelChunk;
  hipStream_t s = (hipStream_t)stream;
  int rc;
  if (!hist) {
    uint32_t* own = reinterpret_cast<uint32_t*>(base + drift_head_bytes(njobs, span) + drift_cand_bytes(njobs, span));
    const int64_t words = (int64_t)njobs * kKeyDigitBins;
    hipLaunchKernelGGL(drift_zero_kernel, dim3((unsigned)std::min<int64_t>((words + 255) / 256, 1024)), dim3(256), 0,
                       s, own, words);
    if ((rc = check_launch("hc_drift_select(hist zero)"))) return rc;
    hipLaunchKernelGGL(drift_hist_kernel, dim3((span + kDriftHistSpan - 1) / kDriftHistSpan, njobs),
                       dim3(kDriftHistThreads), 0, s, scores, score_stride, span, own);
    if ((rc = check_launch("hc_drift_select(hist)"))) return rc;
    hist = own;
  }
  hipLaunchKernelGGL(drift_pick_kernel, dim3(njobs), dim3(256), 0, s, hist, caps, span, state);
  if ((rc = check_launch("hc_drift_select(pick)"))) return rc;
  hipLaunchKernelGGL(drift_compact_kernel, dim3(nchunks, njobs), dim3(kSelThreads), 0, s, scores, score_stride, span,
                     state, bits, words, steps, chunk_info, cand, cand_stride);
  if ((rc = check_launch("hc_drift_select(compact)"))) return rc;
  hipLaunchKernelGGL(drift_resolve_kernel, dim3(njobs), dim3(kResolveThreads), 0, s, state, chunk_info, nchunks, cand,
                     cand_stride, bits, words, steps, overlap, thr);
  if ((rc = check_launch("hc_drift_select(resolve)"))) return rc;
  rc = hc_drift_decide(overlap, nlead, batch, steps, K, threshold, nullptr, nullptr, trigger, stream);
  if (rc) return rc;
  hipLaunchKernelGGL(drift_bits_kernel, dim3(nchunks, nsets), dim3(kSelThreads), 0, s, scores, score_stride, span,
                     thr, bits, words, steps, trigger, trig_of, nchunks);
  return check_launch("hc_drift_select(bits)");
}
