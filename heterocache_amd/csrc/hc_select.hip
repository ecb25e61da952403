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
#include "hc_common.h"
#include "hc_internal.h"

namespace hc {

constexpr int kSelThreads = 256;
constexpr int kSelWaves = kSelThreads / 64;
constexpr int kSelChunk = 4096;                      // positions per workgroup
constexpr int kSelRows = kSelChunk / kSelThreads;    // 16 rows of 256 positions
constexpr int kSelBins = 256;
constexpr int kSelMaxChunks = 4096;
constexpr int kSelMatch = 6;  // digits aggregated per wave before per-lane atomics
constexpr int kSelSub = 1;    // LDS sub-histograms per wave (power of two)

__device__ __forceinline__ uint32_t order_key(float f) {
  uint32_t u = __float_as_uint(f);
  if (u == 0x80000000u) u = 0u;  // -0 ranks equal to +0
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

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
    // Lanes sharing a digit are counted by one atomic of their first lane:
    // up to kSelMatch distinct digits per wave this way (score digits
    // cluster in few bins, where per-lane LDS atomics would serialise),
    // the remaining lanes one atomic each.
    uint64_t rem = __ballot(valid);
#pragma unroll
    for (int it = 0; it < kSelMatch; ++it) {
      if (rem == 0) break;
      const int leader = __ffsll((long long)rem) - 1;
      const uint32_t dl = (uint32_t)__builtin_amdgcn_readlane((int)d, leader);
      const uint64_t m = __ballot(valid && d == dl) & rem;
      if ((int)(threadIdx.x & 63) == leader) atomicAdd(&wh[dl], (unsigned)__popcll(m));
      rem &= ~m;
    }
    if ((rem >> (threadIdx.x & 63)) & 1ull) atomicAdd(&wh[d], 1u);
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
                                                                   int32_t* __restrict__ zero_out) {
  const int job = blockIdx.y, chunk = blockIdx.x;
  const SelJob jb = sel_job(caps, job, span, window, idx_stride);
  if (chunk == 0 && threadIdx.x == 0 && counts) counts[job] = jb.body + jb.tail;
  if (chunk == 0 && threadIdx.x == 0 && zero_out) zero_out[job] = 0;
  if (jb.body <= 0 || jb.body >= span) return;
  __shared__ int s_pick[3];
  __shared__ int s_red[2][kSelWaves];
  const SelState st = sel_replay(ghist + (int64_t)job * 4 * kSelBins, jb.body, 4, s_pick);
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
  if (tid == 0) {
    // Kept elements and ties in the chunks before this one.
    int sel = 0, eq = 0;
    for (int c = 0; c < chunk; ++c) {
      const int g = cnt[((int64_t)job * nchunks + c) * 2], e = cnt[((int64_t)job * nchunks + c) * 2 + 1];
      sel += g + (all_ties ? e : max(0, min(e, need_eq - eq)));
      eq += e;
    }
    s_base[0] = sel;
    s_base[1] = eq;
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

// Ties of tau in the chunks before `chunk` (from the count kernel's
// per-chunk counts).
__device__ __forceinline__ int ties_before(const int* __restrict__ cnt, int job, int chunk, int nchunks) {
  int eq = 0;
  for (int c = 0; c < chunk; ++c) eq += cnt[((int64_t)job * nchunks + c) * 2 + 1];
  return eq;
}

// Keep masks of one chunk: selm[r] is, per wave, the ballot over positions
// t0 + r*256 + 64*wave + lane of "kept" -- the key is above tau, or equals it
// and ranks below need_eq among the ties in position order (eq_before ties
// in earlier chunks).  Reached by the whole workgroup.
__device__ __forceinline__ void chunk_keep_masks(const float* __restrict__ s, int span, int t0, uint32_t tau,
                                                 int need_eq, bool all_ties, int eq_before,
                                                 uint64_t (&selm)[kSelRows], int (*s_cnt)[kSelWaves],
                                                 int (*s_off)[kSelWaves]) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint32_t keys[kSelRows];
#pragma unroll
  for (int r = 0; r < kSelRows; ++r) {
    const int t = t0 + r * kSelThreads + tid;
    keys[r] = t < span ? order_key(s[t]) : 0u;
  }
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  uint64_t eqm[kSelRows];
#pragma unroll
  for (int r = 0; r < kSelRows; ++r) {
    const int t = t0 + r * kSelThreads + tid;
    eqm[r] = __ballot(t < span && keys[r] == tau);
    if (lane == 0) s_cnt[r][wave] = __popcll(eqm[r]);
  }
  __syncthreads();
  if (tid == 0) {
    int e = eq_before;
    for (int r = 0; r < kSelRows; ++r)
      for (int w = 0; w < kSelWaves; ++w) {
        s_off[r][w] = e;
        e += s_cnt[r][w];
      }
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < kSelRows; ++r) {
    const int t = t0 + r * kSelThreads + tid;
    bool take = t < span && keys[r] > tau;
    if (t < span && keys[r] == tau) {
      const int rank = s_off[r][wave] + __popcll(eqm[r] & below);
      take = all_ties || rank < need_eq;
    }
    selm[r] = __ballot(take);
  }
  __syncthreads();
}

// 64 bits of a bitmask set starting at a multiple-of-64 position.
__device__ __forceinline__ uint64_t bits64(const uint32_t* __restrict__ b, int64_t words, int pos) {
  const int64_t w = pos >> 5;
  const uint64_t lo = w < words ? b[w] : 0u, hi = w + 1 < words ? b[w + 1] : 0u;
  return lo | (hi << 32);
}

// out[job] += |kept(job) ∩ set(job / steps)| over this chunk (out zeroed by
// the count kernel).  Chunk 0 clears the job's histograms for the next call.
__global__ __launch_bounds__(kSelThreads) void select_overlap_kernel(
    const float* __restrict__ scores, int64_t score_stride, int span, const int32_t* __restrict__ caps,
    unsigned* __restrict__ ghist, const int* __restrict__ state, const int* __restrict__ cnt, int nchunks,
    const uint32_t* __restrict__ bits, int64_t words, int steps, int32_t* __restrict__ out) {
  const int job = blockIdx.y, chunk = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const SelJob jb = sel_job(caps, job, span, 0, span);
  if (chunk == 0)
    for (int i = tid; i < 4 * kSelBins; i += kSelThreads) ghist[(int64_t)job * 4 * kSelBins + i] = 0u;
  if (jb.body <= 0) return;
  __shared__ int s_eq;
  __shared__ int s_cnt[kSelRows][kSelWaves];
  __shared__ int s_off[kSelRows][kSelWaves];
  __shared__ int s_sum[kSelWaves];
  const uint32_t* ref = bits + (int64_t)(job / steps) * words;
  const int t0 = chunk * kSelChunk;
  uint64_t selm[kSelRows];
  if (jb.body >= span) {
#pragma unroll
    for (int r = 0; r < kSelRows; ++r) selm[r] = __ballot(t0 + r * kSelThreads + tid < span);
  } else {
    if (tid == 0) s_eq = ties_before(cnt, job, chunk, nchunks);
    __syncthreads();
    chunk_keep_masks(scores + (int64_t)job * score_stride, span, t0, (uint32_t)state[job * 4], state[job * 4 + 1],
                     state[job * 4 + 2] != 0, s_eq, selm, s_cnt, s_off);
  }
  int c = 0;
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < kSelRows; ++r) c += __popcll(selm[r] & bits64(ref, words, t0 + r * kSelThreads + 64 * wave));
    s_sum[wave] = c;
  }
  __syncthreads();
  if (tid == 0) {
    int tot = 0;
    for (int w = 0; w < kSelWaves; ++w) tot += s_sum[w];
    if (tot) atomicAdd(out + job, tot);
  }
}

// Set j := kept(job j*steps + steps-1) as a bitmask, for sets whose leader
// triggered (trigger[trig_of[j]] != 0); other sets are left as they are.
// Each workgroup writes the words of its chunk (and chunk 0 any words past
// the last chunk), so no set needs clearing first.
__global__ __launch_bounds__(kSelThreads) void select_bits_kernel(
    const float* __restrict__ scores, int64_t score_stride, int span, const int32_t* __restrict__ caps,
    const int* __restrict__ state, const int* __restrict__ cnt, int nchunks, uint32_t* __restrict__ bits,
    int64_t words, int steps, const int32_t* __restrict__ trigger, const int32_t* __restrict__ trig_of) {
  const int set = blockIdx.y, chunk = blockIdx.x;
  if (trigger[trig_of ? trig_of[set] : set] == 0) return;
  const int job = set * steps + steps - 1;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const SelJob jb = sel_job(caps, job, span, 0, span);
  uint32_t* out = bits + (int64_t)set * words;
  const int t0 = chunk * kSelChunk;
  if (chunk == 0)
    for (int64_t w = (int64_t)nchunks * (kSelChunk / 32) + tid; w < words; w += kSelThreads) out[w] = 0u;
  __shared__ int s_eq;
  __shared__ int s_cnt[kSelRows][kSelWaves];
  __shared__ int s_off[kSelRows][kSelWaves];
  uint64_t selm[kSelRows];
  if (jb.body <= 0 || jb.body >= span) {
#pragma unroll
    for (int r = 0; r < kSelRows; ++r) selm[r] = __ballot(jb.body > 0 && t0 + r * kSelThreads + tid < span);
  } else {
    if (tid == 0) s_eq = ties_before(cnt, job, chunk, nchunks);
    __syncthreads();
    chunk_keep_masks(scores + (int64_t)job * score_stride, span, t0, (uint32_t)state[job * 4], state[job * 4 + 1],
                     state[job * 4 + 2] != 0, s_eq, selm, s_cnt, s_off);
  }
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < kSelRows; ++r) {
      const int64_t w = (t0 + r * kSelThreads + 64 * wave) >> 5;
      if (w < words) out[w] = (uint32_t)selm[r];
      if (w + 1 < words) out[w + 1] = (uint32_t)(selm[r] >> 32);
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
                              size_t hist_bytes, void* scratch, size_t scratch_bytes, void* stream) {
  clear_error();
  if (njobs < 0 || njobs > 65535 || span < 0 || window < 0)
    return set_error(HC_ERR_INVALID, "hc_select_topk: njobs=%d span=%d window=%d", njobs, span, window);
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
    for (int pass = 0; pass < 4; ++pass) {
      hipLaunchKernelGGL(select_hist_kernel, grid, dim3(kSelThreads), 0, s, scores, score_stride, span, caps, window,
                         idx_stride, ghist, pass);
      int rc = check_launch("hc_select_topk(hist)");
      if (rc) return rc;
    }
  }
  hipLaunchKernelGGL(select_count_kernel, grid, dim3(kSelThreads), 0, s, scores, score_stride, span, caps, window,
                     idx_stride, ghist, state, cnt, counts, nchunks, (int32_t*)nullptr);
  int rc = check_launch("hc_select_topk(count)");
  if (rc) return rc;
  hipLaunchKernelGGL(select_write_kernel, grid, dim3(kSelThreads), 0, s, scores, score_stride, span, caps, window,
                     idx, idx_stride, ghist, state, cnt, nchunks);
  return check_launch("hc_select_topk(write)");
}

extern "C" int hc_drift_select(const float* scores, int64_t score_stride, int nsets, int steps, int batch, int span,
                               const int32_t* caps, int K, uint32_t* bits, int64_t words, const int32_t* trig_of,
                               int nlead, double threshold, int32_t* overlap, int32_t* trigger, void* hist,
                               size_t hist_bytes, void* scratch, size_t scratch_bytes, void* stream) {
  clear_error();
  const int64_t njobs64 = (int64_t)nsets * steps;
  if (nsets < 0 || steps < 1 || steps > 64 || batch < 1 || span < 1 || K < 1 || njobs64 > 65535 ||
      (int64_t)nlead * batch != nsets || words < (span + 31) / 32)
    return set_error(HC_ERR_INVALID, "hc_drift_select: nsets=%d steps=%d batch=%d span=%d K=%d nlead=%d words=%lld",
                     nsets, steps, batch, span, K, nlead, (long long)words);
  if (nsets == 0) return HC_OK;
  if (!scores || !caps || !bits || !overlap || !trigger || !hist || !scratch)
    return set_error(HC_ERR_INVALID, "hc_drift_select: null pointer argument");
  const int njobs = (int)njobs64;
  if (score_stride < span) return set_error(HC_ERR_INVALID, "hc_drift_select: score stride below the span");
  const int nchunks = (span + kSelChunk - 1) / kSelChunk;
  if (nchunks > kSelMaxChunks) return set_error(HC_ERR_INVALID, "hc_drift_select: span %d too long", span);
  if (hist_bytes < select_hist_bytes(njobs) || scratch_bytes < select_scratch_bytes(njobs, span))
    return set_error(HC_ERR_INVALID, "hc_drift_select: histogram or scratch buffer too small");
  unsigned* ghist = reinterpret_cast<unsigned*>(hist);
  int* state = reinterpret_cast<int*>(scratch);
  int* cnt = state + (size_t)njobs * 4;
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid(nchunks, njobs);
  for (int pass = 0; pass < 4; ++pass) {
    hipLaunchKernelGGL(select_hist_kernel, grid, dim3(kSelThreads), 0, s, scores, score_stride, span, caps, 0,
                       (int64_t)span, ghist, pass);
    int rc = check_launch("hc_drift_select(hist)");
    if (rc) return rc;
  }
  hipLaunchKernelGGL(select_count_kernel, grid, dim3(kSelThreads), 0, s, scores, score_stride, span, caps, 0,
                     (int64_t)span, ghist, state, cnt, (int32_t*)nullptr, nchunks, overlap);
  int rc = check_launch("hc_drift_select(count)");
  if (rc) return rc;
  hipLaunchKernelGGL(select_overlap_kernel, grid, dim3(kSelThreads), 0, s, scores, score_stride, span, caps, ghist,
                     state, cnt, nchunks, bits, words, steps, overlap);
  rc = check_launch("hc_drift_select(overlap)");
  if (rc) return rc;
  rc = hc_drift_decide(overlap, nlead, batch, steps, K, threshold, nullptr, nullptr, trigger, stream);
  if (rc) return rc;
  hipLaunchKernelGGL(select_bits_kernel, dim3(nchunks, nsets), dim3(kSelThreads), 0, s, scores, score_stride, span,
                     caps, state, cnt, nchunks, bits, words, steps, trigger, trig_of);
  return check_launch("hc_drift_select(bits)");
}
