// Observation-window attention scores, pooled and maxed over the GQA group.
//
//   S_j[w'][t] = max_g round(pool_k(round(sum_w round(softmax_t(q_{g,w}.k_t * scale + mask)))))
//
// One implementation serves every scorer of the path:
//  * prefill budget scoring, last query (W = 1): HeteroCache.prefill_select
//    and init_coefficient (heterocache/cache_utils.py:807-829, :1158-1187);
//  * SnapKV window scoring (W = 32, causal window, sum over the window, span
//    L - W): SnapKVCluster.update_kv (heterocache/kv_cluster.py:165-185);
//  * pivot drift scoring of the buffered decode queries against a pivot's
//    prefill keys read in place from the tiled store (W = decode_step rows,
//    no sum): HeteroCache.decode_select (heterocache/cache_utils.py:1030-1057).
// `round` reproduces the reference's casts to the model dtype when asked
// (HC_SCORE_ROUND_BF16 / _F16); by default everything stays float32.
//
// Phases (all launched by hc_score):
//  1. score_stats_kernel: per (job, run of 256-token chunks) the logits of
//     all G*W query rows against 16-token key sub-tiles on the MFMA (K is
//     the A operand, loaded straight from HBM; queries are B operands staged
//     in LDS once per workgroup), reduced to a (max, sum exp) per row; with
//     fewer than 32 rows the logits are stored too.
//  2. score_stats_merge_kernel: fold the workgroups' (max, sum) per row
//     (on the stored-logit path, phase 3b folds them itself unless the
//     drift histograms need clearing).
//  3a. (>= 32 rows) score_probs_kernel: recompute the logits, normalise, sum
//     over the window rows of each query head (xor-shuffle tree: fixed
//     order), write A[job][w'][g][t]; score_pool_kernel: pooling over t and
//     max over g -> S[job][w'][t].
//  3b. (< 32 rows) score_finish_kernel: the same from the stored logits
//     (score_finish_reg_kernel for pool kernels 5 and 7: pooling in
//     registers).
// CAKE scoring (hc_cake_score) runs phases 1-2, the probability pass with
// window moments, and its own pooling and reductions.
// With the rows' softmax statistics already known (prefill attention reports
// them for its last queries, decode attention for each step query), phases
// 1-2 drop out: hc_score_with_stats runs phase 3a alone (one key pass), and
// hc_score_given_stats is the fused one-pass kernel of the drift check
// (fewer than 32 rows, tiled store, pooling in LDS).
#include <cfloat>
#include <algorithm>
#include <cmath>
#include <mutex>
#include <type_traits>
#include <vector>

#include "hc_common.h"
#include "hc_internal.h"

namespace hc {

constexpr int kScoreWaves = 4;
constexpr int kSubTiles = 4;                      // 16-token sub-tiles per wave
constexpr int kScoreChunk = kScoreWaves * 16 * kSubTiles;  // 256 tokens per workgroup
constexpr int kQPitch = HC_HEAD_DIM + 8;

struct ScoreArgs {
  const void* q;
  const int64_t* q_off;
  int64_t q_head_stride, q_row_stride;
  const void* k;
  const int64_t* k_off;
  int64_t k_tok_stride;
  const int64_t* row_tile_off;
  const int32_t* k_row;
  int L, G, W, R, NT, flags, span;
  int cpw;  // 256-token chunks per workgroup of the statistics and probability passes
  float scale;
  float scale2;  // scale * log2(e): base-2 logits without the reference's casts
};


__device__ __forceinline__ float round_mode(float x, int flags) {
  if (flags & HC_SCORE_ROUND_BF16) return (float)(__bf16)x;
  if (flags & HC_SCORE_ROUND_F16) return (float)(_Float16)x;
  return x;
}

// Stage the query rows (row r = g*W + w) of a job in LDS, zero-padded to NT*16.
template <typename T>
__device__ __forceinline__ void stage_queries(const ScoreArgs& a, int job, T* s_q) {
  const T* q = reinterpret_cast<const T*>(a.q) + a.q_off[job];
  const int rows = a.NT * 16;
  for (int c = threadIdx.x; c < rows * 16; c += kScoreWaves * 64) {
    const int r = c >> 4, ch = c & 15;
    typename Elem<T>::vec8 v = zero8<T>();
    if (r < a.R) {
      const int g = r / a.W, w = r % a.W;
      v = load8<T>(q + g * a.q_head_stride + w * a.q_row_stride + ch * 8);
    }
    *reinterpret_cast<typename Elem<T>::vec8*>(s_q + r * kQPitch + ch * 8) = v;
  }
}

// K operand of one 16-token sub-tile: lane holds token t0 + (lane & 15),
// channels 32s + 8*(lane >> 4) + [0, 8).
// The job's keys: its first tile in the store, or its first row in natural
// layout.  Read once per kernel: the offset tables sit in global memory, and
// read again in a chunk loop after the loop's own stores (which could alias
// them) each read was a chain of waits that drained every load in flight.
template <typename T, bool STORE>
__device__ __forceinline__ const T* job_keys(const ScoreArgs& a, int job) {
  if constexpr (STORE) return reinterpret_cast<const T*>(a.k) + a.row_tile_off[a.k_row[job]] * (int64_t)HC_TILE_ELEMS;
  return reinterpret_cast<const T*>(a.k) + a.k_off[job];
}

template <typename T, bool STORE>
__device__ __forceinline__ void load_k_subtile(const ScoreArgs& a, const T* kj, int t0, int lane,
                                               typename Elem<T>::vec8 (&kr)[4]) {
  if constexpr (STORE) {
    if (t0 >= a.L) {  // the sub-tile may lie past the row's capacity
#pragma unroll
      for (int s = 0; s < 4; ++s) kr[s] = zero8<T>();
      return;
    }
    const T* base = kj + (t0 / HC_TILE) * (int64_t)HC_TILE_ELEMS;
    const int h = (t0 / 16) & 1;
#pragma unroll
    // Keys read in place from the store are read once per launch: streamed
    // past L2 (260 -> 247 us for the 33-pivot drift check at 128K).  The
    // natural-layout callers keep ordinary loads: their second pass over
    // the same keys hits in the caches (nontemporal: 0.137 -> 0.150 ms for
    // the two-pass window scorer).
    for (int s = 0; s < 4; ++s) kr[s] = load8_stream<T>(base + (h * 4 + s) * 512 + lane * 8);
  } else {
    const int t = t0 + (lane & 15);
    if (t < a.L) {
      const T* p = kj + (int64_t)t * a.k_tok_stride + 8 * (lane >> 4);
#pragma unroll
      for (int s = 0; s < 4; ++s) kr[s] = load8<T>(p + 32 * s);
    } else {
#pragma unroll
      for (int s = 0; s < 4; ++s) kr[s] = zero8<T>();
    }
  }
}

// Last key position row r may see: L - W + w under the causal window mask,
// else L - 1; -1 for padding rows (r >= R).  Computed once per row tile, so
// the inner loops hold no integer division.
__device__ __forceinline__ int row_limit(const ScoreArgs& a, int r) {
  if (r >= a.R) return -1;
  return (a.flags & HC_SCORE_CAUSAL_WINDOW) ? a.L - a.W + r % a.W : a.L - 1;
}

template <int RM>
__device__ __forceinline__ float scaled_logit(const ScoreArgs& a, float acc) {
  if constexpr (RM == 0) return acc * a.scale2;
  return round_fixed<RM>(round_fixed<RM>(acc) * a.scale) * 1.4426950408889634f;
}

// Logits (base 2) of row 16nt + (lane & 15) (visible up to `limit`) for
// tokens t0 + 4*(lane>>4) + j; keys are the A operand.  RAW (no casts):
// the unscaled dot products, the caller folds scale2 into its exp2 argument.
template <typename T, int RM, bool MASK, bool RAW = false>
__device__ __forceinline__ void subtile_logits(const ScoreArgs& a, const typename Elem<T>::vec8 (&kr)[4],
                                               const T* s_q, int nt, int t0, int lane, int limit, float (&x)[4]) {
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  const T* qrow = s_q + (16 * nt + (lane & 15)) * kQPitch + 8 * (lane >> 4);
#pragma unroll
  for (int s = 0; s < 4; ++s) acc = mma_16x16x32(kr[s], load8<T>(qrow + 32 * s), acc);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int t = t0 + 4 * (lane >> 4) + j;
    x[j] = (!MASK || t <= limit) ? (RAW ? acc[j] : scaled_logit<RM>(a, acc[j])) : -INFINITY;
  }
}

__device__ __forceinline__ void merge_ml(float& m, float& l, float m2, float l2) {
  const float mn = fmaxf(m, m2);
  if (mn == -INFINITY) return;
  l = l * fast_exp2(m - mn) + l2 * fast_exp2(m2 - mn);
  m = mn;
}

// Key registers of one wave's kSubTiles sub-tiles.
template <typename T>
struct KRegs {
  typename Elem<T>::vec8 v[kSubTiles][4];
};

template <typename T, bool STORE>
__device__ __forceinline__ void load_k_chunk(const ScoreArgs& a, const T* kj, int tw, int lane, KRegs<T>& k) {
#pragma unroll
  for (int u = 0; u < kSubTiles; ++u) load_k_subtile<T, STORE>(a, kj, tw + 16 * u, lane, k.v[u]);
}

// Statistics of one 256-token chunk: the (max, sum) of every row over this
// wave's 64 tokens (lane l holds row 16nt + l%16, tokens 4*(l/16) + j of
// each sub-tile), merged into the wave's LDS entry of the row.  One 16-row
// tile at a time, in a rolled loop: unrolled over the 16 tiles and the mask
// variants the kernel outgrows the instruction cache.
template <typename T, int RM, bool LOGITS, bool MASK>
__device__ __forceinline__ void stats_chunk(const ScoreArgs& a, const KRegs<T>& k, const T* s_q, float* my, int job,
                                            int tw, int lane, float* __restrict__ logits) {
  const bool vec_logits = (a.span & 3) == 0;
  for (int nt = 0; nt < a.NT; ++nt) {
    const int limit = row_limit(a, 16 * nt + (lane & 15));
    // All sub-tiles' logits first (independent MFMA chains, no branch
    // between them); then the row's maximum over its four lanes, and one sum
    // of exp2 against it (no rescaling).  Without casts the maximum is taken
    // on the unscaled products and the scale folds into each exp2's fma.
    constexpr bool RAW = RM == 0 && !LOGITS;
    float x[kSubTiles][4];
#pragma unroll
    for (int u = 0; u < kSubTiles; ++u) {
      subtile_logits<T, RM, MASK, RAW>(a, k.v[u], s_q, nt, tw + 16 * u, lane, limit, x[u]);
      if constexpr (LOGITS) {
        // Row r, tokens t..t+3 (16 bytes) of the job's [R][span] logits.
        const int r = 16 * nt + (lane & 15), t = tw + 16 * u + 4 * (lane >> 4);
        float* o = logits + ((int64_t)job * a.R + r) * a.span + t;
        if (r < a.R) {
          if (vec_logits && t + 4 <= a.span) {
            *reinterpret_cast<f32x4*>(o) = f32x4{x[u][0], x[u][1], x[u][2], x[u][3]};
          } else {
#pragma unroll
            for (int j = 0; j < 4; ++j)
              if (t + j < a.span) o[j] = x[u][j];
          }
        }
      }
    }
    // -FLT_MAX (not -inf) as the empty maximum: exp2(-inf - m) = 0 for a
    // row with no visible value, never NaN.
    // IEEE maximum (v_maximum3 on gfx950): the raw accumulators need no
    // canonicalising, three operands per instruction.
    float m = -FLT_MAX;
#pragma unroll
    for (int u = 0; u < kSubTiles; ++u)
      m = __builtin_elementwise_maximum(
          m, __builtin_elementwise_maximum(__builtin_elementwise_maximum(x[u][0], x[u][1]),
                                           __builtin_elementwise_maximum(x[u][2], x[u][3])));
    m = rows4_max(m);
    float l = 0.f;
    if constexpr (RAW) {
      m = fmaxf(m * a.scale2, -FLT_MAX);  // base-2 scaled maximum, finite
#pragma unroll
      for (int u = 0; u < kSubTiles; ++u)
        l += (fast_exp2(fmaf(x[u][0], a.scale2, -m)) + fast_exp2(fmaf(x[u][1], a.scale2, -m))) +
             (fast_exp2(fmaf(x[u][2], a.scale2, -m)) + fast_exp2(fmaf(x[u][3], a.scale2, -m)));
    } else {
#pragma unroll
      for (int u = 0; u < kSubTiles; ++u)
        l += (fast_exp2(x[u][0] - m) + fast_exp2(x[u][1] - m)) + (fast_exp2(x[u][2] - m) + fast_exp2(x[u][3] - m));
    }
    l = rows4_sum(l);
    if (lane < 16) {  // each row entry belongs to one lane of this wave
      float* e = my + 2 * (16 * nt + lane);
      float em = e[0], el = e[1];
      merge_ml(em, el, m, l);
      e[0] = em;
      e[1] = el;
    }
  }
}

// Each workgroup takes a.cpw consecutive 256-token chunks of one job; its
// queries are staged in LDS once.  One (max, sum) partial per workgroup and
// row.  (A second register set for the next chunk's keys halves occupancy
// and was slower: the passes are bound by latency within a chunk.)
template <typename T, bool STORE, int RM, bool LOGITS>
__global__ __launch_bounds__(kScoreWaves * 64) void score_stats_kernel(ScoreArgs a, float* __restrict__ part,
                                                                      float* __restrict__ logits) {
  extern __shared__ __align__(16) unsigned char smem[];
  T* s_q = reinterpret_cast<T*>(smem);
  float* s_st = reinterpret_cast<float*>(smem + (size_t)a.NT * 16 * kQPitch * sizeof(T));  // [waves][rows][2]
  const int job = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rows = a.NT * 16;
  const int nchunks = (a.L + kScoreChunk - 1) / kScoreChunk;
  const int c0 = blockIdx.x * a.cpw, c1 = min(c0 + a.cpw, nchunks);
  // Each wave owns kSubTiles consecutive 16-token sub-tiles of a chunk.
  const int woff = wave * 16 * kSubTiles;
  const T* const kj = job_keys<T, STORE>(a, job);
  KRegs<T> ka;
  load_k_chunk<T, STORE>(a, kj, c0 * kScoreChunk + woff, lane, ka);
  stage_queries<T>(a, job, s_q);
  float* my = s_st + (size_t)wave * rows * 2;
  for (int r = lane; r < rows; r += 64) {
    my[2 * r] = -INFINITY;
    my[2 * r + 1] = 0.f;
  }
  __syncthreads();
  // Masks matter only where a chunk reaches past the lowest row limit (the
  // causal window or the end of the keys); elsewhere every logit is visible
  // and the per-value test is skipped.
  const int min_limit = (a.flags & HC_SCORE_CAUSAL_WINDOW) ? a.L - a.W : a.L - 1;
  auto chunk_stats = [&](const KRegs<T>& k, int c) {
    const int tw = c * kScoreChunk + woff;
    if (c * kScoreChunk + kScoreChunk - 1 > min_limit)
      stats_chunk<T, RM, LOGITS, true>(a, k, s_q, my, job, tw, lane, logits);
    else
      stats_chunk<T, RM, LOGITS, false>(a, k, s_q, my, job, tw, lane, logits);
  };
  for (int c = c0; c < c1; ++c) {
    if (c > c0) load_k_chunk<T, STORE>(a, kj, c * kScoreChunk + woff, lane, ka);
    chunk_stats(ka, c);
  }
  __syncthreads();
  const int nparts = gridDim.x;
  for (int r = threadIdx.x; r < a.R; r += kScoreWaves * 64) {
    float mm = -INFINITY, ll = 0.f;
#pragma unroll
    for (int w = 0; w < kScoreWaves; ++w) merge_ml(mm, ll, s_st[(w * rows + r) * 2], s_st[(w * rows + r) * 2 + 1]);
    float* o = part + (((int64_t)job * nparts + blockIdx.x) * a.R + r) * 2;
    o[0] = mm;
    o[1] = ll;
  }
}

// Statistics pass for few query rows (R <= 16) over natural-layout keys, on
// the vector ALUs.  With at most 16 rows the contraction is 2*R*128 flops
// per 256-byte key row, so the pass is bound by streaming the keys -- and
// the MFMA operand layout of score_stats_kernel makes every wave load touch
// 16 rows of 64 bytes each.  Here the 16 lanes of group s hold channels
// 8c..8c+7 (c = lane % 16) of token 4*step + s, so a wave load reads four
// whole 256-byte token rows; the groups' partial dot products of all NR
// rows are summed by one DPP reduce-scatter (row16_sum_scatter), after which
// lane c < R of a group holds row c's logit of its token.  Logits are stored as score_stats_kernel stores them (base-2
// scaled and masked, [job][R][span]) and every workgroup writes one
// (max, sum) partial per row, so the merge and finish passes are shared.
// NR: rows held per lane (R rounded up to 4, 8 or 16).
constexpr int kRowsSteps = 8;  // 4-token steps per wave and iteration

// Two products per instruction for 16-bit inputs: v_dot2_f32_bf16 /
// v_dot2_f32_f16 multiply packed pairs exactly and accumulate in float32,
// so the queries stay in the input type (half the registers) and the keys
// need no conversion.  Float32 inputs take FMAs.
template <typename T>
struct Dot2 {
  typedef float pair;
};
template <>
struct Dot2<__bf16> {
  typedef __attribute__((ext_vector_type(2))) __bf16 pair;
  static __device__ __forceinline__ float dot(pair a, pair b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(a, b, c, false);
  }
};
template <>
struct Dot2<_Float16> {
  typedef __attribute__((ext_vector_type(2))) _Float16 pair;
  static __device__ __forceinline__ float dot(pair a, pair b, float c) { return __builtin_amdgcn_fdot2(a, b, c, false); }
};
// Pair j (elements 2j, 2j + 1) of eight 16-bit values.
template <typename T>
__device__ __forceinline__ typename Dot2<T>::pair pair_at(const typename Elem<T>::vec8& v, int j) {
  typename Dot2<T>::pair p;
  p.x = v[2 * j];
  p.y = v[2 * j + 1];
  return p;
}

template <typename T, int NR, int RM>
__global__ __launch_bounds__(kScoreWaves * 64) void score_rows_valu_kernel(ScoreArgs a, float* __restrict__ part,
                                                                          float* __restrict__ logits) {
  typedef typename Elem<T>::vec8 vec8;
  __shared__ float s_st[kScoreWaves][16][2];
  const int job = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane >> 4, c = lane & 15;
  // This lane's 8 channels of every query row (zero past R): four packed
  // pairs of the input type for 16-bit inputs, eight floats for float32.
  constexpr bool kPairs = sizeof(T) == 2;
  typedef typename Dot2<T>::pair QP;
  constexpr int QW = kPairs ? 4 : 8;
  typedef std::conditional_t<kPairs, QP, float> QE;
  QE qr[NR][QW];
  {
    const T* q = reinterpret_cast<const T*>(a.q) + a.q_off[job] + 8 * c;
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const vec8 v = r < a.R ? load8<T>(q + (r / a.W) * a.q_head_stride + (r % a.W) * a.q_row_stride) : zero8<T>();
      if constexpr (kPairs) {
#pragma unroll
        for (int j = 0; j < 4; ++j) qr[r][j] = pair_at<T>(v, j);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) qr[r][e] = vec8_at<T>(v, e);
      }
    }
  }
  const bool owner = c < a.R;  // lane c post-processes row c of its group's token
  const int limit = owner ? row_limit(a, c) : -1;
  const int nchunks = (a.L + kScoreChunk - 1) / kScoreChunk;
  const int c0 = blockIdx.x * a.cpw, c1 = min(c0 + a.cpw, nchunks);
  const int t_end = min(c1 * kScoreChunk, a.L);
  const T* kb = reinterpret_cast<const T*>(a.k) + a.k_off[job] + 8 * c;
  float* lrow = logits + ((int64_t)job * a.R + (owner ? c : 0)) * a.span;
  float m = -FLT_MAX, l = 0.f;
  constexpr int kIter = kScoreWaves * kRowsSteps * 4;  // tokens per workgroup iteration
  // Keys of one iteration, streamed past L2 (this pass reads them once):
  // with ordinary loads the pass took 69-71 us per 128K Llama-3-8B layer
  // (eight heads), nontemporal 50 us, while the gather that follows loses
  // ~4 us of cache hits.  Token addresses are clamped into [0, L) (a token
  // past the keys is read from the last one and its logit masked below), so
  // the loads take no branches.  A second key buffer, the next iteration's
  // loads in flight during this one, measured the same (50.4 against 50.7
  // us) at 132 instead of 76 registers.
  auto load_keys = [&](vec8 (&kr)[kRowsSteps], int t0) {
#pragma unroll
    for (int st = 0; st < kRowsSteps; ++st)
      kr[st] = load8_stream<T>(kb + (int64_t)min(t0 + 4 * st + sub, a.L - 1) * a.k_tok_stride);
  };
  auto consume = [&](const vec8 (&kr)[kRowsSteps], int t0) {
    float x[kRowsSteps];
#pragma unroll
    for (int st = 0; st < kRowsSteps; ++st) {
      float acc[NR];
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        float d = 0.f;
        if constexpr (kPairs) {
#pragma unroll
          for (int j = 0; j < 4; ++j) d = Dot2<T>::dot(qr[r][j], pair_at<T>(kr[st], j), d);
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) d = fmaf(qr[r][e], vec8_at<T>(kr[st], e), d);
        }
        acc[r] = d;
      }
      const float mine = row16_sum_scatter<NR>(acc, lane);  // row c % NR
      const int t = t0 + 4 * st + sub;
      x[st] = t <= limit ? scaled_logit<RM>(a, mine) : -INFINITY;
    }
    // The logits are stored after all the iteration's keys are consumed:
    // stores between the key waits count against the same in-order counter,
    // so each wait also waited for the next key (prefill compression 0.192-
    // 0.193 -> 0.191 ms per 128K layer).
#pragma unroll
    for (int st = 0; st < kRowsSteps; ++st) {
      const int t = t0 + 4 * st + sub;
      if (owner && t < a.span) lrow[t] = x[st];
    }
    float mx = x[0];
#pragma unroll
    for (int st = 1; st < kRowsSteps; ++st) mx = __builtin_elementwise_maximum(mx, x[st]);
    const float mn = __builtin_elementwise_maximum(m, mx);
    float add = 0.f;
#pragma unroll
    for (int st = 0; st < kRowsSteps; ++st) add += fast_exp2(x[st] - mn);
    l = fmaf(l, fast_exp2(m - mn), add);
    m = mn;
  };
  for (int t0 = c0 * kScoreChunk + wave * kRowsSteps * 4; t0 < t_end; t0 += kIter) {
    vec8 kr[kRowsSteps];
    load_keys(kr, t0);
    consume(kr, t0);
  }
  // Rows are held by lanes c, c+16, c+32, c+48 of each wave; then the waves.
  const float M = rows4_max(m);
  const float Ls = rows4_sum(l * fast_exp2(m - M));
  if (sub == 0) {
    s_st[wave][c][0] = M;
    s_st[wave][c][1] = Ls;
  }
  __syncthreads();
  if (threadIdx.x < a.R) {
    const int r = threadIdx.x;
    float mm = -INFINITY, ll = 0.f;
#pragma unroll
    for (int w = 0; w < kScoreWaves; ++w) merge_ml(mm, ll, s_st[w][r][0], s_st[w][r][1]);
    float* o = part + (((int64_t)job * gridDim.x + blockIdx.x) * a.R + r) * 2;
    o[0] = mm;
    o[1] = ll;
  }
}

// One wave per (job, row): lanes stride over the chunks, then a xor tree.
__global__ __launch_bounds__(256) void score_stats_merge_kernel(const float* __restrict__ part, int nchunks, int R,
                                                                int njobs, float* __restrict__ stats,
                                                                uint32_t* __restrict__ hist, int64_t hist_words) {
  // Zero the optional score histogram the finish pass accumulates into.
  for (int64_t w = (int64_t)blockIdx.x * 256 + threadIdx.x; w < hist_words; w += (int64_t)gridDim.x * 256) hist[w] = 0u;
  const int i = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (i >= njobs * R) return;
  const int job = i / R, r = i % R;
  float m = -INFINITY, l = 0.f;
  for (int c = lane; c < nchunks; c += 64) {
    const float* p = part + (((int64_t)job * nchunks + c) * R + r) * 2;
    merge_ml(m, l, p[0], p[1]);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float m2 = __shfl_xor(m, off, 64), l2 = __shfl_xor(l, off, 64);
    merge_ml(m, l, m2, l2);
  }
  if (lane == 0) {
    stats[2 * i] = m;
    stats[2 * i + 1] = l;
  }
}

// Logits (base 2) with the queries as the A operand: lane holds rows
// 16nt + 4*(lane>>4) + j (visible up to limit[j]) of token t0 + lane%16, so
// sums over a query head's window rows are in-lane adds plus at most two
// cross-lane steps.  RAW as for subtile_logits.
template <typename T, int RM, bool MASK, bool RAW = false>
__device__ __forceinline__ void subtile_logits_rows(const ScoreArgs& a, const typename Elem<T>::vec8 (&kr)[4],
                                                    const T* s_q, int nt, int t0, int lane, const int (&limit)[4],
                                                    float (&x)[4]) {
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  const T* qrow = s_q + (16 * nt + (lane & 15)) * kQPitch + 8 * (lane >> 4);
#pragma unroll
  for (int s = 0; s < 4; ++s) acc = mma_16x16x32(load8<T>(qrow + 32 * s), kr[s], acc);
  const int t = t0 + (lane & 15);
#pragma unroll
  for (int j = 0; j < 4; ++j)
    x[j] = (!MASK || t <= limit[j]) ? (RAW ? acc[j] : scaled_logit<RM>(a, acc[j])) : -INFINITY;
}

// Window modes of the probability pass, fixed per kernel instance so each
// instance holds one output path (with all of them, and the 16 row tiles
// unrolled, the kernel outgrew the instruction cache).
enum WinMode { kWinNone = 0, kWin16 = 1, kWin8 = 2, kWin4 = 3, kWin2 = 4, kWin1 = 5 };

// Probabilities of every (row, token) of the workgroup's chunk, summed over
// the window rows of each query head per WM (kWinNone: no sum).
// MOM (CAKE scoring, kWin16): besides the window sum A, write the window sum
// of squares A2 unrounded and one partial of sum p*log(p + 1e-10) over
// t < span per (job, chunk) into ent.
// Where the probability pass finds row r = g*W + w's statistics (M, L) of
// job j: at p + base + 2r with base = off ? off[j] : 2*R*j, or, with a
// nonzero head_stride, at p + base + g*head_stride + 2w (statistics laid out
// per query head, such as the ones prefill attention reports).
struct StatsView {
  const float* p;
  const int64_t* off;
  int64_t head_stride;
  __device__ __forceinline__ const float* row(const ScoreArgs& a, int job, int r) const {
    const int64_t base = off ? off[job] : (int64_t)job * a.R * 2;
    return p + base + (head_stride ? (r / a.W) * head_stride + 2 * (r % a.W) : 2 * (int64_t)r);
  }
};

template <typename T, bool STORE, int RM, int WM, bool MOM>
__global__ __launch_bounds__(kScoreWaves * 64) void score_probs_kernel(ScoreArgs a, StatsView stats,
                                                                      float* __restrict__ A, float* __restrict__ A2,
                                                                      float* __restrict__ ent) {
  extern __shared__ __align__(16) unsigned char smem[];
  T* s_q = reinterpret_cast<T*>(smem);
  const int rows = a.NT * 16;
  float* s_m = reinterpret_cast<float*>(smem + (size_t)rows * kQPitch * sizeof(T));  // [rows] row max
  float* s_iz = s_m + rows;                                                           // [rows] 1 / row sum
  const int job = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rg = lane >> 4;
  const int nchunks = (a.span + kScoreChunk - 1) / kScoreChunk;
  const int c0 = blockIdx.x * a.cpw, c1 = min(c0 + a.cpw, nchunks);
  const int woff = wave * 16 * kSubTiles;
  const T* const kj = job_keys<T, STORE>(a, job);
  KRegs<T> ka;
  load_k_chunk<T, STORE>(a, kj, c0 * kScoreChunk + woff, lane, ka);
  stage_queries<T>(a, job, s_q);
  for (int r = threadIdx.x; r < rows; r += kScoreWaves * 64) {
    // Padding rows get probability 0 even where logits are not masked.
    const float* st = r < a.R ? stats.row(a, job, r) : nullptr;
    if constexpr (RM == 0) {
      // Without casts p = exp2(x - (m + log2 l)): one subtract, no divide.
      s_m[r] = st ? st[0] + __log2f(st[1]) : INFINITY;
    } else {
      s_m[r] = st ? st[0] : 0.f;
      s_iz[r] = st ? 1.f / st[1] : 0.f;
    }
  }
  const int wout = WM == kWinNone ? a.W : 1;
  __syncthreads();
  float gsum[kSubTiles], gsq[kSubTiles];  // running window sum (and sum of squares) per sub-tile (kWin16)
#pragma unroll
  for (int u = 0; u < kSubTiles; ++u) gsum[u] = gsq[u] = 0.f;
  float ent_acc = 0.f;
  const int min_limit = (a.flags & HC_SCORE_CAUSAL_WINDOW) ? a.L - a.W : a.L - 1;
  auto body = [&](auto mask_tag, const KRegs<T>& k, int tw) {
    constexpr bool MASK = decltype(mask_tag)::value;
    for (int nt = 0; nt < a.NT; ++nt) {
      {
        const int r0 = 16 * nt + 4 * rg;
        float M[4], IZ[4];
        int limit[4];
        int64_t orow[4];  // output row of each j without the window sum: A[job][w][g]
  #pragma unroll
        for (int j = 0; j < 4; ++j) {
          M[j] = s_m[r0 + j];
          IZ[j] = s_iz[r0 + j];
          limit[j] = row_limit(a, r0 + j);
          if constexpr (WM == kWinNone) orow[j] = (((int64_t)job * wout + (r0 + j) % a.W) * a.G + (r0 + j) / a.W) * a.span;
        }
        // All sub-tiles' logits first (independent MFMA chains, no branch
        // between them), then the probabilities and their sums.
        float x[kSubTiles][4];
  #pragma unroll
        for (int u = 0; u < kSubTiles; ++u)
          subtile_logits_rows<T, RM, MASK, RM == 0>(a, k.v[u], s_q, nt, tw + 16 * u, lane, limit, x[u]);
  #pragma unroll
        for (int u = 0; u < kSubTiles; ++u) {
          const int t = tw + 16 * u + (lane & 15);
          float p[4];
  #pragma unroll
          for (int j = 0; j < 4; ++j) {
            if constexpr (RM == 0)  // x: unscaled products; M holds m + log2 l; masked logits give 0
              p[j] = fast_exp2(fmaf(x[u][j], a.scale2, -M[j]));
            else
              p[j] = x[u][j] == -INFINITY ? 0.f : round_fixed<RM>(fast_exp2(x[u][j] - M[j]) * IZ[j]);
          }
          if constexpr (MOM) {
            // Padding rows have p = 0 and add 0 * log(1e-10) = 0.
            float e = 0.f;
  #pragma unroll
            for (int j = 0; j < 4; ++j) e += p[j] * __logf(p[j] + 1e-10f);
            ent_acc += t < a.span ? e : 0.f;
          }
          if constexpr (WM == kWinNone) {
            // Row r = g*W + w -> A[job][w][g][t].
  #pragma unroll
            for (int j = 0; j < 4; ++j)
              if (r0 + j < a.R && t < a.span) A[orow[j] + t] = p[j];
          } else if constexpr (WM == kWin16) {
            // The 16 rows of this tile all belong to one query head; each
            // lane sums its 4 rows over the head's tiles, and the 4 lane
            // groups are combined once per head (below).
            gsum[u] += (p[0] + p[1]) + (p[2] + p[3]);
            if constexpr (MOM) gsq[u] += (p[0] * p[0] + p[1] * p[1]) + (p[2] * p[2] + p[3] * p[3]);
          } else if constexpr (WM == kWin8) {
            float v = (p[0] + p[1]) + (p[2] + p[3]);
            v = rows2_sum(v);
            const int g = r0 / 8;
            if ((rg & 1) == 0 && r0 < a.R && t < a.span) A[((int64_t)job * a.G + g) * a.span + t] = round_fixed<RM>(v);
          } else if constexpr (WM == kWin4) {
            // A head's rows are the four j of this lane.
            const float v = (p[0] + p[1]) + (p[2] + p[3]);
            if (r0 < a.R && t < a.span) A[((int64_t)job * a.G + r0 / 4) * a.span + t] = round_fixed<RM>(v);
          } else if constexpr (WM == kWin2) {
            const float v0 = p[0] + p[1], v1 = p[2] + p[3];
            if (r0 < a.R && t < a.span) A[((int64_t)job * a.G + r0 / 2) * a.span + t] = round_fixed<RM>(v0);
            if (r0 + 2 < a.R && t < a.span) A[((int64_t)job * a.G + r0 / 2 + 1) * a.span + t] = round_fixed<RM>(v1);
          } else {
            // W == 1: every row is its own query head.
  #pragma unroll
            for (int j = 0; j < 4; ++j)
              if (r0 + j < a.R && t < a.span) A[((int64_t)job * a.G + r0 + j) * a.span + t] = round_fixed<RM>(p[j]);
          }
        }
        if constexpr (WM == kWin16) {
          if (((16 * (nt + 1)) % a.W) == 0) {  // the last tile of a query head
            const int g = (16 * nt) / a.W;
  #pragma unroll
            for (int u = 0; u < kSubTiles; ++u) {
              const int t = tw + 16 * u + (lane & 15);
              float v = gsum[u];
              v = rows4_sum(v);
              const int64_t o = ((int64_t)job * a.G + g) * a.span + t;
              if constexpr (MOM) {
                float v2 = gsq[u];
                v2 = rows4_sum(v2);
                if (rg == 0 && g < a.G && t < a.span) {
                  A[o] = v;
                  A2[o] = v2;
                }
                gsq[u] = 0.f;
              } else {
                if (rg == 0 && g < a.G && t < a.span) A[o] = round_fixed<RM>(v);
              }
              gsum[u] = 0.f;
            }
          }
        }
      }
    }
  };
  // The workgroup's chunks in order (queries and row statistics staged once).
  auto chunk_probs = [&](const KRegs<T>& k, int c) {
    const int tw = c * kScoreChunk + woff;
    if (c * kScoreChunk + kScoreChunk - 1 > min_limit)
      body(std::true_type{}, k, tw);
    else
      body(std::false_type{}, k, tw);
  };
  for (int c = c0; c < c1; ++c) {
    if (c > c0) load_k_chunk<T, STORE>(a, kj, c * kScoreChunk + woff, lane, ka);
    chunk_probs(ka, c);
  }
  if constexpr (MOM) {
    __shared__ float s_ent[kScoreWaves];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) ent_acc += __shfl_xor(ent_acc, off, 64);
    if (lane == 0) s_ent[wave] = ent_acc;
    __syncthreads();
    if (threadIdx.x == 0) ent[(int64_t)job * gridDim.x + blockIdx.x] = (s_ent[0] + s_ent[1]) + (s_ent[2] + s_ent[3]);
  }
}

// ---------------------------------------------------------------------------
// Probability pass with the pooling fused (summed windows of whole 16-row
// tiles, W a multiple of 16, pooling kernels up to 2 * kPpMaxHalf + 1): the
// window sums of the workgroup's chunk stay in LDS (one strip row per query
// head) and the chunk is pooled and maxed over the group there, so neither
// the window sums nor a pooling launch go through HBM.  A workgroup runs the
// chunks [c0, c1) in order: the pooled output trails the chunk by the pool
// half-width P (its last P positions wait for the next chunk's first ones),
// and the 16 positions before the run and after it are recomputed as one
// extra sub-tile each (by waves 0 and kScoreWaves - 1).  Same arithmetic, in
// the same order, as score_probs_kernel followed by score_pool_kernel.
// ---------------------------------------------------------------------------
constexpr int kPpMargin = 16;                       // positions of a margin sub-tile
constexpr int kPpPitch = kScoreChunk + kPpMargin;   // strip row: the chunk, then the run's right margin
constexpr int kPpMaxHalf = 4;

// Window sums of query head g over tokens tw + 16u + (lane & 15), u < NU,
// written (by the lanes of row group 0) to dst[g * pitch + 16u + (lane & 15)],
// the pad value for tokens outside [0, span).
template <typename T, int RM, bool MASK, int NU>
__device__ __forceinline__ void window_sums(const ScoreArgs& a, const typename Elem<T>::vec8 (&k)[NU][4],
                                            const T* s_q, const float* s_m, const float* s_iz, int tw, int lane,
                                            float* dst, int pitch, float pad) {
  const int rg = lane >> 4;
  float gsum[NU];
#pragma unroll
  for (int u = 0; u < NU; ++u) gsum[u] = 0.f;
  for (int nt = 0; nt < a.NT; ++nt) {
    const int r0 = 16 * nt + 4 * rg;
    float M[4], IZ[4];
    int limit[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      M[j] = s_m[r0 + j];
      IZ[j] = RM != 0 ? s_iz[r0 + j] : 0.f;
      limit[j] = row_limit(a, r0 + j);
    }
    float x[NU][4];
#pragma unroll
    for (int u = 0; u < NU; ++u) subtile_logits_rows<T, RM, MASK, RM == 0>(a, k[u], s_q, nt, tw + 16 * u, lane, limit, x[u]);
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      float p[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if constexpr (RM == 0)
          p[j] = fast_exp2(fmaf(x[u][j], a.scale2, -M[j]));
        else
          p[j] = x[u][j] == -INFINITY ? 0.f : round_fixed<RM>(fast_exp2(x[u][j] - M[j]) * IZ[j]);
      }
      gsum[u] += (p[0] + p[1]) + (p[2] + p[3]);
    }
    if (((16 * (nt + 1)) % a.W) == 0) {  // the last tile of a query head
      const int g = (16 * nt) / a.W;
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        const int t = tw + 16 * u + (lane & 15);
        const float v = rows4_sum(gsum[u]);
        if (rg == 0) dst[g * pitch + 16 * u + (lane & 15)] = t >= 0 && t < a.span ? round_fixed<RM>(v) : pad;
        gsum[u] = 0.f;
      }
    }
  }
}

// Keys of NU sub-tiles from tw on, natural layout, each lane's row clamped
// to the job's last key (L >= 1): no branch around the loads, so the waits
// on one half of a double buffer leave the other half's loads in flight.
// Clamped rows only feed masked logits: a chunk holding a token at or past
// L - 1 takes the masked path, where every such token is past its row's
// limit.
// `base` is the lane's column in the job's key rows (job_keys).
template <typename T, int NU>
__device__ __forceinline__ void load_k_clamped(const ScoreArgs& a, const T* base, int tw, int lane,
                                               typename Elem<T>::vec8 (&k)[NU][4]) {
#pragma unroll
  for (int u = 0; u < NU; ++u) {
    const int t = min(tw + 16 * u + (lane & 15), a.L - 1);
    const T* p = base + (int64_t)t * a.k_tok_stride;
#pragma unroll
    for (int s = 0; s < 4; ++s) k[u][s] = load8<T>(p + 32 * s);
  }
}

// Natural-layout keys only (STORE is false in every instance).  Each wave's
// 64 tokens of a chunk are two halves of two sub-tiles in two register
// sets: a half's keys for the next chunk are requested as soon as the half
// has been consumed, so every load has the other half's work to land in.
// In the run's last chunk the "next" keys are the same keys again, so the
// loads stay unconditional.  Against one buffer reloaded after the whole
// chunk (8 heads x 128K, W = 32, max pool 7): 70.0 against 70.1 us per
// launch, so the key loads were not what bounds the pass; VALU issue and
// latency are.
template <typename T, bool STORE, int RM, int POOL, int P>
__global__ __launch_bounds__(kScoreWaves * 64, sizeof(T) == 4 ? 1 : RM == 0 ? 4 : 3) void score_probs_pool_kernel(ScoreArgs a, StatsView stats,
                                                                           float* __restrict__ S) {
  static_assert(!STORE, "the fused pass reads natural-layout keys");
  constexpr int kHalf = kSubTiles / 2;
  extern __shared__ __align__(16) unsigned char smem[];
  constexpr float kPad = POOL == 0 ? 0.f : -INFINITY;
  T* s_q = reinterpret_cast<T*>(smem);
  const int rows = a.NT * 16;
  float* s_m = reinterpret_cast<float*>(smem + (size_t)rows * kQPitch * sizeof(T));  // [rows]
  float* s_iz = s_m + rows;                                                           // [rows], casts only
  float* strip = s_iz + (RM != 0 ? rows : 0);  // [G][kPpPitch]
  float* mrg = strip + a.G * kPpPitch;         // [2][G][kPpMargin]: the 16 positions before the chunk
  const int job = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nchunks = (a.span + kScoreChunk - 1) / kScoreChunk;
  const int c0 = blockIdx.x * a.cpw, c1 = min(c0 + a.cpw, nchunks);
  if (c0 >= c1 || a.L <= 0) return;  // uniform per workgroup
  const int woff = wave * 16 * kSubTiles;
  const T* const kj = job_keys<T, STORE>(a, job);
  const T* const kbase = kj + 8 * (lane >> 4);
  typename Elem<T>::vec8 kh0[kHalf][4], kh1[kHalf][4];
  load_k_clamped<T, kHalf>(a, kbase, c0 * kScoreChunk + woff, lane, kh0);
  load_k_clamped<T, kHalf>(a, kbase, c0 * kScoreChunk + woff + 16 * kHalf, lane, kh1);
  stage_queries<T>(a, job, s_q);
  for (int r = threadIdx.x; r < rows; r += kScoreWaves * 64) {
    const float* st = stats.row(a, job, r);  // rows = R here: W is a multiple of 16
    if constexpr (RM == 0) {
      s_m[r] = st[0] + __log2f(st[1]);
    } else {
      s_m[r] = st[0];
      s_iz[r] = 1.f / st[1];
    }
  }
  __syncthreads();
  if (wave == 0) {
    // The run's left margin: positions c0 * kScoreChunk - 16 .. - 1.
    const int cb = c0 * kScoreChunk;
    if (cb > 0) {
      typename Elem<T>::vec8 km[1][4];
      load_k_subtile<T, STORE>(a, kj, cb - kPpMargin, lane, km[0]);
      window_sums<T, RM, true, 1>(a, km, s_q, s_m, s_iz, cb - kPpMargin, lane, mrg, kPpMargin, kPad);
    } else {
      for (int i = lane; i < a.G * kPpMargin; i += 64) mrg[i] = kPad;
    }
  }
  // Drain every load of the set-up (the first chunk's keys included).  The
  // staging loops and the margin leave a count of loads in flight that the
  // compiler cannot bound; with that state at the loop head it made each
  // chunk's first key wait a wait for every load, the prefetch included.
  __builtin_amdgcn_s_waitcnt(0);
  const int min_limit = (a.flags & HC_SCORE_CAUSAL_WINDOW) ? a.L - a.W : a.L - 1;
  const bool acc_out = (a.flags & HC_SCORE_ACCUMULATE) != 0;
  float* const out = S + (int64_t)job * a.span;
  for (int c = c0; c < c1; ++c) {
    const int cb = c * kScoreChunk;
    const int nb = (c + 1 < c1 ? cb + kScoreChunk : cb) + woff;  // next chunk's keys (or these again)
    float* mcur = mrg + ((c - c0) & 1) * a.G * kPpMargin;
    float* mnext = mrg + ((c - c0 + 1) & 1) * a.G * kPpMargin;
    const bool masked = cb + kScoreChunk - 1 > min_limit;
    if (masked)
      window_sums<T, RM, true, kHalf>(a, kh0, s_q, s_m, s_iz, cb + woff, lane, strip + woff, kPpPitch, kPad);
    else
      window_sums<T, RM, false, kHalf>(a, kh0, s_q, s_m, s_iz, cb + woff, lane, strip + woff, kPpPitch, kPad);
    load_k_clamped<T, kHalf>(a, kbase, nb, lane, kh0);
    if (masked)
      window_sums<T, RM, true, kHalf>(a, kh1, s_q, s_m, s_iz, cb + woff + 16 * kHalf, lane,
                                      strip + woff + 16 * kHalf, kPpPitch, kPad);
    else
      window_sums<T, RM, false, kHalf>(a, kh1, s_q, s_m, s_iz, cb + woff + 16 * kHalf, lane,
                                       strip + woff + 16 * kHalf, kPpPitch, kPad);
    load_k_clamped<T, kHalf>(a, kbase, nb + 16 * kHalf, lane, kh1);
    if (c == c1 - 1 && wave == kScoreWaves - 1) {
      // The run's right margin: positions cb + 256 .. cb + 271.
      const int te = cb + kScoreChunk;
      if (te < a.span) {
        typename Elem<T>::vec8 km[1][4];
        load_k_subtile<T, STORE>(a, kj, te, lane, km[0]);
        window_sums<T, RM, true, 1>(a, km, s_q, s_m, s_iz, te, lane, strip + kScoreChunk, kPpPitch, kPad);
      } else {
        for (int i = lane; i < a.G * kPpMargin; i += 64) strip[(i / kPpMargin) * kPpPitch + kScoreChunk + i % kPpMargin] = kPad;
      }
      __builtin_amdgcn_s_waitcnt(0);  // the run's last chunk: only the unused reloads are in flight
    }
    __syncthreads();
    // Pool positions [lo, hi): the previous chunk's last P, then this chunk's
    // up to its last P (all of them in the run's last chunk), at most two
    // per thread.  Straight-line code, not a loop: stores count against the
    // same wait counter as the key loads in flight, and after a loop of
    // stores the compiler can no longer tell how many are pending, so the
    // next chunk's first key wait became a wait for every load.
    static_assert(kScoreChunk + kPpMaxHalf <= 2 * kScoreWaves * 64, "two pooled positions per thread");
    const int lo = c == c0 ? cb : cb - P;
    const int hi = min(c == c1 - 1 ? cb + kScoreChunk : cb + kScoreChunk - P, a.span);
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int x = lo + (int)threadIdx.x + q * kScoreWaves * 64;
      if (x >= hi) continue;
      const int i = x - cb;
      float best = -INFINITY;
      for (int g = 0; g < a.G; ++g) {
        const float* srow = strip + g * kPpPitch;
        const float* mrow = mcur + g * kPpMargin + kPpMargin;
        float acc = kPad;
#pragma unroll
        for (int d = -P; d <= P; ++d) {
          const int li = i + d;
          const float v = li < 0 ? mrow[li] : srow[li];
          acc = POOL == 0 ? acc + v : fmaxf(acc, v);
        }
        if constexpr (POOL == 0) acc = acc / (float)(2 * P + 1);
        best = fmaxf(best, round_fixed<RM>(acc));
      }
      out[x] = acc_out ? out[x] + best : best;
    }
    // The chunk's last 16 positions are the next chunk's left neighbours.
    if (c + 1 < c1)
      for (int i = threadIdx.x; i < a.G * kPpMargin; i += kScoreWaves * 64)
        mnext[i] = strip[(i / kPpMargin) * kPpPitch + kScoreChunk - kPpMargin + i % kPpMargin];
    __syncthreads();
  }
}

// kPoolTile consecutive positions of one (job, w') per workgroup, four
// consecutive ones per thread (one 16-byte load per query head); each head's
// strip and its pooling halo are staged in LDS in turn.  Kernels up to
// 2 * kPoolRegHalf + 1 pool from three 16-byte LDS reads held in registers;
// wider ones walk the window in LDS.
constexpr int kPoolThreads = 256;
constexpr int kPoolTile = 4 * kPoolThreads;
constexpr int kPoolMaxKernel = 63;  // widest pooling kernel: half-width 31
constexpr int kPoolHalo = 32;       // >= kPoolMaxKernel / 2, keeps the strip 16-byte aligned
static_assert(kPoolHalo >= kPoolMaxKernel / 2, "pooling halo narrower than the widest kernel");
constexpr int kPoolRegHalf = 4;   // register path: kernel <= 9
constexpr int kPoolHeads = 4;     // heads whose loads are in flight together

__global__ __launch_bounds__(kPoolThreads) void score_pool_kernel(const float* __restrict__ A, int G, int span,
                                                                  int pooling, int kernel, int flags,
                                                                  float* __restrict__ S) {
  __shared__ __align__(16) float s_a[kPoolTile + 2 * kPoolHalo];
  const int t0 = blockIdx.x * kPoolTile;
  const int jw = blockIdx.y;  // job * wout + w'
  const int p = kernel / 2;
  const float pad = pooling == 0 ? 0.f : -INFINITY;
  const int tb = t0 + 4 * threadIdx.x;
  const bool vec_ok = (span & 3) == 0 && tb + 4 <= span;
  // Halo of hw positions each side (at least kPoolRegHalf, so the register
  // path reads only loaded values): threads [0, hw) load t0 - hw + x,
  // threads [hw, 2hw) load t0 + kPoolTile + (x - hw).
  const int hw = max(p, kPoolRegHalf);
  const bool halo = threadIdx.x < 2 * hw;
  const int th = threadIdx.x < hw ? t0 - hw + threadIdx.x : t0 + kPoolTile + (threadIdx.x - hw);
  const int sh = threadIdx.x < hw ? kPoolHalo - hw + threadIdx.x : kPoolHalo + kPoolTile + (threadIdx.x - hw);
  float best[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
  for (int g0 = 0; g0 < G; g0 += kPoolHeads) {
    f32x4 v[kPoolHeads];
    float hv[kPoolHeads];
#pragma unroll
    for (int gg = 0; gg < kPoolHeads; ++gg) {
      const int g = min(g0 + gg, G - 1);  // past G: a repeated (unused) head
      const float* a = A + ((int64_t)jw * G + g) * span;
      if (vec_ok) {
        v[gg] = *reinterpret_cast<const f32x4*>(a + tb);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[gg][e] = tb + e < span ? a[tb + e] : pad;
      }
      hv[gg] = halo && th >= 0 && th < span ? a[th] : pad;
    }
#pragma unroll
    for (int gg = 0; gg < kPoolHeads; ++gg) {
      if (g0 + gg >= G) break;
      __syncthreads();  // the previous strip has been pooled
      *reinterpret_cast<f32x4*>(&s_a[kPoolHalo + 4 * threadIdx.x]) = v[gg];
      if (halo) s_a[sh] = hv[gg];
      __syncthreads();
      float r[4];
      if (p <= kPoolRegHalf) {
        // w[i] = position 4*tid - 4 + i of the strip.
        float w[12];
#pragma unroll
        for (int c = 0; c < 3; ++c) {
          const f32x4 x = *reinterpret_cast<const f32x4*>(&s_a[kPoolHalo + 4 * threadIdx.x - 4 + 4 * c]);
#pragma unroll
          for (int e = 0; e < 4; ++e) w[4 * c + e] = x[e];
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float acc = pad;
#pragma unroll
          for (int d = -kPoolRegHalf; d <= kPoolRegHalf; ++d) {
            const float x = w[4 + e + d];
            const float y = pooling == 0 ? acc + x : fmaxf(acc, x);
            acc = (d >= -p && d <= p) ? y : acc;
          }
          r[e] = acc;
        }
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float* win = s_a + kPoolHalo + 4 * threadIdx.x + e - p;
          float acc = pad;
          for (int d = 0; d <= 2 * p; ++d) acc = pooling == 0 ? acc + win[d] : fmaxf(acc, win[d]);
          r[e] = acc;
        }
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float acc = pooling == 0 ? r[e] / (float)kernel : r[e];
        best[e] = fmaxf(best[e], round_mode(acc, flags));
      }
    }
  }
  float* o = S + (int64_t)jw * span + tb;
  const bool acc_out = (flags & HC_SCORE_ACCUMULATE) != 0;
  if (vec_ok) {
    f32x4 b = {best[0], best[1], best[2], best[3]};
    if (acc_out) b += *reinterpret_cast<const f32x4*>(o);
    *reinterpret_cast<f32x4*>(o) = b;
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (tb + e < span) o[e] = acc_out ? o[e] + best[e] : best[e];
  }
}

// Small query sets (R < 32 rows): the statistics pass stored the logits,
// so probabilities, the window sum, pooling and the group max are formed in
// one pass over them instead of a second pass over K.  One workgroup per
// (job, w', kFinTile positions); each query head's strip plus its pooling
// halo is built in LDS.
constexpr int kFinTile = 1024;
constexpr int kLogitRowsMax = 32;  // rows of the logit-store path (R < 32)

// Probability of one logit (0 for a masked position), as the probability
// pass forms it.
template <int RMODE>
__device__ __forceinline__ float fin_prob(float x, float m, float iz) {
  return x == -INFINITY ? 0.f : round_fixed<RMODE>(fast_exp2(x - m) * iz);
}

constexpr int kFinHalo = 32;  // >= kPoolMaxKernel / 2, keeps the strip 16-byte aligned
constexpr int kFinHeads = 4;  // query heads whose loads are in flight together
constexpr int kFinWaveSlots = 6;  // the left halo, the four waves of a tile, the right halo

// With HIST, every output row also gets a kKeyDigitBins histogram of the
// top kKeyDigitBits bits of its scores' order keys (hist[row][digit], zeroed
// by the statistics merge): the first digit of the drift check's selection,
// built while the scores are in registers.  Workgroups then take several
// tiles of their row (gridDim.x < tiles) so that each flushes its LDS
// histogram to the row's once.
// Row statistics of the finish passes.  From the merged (max, sum) pairs,
// or, with `part` given, folded here from the statistics pass's
// per-workgroup partials (one wave per row, in the order of
// score_stats_merge_kernel, so the same values), which spares the merge
// launch.  LOG2: s_m = max + log2(sum) (p = exp2(x - s_m)); otherwise
// s_m = max and s_iz = 1 / sum.
template <bool LOG2>
__device__ __forceinline__ void finish_row_stats(const float* __restrict__ stats, const float* __restrict__ part,
                                                 int nparts, int job, int R, float* s_m, float* s_iz) {
  auto set = [&](int r, float m, float l) {
    if constexpr (LOG2) {
      s_m[r] = m + __log2f(l);
    } else {
      s_m[r] = m;
      s_iz[r] = 1.f / l;
    }
  };
  if (part) {
    const int lane = threadIdx.x & 63;
    for (int r = threadIdx.x >> 6; r < R; r += blockDim.x >> 6) {
      float m = -INFINITY, l = 0.f;
      for (int c = lane; c < nparts; c += 64) {
        const float* q = part + (((int64_t)job * nparts + c) * R + r) * 2;
        merge_ml(m, l, q[0], q[1]);
      }
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) {
        const float m2 = __shfl_xor(m, off, 64), l2 = __shfl_xor(l, off, 64);
        merge_ml(m, l, m2, l2);
      }
      if (lane == 0) set(r, m, l);
    }
  } else {
    for (int r = threadIdx.x; r < R; r += blockDim.x)
      set(r, stats[((int64_t)job * R + r) * 2], stats[((int64_t)job * R + r) * 2 + 1]);
  }
}

template <int RMODE, int POOL, bool HIST>
__global__ __launch_bounds__(256) void score_finish_kernel(const float* __restrict__ logits,
                                                           const float* __restrict__ stats,
                                                           const float* __restrict__ part, int nparts, int R, int G, int W,
                                                           int span, int sum_w, int kernel, int accumulate,
                                                           float* __restrict__ S, uint32_t* __restrict__ hist) {
  // s_a[kFinHalo + i] holds position t0 + i of the current head's strip,
  // i in [-p, kFinTile + p).  Thread x loads positions t0 + 4x .. +3 (one
  // 16-byte load per row) and pools positions t0 + x + 256k, so LDS reads
  // of neighbouring lanes are consecutive words.
  __shared__ __align__(16) float s_a[kFinTile + 2 * kFinHalo];
  __shared__ float s_m[kLogitRowsMax], s_iz[kLogitRowsMax];  // row max, 1 / row sum
  __shared__ uint32_t s_hist[HIST ? kKeyDigitBins : 1];
  const int wout = sum_w ? 1 : W;
  const int job = blockIdx.y / wout, wo = blockIdx.y % wout;
  const int ntiles = (span + kFinTile - 1) / kFinTile;
  const int p = kernel / 2;
  constexpr float pad = POOL == 0 ? 0.f : -INFINITY;
  finish_row_stats<false>(stats, part, nparts, job, R, s_m, s_iz);
  if constexpr (HIST)
    for (int b = threadIdx.x; b < kKeyDigitBins; b += 256) s_hist[b] = 0u;
  const int w_lo = sum_w ? 0 : wo, w_hi = sum_w ? W : wo + 1;
  const bool halo = threadIdx.x < 2 * p;
  const float inv_k = 1.f / (float)kernel;
  float* o = S + ((int64_t)job * wout + wo) * span;
  __syncthreads();
  for (int tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
    const int t0 = tile * kFinTile;
    const int tb = t0 + 4 * threadIdx.x;
    const bool vec_ok = (span & 3) == 0 && tb + 4 <= span;
    // Halo: threads [0, p) load t0 - p + x (left), threads [p, 2p) load
    // t0 + kFinTile + (x - p) (right).
    const int th = threadIdx.x < p ? t0 - p + threadIdx.x : t0 + kFinTile + (threadIdx.x - p);
    const int sh = threadIdx.x < p ? kFinHalo - p + threadIdx.x : kFinHalo + kFinTile + (threadIdx.x - p);
    float best[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    // Heads are taken kFinHeads at a time: all their rows' loads are issued
    // before any strip is pooled.
    for (int g0 = 0; g0 < G; g0 += kFinHeads) {
      f32x4 a4[kFinHeads];
      float ah[kFinHeads];
#pragma unroll
      for (int gg = 0; gg < kFinHeads; ++gg) {
        const int g = g0 + gg;
        a4[gg] = f32x4{pad, pad, pad, pad};
        ah[gg] = pad;
        if (g >= G) continue;
        if (tb < span) {
          f32x4 acc = {0.f, 0.f, 0.f, 0.f};
          for (int w = w_lo; w < w_hi; ++w) {
            const int r = g * W + w;
            const float* row = logits + ((int64_t)job * R + r) * span;
            const float m = s_m[r], iz = s_iz[r];
            if (vec_ok) {
              const f32x4 x = *reinterpret_cast<const f32x4*>(row + tb);
#pragma unroll
              for (int e = 0; e < 4; ++e) acc[e] += fin_prob<RMODE>(x[e], m, iz);
            } else {
#pragma unroll
              for (int e = 0; e < 4; ++e)
                if (tb + e < span) acc[e] += fin_prob<RMODE>(row[tb + e], m, iz);
            }
          }
#pragma unroll
          for (int e = 0; e < 4; ++e) a4[gg][e] = tb + e < span ? round_fixed<RMODE>(acc[e]) : pad;
        }
        if (halo && th >= 0 && th < span) {
          float acc = 0.f;
          for (int w = w_lo; w < w_hi; ++w) {
            const int r = g * W + w;
            acc += fin_prob<RMODE>(logits[((int64_t)job * R + r) * span + th], s_m[r], s_iz[r]);
          }
          ah[gg] = round_fixed<RMODE>(acc);
        }
      }
#pragma unroll
      for (int gg = 0; gg < kFinHeads; ++gg) {
        if (g0 + gg >= G) break;
        __syncthreads();  // the previous strip has been pooled
        *reinterpret_cast<f32x4*>(&s_a[kFinHalo + 4 * threadIdx.x]) = a4[gg];
        if (halo) s_a[sh] = ah[gg];
        __syncthreads();
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int c = threadIdx.x + 256 * k;  // output position t0 + c
          const float* win = s_a + kFinHalo + c - p;
          float v = pad;
          for (int d = 0; d <= 2 * p; ++d) v = POOL == 0 ? v + win[d] : fmaxf(v, win[d]);
          if constexpr (POOL == 0) v *= inv_k;
          best[k] = fmaxf(best[k], round_fixed<RMODE>(v));
        }
      }
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int t = t0 + threadIdx.x + 256 * k;
      if (t < span) {
        o[t] = accumulate ? o[t] + best[k] : best[k];
        if constexpr (HIST) atomicAdd(&s_hist[order_key(best[k]) >> kKeyDigitShift], 1u);
      }
    }
  }
  if constexpr (HIST) {
    __syncthreads();
    uint32_t* h = hist + ((int64_t)job * wout + wo) * kKeyDigitBins;
    for (int b = threadIdx.x; b < kKeyDigitBins; b += 256)
      if (s_hist[b]) atomicAdd(&h[b], s_hist[b]);
  }
}

// Tiles per workgroup of the histogram-building finish: each workgroup
// flushes its histogram once, so a row's histogram takes tiles / this many
// flushes (global atomics on the same few lines serialise).
constexpr int kFinHistTiles = 4;

// Pool kernels 5 and 7 (the half-width P a template parameter, so the taps
// unroll without per-tap selects): each thread pools its own kFinRegPos
// consecutive positions in registers (tiles of kFinRegTile positions, two
// 16-byte loads per row and thread).  The P neighbours on either side come
// from the adjacent lanes by shuffles; only each wave's edge values and the
// tile's halo go through LDS, one barrier per group of kFinHeads query heads
// (the edge buffer alternates between groups).  Sums and maxima run in
// score_finish_kernel's order; with the reference's casts the scores are the
// same bit for bit, without them the row sum is folded into the exponent
// (within a few ulp of the reciprocal form).
constexpr int kFinRegHalf = 4;  // widest half-width the window registers hold
// Probability of one logit: without casts m holds m + log2 l (the row sum
// folded into the exponent); with casts as fin_prob.
template <int RMODE>
__device__ __forceinline__ float fin_prob_reg(float x, float m, float iz) {
  if constexpr (RMODE == 0) return fast_exp2(x - m);
  return fin_prob<RMODE>(x, m, iz);
}
constexpr int kFinRegPos = 8;
constexpr int kFinRegTile = 256 * kFinRegPos;
constexpr int kFinRegHistTiles = 2;
template <int RMODE, int POOL, bool HIST, int P>
__global__ __launch_bounds__(256) void score_finish_reg_kernel(const float* __restrict__ logits,
                                                               const float* __restrict__ stats,
                                                               const float* __restrict__ part, int nparts, int R,
                                                               int G, int W,
                                                               int span, int sum_w, int kernel, int accumulate,
                                                               float* __restrict__ S, uint32_t* __restrict__ hist) {
  constexpr int NV = kFinRegPos / 4;  // 16-byte vectors per thread and row
  // s_edge[buffer][head][slot][side]: slot 0 = the tile's left halo, 1 + w =
  // wave w, 5 = the right halo; side 0 = first four positions, 1 = last four.
  __shared__ f32x4 s_edge[2][kFinHeads][kFinWaveSlots][2];
  __shared__ float s_m[kLogitRowsMax], s_iz[kLogitRowsMax];
  __shared__ uint32_t s_hist[HIST ? kKeyDigitBins : 1];
  const int wout = sum_w ? 1 : W;
  const int job = blockIdx.y / wout, wo = blockIdx.y % wout;
  static_assert(P >= 0 && P <= kFinRegHalf, "pool half-width");
  const int ntiles = (span + kFinRegTile - 1) / kFinRegTile;
  constexpr int p = P;  // kernel == 2P + 1
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  constexpr float pad = POOL == 0 ? 0.f : -INFINITY;
  finish_row_stats<RMODE == 0>(stats, part, nparts, job, R, s_m, s_iz);
  if constexpr (HIST)
    for (int b = threadIdx.x; b < kKeyDigitBins; b += 256) s_hist[b] = 0u;
  const int w_lo = sum_w ? 0 : wo, w_hi = sum_w ? W : wo + 1;
  const bool halo = threadIdx.x < 2 * p;
  const float inv_k = 1.f / (float)kernel;
  float* o = S + ((int64_t)job * wout + wo) * span;
  int buf = 0;
  __syncthreads();
  for (int tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
    const int t0 = tile * kFinRegTile;
    const int tb = t0 + kFinRegPos * threadIdx.x;
    const bool vec_ok = (span & 3) == 0 && tb + kFinRegPos <= span;
    // Halo threads: [0, p) positions t0 - p + x, [p, 2p) t0 + kFinRegTile + (x - p).
    const int th = threadIdx.x < p ? t0 - p + threadIdx.x : t0 + kFinRegTile + (threadIdx.x - p);
    float best[kFinRegPos];
#pragma unroll
    for (int i = 0; i < kFinRegPos; ++i) best[i] = -INFINITY;
    for (int g0 = 0; g0 < G; g0 += kFinHeads) {
      float a[kFinHeads][kFinRegPos];
      float ah[kFinHeads];
#pragma unroll
      for (int gg = 0; gg < kFinHeads; ++gg) {
        const int g = g0 + gg;
#pragma unroll
        for (int i = 0; i < kFinRegPos; ++i) a[gg][i] = pad;
        ah[gg] = pad;
        if (g >= G) continue;
        if (tb < span) {
          float acc[kFinRegPos];
#pragma unroll
          for (int i = 0; i < kFinRegPos; ++i) acc[i] = 0.f;
          for (int w = w_lo; w < w_hi; ++w) {
            const int r = g * W + w;
            const float* row = logits + ((int64_t)job * R + r) * span;
            const float m = s_m[r], iz = s_iz[r];
            if (vec_ok) {
              f32x4 x[NV];
#pragma unroll
              for (int v = 0; v < NV; ++v) x[v] = *reinterpret_cast<const f32x4*>(row + tb + 4 * v);
#pragma unroll
              for (int v = 0; v < NV; ++v)
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[4 * v + e] += fin_prob_reg<RMODE>(x[v][e], m, iz);
            } else {
#pragma unroll
              for (int i = 0; i < kFinRegPos; ++i)
                if (tb + i < span) acc[i] += fin_prob_reg<RMODE>(row[tb + i], m, iz);
            }
          }
#pragma unroll
          for (int i = 0; i < kFinRegPos; ++i) a[gg][i] = tb + i < span ? round_fixed<RMODE>(acc[i]) : pad;
        }
        if (halo && th >= 0 && th < span) {
          float acc = 0.f;
          for (int w = w_lo; w < w_hi; ++w) {
            const int r = g * W + w;
            acc += fin_prob_reg<RMODE>(logits[((int64_t)job * R + r) * span + th], s_m[r], s_iz[r]);
          }
          ah[gg] = round_fixed<RMODE>(acc);
        }
      }
      // Edges and halo to LDS; the buffer alternates, so a group's writes
      // never meet the previous group's reads.
#pragma unroll
      for (int gg = 0; gg < kFinHeads; ++gg) {
        if (lane == 0) s_edge[buf][gg][1 + wave][0] = f32x4{a[gg][0], a[gg][1], a[gg][2], a[gg][3]};
        if (lane == 63)
          s_edge[buf][gg][1 + wave][1] = f32x4{a[gg][kFinRegPos - 4], a[gg][kFinRegPos - 3], a[gg][kFinRegPos - 2],
                                               a[gg][kFinRegPos - 1]};
        if (halo) {
          if (threadIdx.x < p)
            s_edge[buf][gg][0][1][kFinRegHalf - p + threadIdx.x] = ah[gg];
          else
            s_edge[buf][gg][kFinWaveSlots - 1][0][threadIdx.x - p] = ah[gg];
        }
      }
      __syncthreads();
#pragma unroll
      for (int gg = 0; gg < kFinHeads; ++gg) {
        if (g0 + gg >= G) break;
        // w[4 + d] = position tb + d, d in [-4, kFinRegPos + 4).
        float w[kFinRegPos + 8];
#pragma unroll
        for (int i = 0; i < kFinRegPos; ++i) w[4 + i] = a[gg][i];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          w[e] = __shfl_up(a[gg][kFinRegPos - 4 + e], 1, 64);
          w[kFinRegPos + 4 + e] = __shfl_down(a[gg][e], 1, 64);
        }
        if (lane == 0) {
          const f32x4 l = s_edge[buf][gg][wave][1];
#pragma unroll
          for (int e = 0; e < 4; ++e) w[e] = l[e];
        }
        if (lane == 63) {
          const f32x4 r = s_edge[buf][gg][wave + 2][0];
#pragma unroll
          for (int e = 0; e < 4; ++e) w[kFinRegPos + 4 + e] = r[e];
        }
#pragma unroll
        for (int i = 0; i < kFinRegPos; ++i) {
          float v = pad;
#pragma unroll
          for (int off = -P; off <= P; ++off) v = POOL == 0 ? v + w[4 + i + off] : fmaxf(v, w[4 + i + off]);
          if constexpr (POOL == 0) v *= inv_k;
          best[i] = fmaxf(best[i], round_fixed<RMODE>(v));
        }
      }
      buf ^= 1;
    }
    if (vec_ok && !accumulate) {
#pragma unroll
      for (int v = 0; v < NV; ++v)
        *reinterpret_cast<f32x4*>(o + tb + 4 * v) = f32x4{best[4 * v], best[4 * v + 1], best[4 * v + 2], best[4 * v + 3]};
    } else {
#pragma unroll
      for (int i = 0; i < kFinRegPos; ++i)
        if (tb + i < span) o[tb + i] = accumulate ? o[tb + i] + best[i] : best[i];
    }
    if constexpr (HIST) {
#pragma unroll
      for (int i = 0; i < kFinRegPos; ++i)
        if (tb + i < span) atomicAdd(&s_hist[order_key(best[i]) >> kKeyDigitShift], 1u);
    }
  }
  if constexpr (HIST) {
    __syncthreads();
    uint32_t* h = hist + ((int64_t)job * wout + wo) * kKeyDigitBins;
    for (int b = threadIdx.x; b < kKeyDigitBins; b += 256)
      if (s_hist[b]) atomicAdd(&h[b], s_hist[b]);
  }
}

// ---------------------------------------------------------------------------
// One-pass scoring with given softmax statistics (hc_score_given_stats).
// When the normaliser of every query row over the keys is already known --
// the drift check's buffered decode queries, whose decode attention launches
// (hc_decode_attn_stats) reported (M, L) over the pivot's prefill keys --
// the probabilities need no statistics pass and no stored logits:
//   p = exp2(s - (M + log2 L)),  S[w'][t] = max_g pool(p[g*W + w'])[t].
// Each workgroup takes a run of 256-token chunks of one job.  Per chunk its
// four waves form the probabilities of all R rows (keys from the tiled
// store as the MFMA A operand, queries staged in LDS once) into an LDS strip
// of the chunk's 256 positions, and the pooling runs 16 positions behind:
// positions [cb - 16, cb + 240) of chunk c, whose right neighbours are now
// in the strip.  The left neighbours -- the previous chunk's last 32
// positions -- sit in one of two margin buffers, which the pooling of chunk
// c also fills for chunk c + 1, so each chunk costs two barriers (strip
// written; strip read).  Only a run's ends cost an extra 16-token sub-tile:
// the left margin of its first chunk and the right margin of its last 16
// positions.  Each wave's keys are two double-buffered halves: a half's next
// keys are requested as soon as its products are formed, so they land while
// the other half is scored and the chunk pools.  The first-digit key
// histograms that hc_drift_select needs are left to its own pass over the
// scores (24 us at
// 33 pivots x 5 steps x 128K): counted here, in LDS as 16-bit counters of
// the 1024 digits a probability can have, they took the kernel from 0.25 to
// 0.39 ms, and counted into global memory, 0.69 ms.
// (Four independent waves per workgroup, each with its own 128-position ring
// and no barriers, measured slower: 0.32 against 0.25 ms at 33 pivots x 5
// steps x 128K, at three waves per SIMD instead of four.  With one key
// buffer, so did requesting the next chunk's keys earlier -- sub-tile by
// sub-tile as each one's products are issued (270 against 260 us: two MFMA
// chains per step instead of eight), or all four right after the last row
// tile's products (263).)
// ---------------------------------------------------------------------------
constexpr int kGsMargin = 32;                     // margin positions before a chunk
constexpr int kGsRight = 16;                      // the run's right margin
constexpr int kGsPitch = kScoreChunk + kGsRight + 4;   // strip row: chunk + right margin + bank skew
constexpr int kGsMPitch = kGsMargin + 4;          // margin row
constexpr int kGsPosPerTask = 4;                  // pooled positions per task

// Strip view of one chunk: position cb + i (i in [-32, 272)) of row r is
// margin[r][i + 32] for i < 0, strip[r][i] otherwise.
struct GsView {
  float* strip;        // [R][kGsPitch]
  const float* mrg;    // [R][kGsMPitch] (previous chunk's last 32 positions)
  __device__ __forceinline__ f32x4 read4(int r, int i) const {  // i a multiple of 4
    return i < 0 ? *reinterpret_cast<const f32x4*>(mrg + r * kGsMPitch + kGsMargin + i)
                 : *reinterpret_cast<const f32x4*>(strip + r * kGsPitch + i);
  }
};

// Probabilities of the 16-token sub-tiles tw + 16u (u < NU) of every row,
// written to dst + r * pitch + (token - base); positions outside [0, span)
// get the pooling pad.  Per row tile the NU sub-tiles' MFMA chains are
// issued before any exponential.  RM == 0: p = exp2(s - s_mz[r]) with s_mz
// = M + log2 L; otherwise the cast chain of the probability pass,
// p = round(exp2(x - M) * (1 / L)) of the rounded logit x, with s_mz = M
// and s_iz = 1 / L.
template <typename T, int POOL, int NU, int RM>
__device__ __forceinline__ void gs_subtiles(const ScoreArgs& a, const typename Elem<T>::vec8 (*kr)[4], const T* s_q,
                                            const float* s_mz, const float* s_iz, float* dst, int pitch, int base,
                                            int tw, int lane) {
  constexpr float pad = POOL == 0 ? 0.f : -INFINITY;
  const bool mask = tw + 16 * NU - 1 >= a.L;
  // At most two row tiles (R < 32): unrolled, so the code holds no loop and
  // the compiler's waits for the keys are exact (inside a rolled loop they
  // also waited for the other key buffer in flight).
  static_assert(kLogitRowsMax <= 32, "two row tiles at most");
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    if (nt >= a.NT) break;
    const int r = 16 * nt + (lane & 15);
    float x[NU][4];
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      if (mask)
        subtile_logits<T, RM, true, RM == 0>(a, kr[u], s_q, nt, tw + 16 * u, lane, a.L - 1, x[u]);
      else
        subtile_logits<T, RM, false, RM == 0>(a, kr[u], s_q, nt, tw + 16 * u, lane, a.L - 1, x[u]);
    }
    if (r < a.R) {
      const float mz = s_mz[r];
      const float iz = RM == 0 ? 0.f : s_iz[r];
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        const int tb = tw + 16 * u + 4 * (lane >> 4);
        f32x4 v;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int t = tb + j;
          float p;
          if constexpr (RM == 0)
            p = fast_exp2(fmaf(x[u][j], a.scale2, -mz));
          else
            p = x[u][j] == -INFINITY ? 0.f : round_fixed<RM>(fast_exp2(x[u][j] - mz) * iz);
          v[j] = (t >= 0 && t < a.span) ? p : pad;
        }
        *reinterpret_cast<f32x4*>(dst + r * pitch + (tb - base)) = v;
      }
    }
  }
}

// Pool chunk positions cb + [i0, i0 + n) (i0, n multiples of 4), take the
// group max and write the scores: task = (output row w', four consecutive
// positions), reading its 4 + 2P window values per query head as three
// 16-byte LDS reads.  RM: the pooled value is rounded before the group max,
// as in the cast chain.
template <int POOL, int P, int RM>
__device__ __forceinline__ void gs_pool(const ScoreArgs& a, const GsView& v, int cb, int i0, int n, int job,
                                        float* __restrict__ S) {
  static_assert(P <= 4, "window registers hold 4 values on either side");
  constexpr float pad = POOL == 0 ? 0.f : -INFINITY;
  const float inv_k = 1.f / (float)(2 * P + 1);
  const int per_row = n / kGsPosPerTask;
  for (int task = threadIdx.x; task < a.W * per_row; task += kScoreWaves * 64) {
    const int w = task / per_row, i = i0 + (task % per_row) * kGsPosPerTask;
    float best[kGsPosPerTask];
#pragma unroll
    for (int e = 0; e < kGsPosPerTask; ++e) best[e] = -INFINITY;
    for (int g = 0; g < a.G; ++g) {
      const int r = g * a.W + w;
      // win[d] = position cb + i - 4 + d, d in [0, 12).
      const f32x4 lo = v.read4(r, i - 4), mid = v.read4(r, i), hi = v.read4(r, i + 4);
      const float win[12] = {lo[0], lo[1], lo[2], lo[3], mid[0], mid[1], mid[2], mid[3], hi[0], hi[1], hi[2], hi[3]};
#pragma unroll
      for (int e = 0; e < kGsPosPerTask; ++e) {
        float x = pad;
#pragma unroll
        for (int d = -P; d <= P; ++d) x = POOL == 0 ? x + win[4 + e + d] : fmaxf(x, win[4 + e + d]);
        if constexpr (POOL == 0) x *= inv_k;
        best[e] = fmaxf(best[e], round_fixed<RM>(x));
      }
    }
    const int t = cb + i;
    float* o = S + ((int64_t)job * a.W + w) * a.span + t;
    if (t + kGsPosPerTask <= a.span && (a.span & 3) == 0) {
      *reinterpret_cast<f32x4*>(o) = f32x4{best[0], best[1], best[2], best[3]};
    } else {
#pragma unroll
      for (int e = 0; e < kGsPosPerTask; ++e)
        if (t + e < a.span) o[e] = best[e];
    }
  }
}

// Keys of NU 16-token sub-tiles from tw on, read in place from the tiled
// store past L2.  A sub-tile past the job's last key is read at the last
// sub-tile holding a key instead (inside the row's tiles; its tokens are
// masked), so no lane branches around the loads.
template <typename T, int NU>
__device__ __forceinline__ void load_k_run(const ScoreArgs& a, const T* kj, int tw, int lane,
                                           typename Elem<T>::vec8 (&k)[NU][4]) {
  const int last = ((a.L - 1) / 16) * 16;
#pragma unroll
  for (int u = 0; u < NU; ++u) {
    const int t0 = min(tw + 16 * u, last);
    const T* base = kj + (t0 / HC_TILE) * (int64_t)HC_TILE_ELEMS + ((t0 / 16) & 1) * 4 * 512 + lane * 8;
#pragma unroll
    for (int s = 0; s < 4; ++s) k[u][s] = load8_stream<T>(base + s * 512);
  }
}

template <typename T, bool STORE, int POOL, int P, int RM>
__global__ __launch_bounds__(kScoreWaves * 64) void score_given_stats_kernel(ScoreArgs a,
                                                                            const float* __restrict__ stats,
                                                                            const int64_t* __restrict__ st_off,
                                                                            float* __restrict__ S) {
  static_assert(STORE, "keys are read in place from the tiled store");
  extern __shared__ __align__(16) unsigned char smem[];
  T* s_q = reinterpret_cast<T*>(smem);
  float* strip = reinterpret_cast<float*>(smem + (size_t)a.NT * 16 * kQPitch * sizeof(T));  // [R][kGsPitch]
  // Two margin buffers [R][kGsMPitch] after the strip.  Addressed by
  // arithmetic on the strip pointer: picked from an array of pointers, the
  // buffer's address lost its LDS address space, so the margin reads and
  // writes were flat instructions, which count against both wait counters
  // and made every wait in the chunk loop a wait for all loads and stores.
  float* const mrg0 = strip + a.R * kGsPitch;
  const int mstride = a.R * kGsMPitch;
  __shared__ float s_mz[kLogitRowsMax];
  __shared__ float s_iz[RM == 0 ? 1 : kLogitRowsMax];
  constexpr float pad = POOL == 0 ? 0.f : -INFINITY;
  typedef typename Elem<T>::vec8 vec8;
  const int job = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nchunks = (a.L + kScoreChunk - 1) / kScoreChunk;
  const int c0 = blockIdx.x * a.cpw, c1 = min(c0 + a.cpw, nchunks);
  if (c0 >= c1) return;  // uniform per workgroup (the grid holds none such)
  const int woff = wave * 16 * kSubTiles;
  const T* const kj = job_keys<T, STORE>(a, job);
  // A wave's 64 tokens of a chunk in two halves, double-buffered: a half's
  // keys for the next chunk are requested as soon as its products are
  // formed, so they land while the other half is scored and the chunk pools.
  constexpr int kHalf = kSubTiles / 2;
  vec8 ka0[kHalf][4], ka1[kHalf][4];
  vec8 kh[1][4];  // wave 1: the run's left margin; wave 0: its right margin
  load_k_run<T, kHalf>(a, kj, c0 * kScoreChunk + woff, lane, ka0);
  load_k_run<T, kHalf>(a, kj, c0 * kScoreChunk + woff + 16 * kHalf, lane, ka1);
  if (wave == 1 && c0 > 0) load_k_subtile<T, STORE>(a, kj, c0 * kScoreChunk - 16, lane, kh[0]);
  stage_queries<T>(a, job, s_q);
  for (int r = threadIdx.x; r < a.R; r += kScoreWaves * 64) {
    const float* st = stats + st_off[job] + 2 * r;
    // p = exp2(s - (M + log2 L)); a row without keys (L = 0) gives p = 0.
    if constexpr (RM == 0) {
      s_mz[r] = st[1] > 0.f ? st[0] + __log2f(st[1]) : INFINITY;
    } else {
      s_mz[r] = st[1] > 0.f ? st[0] : INFINITY;
      s_iz[r] = st[1] > 0.f ? 1.f / st[1] : 0.f;
    }
  }
  __syncthreads();
  // The run's left margin: positions c0*256 - 16 .. - 1 (margin entries
  // [16, 32) of buffer 1, which the first chunk reads).
  if (wave == 1) {
    const int cb0 = c0 * kScoreChunk;
    if (c0 > 0) {
      gs_subtiles<T, POOL, 1, RM>(a, kh, s_q, s_mz, s_iz, mrg0 + mstride, kGsMPitch, cb0 - kGsMargin, cb0 - 16, lane);
    } else {
      for (int i = lane; i < a.R * 16; i += 64) mrg0[mstride + (i / 16) * kGsMPitch + 16 + i % 16] = pad;
    }
  }
  // Drain the set-up's loads: the staging loops leave a count in flight that
  // the compiler cannot bound, and with that state at the loop head its
  // waits for a half's keys would wait for the other half's as well.
  __builtin_amdgcn_s_waitcnt(0);
  // The chunk loop with the run's last chunk peeled: a chunk requests the
  // next chunk's keys unconditionally, so the compiler's waits count every
  // load in flight (behind a branch around the requests its waits for one
  // half also waited for the other).
  auto run_chunk = [&](int c, auto load_next) {
    const int cb = c * kScoreChunk;
    gs_subtiles<T, POOL, kHalf, RM>(a, ka0, s_q, s_mz, s_iz, strip, kGsPitch, cb, cb + woff, lane);
    if constexpr (decltype(load_next)::value) load_k_run<T, kHalf>(a, kj, cb + kScoreChunk + woff, lane, ka0);
    gs_subtiles<T, POOL, kHalf, RM>(a, ka1, s_q, s_mz, s_iz, strip, kGsPitch, cb, cb + woff + 16 * kHalf, lane);
    if constexpr (decltype(load_next)::value)
      load_k_run<T, kHalf>(a, kj, cb + kScoreChunk + woff + 16 * kHalf, lane, ka1);
    __syncthreads();  // strip written (and the margin of the previous chunk)
    const int mb = (c - c0 + 1) & 1;  // margin buffer holding the previous chunk's tail
    GsView v{strip, mrg0 + mb * mstride};
    // Positions [cb - 16, cb + 240) (the run's first chunk: from cb).
    if (c == c0)
      gs_pool<POOL, P, RM>(a, v, cb, 0, kScoreChunk - 16, job, S);
    else
      gs_pool<POOL, P, RM>(a, v, cb, -16, kScoreChunk, job, S);
    // This chunk's last 32 positions are the next chunk's margin.
    float* nm = mrg0 + (mb ^ 1) * mstride;
    for (int i = threadIdx.x; i < a.R * kGsMargin; i += kScoreWaves * 64) {
      const int r = i / kGsMargin, e = i % kGsMargin;
      nm[r * kGsMPitch + e] = strip[r * kGsPitch + kScoreChunk - kGsMargin + e];
    }
    __syncthreads();  // strip read
  };
  for (int c = c0; c < c1 - 1; ++c) run_chunk(c, std::true_type{});
  run_chunk(c1 - 1, std::false_type{});
  // The run's last 16 positions, with its right margin c1*256 .. +15 at
  // strip entries [256, 272).
  if (wave == 0) {
    const int tr = c1 * kScoreChunk;
    load_k_subtile<T, STORE>(a, kj, tr, lane, kh[0]);
    gs_subtiles<T, POOL, 1, RM>(a, kh, s_q, s_mz, s_iz, strip, kGsPitch, tr - kScoreChunk, tr, lane);
  }
  __syncthreads();
  const int mb = (c1 - c0) & 1;
  gs_pool<POOL, P, RM>(a, GsView{strip, mrg0 + mb * mstride}, (c1 - 1) * kScoreChunk, kScoreChunk - 16, 16, job, S);
}

static size_t align256(size_t x) { return (x + 255) / 256 * 256; }

// Query sets below this many rows take the logit-store path.
constexpr int kLogitRows = 32;

size_t score_workspace_bytes(int njobs, int L, int G, int W, int flags) {
  const int R = G * W;
  const int nchunks = (L + kScoreChunk - 1) / kScoreChunk;
  const int wout = (flags & HC_SCORE_SUM_WINDOW) ? 1 : W;
  const size_t tail = R < kLogitRows ? (size_t)njobs * R * L * sizeof(float)          // logits
                                     : (size_t)njobs * wout * G * L * sizeof(float);  // probabilities
  return align256((size_t)njobs * nchunks * R * 2 * sizeof(float)) +
         align256((size_t)njobs * R * 2 * sizeof(float)) + align256(tail);
}

// Workgroups of one score kernel instance (kScoreWaves * 64 threads, `lds`
// bytes of dynamic LDS) resident on the current device at once, cached per
// (device, instance, lds); 0 when the query fails.
static int resident_wgs(const void* fn, size_t lds) {
  struct Entry {
    int dev;
    const void* fn;
    size_t lds;
    int slots;
  };
  static std::mutex mu;
  static std::vector<Entry> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  std::lock_guard<std::mutex> lock(mu);
  for (const Entry& e : cache)
    if (e.dev == dev && e.fn == fn && e.lds == lds) return e.slots;
  int per_cu = 0, cus = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kScoreWaves * 64, lds) != hipSuccess) return 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  const int slots = (per_cu > 0 ? per_cu : 1) * (cus > 0 ? cus : 1);
  cache.push_back({dev, fn, lds, slots});
  return slots;
}

// Chunks per workgroup so that one resident round of workgroups covers the
// njobs * nchunks chunks (queries staged once per workgroup); sets a.cpw,
// returns the grid's x extent.  The statistics pass that also stores every
// logit takes one chunk per workgroup (multi = false), measured faster
// there: vmcnt counts stores as well as loads, so a workgroup's wait for its
// next chunk's keys also waits for its previous chunk's 4R-byte-per-token
// stores, while a finished workgroup leaves them draining behind the next.
static int plan_chunks(const void* fn, size_t lds, int njobs, int nchunks, ScoreArgs& a, bool multi = true) {
  const int slots = multi ? resident_wgs(fn, lds) : 0;
  const int64_t total = (int64_t)njobs * nchunks;
  a.cpw = slots > 0 ? (int)std::max<int64_t>(1, (total + slots - 1) / slots) : 1;
  return (nchunks + a.cpw - 1) / a.cpw;
}

template <typename T, int RM, int POOL, int P>
static void launch_fused(ScoreArgs a, int njobs, StatsView sv, float* scores, hipStream_t s) {
  const int rows = a.NT * 16;
  const size_t lds = (size_t)rows * kQPitch * sizeof(T) + (size_t)rows * (RM != 0 ? 2 : 1) * sizeof(float) +
                     (size_t)a.G * (kPpPitch + 2 * kPpMargin) * sizeof(float);
  auto fn = score_probs_pool_kernel<T, false, RM, POOL, P>;
  const int nchunks = (a.span + kScoreChunk - 1) / kScoreChunk;
  const int gx = plan_chunks(reinterpret_cast<const void*>(fn), lds, njobs, nchunks, a);
  hipLaunchKernelGGL(fn, dim3(gx, njobs), dim3(kScoreWaves * 64), lds, s, a, sv, scores);
}

// The fused probability + pooling pass over natural-layout keys; the
// rounding mode of an instance is the one its key type takes (or none).
template <typename T>
static int launch_probs_pool_fused(ScoreArgs a, int njobs, int pooling, int kernel, StatsView sv, float* scores,
                                   hipStream_t s) {
  constexpr int kRm = std::is_same<T, __bf16>::value ? 1 : std::is_same<T, _Float16>::value ? 2 : 0;
  const bool cast = (a.flags & (HC_SCORE_ROUND_BF16 | HC_SCORE_ROUND_F16)) != 0;
#define HC_FUSED_P(RM, PL)                                                           \
  switch (kernel / 2) {                                                              \
    case 0: launch_fused<T, RM, PL, 0>(a, njobs, sv, scores, s); break;              \
    case 1: launch_fused<T, RM, PL, 1>(a, njobs, sv, scores, s); break;              \
    case 2: launch_fused<T, RM, PL, 2>(a, njobs, sv, scores, s); break;              \
    case 3: launch_fused<T, RM, PL, 3>(a, njobs, sv, scores, s); break;              \
    default: launch_fused<T, RM, PL, 4>(a, njobs, sv, scores, s); break;             \
  }
  if (!cast) {
    if (pooling == 0) { HC_FUSED_P(0, 0) } else { HC_FUSED_P(0, 1) }
  } else if constexpr (kRm != 0) {
    if (pooling == 0) { HC_FUSED_P(kRm, 0) } else { HC_FUSED_P(kRm, 1) }
  }
#undef HC_FUSED_P
  return check_launch("hc_score(probs+pool)");
}

// The probability pass (row statistics given) and the pooling pass:
// scores over [0, a.span), A = the window-summed probabilities.
template <typename T, bool STORE>
static int launch_probs_pool(ScoreArgs a, int njobs, int pooling, int kernel, StatsView sv, float* A, float* scores,
                             hipStream_t s) {
  const int wout = (a.flags & HC_SCORE_SUM_WINDOW) ? 1 : a.W;
  const size_t lds3 = (size_t)a.NT * 16 * kQPitch * sizeof(T) + (size_t)a.NT * 16 * 2 * sizeof(float);
  const int rm = (a.flags & HC_SCORE_ROUND_BF16) ? 1 : (a.flags & HC_SCORE_ROUND_F16) ? 2 : 0;
  int rc;
  const int nchunks_span = (a.span + kScoreChunk - 1) / kScoreChunk;
  if (nchunks_span > 0 && !STORE && (a.flags & HC_SCORE_SUM_WINDOW) && a.W % 16 == 0 && kernel / 2 <= kPpMaxHalf &&
      (rm == 0 || rm == (std::is_same<T, __bf16>::value ? 1 : std::is_same<T, _Float16>::value ? 2 : -1)))
    return launch_probs_pool_fused<T>(a, njobs, pooling, kernel, sv, scores, s);
  if (nchunks_span > 0) {
    const int wm = !(a.flags & HC_SCORE_SUM_WINDOW) ? kWinNone
                   : a.W >= 16                       ? kWin16
                   : a.W == 8                        ? kWin8
                   : a.W == 4                        ? kWin4
                   : a.W == 2                        ? kWin2
                                                     : kWin1;
#define HC_PROBS(RM, WM)                                                                                    \
  do {                                                                                                      \
    auto fn = score_probs_kernel<T, STORE, RM, WM, false>;                                                  \
    ScoreArgs as = a;                                                                                       \
    const int gx = plan_chunks(reinterpret_cast<const void*>(fn), lds3, njobs, nchunks_span, as);           \
    hipLaunchKernelGGL(fn, dim3(gx, njobs), dim3(kScoreWaves * 64), lds3, s, as, sv, A, nullptr, nullptr);    \
  } while (0)
#define HC_PROBS_RM(RM)                                     \
  switch (wm) {                                             \
    case kWinNone: HC_PROBS(RM, kWinNone); break;           \
    case kWin16: HC_PROBS(RM, kWin16); break;               \
    case kWin8: HC_PROBS(RM, kWin8); break;                 \
    case kWin4: HC_PROBS(RM, kWin4); break;                 \
    case kWin2: HC_PROBS(RM, kWin2); break;                 \
    default: HC_PROBS(RM, kWin1); break;                    \
  }
    if (rm == 0) { HC_PROBS_RM(0) } else if (rm == 1) { HC_PROBS_RM(1) } else { HC_PROBS_RM(2) }
#undef HC_PROBS_RM
#undef HC_PROBS
    if ((rc = check_launch("hc_score(probs)"))) return rc;
    hipLaunchKernelGGL(score_pool_kernel, dim3((a.span + kPoolTile - 1) / kPoolTile, njobs * wout),
                       dim3(kPoolThreads), 0, s, A, a.G, a.span, pooling, kernel, a.flags, scores);
    if ((rc = check_launch("hc_score(pool)"))) return rc;
  }
  return HC_OK;
}

template <typename T, bool STORE>
static int launch_score(ScoreArgs a, int njobs, int pooling, int kernel, float* scores, void* ws, uint32_t* hist,
                        hipStream_t s) {
  const int nchunks = (a.L + kScoreChunk - 1) / kScoreChunk;
  const int wout = (a.flags & HC_SCORE_SUM_WINDOW) ? 1 : a.W;
  float* part = reinterpret_cast<float*>(ws);
  float* stats = reinterpret_cast<float*>(reinterpret_cast<char*>(ws) +
                                          align256((size_t)njobs * nchunks * a.R * 2 * sizeof(float)));
  float* A = reinterpret_cast<float*>(reinterpret_cast<char*>(stats) + align256((size_t)njobs * a.R * 2 * sizeof(float)));
  const size_t qbytes = (size_t)a.NT * 16 * kQPitch * sizeof(T);
  const size_t lds1 = qbytes + (size_t)kScoreWaves * a.NT * 16 * 2 * sizeof(float);
  const bool via_logits = a.R < kLogitRows;
  const int rm = (a.flags & HC_SCORE_ROUND_BF16) ? 1 : (a.flags & HC_SCORE_ROUND_F16) ? 2 : 0;
  int nparts = 0;  // statistics partials per job: the stats grid's x extent
  if (!STORE && via_logits && a.R <= 16) {
#define HC_ROWS(NR, RM)                                                                                     \
  do {                                                                                                      \
    auto fn = score_rows_valu_kernel<T, NR, RM>;                                                            \
    ScoreArgs as = a;                                                                                       \
    nparts = plan_chunks(reinterpret_cast<const void*>(fn), 0, njobs, nchunks, as);                         \
    hipLaunchKernelGGL(fn, dim3(nparts, njobs), dim3(kScoreWaves * 64), 0, s, as, part, A);                 \
  } while (0)
#define HC_ROWS_RM(NR) \
  if (rm == 0) HC_ROWS(NR, 0); else if (rm == 1) HC_ROWS(NR, 1); else HC_ROWS(NR, 2);
    if (a.R <= 4) { HC_ROWS_RM(4) } else if (a.R <= 8) { HC_ROWS_RM(8) } else { HC_ROWS_RM(16) }
#undef HC_ROWS_RM
#undef HC_ROWS
  } else {
#define HC_STATS(RM, LG)                                                                                    \
  do {                                                                                                      \
    auto fn = score_stats_kernel<T, STORE, RM, LG>;                                                         \
    ScoreArgs as = a;                                                                                       \
    nparts = plan_chunks(reinterpret_cast<const void*>(fn), lds1, njobs, nchunks, as, !LG);                 \
    hipLaunchKernelGGL(fn, dim3(nparts, njobs), dim3(kScoreWaves * 64), lds1, s, as, part, LG ? A : nullptr); \
  } while (0)
  if (via_logits) {
    if (rm == 0) HC_STATS(0, true); else if (rm == 1) HC_STATS(1, true); else HC_STATS(2, true);
  } else {
    if (rm == 0) HC_STATS(0, false); else if (rm == 1) HC_STATS(1, false); else HC_STATS(2, false);
  }
#undef HC_STATS
  }
  int rc = check_launch("hc_score(stats)");
  if (rc) return rc;
  // The logit path's finish folds the partials itself, unless the merge
  // launch also has the histograms to clear.
  const bool fold_in_finish = via_logits && !hist;
  if (!fold_in_finish) {
    hipLaunchKernelGGL(score_stats_merge_kernel, dim3((njobs * a.R + 3) / 4), dim3(256), 0, s, part, nparts, a.R,
                       njobs, stats, hist, hist ? (int64_t)njobs * wout * kKeyDigitBins : (int64_t)0);
    if ((rc = check_launch("hc_score(merge)"))) return rc;
  }
  const float* fpart = fold_in_finish ? part : nullptr;
  if (via_logits) {
    if (a.span > 0) {
      const bool reg_pool = kernel == 5 || kernel == 7;
      const int ntiles = (a.span + (reg_pool ? kFinRegTile : kFinTile) - 1) / (reg_pool ? kFinRegTile : kFinTile);
      const int rows = njobs * wout;
      const int ht = reg_pool ? kFinRegHistTiles : kFinHistTiles;
      const int per_row = hist ? (ntiles + ht - 1) / ht : ntiles;
      const dim3 fgrid(per_row, rows);
      const int sum_w = (a.flags & HC_SCORE_SUM_WINDOW) ? 1 : 0;
      const int rmode = rm;
#define HC_FINISH2(RM, PL, HI)                                                                              \
  do {                                                                                                      \
    if (kernel == 5)                                                                                        \
      hipLaunchKernelGGL((score_finish_reg_kernel<RM, PL, HI, 2>), fgrid, dim3(256), 0, s, A, stats, fpart,   \
                         nparts, a.R,                                                                 \
                         a.G, a.W, a.span, sum_w, kernel, (a.flags & HC_SCORE_ACCUMULATE) ? 1 : 0, scores,    \
                         hist);                                                                             \
    else if (kernel == 7)                                                                                   \
      hipLaunchKernelGGL((score_finish_reg_kernel<RM, PL, HI, 3>), fgrid, dim3(256), 0, s, A, stats, fpart,   \
                         nparts, a.R,                                                                 \
                         a.G, a.W, a.span, sum_w, kernel, (a.flags & HC_SCORE_ACCUMULATE) ? 1 : 0, scores,    \
                         hist);                                                                             \
    else                                                                                                    \
      hipLaunchKernelGGL((score_finish_kernel<RM, PL, HI>), fgrid, dim3(256), 0, s, A, stats, fpart, nparts,  \
                         a.R, a.G, a.W,                                                               \
                         a.span, sum_w, kernel, (a.flags & HC_SCORE_ACCUMULATE) ? 1 : 0, scores, hist);      \
  } while (0)
#define HC_FINISH(RM, PL)          \
  do {                             \
    if (hist)                      \
      HC_FINISH2(RM, PL, true);    \
    else                           \
      HC_FINISH2(RM, PL, false);   \
  } while (0)
      if (rmode == 0) { if (pooling == 0) HC_FINISH(0, 0); else HC_FINISH(0, 1); }
      else if (rmode == 1) { if (pooling == 0) HC_FINISH(1, 0); else HC_FINISH(1, 1); }
      else { if (pooling == 0) HC_FINISH(2, 0); else HC_FINISH(2, 1); }
#undef HC_FINISH
#undef HC_FINISH2
      if ((rc = check_launch("hc_score(finish)"))) return rc;
    }
    return HC_OK;
  }
  return launch_probs_pool<T, STORE>(a, njobs, pooling, kernel, StatsView{stats, nullptr, 0}, A, scores, s);
}

// ---------------------------------------------------------------------------
// CAKE layer scoring (heterocache/kv_cluster.py:284-315).  From the window
// sum s1 and sum of squares s2 of the cast probabilities of one query head:
//   mean = s1 / W, var = unbiased variance over the W rows,
//   hh   = max_g avg_pool5(round(round(mean) + round(gamma * round(var)))),
//   entropy = -sum p log(p + 1e-10) and the variance sum over t < span,
// with the reference's casts (round) when its model dtype is 16-bit.
// ---------------------------------------------------------------------------
constexpr int kCakeThreads = 256;
constexpr int kCakeHalf = 2;  // avg_pool1d(kernel_size=5, padding=2), kv_cluster.py:309

template <int RM>
__device__ __forceinline__ float cake_var(float s1, float s2, int W) {
  return round_fixed<RM>(fmaxf(s2 - s1 * (s1 * (1.f / (float)W)), 0.f) / (float)(W - 1));
}

template <int RM>
__device__ __forceinline__ float cake_score(float s1, float s2, int W, float gamma) {
  const float mean = round_fixed<RM>(s1 * (1.f / (float)W));
  return round_fixed<RM>(mean + round_fixed<RM>(gamma * cake_var<RM>(s1, s2, W)));
}

// hh[job][t]: one workgroup per (job, 256 positions); each query head's
// scores plus the pooling halo are formed in LDS (zero outside [0, span)).
template <int RM>
__global__ __launch_bounds__(kCakeThreads) void cake_pool_kernel(const float* __restrict__ A1,
                                                                 const float* __restrict__ A2, int G, int W, int span,
                                                                 float gamma, float* __restrict__ S) {
  __shared__ float s_a[kCakeThreads + 2 * kCakeHalf];
  const int t0 = blockIdx.x * kCakeThreads, t = t0 + threadIdx.x;
  const int job = blockIdx.y;
  float best = -INFINITY;
  for (int g = 0; g < G; ++g) {
    const int64_t base = ((int64_t)job * G + g) * span;
    __syncthreads();
    for (int i = threadIdx.x; i < kCakeThreads + 2 * kCakeHalf; i += kCakeThreads) {
      const int u = t0 - kCakeHalf + i;
      s_a[i] = (u >= 0 && u < span) ? cake_score<RM>(A1[base + u], A2[base + u], W, gamma) : 0.f;
    }
    __syncthreads();
    float acc = 0.f;
#pragma unroll
    for (int d = 0; d <= 2 * kCakeHalf; ++d) acc += s_a[threadIdx.x + d];
    best = fmaxf(best, round_fixed<RM>(acc / (float)(2 * kCakeHalf + 1)));
  }
  if (t < span) S[(int64_t)job * span + t] = best;
}

// Variance sum in the reference's order: var[B][H][span].sum(0) (cast),
// .sum(0) over heads (cast), then over positions; one partial per 256
// positions.  Query head h of batch b is plane b*heads + h of A1 / A2.
template <int RM>
__global__ __launch_bounds__(kCakeThreads) void cake_varsum_kernel(const float* __restrict__ A1,
                                                                   const float* __restrict__ A2, int batch, int heads,
                                                                   int W, int span, float* __restrict__ part) {
  __shared__ float s_p[kCakeThreads / 64];
  const int t = blockIdx.x * kCakeThreads + threadIdx.x;
  float y = 0.f;
  if (t < span) {
    for (int h = 0; h < heads; ++h) {
      float x = 0.f;
      for (int b = 0; b < batch; ++b) {
        const int64_t o = ((int64_t)b * heads + h) * span + t;
        x += cake_var<RM>(A1[o], A2[o], W);
      }
      y += round_fixed<RM>(x);
    }
    y = round_fixed<RM>(y);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) y += __shfl_xor(y, off, 64);
  if ((threadIdx.x & 63) == 0) s_p[threadIdx.x >> 6] = y;
  __syncthreads();
  if (threadIdx.x == 0) part[blockIdx.x] = (s_p[0] + s_p[1]) + (s_p[2] + s_p[3]);
}

// out = {entropy, variance sum, preference}; preference = entropy * variance
// sum, or 0 when either is NaN (kv_cluster.py:297-303, tau1 = tau2 = 1).
template <int RM>
__global__ __launch_bounds__(kCakeThreads) void cake_final_kernel(const float* __restrict__ ent, int n_ent,
                                                                  const float* __restrict__ part, int n_part,
                                                                  float* __restrict__ out) {
  __shared__ float s_e[kCakeThreads / 64], s_v[kCakeThreads / 64];
  float e = 0.f, v = 0.f;
  for (int i = threadIdx.x; i < n_ent; i += kCakeThreads) e += ent[i];
  for (int i = threadIdx.x; i < n_part; i += kCakeThreads) v += part[i];
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    e += __shfl_xor(e, off, 64);
    v += __shfl_xor(v, off, 64);
  }
  if ((threadIdx.x & 63) == 0) {
    s_e[threadIdx.x >> 6] = e;
    s_v[threadIdx.x >> 6] = v;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    const float disp = -((s_e[0] + s_e[1]) + (s_e[2] + s_e[3]));
    const float var = round_fixed<RM>((s_v[0] + s_v[1]) + (s_v[2] + s_v[3]));
    out[0] = disp;
    out[1] = var;
    out[2] = (isnan(disp) || isnan(var)) ? 0.f : disp * var;
  }
}

size_t cake_workspace_bytes(int njobs, int L, int G, int W) {
  const int R = G * W;
  const size_t nchunks = (L + kScoreChunk - 1) / kScoreChunk;
  const size_t span = L - W, nspan = (span + kScoreChunk - 1) / kScoreChunk;
  return align256(njobs * nchunks * R * 2 * sizeof(float)) + align256((size_t)njobs * R * 2 * sizeof(float)) +
         2 * align256((size_t)njobs * G * span * sizeof(float)) + align256(njobs * nspan * sizeof(float)) +
         align256(nspan * sizeof(float));
}

template <typename T, int RM>
static int launch_cake(ScoreArgs a, int njobs, int batch, int heads, float gamma, float* scores, float* out, void* ws,
                       hipStream_t s) {
  const int nchunks = (a.L + kScoreChunk - 1) / kScoreChunk;
  const int nspan = (a.span + kScoreChunk - 1) / kScoreChunk;
  char* w = reinterpret_cast<char*>(ws);
  float* part = reinterpret_cast<float*>(w);
  w += align256((size_t)njobs * nchunks * a.R * 2 * sizeof(float));
  float* stats = reinterpret_cast<float*>(w);
  w += align256((size_t)njobs * a.R * 2 * sizeof(float));
  float* A1 = reinterpret_cast<float*>(w);
  w += align256((size_t)njobs * a.G * a.span * sizeof(float));
  float* A2 = reinterpret_cast<float*>(w);
  w += align256((size_t)njobs * a.G * a.span * sizeof(float));
  float* ent = reinterpret_cast<float*>(w);
  w += align256((size_t)njobs * nspan * sizeof(float));
  float* vpart = reinterpret_cast<float*>(w);
  const size_t qbytes = (size_t)a.NT * 16 * kQPitch * sizeof(T);
  const size_t lds1 = qbytes + (size_t)kScoreWaves * a.NT * 16 * 2 * sizeof(float);
  const size_t lds3 = qbytes + (size_t)a.NT * 16 * 2 * sizeof(float);
  int rc;
  auto fstats = score_stats_kernel<T, false, RM, false>;
  ScoreArgs as = a;
  const int nparts = plan_chunks(reinterpret_cast<const void*>(fstats), lds1, njobs, nchunks, as);
  hipLaunchKernelGGL(fstats, dim3(nparts, njobs), dim3(kScoreWaves * 64), lds1, s, as, part, nullptr);
  if ((rc = check_launch("hc_cake_score(stats)"))) return rc;
  hipLaunchKernelGGL(score_stats_merge_kernel, dim3((njobs * a.R + 3) / 4), dim3(256), 0, s, part, nparts, a.R,
                     njobs, stats, (uint32_t*)nullptr, (int64_t)0);
  if ((rc = check_launch("hc_cake_score(merge)"))) return rc;
  auto fprobs = score_probs_kernel<T, false, RM, kWin16, true>;
  ScoreArgs ap = a;
  const int nprob = plan_chunks(reinterpret_cast<const void*>(fprobs), lds3, njobs, nspan, ap);
  hipLaunchKernelGGL(fprobs, dim3(nprob, njobs), dim3(kScoreWaves * 64), lds3, s, ap, StatsView{stats, nullptr, 0}, A1,
                     A2, ent);
  if ((rc = check_launch("hc_cake_score(probs)"))) return rc;
  hipLaunchKernelGGL((cake_pool_kernel<RM>), dim3((a.span + kCakeThreads - 1) / kCakeThreads, njobs),
                     dim3(kCakeThreads), 0, s, A1, A2, a.G, a.W, a.span, gamma, scores);
  if ((rc = check_launch("hc_cake_score(pool)"))) return rc;
  const int nvar = (a.span + kCakeThreads - 1) / kCakeThreads;
  hipLaunchKernelGGL((cake_varsum_kernel<RM>), dim3(nvar), dim3(kCakeThreads), 0, s, A1, A2, batch, heads, a.W,
                     a.span, vpart);
  if ((rc = check_launch("hc_cake_score(varsum)"))) return rc;
  hipLaunchKernelGGL((cake_final_kernel<RM>), dim3(1), dim3(kCakeThreads), 0, s, ent, njobs * nprob, vpart, nvar,
                     out);
  return check_launch("hc_cake_score(final)");
}

}  // namespace hc

using namespace hc;

extern "C" size_t hc_score_workspace_size(int njobs, int seq_len, int group, int window, int flags) {
  if (njobs <= 0 || seq_len <= 0 || group <= 0 || window <= 0) return 0;
  return score_workspace_bytes(njobs, seq_len, group, window, flags);
}

extern "C" int hc_score(int dtype, const void* q, const int64_t* q_off, int64_t q_head_stride, int64_t q_row_stride,
                        const void* k, const int64_t* k_off, int64_t k_tok_stride, const int64_t* row_tile_off,
                        const int32_t* k_row, int njobs, int seq_len, int group, int window, int flags, int span,
                        int pooling, int kernel, float scale, float* scores, void* workspace,
                        size_t workspace_bytes, uint32_t* hist, void* stream) {
  clear_error();
  if (njobs < 0 || njobs > 65535 || seq_len < 0 || group < 1 || window < 1)
    return set_error(HC_ERR_INVALID, "hc_score: njobs=%d seq_len=%d group=%d window=%d", njobs, seq_len, group,
                     window);
  if (njobs == 0 || seq_len == 0) return HC_OK;
  const bool sum_w = (flags & HC_SCORE_SUM_WINDOW) != 0;
  if (sum_w && window >= 16 ? (window % 16) != 0 : (sum_w && (window & (window - 1)) != 0))
    return set_error(HC_ERR_INVALID, "hc_score: a summed window must be 1, 2, 4, 8 or a multiple of 16 (got %d)",
                     window);
  if (span < 0 || span > seq_len) return set_error(HC_ERR_INVALID, "hc_score: span %d outside [0, %d]", span, seq_len);
  if (pooling != 0 && pooling != 1) return set_error(HC_ERR_INVALID, "hc_score: pooling must be 0 (avg) or 1 (max)");
  if (kernel < 1 || (kernel % 2) == 0 || kernel > kPoolMaxKernel)
    return set_error(HC_ERR_INVALID, "hc_score: pooling kernel must be odd and <= %d (got %d)", kPoolMaxKernel, kernel);
  const int R = group * window;
  if ((int64_t)njobs * ((flags & HC_SCORE_SUM_WINDOW) ? 1 : window) > 65535)
    return set_error(HC_ERR_INVALID, "hc_score: njobs x window rows %lld exceed 65535",
                     (long long)njobs * window);
  int NT = (R + 15) / 16;
  if (NT > 16) return set_error(HC_ERR_INVALID, "hc_score: group*window = %d exceeds 256 rows", R);
  if (dtype == HC_DTYPE_F32 && NT > 8)
    return set_error(HC_ERR_INVALID, "hc_score: float32 supports group*window <= 128 (got %d)", R);
  if (!q || !q_off || !k || !scores || !workspace)
    return set_error(HC_ERR_INVALID, "hc_score: null pointer argument");
  const bool store = row_tile_off != nullptr;
  if (store ? !k_row : !k_off) return set_error(HC_ERR_INVALID, "hc_score: missing key addressing");
  if (!store && (k_tok_stride < HC_HEAD_DIM || (k_tok_stride % 8) != 0))
    return set_error(HC_ERR_INVALID, "hc_score: key token stride %lld", (long long)k_tok_stride);
  if (workspace_bytes < score_workspace_bytes(njobs, seq_len, group, window, flags))
    return set_error(HC_ERR_INVALID, "hc_score: workspace too small");
  if (hist && (R >= kLogitRows || (flags & HC_SCORE_ACCUMULATE)))
    return set_error(HC_ERR_INVALID, "hc_score: a score histogram needs fewer than %d query rows and no accumulation",
                     kLogitRows);
  ScoreArgs a;
  a.q = q;
  a.q_off = q_off;
  a.q_head_stride = q_head_stride;
  a.q_row_stride = q_row_stride;
  a.k = k;
  a.k_off = k_off;
  a.k_tok_stride = k_tok_stride;
  a.row_tile_off = row_tile_off;
  a.k_row = k_row;
  a.L = seq_len;
  a.G = group;
  a.W = window;
  a.R = R;
  a.NT = NT;
  a.flags = flags;
  a.span = span;
  a.scale = scale;
  a.scale2 = scale * 1.4426950408889634f;
  a.cpw = 1;
  hipStream_t s = (hipStream_t)stream;
#define HC_SCORE_DISPATCH(T)                                                                          \
  return store ? launch_score<T, true>(a, njobs, pooling, kernel, scores, workspace, hist, s)         \
               : launch_score<T, false>(a, njobs, pooling, kernel, scores, workspace, hist, s);
  switch (dtype) {
    case HC_DTYPE_BF16: { HC_SCORE_DISPATCH(__bf16) }
    case HC_DTYPE_F16: { HC_SCORE_DISPATCH(_Float16) }
    case HC_DTYPE_F32: { HC_SCORE_DISPATCH(float) }
    default:
      return set_error(HC_ERR_INVALID, "hc_score: unknown dtype %d", dtype);
  }
#undef HC_SCORE_DISPATCH
}

template <typename T, int POOL, int P, int RM>
static int launch_given_stats(ScoreArgs a, int njobs, const float* stats, const int64_t* st_off, float* scores,
                              hipStream_t s) {
  const int nchunks = (a.L + kScoreChunk - 1) / kScoreChunk;
  const size_t lds =
      (size_t)a.NT * 16 * kQPitch * sizeof(T) + (size_t)a.R * (kGsPitch + 2 * kGsMPitch) * sizeof(float);
  auto fn = score_given_stats_kernel<T, true, POOL, P, RM>;
  const int gx = plan_chunks(reinterpret_cast<const void*>(fn), lds, njobs, nchunks, a);
  hipLaunchKernelGGL(fn, dim3(gx, njobs), dim3(kScoreWaves * 64), lds, s, a, stats, st_off, scores);
  return check_launch("hc_score_given_stats");
}

template <typename T, int RM>
static int dispatch_given_stats(const ScoreArgs& a, int njobs, int pooling, int kernel, const float* stats,
                                const int64_t* st_off, float* scores, hipStream_t s) {
#define HC_GS(PL)                                                                              \
  switch (kernel / 2) {                                                                        \
    case 0: return launch_given_stats<T, PL, 0, RM>(a, njobs, stats, st_off, scores, s);  \
    case 1: return launch_given_stats<T, PL, 1, RM>(a, njobs, stats, st_off, scores, s);  \
    case 2: return launch_given_stats<T, PL, 2, RM>(a, njobs, stats, st_off, scores, s);  \
    case 3: return launch_given_stats<T, PL, 3, RM>(a, njobs, stats, st_off, scores, s);  \
    default: return launch_given_stats<T, PL, 4, RM>(a, njobs, stats, st_off, scores, s); \
  }
  if (pooling == 0) { HC_GS(0) } else { HC_GS(1) }
#undef HC_GS
}

// Rounding mode of the flags' cast chain (0: the uncast chain).
template <typename T>
static int dispatch_given_stats_flags(const ScoreArgs& a, int njobs, int pooling, int kernel, int flags,
                                      const float* stats, const int64_t* st_off, float* scores, hipStream_t s) {
  if (flags == HC_SCORE_ROUND_BF16) return dispatch_given_stats<T, 1>(a, njobs, pooling, kernel, stats, st_off, scores, s);
  if (flags == HC_SCORE_ROUND_F16) return dispatch_given_stats<T, 2>(a, njobs, pooling, kernel, stats, st_off, scores, s);
  return dispatch_given_stats<T, 0>(a, njobs, pooling, kernel, stats, st_off, scores, s);
}

extern "C" int hc_score_given_stats(int dtype, const void* q, const int64_t* q_off, int64_t q_head_stride,
                                    int64_t q_row_stride, const void* kstore, const int64_t* row_tile_off,
                                    const int32_t* k_row, int njobs, int seq_len, int group, int window, int flags,
                                    int pooling, int kernel, float scale, const float* stats, const int64_t* stat_off,
                                    float* scores, void* stream) {
  clear_error();
  if (njobs < 0 || njobs > 65535 || seq_len < 0 || group < 1 || window < 1)
    return set_error(HC_ERR_INVALID, "hc_score_given_stats: njobs=%d seq_len=%d group=%d window=%d", njobs, seq_len,
                     group, window);
  if (njobs == 0 || seq_len == 0) return HC_OK;
  const int R = group * window;
  if (R >= kLogitRowsMax)
    return set_error(HC_ERR_INVALID, "hc_score_given_stats: group*window = %d, at most %d rows", R, kLogitRowsMax - 1);
  if (pooling != 0 && pooling != 1)
    return set_error(HC_ERR_INVALID, "hc_score_given_stats: pooling must be 0 (avg) or 1 (max)");
  if (flags != 0 && flags != HC_SCORE_ROUND_BF16 && flags != HC_SCORE_ROUND_F16)
    return set_error(HC_ERR_INVALID, "hc_score_given_stats: flags=%d (0, HC_SCORE_ROUND_BF16 or _F16)", flags);
  if (kernel < 1 || (kernel % 2) == 0 || kernel / 2 > 4)
    return set_error(HC_ERR_INVALID, "hc_score_given_stats: pooling kernel must be 1, 3, 5, 7 or 9 (got %d)", kernel);
  if (!q || !q_off || !kstore || !row_tile_off || !k_row || !stats || !stat_off || !scores)
    return set_error(HC_ERR_INVALID, "hc_score_given_stats: null pointer argument");
  ScoreArgs a;
  a.q = q;
  a.q_off = q_off;
  a.q_head_stride = q_head_stride;
  a.q_row_stride = q_row_stride;
  a.k = kstore;
  a.k_off = nullptr;
  a.k_tok_stride = 0;
  a.row_tile_off = row_tile_off;
  a.k_row = k_row;
  a.L = seq_len;
  a.G = group;
  a.W = window;
  a.R = R;
  a.NT = (R + 15) / 16;
  a.flags = 0;
  a.span = seq_len;
  a.scale = scale;
  a.scale2 = scale * 1.4426950408889634f;
  a.cpw = 1;
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case HC_DTYPE_BF16:
      return dispatch_given_stats_flags<__bf16>(a, njobs, pooling, kernel, flags, stats, stat_off, scores, s);
    case HC_DTYPE_F16:
      return dispatch_given_stats_flags<_Float16>(a, njobs, pooling, kernel, flags, stats, stat_off, scores, s);
    case HC_DTYPE_F32:
      return dispatch_given_stats_flags<float>(a, njobs, pooling, kernel, flags, stats, stat_off, scores, s);
    default: return set_error(HC_ERR_INVALID, "hc_score_given_stats: unknown dtype %d", dtype);
  }
}

extern "C" int hc_score_with_stats(int dtype, const void* q, const int64_t* q_off, int64_t q_head_stride,
                                   int64_t q_row_stride, const void* k, const int64_t* k_off, int64_t k_tok_stride,
                                   const int64_t* row_tile_off, const int32_t* k_row, int njobs, int seq_len,
                                   int group, int window, int flags, int span, int pooling, int kernel, float scale,
                                   const float* stats, const int64_t* stat_off, int64_t stat_head_stride,
                                   float* scores, void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  if (njobs < 0 || njobs > 65535 || seq_len < 0 || group < 1 || window < 1)
    return set_error(HC_ERR_INVALID, "hc_score_with_stats: njobs=%d seq_len=%d group=%d window=%d", njobs, seq_len,
                     group, window);
  if (njobs == 0 || seq_len == 0) return HC_OK;
  if (flags & ~(HC_SCORE_CAUSAL_WINDOW | HC_SCORE_SUM_WINDOW | HC_SCORE_ACCUMULATE))
    return set_error(HC_ERR_INVALID,
                     "hc_score_with_stats: flags 0x%x (the given statistics are of unrounded logits: no rounding "
                     "flag)",
                     flags);
  const bool sum_w = (flags & HC_SCORE_SUM_WINDOW) != 0;
  if (sum_w && window >= 16 ? (window % 16) != 0 : (sum_w && (window & (window - 1)) != 0))
    return set_error(HC_ERR_INVALID,
                     "hc_score_with_stats: a summed window must be 1, 2, 4, 8 or a multiple of 16 (got %d)", window);
  if (span < 0 || span > seq_len)
    return set_error(HC_ERR_INVALID, "hc_score_with_stats: span %d outside [0, %d]", span, seq_len);
  if (pooling != 0 && pooling != 1)
    return set_error(HC_ERR_INVALID, "hc_score_with_stats: pooling must be 0 (avg) or 1 (max)");
  if (kernel < 1 || (kernel % 2) == 0 || kernel > kPoolMaxKernel)
    return set_error(HC_ERR_INVALID, "hc_score_with_stats: pooling kernel must be odd and <= %d (got %d)",
                     kPoolMaxKernel, kernel);
  const int R = group * window;
  const int wout = sum_w ? 1 : window;
  if ((int64_t)njobs * wout > 65535)
    return set_error(HC_ERR_INVALID, "hc_score_with_stats: njobs x window rows %lld exceed 65535",
                     (long long)njobs * wout);
  const int NT = (R + 15) / 16;
  if (NT > 16) return set_error(HC_ERR_INVALID, "hc_score_with_stats: group*window = %d exceeds 256 rows", R);
  if (dtype == HC_DTYPE_F32 && NT > 8)
    return set_error(HC_ERR_INVALID, "hc_score_with_stats: float32 supports group*window <= 128 (got %d)", R);
  if (!q || !q_off || !k || !stats || !scores || (span > 0 && !workspace))
    return set_error(HC_ERR_INVALID, "hc_score_with_stats: null pointer argument");
  if (stat_head_stride < 0 || (stat_head_stride > 0 && stat_head_stride < 2 * (int64_t)window))
    return set_error(HC_ERR_INVALID, "hc_score_with_stats: stat_head_stride %lld (0, or >= 2 * window)",
                     (long long)stat_head_stride);
  const bool store = row_tile_off != nullptr;
  if (store ? !k_row : !k_off) return set_error(HC_ERR_INVALID, "hc_score_with_stats: missing key addressing");
  if (!store && (k_tok_stride < HC_HEAD_DIM || (k_tok_stride % 8) != 0))
    return set_error(HC_ERR_INVALID, "hc_score_with_stats: key token stride %lld", (long long)k_tok_stride);
  if (workspace_bytes < (size_t)njobs * wout * group * span * sizeof(float))
    return set_error(HC_ERR_INVALID, "hc_score_with_stats: workspace too small");
  ScoreArgs a;
  a.q = q;
  a.q_off = q_off;
  a.q_head_stride = q_head_stride;
  a.q_row_stride = q_row_stride;
  a.k = k;
  a.k_off = k_off;
  a.k_tok_stride = k_tok_stride;
  a.row_tile_off = row_tile_off;
  a.k_row = k_row;
  a.L = seq_len;
  a.G = group;
  a.W = window;
  a.R = R;
  a.NT = NT;
  a.flags = flags;
  a.span = span;
  a.scale = scale;
  a.scale2 = scale * 1.4426950408889634f;
  a.cpw = 1;
  const StatsView sv{stats, stat_off, stat_head_stride};
  float* A = reinterpret_cast<float*>(workspace);
  hipStream_t s = (hipStream_t)stream;
#define HC_WS_DISPATCH(T)                                                                            \
  return store ? launch_probs_pool<T, true>(a, njobs, pooling, kernel, sv, A, scores, s)            \
               : launch_probs_pool<T, false>(a, njobs, pooling, kernel, sv, A, scores, s);
  switch (dtype) {
    case HC_DTYPE_BF16: { HC_WS_DISPATCH(__bf16) }
    case HC_DTYPE_F16: { HC_WS_DISPATCH(_Float16) }
    case HC_DTYPE_F32: { HC_WS_DISPATCH(float) }
    default:
      return set_error(HC_ERR_INVALID, "hc_score_with_stats: unknown dtype %d", dtype);
  }
#undef HC_WS_DISPATCH
}

extern "C" size_t hc_cake_workspace_size(int batch, int kv_heads, int seq_len, int group, int window) {
  if (batch <= 0 || kv_heads <= 0 || group <= 0 || window <= 0 || seq_len <= window) return 0;
  return cake_workspace_bytes(batch * kv_heads, seq_len, group, window);
}

extern "C" int hc_cake_score(int dtype, const void* q, const int64_t* q_off, int64_t q_head_stride,
                             int64_t q_row_stride, const void* k, const int64_t* k_off, int64_t k_tok_stride,
                             int batch, int kv_heads, int seq_len, int group, int window, int flags, float scale,
                             float gamma, float* scores, float* stats_out, void* workspace, size_t workspace_bytes,
                             void* stream) {
  clear_error();
  if (batch < 1 || kv_heads < 1 || group < 1 || (int64_t)batch * kv_heads > 65535)
    return set_error(HC_ERR_INVALID, "hc_cake_score: batch=%d kv_heads=%d group=%d", batch, kv_heads, group);
  if (window < 16 || (window % 16) != 0)
    return set_error(HC_ERR_INVALID, "hc_cake_score: the window must be a positive multiple of 16 (got %d)", window);
  if (seq_len <= window)
    return set_error(HC_ERR_INVALID, "hc_cake_score: seq_len %d must exceed the window %d", seq_len, window);
  if ((flags & ~(HC_SCORE_ROUND_BF16 | HC_SCORE_ROUND_F16)) != 0 ||
      (flags & (HC_SCORE_ROUND_BF16 | HC_SCORE_ROUND_F16)) == (HC_SCORE_ROUND_BF16 | HC_SCORE_ROUND_F16))
    return set_error(HC_ERR_INVALID, "hc_cake_score: flags 0x%x (only one rounding flag is accepted)", flags);
  if (!(scale > 0.f) || !std::isfinite(gamma))
    return set_error(HC_ERR_INVALID, "hc_cake_score: scale %g, gamma %g", (double)scale, (double)gamma);
  const int R = group * window;
  const int NT = (R + 15) / 16;
  if (NT > 16) return set_error(HC_ERR_INVALID, "hc_cake_score: group*window = %d exceeds 256 rows", R);
  if (dtype == HC_DTYPE_F32 && NT > 8)
    return set_error(HC_ERR_INVALID, "hc_cake_score: float32 supports group*window <= 128 (got %d)", R);
  if (!q || !q_off || !k || !k_off || !scores || !stats_out || !workspace)
    return set_error(HC_ERR_INVALID, "hc_cake_score: null pointer argument");
  if (k_tok_stride < HC_HEAD_DIM || (k_tok_stride % 8) != 0)
    return set_error(HC_ERR_INVALID, "hc_cake_score: key token stride %lld", (long long)k_tok_stride);
  const int njobs = batch * kv_heads;
  if (workspace_bytes < cake_workspace_bytes(njobs, seq_len, group, window))
    return set_error(HC_ERR_INVALID, "hc_cake_score: workspace too small");
  ScoreArgs a;
  a.q = q;
  a.q_off = q_off;
  a.q_head_stride = q_head_stride;
  a.q_row_stride = q_row_stride;
  a.k = k;
  a.k_off = k_off;
  a.k_tok_stride = k_tok_stride;
  a.row_tile_off = nullptr;
  a.k_row = nullptr;
  a.L = seq_len;
  a.G = group;
  a.W = window;
  a.R = R;
  a.NT = NT;
  a.flags = flags | HC_SCORE_CAUSAL_WINDOW | HC_SCORE_SUM_WINDOW;
  a.span = seq_len - window;
  a.scale = scale;
  a.scale2 = scale * 1.4426950408889634f;
  a.cpw = 1;
  hipStream_t s = (hipStream_t)stream;
  const int rm = (flags & HC_SCORE_ROUND_BF16) ? 1 : (flags & HC_SCORE_ROUND_F16) ? 2 : 0;
  const int heads = kv_heads * group;
#define HC_CAKE_DISPATCH(T)                                                                          \
  return rm == 0   ? launch_cake<T, 0>(a, njobs, batch, heads, gamma, scores, stats_out, workspace, s) \
         : rm == 1 ? launch_cake<T, 1>(a, njobs, batch, heads, gamma, scores, stats_out, workspace, s) \
                   : launch_cake<T, 2>(a, njobs, batch, heads, gamma, scores, stats_out, workspace, s);
  switch (dtype) {
    case HC_DTYPE_BF16: { HC_CAKE_DISPATCH(__bf16) }
    case HC_DTYPE_F16: { HC_CAKE_DISPATCH(_Float16) }
    case HC_DTYPE_F32: { HC_CAKE_DISPATCH(float) }
    default:
      return set_error(HC_ERR_INVALID, "hc_cake_score: unknown dtype %d", dtype);
  }
#undef HC_CAKE_DISPATCH
}
