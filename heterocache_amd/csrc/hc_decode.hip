// Split-K GQA flash-decode over the ragged per-head tiled KV store.
//
// Replaces the paged `flash_attn_with_kvcache(q, k_pool, v_pool,
// cache_seqlens, block_table, causal=False)` call of the reference decode
// step (heterocache/llama_model.py:382-389, heterocache/qwen_model.py:194-201)
// and, optionally, the decode-token append that precedes it
// (heterocache/cache_utils.py:970-1005).
//
// Two back-to-back launches per layer and step, no cross-workgroup
// synchronisation inside a kernel (an agent-scope fence costs an L2
// write-back per workgroup on a multi-XCD part):
//  * decode_partial_kernel: every row (batch, kv-head) is cut into chunks of
//    chunk_tiles 32-token tiles, one workgroup per chunk (its NWAVES waves
//    split the chunk evenly), rows
//    visited in row_order (longest first).  Each wave streams its run of
//    tiles with nontemporal loads, computes S = K.Q^T on the matrix cores
//    (the G query heads of the group share every K load), an online base-2
//    softmax and O^T += V^T.P^T on the matrix cores; the waves' states are
//    combined through LDS into one (m, l, O) partial per workgroup.
//  * decode_merge_kernel: one workgroup per (row, query, 32-channel slice)
//    folds the row's partials.
//  * with k_new/v_new the new token is attended at slot len by the wave
//    owning that slot (folded into its softmax state after its stored
//    tiles) and written into the store by that wave; the merge advances
//    row_len by one.
#include <mutex>

#include "hc_common.h"
#include "hc_internal.h"

namespace hc {

struct ChunkLoc {
  int row;        // store row
  int chunk;      // chunk index inside the row
  int len;        // tokens attended (stored length, +1 with a fused append)
  int nparts;     // chunks of the row
  int p0;         // global part index of the row's first chunk
  int total;      // chunks of all rows
  int64_t tiles;  // first tile of the row in the store (row_tile_off[row])
  bool found;
  bool full;      // a fused append was asked for but the row is at capacity
};

__device__ __forceinline__ int chunks_of(int len, int chunk_tiles) {
  const int nt = (len + HC_TILE - 1) / HC_TILE;
  // An empty row still gets one workgroup, which writes its zero output.
  return nt > 0 ? (nt + chunk_tiles - 1) / chunk_tiles : 1;
}

__device__ __forceinline__ int wave_inclusive_scan(int v, int lane) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int u = __shfl_up(v, d, 64);
    if (lane >= d) v += u;
  }
  return v;
}

// Map workgroup index b onto (row, chunk) from the device-resident lengths.
// Each wave scans the rows 64 at a time, one row per lane: the per-row loads
// of a block are issued together (for up to 64 rows, row_order, row_len,
// row_cap and row_tile_off are all read in one round trip and the order is
// applied by a lane permute), so locating costs one or two memory latencies,
// not one per row.  With a fused append (extra = 1) a row attends one more
// token unless it is at capacity (row_cap), in which case it is marked full
// and attends nothing new.
__device__ __forceinline__ ChunkLoc locate_chunk(const int* __restrict__ row_len, const int* __restrict__ row_cap,
                                                 const int* __restrict__ row_order,
                                                 const int64_t* __restrict__ row_tile_off, int rows, int extra,
                                                 int chunk_tiles, int b) {
  const int lane = threadIdx.x & 63;
  ChunkLoc c;
  c.found = false;
  c.full = false;
  c.row = 0;
  c.chunk = 0;
  c.len = 0;
  c.nparts = 0;
  c.p0 = 0;
  c.tiles = 0;
  int acc = 0;
  if (rows <= 64) {
    const bool live = lane < rows;
    const int own_len = live ? row_len[lane] : 0;
    const int own_cap = (live && extra) ? row_cap[lane] : 0;
    const int64_t own_off = live ? row_tile_off[lane] : 0;
    const int r = live ? (row_order ? row_order[lane] : lane) : 0;
    const int own_ext = (extra && own_len < own_cap) ? 1 : 0;
    const int l = __shfl(own_len + own_ext, r, 64);
    const int fl = __shfl(extra - own_ext, r, 64);
    const int nc = live ? chunks_of(l, chunk_tiles) : 0;
    const int incl = wave_inclusive_scan(nc, lane);
    const int excl = incl - nc;
    const uint64_t hit = __ballot(live && b >= excl && b < incl);
    acc = __shfl(incl, 63, 64);
    if (hit) {
      const int src = __builtin_ctzll(hit);
      c.found = true;
      c.row = __shfl(r, src, 64);
      c.len = __shfl(l, src, 64);
      c.full = __shfl(fl, src, 64) != 0;
      c.nparts = __shfl(nc, src, 64);
      c.p0 = __shfl(excl, src, 64);
      c.chunk = b - c.p0;
      c.tiles = __shfl(own_off, c.row, 64);
    }
  } else {
    for (int base = 0; base < rows; base += 64) {
      const int k = base + lane;
      const bool live = k < rows;
      const int r = live ? (row_order ? row_order[k] : k) : 0;
      const int len0 = live ? row_len[r] : 0;
      const int ext = (live && extra && len0 < row_cap[r]) ? 1 : 0;
      const int l = len0 + ext;
      const int fl = live ? extra - ext : 0;
      const int nc = live ? chunks_of(l, chunk_tiles) : 0;
      const int incl = acc + wave_inclusive_scan(nc, lane);
      const int excl = incl - nc;
      const uint64_t hit = __ballot(live && b >= excl && b < incl);
      if (hit && !c.found) {
        const int src = __builtin_ctzll(hit);
        c.found = true;
        c.row = __shfl(r, src, 64);
        c.len = __shfl(l, src, 64);
        c.full = __shfl(fl, src, 64) != 0;
        c.nparts = __shfl(nc, src, 64);
        c.p0 = __shfl(excl, src, 64);
        c.chunk = b - c.p0;
      }
      acc = __shfl(incl, 63, 64);
    }
    if (c.found) c.tiles = row_tile_off[c.row];
  }
  c.total = acc;
  return c;
}

// Request the K and V parts of tile t (16 wave-loads of 1 KB, contiguous).
template <typename T>
__device__ __forceinline__ void load_tile(typename Elem<T>::vec8 (&kr)[8], typename Elem<T>::vec8 (&vr)[8],
                                          const T* __restrict__ kb, const T* __restrict__ vb, int t) {
#pragma unroll
  for (int x = 0; x < 8; ++x) {
    kr[x] = load8_stream<T>(kb + (int64_t)t * HC_TILE_ELEMS + x * 512);
    vr[x] = load8_stream<T>(vb + (int64_t)t * HC_TILE_ELEMS + x * 512);
  }
}

// Attend the resident tile t: S^T = K.Q^T on the matrix cores, mask of the
// tokens at or beyond len, online base-2 softmax, O^T += V^T.P^T.  Lane
// state: m_run is the running maximum of query n = lane%16 (scaled, base 2),
// l_run this lane's share of the running sum, o[mt][j] = O^T[16mt+4g+j][n].
// STATS: (m_snap, l_snap) also follow the state over the tokens below
// stat_len only (see decode_partial_kernel).  RM (a rounding mode of
// round_fixed, with STATS): that state is the one of the reference's cast
// chain instead, x = round(round(q.k) * scale) * log2(e), which the
// attention itself does not use.
template <typename T, bool STATS, int RM = 0>
__device__ __forceinline__ void attend_tile(typename Elem<T>::vec8 (&kr)[8], typename Elem<T>::vec8 (&vr)[8],
                                            const typename Elem<T>::vec8 (&qreg)[4], int t, int len, int lane,
                                            float scale_log2, float& m_run, float& l_run, f32x4 (&o)[8],
                                            int stat_len, float& m_snap, float& l_snap, float scale = 0.f) {
  typedef typename Elem<T>::vec8 vec8;
  const int g = lane >> 4;
  const int tok0 = t * HC_TILE;
  // S^T(token, query) for the two 16-token halves of the tile.
  f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    s0 = mma_16x16x32(kr[s], qreg[s], s0);
    s1 = mma_16x16x32(kr[4 + s], qreg[s], s1);
  }
  // Element e of this lane holds token 16*(e/4) + 4g + e%4 of the tile.
  float sv[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
  if (tok0 + HC_TILE > len) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int tok = tok0 + 16 * (e >> 2) + 4 * g + (e & 3);
      if (tok >= len) sv[e] = -INFINITY;
    }
#pragma unroll
    for (int mt = 0; mt < 8; ++mt) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int tok = tok0 + 16 * (e >> 2) + 4 * g + (e & 3);
        if (tok >= len) {
          if constexpr (sizeof(T) == 4) {
            if (e < 4) vr[mt].lo[e] = 0.f; else vr[mt].hi[e - 4] = 0.f;
          } else {
            vr[mt][e] = Elem<T>::from_f32(0.f);
          }
        }
      }
    }
  }
  float mx = sv[0];
#pragma unroll
  for (int e = 1; e < 8; ++e) mx = fmaxf(mx, sv[e]);
  mx = rows4_max(mx);
  const float m_new = fmaxf(m_run, mx * scale_log2);
  const float alpha = fast_exp2(m_run - m_new);
  float p[8];
  float psum = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    p[e] = fast_exp2(fmaf(sv[e], scale_log2, -m_new));
    psum += p[e];
  }
  if constexpr (STATS && RM != 0) {
    // The cast chain's own online state over the tile's tokens below
    // stat_len (masked tokens are -inf already, and stay so).
    if (tok0 < stat_len) {
      float xs[8];
      float mxs = -INFINITY;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int tok = tok0 + 16 * (e >> 2) + 4 * g + (e & 3);
        xs[e] = tok < stat_len ? round_fixed<RM>(round_fixed<RM>(sv[e]) * scale) * 1.4426950408889634f : -INFINITY;
        mxs = fmaxf(mxs, xs[e]);
      }
      mxs = rows4_max(mxs);
      const float mn = fmaxf(m_snap, mxs);
      if (mn != -INFINITY) {
        float ps = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) ps += fast_exp2(xs[e] - mn);
        l_snap = fmaf(l_snap, fast_exp2(m_snap - mn), ps);
        m_snap = mn;
      }
    }
  } else if constexpr (STATS) {
    // Tiles are visited in increasing order, so while every tile so far lies
    // below stat_len the snapshot is the running state itself; the tile
    // that crosses stat_len adds only its tokens below it (against the new
    // maximum, which bounds them); later tiles leave it alone.
    if (tok0 + HC_TILE <= stat_len) {
      m_snap = m_new;
      l_snap = fmaf(l_run, alpha, psum);
    } else if (tok0 < stat_len) {
      float ps = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (tok0 + 16 * (e >> 2) + 4 * g + (e & 3) < stat_len) ps += p[e];
      m_snap = m_new;
      l_snap = fmaf(l_run, alpha, ps);
    }
  }
  l_run = fmaf(l_run, alpha, psum);
  m_run = m_new;
  vec8 pb = pack8<T>(p);
#pragma unroll
  for (int mt = 0; mt < 8; ++mt) {
    o[mt] = o[mt] * alpha;
    o[mt] = mma_16x16x32(vr[mt], pb, o[mt]);
  }
}

// Fold the appended token (k_new, v_new of this row) into the lane state of
// attend_tile.  The score is a VALU dot product of the operand registers
// (exact bf16/f16 products, fp32 sums), reduced over the four k-groups; P is
// rounded to T as on the matrix-core path.  Returns the score's dot product.
template <typename T>
__device__ __forceinline__ float attend_new_token(const typename Elem<T>::vec8 (&qreg)[4], const T* __restrict__ kn,
                                                 const T* __restrict__ vn, int lane, float scale_log2, float& m_run,
                                                 float& l_run, f32x4 (&o)[8]) {
  const int g = lane >> 4;
  float dot = 0.f;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const typename Elem<T>::vec8 k8 = load8<T>(kn + 32 * s + 8 * g);
#pragma unroll
    for (int e = 0; e < 8; ++e) dot = fmaf(vec8_at<T>(qreg[s], e), vec8_at<T>(k8, e), dot);
  }
  dot = rows4_sum(dot);
  const float sc = dot * scale_log2;
  const float m_new = fmaxf(m_run, sc);
  const float alpha = fast_exp2(m_run - m_new);
  const float p = Elem<T>::to_f32(Elem<T>::from_f32(fast_exp2(sc - m_new)));
  l_run = fmaf(l_run, alpha, g == 0 ? p : 0.f);
  m_run = m_new;
#pragma unroll
  for (int mt = 0; mt < 8; ++mt)
#pragma unroll
    for (int j = 0; j < 4; ++j) o[mt][j] = fmaf(p, Elem<T>::to_f32(vn[16 * mt + 4 * g + j]), o[mt][j] * alpha);
  return dot;
}

// Stream tiles [t_begin, t_end) of a row through attend_tile (SNAP: with the
// below-stat_len snapshot).  Two tile buffers: the next tile's 16 wave-loads
// are in flight while the current one is consumed.  The buffers alternate by
// name (no register copies) and the loads inside the paired loop are
// unconditional, so every wait leaves the younger tile outstanding.
// Scheduling barriers keep each request between the two consumers (hoisting
// both requests would hold three tiles and spill).
template <typename T, bool SNAP, int RM = 0>
__device__ __forceinline__ void stream_tiles(const T* __restrict__ kstore, const T* __restrict__ vstore,
                                             int64_t row_base, int lane, int t_begin, int t_end,
                                             const typename Elem<T>::vec8 (&qreg)[4], int len_st, float scale_log2,
                                             float& m_run, float& l_run, f32x4 (&o)[8], int stat_len, float& m_snap,
                                             float& l_snap, float scale) {
  typedef typename Elem<T>::vec8 vec8;
  const T* kb = kstore + row_base + lane * 8;
  const T* vb = vstore + row_base + lane * 8;
  vec8 kA[8], vA[8], kB[8], vB[8];
  load_tile<T>(kA, vA, kb, vb, t_begin);
  int t = t_begin;
  for (; t + 2 < t_end; t += 2) {
    load_tile<T>(kB, vB, kb, vb, t + 1);
    __builtin_amdgcn_sched_barrier(0);
    attend_tile<T, SNAP, RM>(kA, vA, qreg, t, len_st, lane, scale_log2, m_run, l_run, o, stat_len, m_snap, l_snap, scale);
    __builtin_amdgcn_sched_barrier(0);
    load_tile<T>(kA, vA, kb, vb, t + 2);
    __builtin_amdgcn_sched_barrier(0);
    attend_tile<T, SNAP, RM>(kB, vB, qreg, t + 1, len_st, lane, scale_log2, m_run, l_run, o, stat_len, m_snap, l_snap, scale);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (t + 1 < t_end) {
    load_tile<T>(kB, vB, kb, vb, t + 1);
    attend_tile<T, SNAP, RM>(kA, vA, qreg, t, len_st, lane, scale_log2, m_run, l_run, o, stat_len, m_snap, l_snap, scale);
    attend_tile<T, SNAP, RM>(kB, vB, qreg, t + 1, len_st, lane, scale_log2, m_run, l_run, o, stat_len, m_snap, l_snap, scale);
  } else {
    attend_tile<T, SNAP, RM>(kA, vA, qreg, t, len_st, lane, scale_log2, m_run, l_run, o, stat_len, m_snap, l_snap, scale);
  }
}

constexpr int kOPitch = HC_HEAD_DIM + 4;

// STATS: besides its (m, l, O) partial, each workgroup writes part_st, the
// (max, sum) of its queries' scaled base-2 scores over the attended tokens
// below stat_len, which the merge folds into the row's softmax statistics
// over its first stat_len tokens (RM != 0: of the cast chain's logits,
// see attend_tile).
template <typename T, int NWAVES, bool STATS, int RM = 0>
__global__ __launch_bounds__(NWAVES * 64, sizeof(T) == 4 ? 1 : 2) void decode_partial_kernel(
    const T* __restrict__ q, T* __restrict__ kstore, T* __restrict__ vstore, const int64_t* __restrict__ row_tile_off,
    const int* __restrict__ row_len, const int* __restrict__ row_cap, const int* __restrict__ row_order, int rows,
    int G, float scale_log2, int chunk_tiles, const T* __restrict__ k_new, const T* __restrict__ v_new,
    float* __restrict__ part_o, float* __restrict__ part_ml, int* __restrict__ row_info, int* __restrict__ status,
    int stat_len, float* __restrict__ part_st, float scale) {
  typedef typename Elem<T>::vec8 vec8;
  constexpr int NT = NWAVES * 64;
  const bool fused_append = (k_new != nullptr);
  const ChunkLoc loc = locate_chunk(row_len, row_cap, row_order, row_tile_off, rows, fused_append ? 1 : 0,
                                    chunk_tiles, (int)blockIdx.x);

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int n = lane & 15;  // query slot owned by this lane
  const int g = lane >> 4;  // k-group of this lane

  __shared__ float s_m[NWAVES][16];
  __shared__ float s_l[NWAVES][16];
  __shared__ float s_ms[STATS ? NWAVES : 1][16];
  __shared__ float s_ls[STATS ? NWAVES : 1][16];
  // Per-wave O^T of the G queries, [wave][query][channel], pitch kOPitch;
  // sized by the launch for G queries.
  extern __shared__ float s_o[];

  if (loc.total > (int)gridDim.x) {
    // The launch grid is smaller than the device lengths need (every
    // workgroup sees the same lengths, so all of them take this branch):
    // flag every row -- workgroup b the rows b, b + grid, ... -- so the
    // merge writes NaN and advances no length, whatever a previous launch
    // left in the workspace.  Nothing is attended or stored.
    for (int64_t r = blockIdx.x + (int64_t)threadIdx.x * gridDim.x; r < rows; r += (int64_t)NT * gridDim.x) {
      row_info[2 * r] = 0;
      row_info[2 * r + 1] = -1;
    }
    return;
  }
  if (!loc.found) return;
  if (loc.full) {
    // Fused append into a row at capacity: the row is left unchanged, its
    // output is NaN (flag) and bit 0 of *status reports it.
    if (threadIdx.x == 0 && loc.chunk == 0) {
      row_info[2 * loc.row] = 0;
      row_info[2 * loc.row + 1] = -1;
      if (status) atomicOr(status, 1);
    }
    return;
  }
  {
    const int row = loc.row, len = loc.len;
    const int new_pos = fused_append ? len - 1 : -1;
    const T* kn = fused_append ? k_new + (int64_t)row * HC_HEAD_DIM : nullptr;
    const T* vn = fused_append ? v_new + (int64_t)row * HC_HEAD_DIM : nullptr;

    // Query operand: lane owns Q[n][32s + 8g + e] (zero for padded slots).
    vec8 qreg[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      if (n < G)
        qreg[s] = load8<T>(q + ((int64_t)row * G + n) * HC_HEAD_DIM + 32 * s + 8 * g);
      else
        qreg[s] = zero8<T>();
    }

    const int ntiles = (len + HC_TILE - 1) / HC_TILE;
    const int t0 = loc.chunk * chunk_tiles;
    const int t_begin = t0 + (wave * chunk_tiles) / NWAVES;
    const int t_end = min(t0 + ((wave + 1) * chunk_tiles) / NWAVES, ntiles);
    // Stored tokens only: the appended token is folded in separately.
    const int len_st = fused_append ? len - 1 : len;
    const int t_end_st = min(t_end, (len_st + HC_TILE - 1) / HC_TILE);

    float m_run = -INFINITY, l_run = 0.f;
    float m_snap = -INFINITY, l_snap = 0.f;  // STATS: the state below stat_len
    f32x4 o[8];
#pragma unroll
    for (int mt = 0; mt < 8; ++mt) o[mt] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int64_t row_base = loc.tiles * (int64_t)HC_TILE_ELEMS;
    if (t_begin < t_end_st) {
      // Only the wave whose tiles straddle stat_len follows the snapshot
      // tile by tile; a wave wholly below it takes its final state, one
      // wholly above leaves the snapshot empty.  The cast chain's state is
      // its own: every wave with tiles below stat_len follows it.
      if constexpr (STATS) {
        const bool cross = RM != 0 ? t_begin * HC_TILE < stat_len
                                   : t_begin * HC_TILE < stat_len && t_end_st * HC_TILE > stat_len;
        if (cross)
          stream_tiles<T, true, RM>(kstore, vstore, row_base, lane, t_begin, t_end_st, qreg, len_st, scale_log2,
                                    m_run, l_run, o, stat_len, m_snap, l_snap, scale);
        else
          stream_tiles<T, false, RM>(kstore, vstore, row_base, lane, t_begin, t_end_st, qreg, len_st, scale_log2,
                                     m_run, l_run, o, stat_len, m_snap, l_snap, scale);
        if (RM == 0 && t_end_st * HC_TILE <= stat_len) {
          m_snap = m_run;
          l_snap = l_run;
        }
      } else {
        // The same loop as stream_tiles, written out: through stream_tiles the
        // compiler schedules the plain instance's MFMAs and waits differently;
        // written out, its code is the one it had before the statistics
        // variant existed.
        const T* kb = kstore + row_base + lane * 8;
        const T* vb = vstore + row_base + lane * 8;
        vec8 kA[8], vA[8], kB[8], vB[8];
        load_tile<T>(kA, vA, kb, vb, t_begin);
        int t = t_begin;
        for (; t + 2 < t_end_st; t += 2) {
          load_tile<T>(kB, vB, kb, vb, t + 1);
          __builtin_amdgcn_sched_barrier(0);
          attend_tile<T, false>(kA, vA, qreg, t, len_st, lane, scale_log2, m_run, l_run, o, stat_len, m_snap, l_snap);
          __builtin_amdgcn_sched_barrier(0);
          load_tile<T>(kA, vA, kb, vb, t + 2);
          __builtin_amdgcn_sched_barrier(0);
          attend_tile<T, false>(kB, vB, qreg, t + 1, len_st, lane, scale_log2, m_run, l_run, o, stat_len, m_snap,
                                l_snap);
          __builtin_amdgcn_sched_barrier(0);
        }
        if (t + 1 < t_end_st) {
          load_tile<T>(kB, vB, kb, vb, t + 1);
          attend_tile<T, false>(kA, vA, qreg, t, len_st, lane, scale_log2, m_run, l_run, o, stat_len, m_snap, l_snap);
          attend_tile<T, false>(kB, vB, qreg, t + 1, len_st, lane, scale_log2, m_run, l_run, o, stat_len, m_snap,
                                l_snap);
        } else {
          attend_tile<T, false>(kA, vA, qreg, t, len_st, lane, scale_log2, m_run, l_run, o, stat_len, m_snap, l_snap);
        }
      }
    }
    // The wave whose tile range holds the new slot attends the new token and
    // stores it (no other workgroup of this launch reads that slot).
    if (fused_append && new_pos >= t_begin * HC_TILE && new_pos < t_end * HC_TILE) {
      const float dot = attend_new_token<T>(qreg, kn, vn, lane, scale_log2, m_run, l_run, o);
      if (STATS && new_pos < stat_len) {  // every earlier token lies below it too
        if constexpr (RM == 0) {
          m_snap = m_run;
          l_snap = l_run;
        } else {
          const float x = round_fixed<RM>(round_fixed<RM>(dot) * scale) * 1.4426950408889634f;
          const float mn = fmaxf(m_snap, x);
          l_snap = fmaf(l_snap, fast_exp2(m_snap - mn), g == 0 ? fast_exp2(x - mn) : 0.f);
          m_snap = mn;
        }
      }
      const int64_t tb = row_base + (int64_t)(new_pos / HC_TILE) * HC_TILE_ELEMS;
      const int tn = new_pos % HC_TILE;
      for (int d = lane; d < HC_HEAD_DIM; d += 64) {
        kstore[tb + k_tile_offset(tn, d)] = kn[d];
        vstore[tb + v_tile_offset(tn, d)] = vn[d];
      }
    }
    l_run = rows4_sum(l_run);
    if constexpr (STATS) l_snap = rows4_sum(l_snap);

    // Wave states -> LDS.  Lane holds O^T[d = 16mt + 4g + j][q = n].
    if (n < G) {
      if (g == 0) {
        s_m[wave][n] = m_run;
        s_l[wave][n] = l_run;
        if constexpr (STATS) {
          s_ms[wave][n] = m_snap;
          s_ls[wave][n] = l_snap;
        }
      }
#pragma unroll
      for (int mt = 0; mt < 8; ++mt)
#pragma unroll
        for (int j = 0; j < 4; ++j) s_o[(wave * G + n) * kOPitch + 16 * mt + 4 * g + j] = o[mt][j];
    }
    __syncthreads();

    const int64_t part = loc.p0 + loc.chunk;
    for (int idx = threadIdx.x; idx < G * HC_HEAD_DIM; idx += NT) {
      const int qq = idx / HC_HEAD_DIM, d = idx % HC_HEAD_DIM;
      float M = -INFINITY;
#pragma unroll
      for (int w = 0; w < NWAVES; ++w) M = fmaxf(M, s_m[w][qq]);
      float acc = 0.f, lsum = 0.f;
#pragma unroll
      for (int w = 0; w < NWAVES; ++w) {
        const float f = (s_m[w][qq] == -INFINITY) ? 0.f : fast_exp2(s_m[w][qq] - M);
        acc = fmaf(s_o[(w * G + qq) * kOPitch + d], f, acc);
        lsum = fmaf(s_l[w][qq], f, lsum);
      }
      part_o[(part * G + qq) * HC_HEAD_DIM + d] = acc;
      if (d == 0) {
        part_ml[(part * G + qq) * 2 + 0] = M;
        part_ml[(part * G + qq) * 2 + 1] = lsum;
      }
    }
    if constexpr (STATS) {
      for (int qq = threadIdx.x; qq < G; qq += NT) {
        float M = -INFINITY, Ls = 0.f;
#pragma unroll
        for (int w = 0; w < NWAVES; ++w) M = fmaxf(M, s_ms[w][qq]);
        if (M != -INFINITY) {
#pragma unroll
          for (int w = 0; w < NWAVES; ++w)
            if (s_ms[w][qq] != -INFINITY) Ls = fmaf(s_ls[w][qq], fast_exp2(s_ms[w][qq] - M), Ls);
        }
        part_st[(part * G + qq) * 2 + 0] = M;
        part_st[(part * G + qq) * 2 + 1] = Ls;
      }
    }
    if (threadIdx.x == 0 && loc.chunk == 0) {
      row_info[2 * row] = (int)loc.p0;
      row_info[2 * row + 1] = loc.nparts;
    }
  }
}

// Fold the partials of one row for one query slot and kMergeSlice channels;
// the (row, 0, 0) workgroup also advances row_len after a fused append.
// Thread (group, channel) takes parts group, group + kMergeGroups, ...: its
// kBatch O and (m, l) loads are issued unconditionally (addresses clamped
// into the row, values masked after), so they are in flight together, and
// are folded in registers; the groups' (m, l, o) are combined once through
// LDS.  The merge is latency-bound, not bandwidth-bound: loads under a
// per-part branch, or a separate block reduction for the row maximum and
// sum, each add a dependent round.
constexpr int kMergeSlice = 16;
constexpr int kMergeGroups = 16;
constexpr int kMergeThreads = kMergeSlice * kMergeGroups;

// A row whose part range lies outside this launch's grid_parts partials
// (flagged np = -1 by an undersized grid or a full row) is written as NaN
// and its length is not advanced: only rows whose new token was stored and
// attended advance.
// STATS: the grid has one more channel slice, whose workgroup of (row,
// query) folds the parts' statistics below stat_len instead (its first wave:
// lanes striding over the parts, then a xor tree) into
// stat_out[row * st_row_stride + query * st_head_stride] = (max, sum), NaN
// for a flagged row.  (Folded by one of the merge waves of slice 0 the
// statistics cost 0.6 us per layer; by a fifth wave of every merge
// workgroup, 0.3.)
__device__ __forceinline__ void merge_ml_pair(float& m, float& l, float m2, float l2) {
  const float mn = fmaxf(m, m2);
  if (mn == -INFINITY) return;
  l = l * fast_exp2(m - mn) + l2 * fast_exp2(m2 - mn);
  m = mn;
}

template <typename T, bool STATS>
__global__ __launch_bounds__(kMergeThreads) void decode_merge_kernel(
    const float* __restrict__ part_o, const float* __restrict__ part_ml, const int* __restrict__ row_info, int G,
    int64_t grid_parts, int* __restrict__ row_len, int advance, T* __restrict__ out, const float* __restrict__ part_st,
    float* __restrict__ stat_out, int64_t st_row_stride, int64_t st_head_stride) {
  constexpr int kBatch = 8;  // parts per thread whose loads are in flight together
  const int row = blockIdx.x, qq = blockIdx.y, d0 = blockIdx.z * kMergeSlice;
  const int tid = threadIdx.x;
  const int p0 = row_info[2 * row], np = row_info[2 * row + 1];
  __shared__ float s_m[kMergeGroups], s_l[kMergeGroups];
  __shared__ float s_o[kMergeGroups][kMergeSlice];
  T* o = out + ((int64_t)row * G + qq) * HC_HEAD_DIM + d0;
  const bool valid = np >= 1 && p0 >= 0 && (int64_t)p0 + np <= grid_parts;
  if constexpr (STATS) {
    if (blockIdx.z == HC_HEAD_DIM / kMergeSlice) {  // the statistics slice
      if (tid >= 64) return;
      float* so = stat_out + row * st_row_stride + qq * st_head_stride;
      if (!valid) {
        if (tid == 0) so[0] = so[1] = NAN;
        return;
      }
      const int ln = tid;
      float sm = -INFINITY, sl = 0.f;
      for (int p = ln; p < np; p += 64) {
        const float2 x = *reinterpret_cast<const float2*>(part_st + ((int64_t)(p0 + p) * G + qq) * 2);
        merge_ml_pair(sm, sl, x.x, x.y);
      }
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) {
        const float m2 = __shfl_xor(sm, off, 64), l2 = __shfl_xor(sl, off, 64);
        merge_ml_pair(sm, sl, m2, l2);
      }
      if (ln == 0) {
        so[0] = sm;
        so[1] = sl;
      }
      return;
    }
  }
  if (advance && valid && qq == 0 && blockIdx.z == 0 && tid == 0) row_len[row] += 1;
  if (!valid) {
    if (tid < kMergeSlice) o[tid] = Elem<T>::from_f32(NAN);
    return;
  }
  // np >= 1 here: an empty row still has its one (empty) part.
  const int dl = tid % kMergeSlice, grp = tid / kMergeSlice;
  const float* ml = part_ml + ((int64_t)p0 * G + qq) * 2;
  const float* po = part_o + ((int64_t)p0 * G + qq) * HC_HEAD_DIM + d0 + dl;
  const int64_t pstride = (int64_t)G * HC_HEAD_DIM;
  float ov[kBatch];
  float2 mv[kBatch];
#pragma unroll
  for (int k = 0; k < kBatch; ++k) {
    const int pc = min(grp + k * kMergeGroups, np - 1);
    ov[k] = po[pc * pstride];
    mv[k] = *reinterpret_cast<const float2*>(ml + (int64_t)pc * G * 2);
  }
  float m = -INFINITY;
#pragma unroll
  for (int k = 0; k < kBatch; ++k)
    if (grp + k * kMergeGroups < np) m = fmaxf(m, mv[k].x);
  float l = 0.f, acc = 0.f;
  if (m != -INFINITY) {
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const float e = grp + k * kMergeGroups < np ? fast_exp2(mv[k].x - m) : 0.f;
      l = fmaf(mv[k].y, e, l);
      acc = fmaf(ov[k], e, acc);
    }
  }
  // Rows of more than kBatch * kMergeGroups parts: online fold of the rest.
  for (int p = grp + kBatch * kMergeGroups; p < np; p += kMergeGroups) {
    const float2 x = *reinterpret_cast<const float2*>(ml + (int64_t)p * G * 2);
    const float y = po[p * pstride];
    const float mn = fmaxf(m, x.x);
    if (mn == -INFINITY) continue;
    const float f = fast_exp2(m - mn), e = fast_exp2(x.x - mn);
    l = fmaf(l, f, x.y * e);
    acc = fmaf(acc, f, y * e);
    m = mn;
  }
  if (dl == 0) {
    s_m[grp] = m;
    s_l[grp] = l;
  }
  s_o[grp][dl] = acc;
  __syncthreads();
  if (grp == 0) {
    float M = -INFINITY;
#pragma unroll
    for (int g = 0; g < kMergeGroups; ++g) M = fmaxf(M, s_m[g]);
    if (M == -INFINITY) {  // empty row
      o[dl] = Elem<T>::from_f32(0.f);
      return;
    }
    float L = 0.f, a = 0.f;
#pragma unroll
    for (int g = 0; g < kMergeGroups; ++g) {
      const float e = fast_exp2(s_m[g] - M);
      L = fmaf(s_l[g], e, L);
      a = fmaf(s_o[g][dl], e, a);
    }
    o[dl] = Elem<T>::from_f32(a / L);
  }
}

constexpr int kDecodeWaves = 4;

// Device-resident workspace of hc_decode_attn_noalloc, for callers that
// cannot allocate.  Each device holds its own copy for the life of the
// process; host code never passes the symbol itself to a kernel (in host
// code it only names the symbol), it uses the address hipGetSymbolAddress
// returns for the current device.
constexpr size_t kNoAllocScratchBytes = (size_t)16 << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

int64_t decode_num_parts(const int* host_row_len, int rows, int chunk_tiles) {
  int64_t total = 0;
  for (int r = 0; r < rows; ++r) {
    int64_t nt = (host_row_len[r] + HC_TILE - 1) / HC_TILE;
    total += nt > 0 ? (nt + chunk_tiles - 1) / chunk_tiles : 1;
  }
  return total;
}

// Workspace: [row_info: (first part, part count) per row, padded to 256 B]
//            [part_o: parts*G*128 f32][part_ml: parts*G*2 f32][part_st: parts*G*2 f32]
// (the 512-byte partial rows first, so each starts on a cache line)
// Every field is written before it is read within one call, so the buffer
// needs no initialisation and may be reused freely by calls on one stream.
static size_t workspace_head(int rows) { return ((size_t)rows * 2 * sizeof(int) + 255) / 256 * 256; }

size_t decode_workspace_bytes_rows(int rows, int group, int64_t num_parts) {
  if (num_parts <= 0 || group <= 0) return workspace_head(rows);
  return workspace_head(rows) + (size_t)num_parts * (size_t)group * (HC_HEAD_DIM + 4) * sizeof(float);
}

// Softmax statistics requested of a decode launch (hc_decode_attn_stats).
struct DecodeStats {
  int len = 0;  // 0: none
  int rm = 0;   // rounding mode of the cast chain the statistics follow (0: none)
  float* out = nullptr;
  int64_t row_stride = 0, head_stride = 0;
};

template <typename T>
static int launch_decode(const void* q, void* kstore, void* vstore, const int64_t* row_tile_off, int* row_len,
                         const int* row_cap, const int* row_order, int rows, int G, float scale, const void* k_new,
                         const void* v_new, void* out, void* workspace, size_t workspace_bytes, int64_t grid_parts,
                         int chunk_tiles, int* status, const DecodeStats& st, hipStream_t stream) {
  if (grid_parts < rows)
    return set_error(HC_ERR_INVALID, "hc_decode_attn: num_parts=%lld below the row count %d", (long long)grid_parts,
                     rows);
  if (grid_parts > 0x7fffffffLL) return set_error(HC_ERR_INVALID, "hc_decode_attn: too many parts");
  const size_t need = decode_workspace_bytes_rows(rows, G, grid_parts);
  if (!workspace || workspace_bytes < need)
    return set_error(HC_ERR_INVALID, "hc_decode_attn: workspace too small (%zu < %zu bytes)", workspace_bytes, need);
  int* row_info = reinterpret_cast<int*>(workspace);
  float* part_o = reinterpret_cast<float*>(reinterpret_cast<char*>(workspace) + workspace_head(rows));
  float* part_ml = part_o + (size_t)grid_parts * G * HC_HEAD_DIM;
  float* part_st = part_ml + (size_t)grid_parts * G * 2;
  const float scale_log2 = scale * 1.4426950408889634f;
  const size_t lds_o = (size_t)kDecodeWaves * G * kOPitch * sizeof(float);
  const dim3 mgrid(rows, G, HC_HEAD_DIM / kMergeSlice), mblock(kMergeSlice * kMergeGroups);
  if (st.len > 0) {
    auto fn = st.rm == 1   ? decode_partial_kernel<T, kDecodeWaves, true, 1>
              : st.rm == 2 ? decode_partial_kernel<T, kDecodeWaves, true, 2>
                           : decode_partial_kernel<T, kDecodeWaves, true, 0>;
    hipLaunchKernelGGL(fn, dim3((unsigned)grid_parts), dim3(kDecodeWaves * 64), lds_o, stream, (const T*)q,
                       (T*)kstore, (T*)vstore, row_tile_off, row_len, row_cap, row_order, rows, G, scale_log2,
                       chunk_tiles, (const T*)k_new, (const T*)v_new, part_o, part_ml, row_info, status, st.len,
                       part_st, scale);
    int rc = check_launch("hc_decode_attn(partial)");
    if (rc) return rc;
    hipLaunchKernelGGL((decode_merge_kernel<T, true>), dim3(rows, G, HC_HEAD_DIM / kMergeSlice + 1), mblock, 0,
                       stream, part_o, part_ml, row_info, G,
                       grid_parts, row_len, k_new ? 1 : 0, (T*)out, part_st, st.out, st.row_stride,
                       st.head_stride);
    return check_launch("hc_decode_attn(merge)");
  }
  hipLaunchKernelGGL((decode_partial_kernel<T, kDecodeWaves, false>), dim3((unsigned)grid_parts),
                     dim3(kDecodeWaves * 64), lds_o, stream, (const T*)q, (T*)kstore, (T*)vstore, row_tile_off,
                     row_len, row_cap, row_order, rows, G, scale_log2, chunk_tiles, (const T*)k_new, (const T*)v_new,
                     part_o, part_ml, row_info, status, 0, nullptr, scale);
  int rc = check_launch("hc_decode_attn(partial)");
  if (rc) return rc;
  hipLaunchKernelGGL((decode_merge_kernel<T, false>), mgrid, mblock, 0, stream, part_o, part_ml, row_info, G,
                     grid_parts, row_len, k_new ? 1 : 0, (T*)out, nullptr, nullptr, (int64_t)0, (int64_t)0);
  return check_launch("hc_decode_attn(merge)");
}

// Workgroups of decode_partial_kernel<T> resident on the current device at
// once (occupancy per CU x CU count), cached per (device, dtype, group).
static int decode_slots(int dtype, int G) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return -1;
  static std::mutex mu;
  static int cache[64][3][17];  // zero = not yet queried
  std::lock_guard<std::mutex> lock(mu);
  int& slot = cache[dev][dtype][G];
  if (slot > 0) return slot;
  const size_t lds = (size_t)kDecodeWaves * G * kOPitch * sizeof(float);
  const void* fn = nullptr;
  switch (dtype) {
    case HC_DTYPE_BF16: fn = reinterpret_cast<const void*>(decode_partial_kernel<__bf16, kDecodeWaves, false>); break;
    case HC_DTYPE_F16: fn = reinterpret_cast<const void*>(decode_partial_kernel<_Float16, kDecodeWaves, false>); break;
    default: fn = reinterpret_cast<const void*>(decode_partial_kernel<float, kDecodeWaves, false>); break;
  }
  int per_cu = 0, cus = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kDecodeWaves * 64, lds) != hipSuccess) return -1;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return -1;
  slot = (per_cu > 0 ? per_cu : 1) * (cus > 0 ? cus : 1);
  return slot;
}

// Smallest chunk (>= one tile per wave) whose grid fits in one resident
// round: a second, partly filled round of workgroups leaves HBM idle at the
// end of the launch, while smaller chunks keep more loads in flight.  Long
// chunks are then rounded up to a whole number of tiles per wave: the
// slowest wave of a workgroup streams ceil(chunk / NWAVES) tiles either way,
// and with equal shares no wave streams alone at the end while the others
// of the chip have finished.  Measured: 128K Llama-3-8B-shape layers
// (chunks of 27-44 tiles) 47.8 -> 47.4 us per layer; 224K layers (46-76)
// unchanged; a Qwen-shaped 16-64K batch (chunks of 6 and 15 tiles, where
// rounding drops 7-25 % of the workgroups) 22.2 -> 22.8 us, so chunks
// below kRoundChunk stay as found.
constexpr int kRoundChunk = 6 * kDecodeWaves;
static int decode_auto_chunk(const int* host_row_len, int rows, int slots) {
  int max_nt = 0;
  for (int r = 0; r < rows; ++r) max_nt = max(max_nt, (host_row_len[r] + HC_TILE - 1) / HC_TILE);
  if (max_nt <= kDecodeWaves) return kDecodeWaves;
  // One part per row already exceeds the resident slots: one chunk per row.
  if (decode_num_parts(host_row_len, rows, max_nt) > slots) return max_nt;
  int lo = kDecodeWaves, hi = max_nt;  // parts(chunk) does not increase with chunk
  while (lo < hi) {
    const int mid = lo + (hi - lo) / 2;
    if (decode_num_parts(host_row_len, rows, mid) <= slots)
      hi = mid;
    else
      lo = mid + 1;
  }
  return lo < kRoundChunk ? lo : (lo + kDecodeWaves - 1) / kDecodeWaves * kDecodeWaves;
}

}  // namespace hc

using namespace hc;

extern "C" size_t hc_decode_workspace_size(int rows, int group, int64_t num_parts) {
  return decode_workspace_bytes_rows(rows, group, num_parts);
}

extern "C" int hc_decode_chunk_tiles(int dtype, const int32_t* host_row_len, int rows, int group) {
  clear_error();
  if (dtype != HC_DTYPE_BF16 && dtype != HC_DTYPE_F16 && dtype != HC_DTYPE_F32)
    return set_error(HC_ERR_INVALID, "hc_decode_chunk_tiles: unknown dtype %d", dtype);
  if (rows < 0 || group < 1 || group > 16 || (rows > 0 && !host_row_len))
    return set_error(HC_ERR_INVALID, "hc_decode_chunk_tiles: rows=%d group=%d", rows, group);
  for (int r = 0; r < rows; ++r)
    if (host_row_len[r] < 0) return set_error(HC_ERR_INVALID, "hc_decode_chunk_tiles: negative length at row %d", r);
  const int slots = decode_slots(dtype, group);
  if (slots <= 0) return set_error(HC_ERR_HIP, "hc_decode_chunk_tiles: occupancy query failed");
  return decode_auto_chunk(host_row_len, rows, slots);
}

extern "C" int64_t hc_decode_num_parts(const int32_t* host_row_len, int rows, int chunk_tiles) {
  if (!host_row_len || rows < 0 || chunk_tiles <= 0) return -1;
  return decode_num_parts(host_row_len, rows, chunk_tiles);
}

// Argument checks and dtype dispatch shared by the decode entry points.
static int decode_entry(int dtype, const void* q, void* kstore, void* vstore, const int64_t* row_tile_off,
                        int32_t* row_len, const int32_t* row_cap, const int32_t* row_order, int rows, int group,
                        float scale, const void* k_new, const void* v_new, void* out, void* workspace,
                        size_t workspace_bytes, int64_t num_parts, int chunk_tiles, int32_t* status, void* stream,
                        const DecodeStats& st = DecodeStats()) {
  if (rows < 0 || group < 1 || group > 16)
    return set_error(HC_ERR_INVALID, "hc_decode_attn: rows=%d group=%d (group must be 1..16)", rows, group);
  if (chunk_tiles < 1 || chunk_tiles > (1 << 22))
    return set_error(HC_ERR_INVALID, "hc_decode_attn: chunk_tiles=%d out of range", chunk_tiles);
  if (rows == 0) return HC_OK;
  if (!q || !kstore || !vstore || !row_tile_off || !row_len || !out)
    return set_error(HC_ERR_INVALID, "hc_decode_attn: null pointer argument");
  if ((k_new == nullptr) != (v_new == nullptr))
    return set_error(HC_ERR_INVALID, "hc_decode_attn: k_new and v_new must be given together");
  if (k_new && !row_cap) return set_error(HC_ERR_INVALID, "hc_decode_attn: a fused append needs row_cap");
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case HC_DTYPE_BF16:
      return launch_decode<__bf16>(q, kstore, vstore, row_tile_off, row_len, row_cap, row_order, rows, group, scale,
                                   k_new, v_new, out, workspace, workspace_bytes, num_parts, chunk_tiles, status, st, s);
    case HC_DTYPE_F16:
      return launch_decode<_Float16>(q, kstore, vstore, row_tile_off, row_len, row_cap, row_order, rows, group, scale,
                                     k_new, v_new, out, workspace, workspace_bytes, num_parts, chunk_tiles, status, st, s);
    case HC_DTYPE_F32:
      return launch_decode<float>(q, kstore, vstore, row_tile_off, row_len, row_cap, row_order, rows, group, scale,
                                  k_new, v_new, out, workspace, workspace_bytes, num_parts, chunk_tiles, status, st, s);
    default:
      return set_error(HC_ERR_INVALID, "hc_decode_attn: unknown dtype %d", dtype);
  }
}

extern "C" int hc_decode_attn(int dtype, const void* q, void* kstore, void* vstore, const int64_t* row_tile_off,
                              int32_t* row_len, const int32_t* row_cap, const int32_t* row_order, int rows, int group,
                              float scale, const void* k_new, const void* v_new, void* out, void* workspace,
                              size_t workspace_bytes, int64_t num_parts, int chunk_tiles, int32_t* status,
                              void* stream) {
  clear_error();
  return decode_entry(dtype, q, kstore, vstore, row_tile_off, row_len, row_cap, row_order, rows, group, scale, k_new,
                      v_new, out, workspace, workspace_bytes, num_parts, chunk_tiles, status, stream);
}

extern "C" int hc_decode_attn_stats(int dtype, const void* q, void* kstore, void* vstore, const int64_t* row_tile_off,
                                    int32_t* row_len, const int32_t* row_cap, const int32_t* row_order, int rows,
                                    int group, float scale, const void* k_new, const void* v_new, void* out,
                                    void* workspace, size_t workspace_bytes, int64_t num_parts, int chunk_tiles,
                                    int32_t* status, int stat_len, float* stat_out, int64_t stat_row_stride,
                                    int64_t stat_head_stride, int stat_flags, void* stream) {
  clear_error();
  if (stat_len < 1 || !stat_out || stat_row_stride < 0 || stat_head_stride < 0)
    return set_error(HC_ERR_INVALID, "hc_decode_attn_stats: stat_len=%d, stat_out %s", stat_len,
                     stat_out ? "given" : "null");
  if (stat_flags != 0 && stat_flags != HC_SCORE_ROUND_BF16 && stat_flags != HC_SCORE_ROUND_F16)
    return set_error(HC_ERR_INVALID, "hc_decode_attn_stats: stat_flags=%d (0, HC_SCORE_ROUND_BF16 or _F16)",
                     stat_flags);
  DecodeStats st;
  st.len = stat_len;
  st.rm = stat_flags == HC_SCORE_ROUND_BF16 ? 1 : stat_flags == HC_SCORE_ROUND_F16 ? 2 : 0;
  st.out = stat_out;
  st.row_stride = stat_row_stride;
  st.head_stride = stat_head_stride;
  return decode_entry(dtype, q, kstore, vstore, row_tile_off, row_len, row_cap, row_order, rows, group, scale, k_new,
                      v_new, out, workspace, workspace_bytes, num_parts, chunk_tiles, status, stream, st);
}

// Address of this device's scratch array, resolved once per device on the
// first call made with that device current.
static int noalloc_scratch(void** ptr) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
    return set_error(HC_ERR_HIP, "hc_decode_attn_noalloc: no current device");
  static std::mutex mu;
  static void* addr[64] = {nullptr};
  std::lock_guard<std::mutex> lock(mu);
  if (!addr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return set_error(HC_ERR_HIP, "hc_decode_attn_noalloc: hipGetSymbolAddress failed: %s", hipGetErrorString(e));
    addr[dev] = p;
  }
  *ptr = addr[dev];
  return HC_OK;
}

extern "C" int hc_decode_attn_noalloc(int dtype, const void* q, void* kstore, void* vstore, const int64_t* row_tile_off,
                                      int32_t* row_len, const int32_t* row_cap, const int32_t* row_order, int rows,
                                      int group, float scale, const void* k_new, const void* v_new, void* out,
                                      int64_t num_parts, int chunk_tiles, int32_t* status, void* stream) {
  clear_error();
  if (rows > 0 && group >= 1 && group <= 16 && num_parts > 0) {
    const size_t need = decode_workspace_bytes_rows(rows, group, num_parts);
    if (need > kNoAllocScratchBytes)
      return set_error(HC_ERR_INVALID,
                       "hc_decode_attn_noalloc: %d rows x group %d x %lld parts need %zu bytes of workspace, above the "
                       "%zu-byte device scratch (use hc_decode_attn with a caller workspace)",
                       rows, group, (long long)num_parts, need, kNoAllocScratchBytes);
  }
  if (rows <= 0 || group < 1 || group > 16 || chunk_tiles < 1)
    return decode_entry(dtype, q, kstore, vstore, row_tile_off, row_len, row_cap, row_order, rows, group, scale,
                        k_new, v_new, out, nullptr, 0, num_parts, chunk_tiles, status, stream);
  void* ws = nullptr;
  const int rc = noalloc_scratch(&ws);
  if (rc) return rc;
  return decode_entry(dtype, q, kstore, vstore, row_tile_off, row_len, row_cap, row_order, rows, group, scale, k_new,
                      v_new, out, ws, kNoAllocScratchBytes, num_parts, chunk_tiles, status, stream);
}
