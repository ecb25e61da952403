// Causal prefill attention (flash-attention forward) on gfx950 MFMA.
//
//   out[b, i, hq, :] = sum_t softmax_t(scale * q[b, hq, i] . k[b, hq/G, t]) v[b, hq/G, t]
//   over keys t <= Lk - Lq + i
//
// The queries are the last Lq positions of the Lk keys (bottom-right causal
// alignment, as flash-attn's causal=True), so one kernel serves a whole
// prompt (Lq == Lk) and each chunk of a chunked prefill (Lq < Lk).  Replaces
// the flash-attn prefill call of LlamaAttention / Qwen2Attention
// (heterocache/llama_model.py:353-361, through transformers'
// flash_attention_forward; heterocache/qwen_model.py follows the same path).
//
// Structure:
//  * a workgroup holds 4 waves x 32 queries of one query head, three
//    workgroups per CU (168 VGPRs, 48 KB LDS); the blockIdx
//    order puts every workgroup of a KV row on the same XCD (rows are
//    interleaved modulo the grid's round-robin over XCDs) and dispatches the
//    query blocks with the most keys first;
//  * keys advance 64 per iteration (two 32-token tiles), staged through
//    double-buffered LDS in the KV store's tile layout so every MFMA operand
//    is one 16-byte LDS read.  K is read in natural layout (arbitrary
//    batch/head/token strides): its 8-channel chunks stay whole in the tile
//    layout.  V is first re-laid out into tiles by v_tiles_kernel (once per
//    tile, into the caller's workspace).  Both are then plain 16-byte copies,
//    issued as LDS-DMA loads (global_load_lds) that hold no registers;
//  * S^T = K Q^T per 16-key x 16-query block (K as the A operand), online
//    base-2 softmax per query column, O^T += V^T P^T with P taken straight
//    from the S accumulators (the tile layout's V token order is the order in
//    which the accumulator holds the scores), fp32 accumulation;
//  * the softmax is VALU work beside the MFMAs (CDNA4 issues a wave64 VALU
//    op over 4 cycles, v_exp at a quarter of that rate), so it is kept lean:
//    the tile maximum is taken on raw scores and the scale folded into the
//    exp2 argument's fma, masking runs only on tiles that cross the
//    diagonal, and O is rescaled only when the running maximum grows by more
//    than 2^8.
#include <algorithm>
#include <cfloat>
#include <cmath>
#include <mutex>

#include "hc_common.h"
#include "hc_internal.h"

namespace hc {
namespace {

constexpr int kPfWaves = 4;
constexpr int kPfWaveQ = 32;                    // queries per wave: two 16-column MFMA blocks
constexpr int kPfBlockQ = kPfWaves * kPfWaveQ;  // queries per workgroup
constexpr int kPfTiles = 2;                     // 32-token tiles per iteration
constexpr int kPfKeys = kPfTiles * HC_TILE;     // keys per iteration
constexpr int kPfThreads = kPfWaves * 64;
constexpr float kPfLazy = 8.f;                  // lazy-rescale threshold, log2 units

struct PfArgs {
  const void* q;
  const void* k;
  const void* v;   // natural layout (read by v_tiles_kernel)
  const void* vt;  // V in tile layout: [rows][vt_tiles][HC_TILE_ELEMS]
  void* out;
  int64_t q_sb, q_sh, q_st;  // element strides: batch, head, token (channels contiguous)
  int64_t k_sb, k_sh, k_st;
  int64_t v_sb, v_sh, v_st;
  int64_t o_sb, o_sh, o_st;
  int Hq, Hkv, Lq, Lk, nqb, rows;  // rows = batch * Hkv
  int vt_tiles;                    // tiles per row of vt
  float scale_log2;
  // Optional softmax statistics of the last st_rows queries of every
  // (batch, query head): st[((b * Hq + hq) * st_rows + w) * 2 + {0, 1}].
  float* st;
  int st_rows;
  // Split over the keys (short query blocks over long key ranges): grid
  // slice `split` of nsplit takes iterations [split * its, (split + 1) * its)
  // and writes its unnormalised partials to part (kPfPartStride floats per
  // (query, split)); prefill_merge_kernel combines them.  nsplit = 1: no split.
  int nsplit, its;
  float* part;
};

// One partial: 128 unnormalised output channels, then (m, l); 16-byte rows.
constexpr int kPfPartStride = HC_HEAD_DIM + 4;

// LDS: two K buffers and one V buffer of kPfTiles tiles each.
template <typename T>
constexpr size_t pf_lds_bytes() {
  return (size_t)3 * kPfTiles * HC_TILE_ELEMS * sizeof(T);
}

// Four elements of T as one vector store (8 bytes for 16-bit types).
template <typename T>
struct Quad {
  typedef T type __attribute__((ext_vector_type(4)));
};

// V rows in natural layout -> the KV store's V tile layout, one 32-token tile
// per workgroup, zeros past kv_len.  The attention kernel then stages V with
// plain 16-byte copies, and the transposition is paid once per tile rather
// than once per (query head, query block) that reads it.
template <typename T>
__global__ __launch_bounds__(256) void v_tiles_kernel(const PfArgs a) {
  typedef typename Elem<T>::vec8 vec8;
  __shared__ T s[HC_TILE][HC_HEAD_DIM + 8];
  const int tile = blockIdx.x, row = blockIdx.y;
  const int b = row / a.Hkv, h = row % a.Hkv;
  const T* src = reinterpret_cast<const T*>(a.v) + b * a.v_sb + h * a.v_sh;
  const int t0 = tile * HC_TILE;
  for (int c = threadIdx.x; c < HC_TILE * 16; c += 256) {
    const int t = c >> 4, d0 = (c & 15) * 8;
    const vec8 x = t0 + t < a.Lk ? load8(src + (int64_t)(t0 + t) * a.v_st + d0) : zero8<T>();
    *reinterpret_cast<vec8*>(&s[t][d0]) = x;
  }
  __syncthreads();
  T* dst = reinterpret_cast<T*>(const_cast<void*>(a.vt)) + ((int64_t)row * a.vt_tiles + tile) * HC_TILE_ELEMS;
  for (int c = threadIdx.x; c < HC_TILE * 16; c += 256) {
    // Output chunk c = (mt*4 + g)*16 + n: channel 16mt+n, tokens
    // {4g + [0,4), 16 + 4g + [0,4)} (the order the scores take in the MFMA
    // accumulator).
    const int n = c & 15, g = (c >> 4) & 3, mt = c >> 6;
    const int d = mt * 16 + n;
    typename Elem<T>::vec8 o;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const T x = s[16 * (i >> 2) + 4 * g + (i & 3)][d];
      if constexpr (sizeof(T) == 4) {
        if (i < 4) o.lo[i] = x; else o.hi[i - 4] = x;
      } else {
        o[i] = x;
      }
    }
    *reinterpret_cast<vec8*>(dst + c * 8) = o;
  }
}

// 16 bytes per lane straight from global memory into LDS: lane i's bytes
// land at lds + 16*i (lds is wave-uniform).
__device__ __forceinline__ void lds_dma16(const void* src, void* lds) {
  __builtin_amdgcn_global_load_lds(src, lds, 16, 0, 0);
}
// s_waitcnt vmcnt(0): every LDS-DMA load of this wave has landed.
__device__ __forceinline__ void wait_lds_dma() { __builtin_amdgcn_s_waitcnt(0x0f70); }
// s_waitcnt vmcnt(N): all but this wave's N most recent vector loads have
// landed (loads complete in order).
template <int N>
__device__ __forceinline__ void wait_lds_dma_but() {
  static_assert(N >= 0 && N < 16, "vmcnt field");
  __builtin_amdgcn_s_waitcnt(0x0f70 | N);
}

template <typename T, bool SPLIT>
__global__ __launch_bounds__(kPfThreads, sizeof(T) == 4 ? 1 : 3) void prefill_attn_kernel(const PfArgs a) {
  typedef typename Elem<T>::vec8 vec8;
  extern __shared__ __attribute__((aligned(16))) unsigned char pf_lds[];
  T* lds = reinterpret_cast<T*>(pf_lds);

  // The wave index is read through readfirstlane so that every quantity
  // derived from it (query range, masking, skipping) is known to be uniform
  // and branches on it stay scalar.
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g4 = lane >> 4, n16 = lane & 15;
  const int G = a.Hq / a.Hkv;
  // Workgroup -> (KV row, query head of its group, query block).
  const int x = blockIdx.x;
  const int row = x % a.rows;
  const int rest = x / a.rows;
  const int gi = rest % G;
  const int rest2 = rest / G;
  const int split = SPLIT ? rest2 % a.nsplit : 0;
  const int qb = a.nqb - 1 - (SPLIT ? rest2 / a.nsplit : rest2);
  const int b = row / a.Hkv, kvh = row % a.Hkv, hq = kvh * G + gi;

  const T* qbase = reinterpret_cast<const T*>(a.q) + b * a.q_sb + hq * a.q_sh;
  const T* kbase = reinterpret_cast<const T*>(a.k) + b * a.k_sb + kvh * a.k_sh;
  T* obase = reinterpret_cast<T*>(a.out) + b * a.o_sb + hq * a.o_sh;

  const int shift = a.Lk - a.Lq;  // position of query i is shift + i
  const int q_last = min(qb * kPfBlockQ + kPfBlockQ - 1, a.Lq - 1);
  const int nit_all = (shift + q_last + 1 + kPfKeys - 1) / kPfKeys;
  // This workgroup's iterations (all of them without a split).
  const int it0 = SPLIT ? min(split * a.its, nit_all) : 0;
  const int nit = SPLIT ? min(it0 + a.its, nit_all) : nit_all;
  const int qw0 = qb * kPfBlockQ + wave * kPfWaveQ;
  const bool active = qw0 < a.Lq;
  const int pos_lo = shift + qw0;                           // first query position of this wave
  const int pos_hi = shift + min(qw0 + kPfWaveQ - 1, a.Lq - 1);

  // Q^T operands: column = query 16j + n16, k-slots = channels 32s + 8*g4 + [0, 8).
  vec8 qop[2][4];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int qi = qw0 + 16 * j + n16;
#pragma unroll
    for (int s = 0; s < 4; ++s)
      qop[j][s] = qi < a.Lq ? load8(qbase + (int64_t)qi * a.q_st + 32 * s + 8 * g4) : zero8<T>();
  }

  f32x4 o[8][2];
#pragma unroll
  for (int db = 0; db < 8; ++db)
#pragma unroll
    for (int j = 0; j < 2; ++j) o[db][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m[2] = {-INFINITY, -INFINITY}, l[2] = {0.f, 0.f};

  // Staging roles: four 16-byte chunks of K and four of V per thread; chunk
  // u = r*256 + tid is tile u/512, tile chunk u%512, written to LDS at
  // u*16 bytes (contiguous per wave).
  //  * K arrives in natural layout.  Tile chunk ((h*4+s)*4+g)*16+m holds
  //    token 16h+m, channels 32s+8g+[0,8): one strided 16-byte read.  Each
  //    load is a uniform per-iteration base plus a fixed 32-bit byte offset
  //    (the host bounds 64 token strides below 2^31 bytes); in the last
  //    window, lanes past Lk read the window's first token instead (a select,
  //    not a branch, so no load waits at a join) and store zeros.
  //  * V arrives already in tile layout (v_tiles_kernel, zeros past Lk), so
  //    its chunks are plain contiguous reads.
  // Staging goes straight from global memory into LDS (global_load_lds:
  // each lane's 16 bytes land at the wave's LDS base + lane*16), so it
  // takes no registers and no LDS store instructions.  The copy runs in
  // 16-byte units, kUnits per 8-element chunk (1 for 16-bit types, 2 for
  // fp32); unit w = r*256 + tid lands at LDS byte 16*w of the K (or V) set,
  // which is chunk w / kUnits of the tile layout.  Keys past Lk read the
  // window's first token: they are masked, as they follow every query.
  constexpr int kUnits = (int)sizeof(T) / 2;
  constexpr int kUnitsPerThread = 4 * kUnits;
  // 16-bit types: unit r is token 16r + tid%16 with fixed channels, so one
  // offset and a uniform step describe all four; fp32 keeps a table.
  uint32_t koff[kUnits == 1 ? 1 : kUnitsPerThread], kch[kUnits == 1 ? 1 : kUnitsPerThread];
  int ktok[kUnits == 1 ? 1 : kUnitsPerThread];
#pragma unroll
  for (int r = 0; r < (kUnits == 1 ? 1 : kUnitsPerThread); ++r) {
    const int w = r * kPfThreads + tid;
    const int u = w / kUnits, half = w % kUnits;
    const int c = u >> 9, v = u & 511;
    const int h = v >> 8, s = (v >> 6) & 3, g = (v >> 4) & 3, mm = v & 15;
    ktok[r] = c * HC_TILE + h * 16 + mm;
    kch[r] = (uint32_t)((32 * s + 8 * g) * (int64_t)sizeof(T) + 16 * half);
    koff[r] = (uint32_t)(ktok[r] * a.k_st * (int64_t)sizeof(T)) + kch[r];
  }
  const uint32_t kstep = (uint32_t)(16 * a.k_st * (int64_t)sizeof(T));
  const char* vtiles = reinterpret_cast<const char*>(a.vt) +
                       ((int64_t)row * a.vt_tiles * HC_TILE_ELEMS) * (int64_t)sizeof(T) + 16 * tid;
  T* const vbuf = lds + 2 * kPfTiles * HC_TILE_ELEMS;

  auto stage_k = [&](int buf, int it) {
    char* sk = reinterpret_cast<char*>(lds + buf * kPfTiles * HC_TILE_ELEMS);
    const int t0 = it * kPfKeys;
    const char* kit = reinterpret_cast<const char*>(kbase) + (int64_t)t0 * a.k_st * (int64_t)sizeof(T);
    const int lim = a.Lk - t0;
#pragma unroll
    for (int r = 0; r < kUnitsPerThread; ++r) {
      const int wb = r * kPfThreads + wave * 64;  // first unit of this wave
      if constexpr (kUnits == 1) {
        const int tok = 16 * r + (tid & 15);
        lds_dma16(kit + (tok < lim ? koff[0] + r * kstep : kch[0]), sk + 16 * wb);
      } else {
        lds_dma16(kit + (ktok[r] < lim ? koff[r] : kch[r]), sk + 16 * wb);
      }
    }
  };
  auto stage_v = [&](int it) {
    char* sv = reinterpret_cast<char*>(vbuf);
    const char* vit = vtiles + (int64_t)it * kPfTiles * HC_TILE_ELEMS * (int64_t)sizeof(T);
#pragma unroll
    for (int r = 0; r < kUnitsPerThread; ++r)
      lds_dma16(vit + 16 * r * kPfThreads, sv + 16 * (r * kPfThreads + wave * 64));
  };

  // K is double-buffered (K(it+1) loads during iteration it); V has one
  // buffer, loaded between two barriers around the P.V step: V(it+1)
  // arrives while the next iteration forms its scores and probabilities.
  // 48 KB of LDS per workgroup leaves room for three workgroups per CU.
  // (An empty split range stages nothing: its first tile would lie past the
  // keys; its partials come out empty.)
  if (it0 < nit) {
    stage_k(0, it0);
    stage_v(it0);
  }
  wait_lds_dma();
  __syncthreads();

  for (int it = it0; it < nit; ++it) {
    const int cur = (it - it0) & 1;
    const int t0 = it * kPfKeys;
    const bool more = it + 1 < nit;
    if (more) stage_k(cur ^ 1, it + 1);
    const bool work = active && t0 <= pos_hi;
    vec8 pb[2][2];  // [tile][query block]: B operand of the P.V step
    if (work) {
      __builtin_amdgcn_s_setprio(0);
      const T* sk = lds + cur * kPfTiles * HC_TILE_ELEMS;
      // S^T blocks: rows = keys 16*tb + 4*g4 + r, column = query 16j + n16.
      f32x4 sacc[4][2];
#pragma unroll
      for (int tb = 0; tb < 4; ++tb)
#pragma unroll
        for (int j = 0; j < 2; ++j) sacc[tb][j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) {
        const T* kt = sk + (tb >> 1) * HC_TILE_ELEMS + (tb & 1) * 4 * 64 * 8;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const vec8 ka = load8(kt + (s * 64 + lane) * 8);
#pragma unroll
          for (int j = 0; j < 2; ++j) sacc[tb][j] = mma_16x16x32(ka, qop[j][s], sacc[tb][j]);
        }
      }
      // The softmax runs at raised wave priority: the SIMD's other wave,
      // in its MFMA phase, then fills the matrix pipe meanwhile.
      __builtin_amdgcn_s_setprio(1);
      const bool need_mask = t0 + kPfKeys - 1 > pos_lo;
      if (need_mask) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int pj = pos_lo + 16 * j + n16;
#pragma unroll
          for (int tb = 0; tb < 4; ++tb)
#pragma unroll
            for (int r = 0; r < 4; ++r)
              if (t0 + 16 * tb + 4 * g4 + r > pj) sacc[tb][j][r] = -INFINITY;
        }
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        // Raw tile maximum (scale > 0), shared by the 4 lanes of a query.
        float mx = -INFINITY;
#pragma unroll
        for (int tb = 0; tb < 4; ++tb)
#pragma unroll
          for (int r = 0; r < 4; ++r) mx = fmaxf(mx, sacc[tb][j][r]);
        mx = rows4_max(mx);
        const float mt = mx * a.scale_log2;
        // Lazy rescaling: the reference maximum m only moves when a tile
        // maximum exceeds it by more than kPfLazy (log2 units), so the O
        // rescale runs on a few tiles per row; probabilities stay below
        // 2^kPfLazy, well inside every input type's range.
        if (__any(mt > m[j] + kPfLazy)) {
          const float mnew = fmaxf(m[j], mt);
          const float alpha = m[j] == -INFINITY ? 0.f : fast_exp2(m[j] - mnew);
          m[j] = mnew;
          l[j] *= alpha;
#pragma unroll
          for (int db = 0; db < 8; ++db)
#pragma unroll
            for (int r = 0; r < 4; ++r) o[db][j][r] *= alpha;
        }
        const float nm = -m[j];
        float p[4][4];
        float ps = 0.f;
#pragma unroll
        for (int tb = 0; tb < 4; ++tb)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            p[tb][r] = fast_exp2(fmaf(sacc[tb][j][r], a.scale_log2, nm));
            ps += p[tb][r];
          }
        l[j] += ps;
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          const float pv[8] = {p[2 * c][0],     p[2 * c][1],     p[2 * c][2],     p[2 * c][3],
                               p[2 * c + 1][0], p[2 * c + 1][1], p[2 * c + 1][2], p[2 * c + 1][3]};
          pb[c][j] = pack8<T>(pv);
        }
      }
      __builtin_amdgcn_s_setprio(0);
    }
    // V(it) (issued before K(it+1)) has landed in every wave's part of the
    // buffer once each wave's older loads are done.  The release fence of
    // __syncthreads() then drains K(it+1) too; a barrier that waits on LDS
    // reads only, keeping K(it+1) in flight over the P.V step, measured no
    // faster, since the loads have landed by then.
    if (more)
      wait_lds_dma_but<kUnitsPerThread>();
    else
      wait_lds_dma();
    __syncthreads();
    if (work) {
      // O^T blocks: rows = channels 16*db + 4*g4 + r, column = query.
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const T* vt = vbuf + c * HC_TILE_ELEMS;
#pragma unroll
        for (int db = 0; db < 8; ++db) {
          const vec8 va = load8(vt + (db * 64 + lane) * 8);
#pragma unroll
          for (int j = 0; j < 2; ++j) o[db][j] = mma_16x16x32(va, pb[c][j], o[db][j]);
        }
      }
    }
    wait_lds_dma();  // K(it+1) has landed
    __syncthreads();  // ... and V(it) is no longer read
    if (more) stage_v(it + 1);
  }

  if (!active) return;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const float lt = rows4_sum(l[j]);
    const int qi = qw0 + 16 * j + n16;
    if (qi >= a.Lq) continue;
    if constexpr (SPLIT) {
      // Split: the unnormalised partial and its (m, l); the merge forms the
      // output (and the statistics).
      float* pp = a.part + (((int64_t)(b * a.Hq + hq) * a.Lq + qi) * a.nsplit + split) * kPfPartStride;
#pragma unroll
      for (int db = 0; db < 8; ++db) *reinterpret_cast<f32x4*>(pp + 16 * db + 4 * g4) = o[db][j];
      if (g4 == 0) {
        pp[HC_HEAD_DIM] = m[j];
        pp[HC_HEAD_DIM + 1] = lt;
      }
      continue;
    }
    const float inv = 1.f / lt;
    // The softmax state of query qi over its visible keys: m is a reference
    // point of the scaled base-2 scores, not a bound -- the lazy rescale
    // lets the true maximum sit up to kPfLazy above it, so a single
    // exp2(score - m) can reach 2^kPfLazy -- and lt is the sum of
    // exp2(score - m).  Consumers use only m + log2(lt), the log-sum-exp,
    // which is exact whatever m is; one that needs p <= 1 per term must
    // renormalise first.
    const int w = qi - (a.Lq - a.st_rows);
    if (a.st && w >= 0 && g4 == 0) {
      float* so = a.st + (((int64_t)b * a.Hq + hq) * a.st_rows + w) * 2;
      so[0] = m[j];
      so[1] = lt;
    }
    T* orow = obase + (int64_t)qi * a.o_st + 4 * g4;
#pragma unroll
    for (int db = 0; db < 8; ++db) {
      typename Quad<T>::type r;
      r.x = Elem<T>::from_f32(o[db][j][0] * inv);
      r.y = Elem<T>::from_f32(o[db][j][1] * inv);
      r.z = Elem<T>::from_f32(o[db][j][2] * inv);
      r.w = Elem<T>::from_f32(o[db][j][3] * inv);
      *reinterpret_cast<typename Quad<T>::type*>(orow + 16 * db) = r;
    }
  }
}

// ---------------------------------------------------------------------------
// Decode-shaped calls (query heads x queries of a KV row <= 16: a decode
// step of the baseline caches, which attend through this entry point, or a
// few-token chunk).  The G*Lq (query head, query) pairs of a KV row are the
// 16 columns of one MFMA block, so each key is read once per row, not once
// per query head; K and V are read in their natural layout (no V re-layout
// pass): K rows are the A operand of S^T = K Q^T as they lie in memory, and
// each wave transposes its V tile through its own LDS buffer into the A
// operand of O^T += V^T P^T, whose k-slots follow the order in which the
// S^T accumulators hold P (k-slot 8g + i <-> token 16*(i/4) + 4g + i%4).
// A workgroup takes one split of the row's 32-token tiles; its four waves
// take every fourth tile of it, are combined in LDS, and the split writes
// one partial of kPfPartStride floats (the split count seen by
// prefill_merge_kernel is the number of splits).
// ---------------------------------------------------------------------------
constexpr int kDvPitch = HC_TILE + 8;            // fp32: transposed V row, 32 k-slots + skew
constexpr int kDvNPitch = HC_HEAD_DIM + 16;      // 16-bit: natural V row, 128 channels + skew
constexpr int kDvWaves = 4;

// Per-wave V buffer (elements): fp32 keeps the tile transposed ([channel][k-slot]);
// 16-bit types keep it in natural layout ([token][channel]) and read the A
// operand with the LDS transpose read.
template <typename T>
constexpr int dv_wave_elems() {
  return sizeof(T) == 4 ? HC_HEAD_DIM * kDvPitch : HC_TILE * kDvNPitch;
}
template <typename T>
constexpr size_t dv_lds_bytes() {
  // The buffers are reused by the end-of-kernel combine of the four waves.
  const size_t v = (size_t)kDvWaves * dv_wave_elems<T>() * sizeof(T);
  const size_t comb = (size_t)kDvWaves * 16 * (HC_HEAD_DIM + 2) * sizeof(float);
  return v > comb ? v : comb;
}

typedef short __attribute__((ext_vector_type(4))) dv_s4;

// gfx950 LDS transpose read (ds_read_b64_tr_b16), 16-bit elements: within
// each 16-lane group, lane i receives {B[i/4 + 4k][i%4] : k < 4}, where
// B[r][e] is element e of the 8 bytes at lane r's address.
__device__ __forceinline__ dv_s4 lds_read_tr16(const void* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) dv_s4*)(p));
}

struct DvArgs {
  PfArgs a;
  int tps;      // tiles per workgroup split
  int ntiles;   // 32-token tiles of the key range
  int ncols;    // G * Lq valid columns
};

template <typename T>
__global__ __launch_bounds__(kDvWaves * 64, sizeof(T) == 4 ? 1 : 2) void prefill_decode_kernel(const DvArgs d) {
  typedef typename Elem<T>::vec8 vec8;
  const PfArgs& a = d.a;
  extern __shared__ __attribute__((aligned(16))) unsigned char dv_lds[];
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g4 = lane >> 4, n16 = lane & 15;
  T* sv = reinterpret_cast<T*>(dv_lds) + wave * dv_wave_elems<T>();
  const int G = a.Hq / a.Hkv;
  const int row = blockIdx.x % a.rows, split = blockIdx.x / a.rows;
  const int b = row / a.Hkv, kvh = row % a.Hkv;
  const int shift = a.Lk - a.Lq;
  // Column n16 of this lane: query head kvh*G + gi, query qi.
  const bool col_ok = n16 < d.ncols;
  const int gi = col_ok ? n16 / a.Lq : 0, qi = col_ok ? n16 % a.Lq : 0;
  const int hq = kvh * G + gi;
  const int lim = shift + qi;  // last visible key of this column
  vec8 qop[4];
  {
    const T* qp = reinterpret_cast<const T*>(a.q) + b * a.q_sb + hq * a.q_sh + (int64_t)qi * a.q_st + 8 * g4;
#pragma unroll
    for (int s = 0; s < 4; ++s) qop[s] = col_ok ? load8(qp + 32 * s) : zero8<T>();
  }
  const T* kb = reinterpret_cast<const T*>(a.k) + b * a.k_sb + kvh * a.k_sh;
  const T* vb = reinterpret_cast<const T*>(a.v) + b * a.v_sb + kvh * a.v_sh;
  const int tile0 = split * d.tps + wave, tile_end = min(split * d.tps + d.tps, d.ntiles);

  // K: A operand rows = tokens t0 + 16h + n16, k-slots = channels 32s + 8*g4 + [0, 8).
  // V: chunk c = lane + 64i of the tile = token c / 16, channels 8*(c % 16) + [0, 8).
  auto load_tile = [&](int tile, vec8 (&kr)[2][4], vec8 (&vr)[8]) {
    const int t0 = tile * HC_TILE;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int t = t0 + 16 * h + n16;
      // Keys past Lk are read from the last one (clamped, branch-free
      // loads); their logits are masked.
      const T* p = kb + (int64_t)min(t, a.Lk - 1) * a.k_st + 8 * g4;
#pragma unroll
      for (int s = 0; s < 4; ++s) kr[h][s] = load8_stream<T>(p + 32 * s);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int c = lane + 64 * i, t = t0 + (c >> 4);
      const vec8 x = load8_stream<T>(vb + (int64_t)min(t, a.Lk - 1) * a.v_st + 8 * (c & 15));
      vr[i] = t < a.Lk ? x : zero8<T>();
    }
  };

  f32x4 o[8];
#pragma unroll
  for (int db = 0; db < 8; ++db) o[db] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;

  auto step = [&](int tile, const vec8 (&kr)[2][4], const vec8 (&vr)[8]) {
    const int t0 = tile * HC_TILE;
    if constexpr (sizeof(T) == 4) {
      // V tile -> transposed LDS rows: channel 8*(c%16) + e, k-slot of token c/16.
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int c = lane + 64 * i, tt = c >> 4, r = tt & 15;
        const int ks = 8 * (r >> 2) + 4 * (tt >> 4) + (r & 3);
#pragma unroll
        for (int e = 0; e < 8; ++e)
          sv[(8 * (c & 15) + e) * kDvPitch + ks] = e < 4 ? vr[i].lo[e] : vr[i].hi[e - 4];
      }
    } else {
      // V tile -> LDS in natural layout, one 16-byte write per chunk.
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int c = lane + 64 * i;
        *reinterpret_cast<vec8*>(sv + (c >> 4) * kDvNPitch + 8 * (c & 15)) = vr[i];
      }
    }
    // S^T = K Q^T: rows = tokens t0 + 16h + 4*g4 + j, column n16.
    f32x4 sacc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int s = 0; s < 4; ++s) sacc[h] = mma_16x16x32(kr[h][s], qop[s], sacc[h]);
    if (t0 + HC_TILE - 1 > shift) {
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (t0 + 16 * h + 4 * g4 + j > lim) sacc[h][j] = -INFINITY;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int j = 0; j < 4; ++j) mx = fmaxf(mx, sacc[h][j]);
    mx = rows4_max(mx);
    const float mt = mx * a.scale_log2;
    if (__any(mt > m + kPfLazy)) {
      const float mnew = fmaxf(m, mt);
      const float alpha = m == -INFINITY ? 0.f : fast_exp2(m - mnew);
      m = mnew;
      l *= alpha;
#pragma unroll
      for (int db = 0; db < 8; ++db) o[db] *= alpha;
    }
    // (m = -inf only while every key so far is masked: p = 0.)
    const float nm = m == -INFINITY ? 0.f : -m;
    float pv[8];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        pv[4 * h + j] = fast_exp2(fmaf(sacc[h][j], a.scale_log2, nm));
        l += pv[4 * h + j];
      }
    const vec8 pb = pack8<T>(pv);
    // The transposed tile is read only after this wave's writes are done.
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int db = 0; db < 8; ++db) {
      vec8 va;
      if constexpr (sizeof(T) == 4) {
        const T* vp = sv + (16 * db + n16) * kDvPitch + 8 * g4;
        va.lo = *reinterpret_cast<const f32x4*>(vp);
        va.hi = *reinterpret_cast<const f32x4*>(vp + 4);
      } else {
        // Lane r of group g4 points at token 16h + 4*g4 + r/4, channels
        // 16db + 4*(r%4) + [0, 4); the transpose hands lane r the channel
        // 16db + r at tokens 16h + 4*g4 + [0, 4): k-slots 4h + [0, 4).
        const T* vp = sv + (4 * g4 + (n16 >> 2)) * kDvNPitch + 16 * db + 4 * (n16 & 3);
        const dv_s4 lo = lds_read_tr16(vp), hi = lds_read_tr16(vp + 16 * kDvNPitch);
        typedef short __attribute__((ext_vector_type(8))) dv_s8;
        const dv_s8 both = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        va = __builtin_bit_cast(vec8, both);
      }
      o[db] = mma_16x16x32(va, pb, o[db]);
    }
    // The next tile's writes follow this tile's reads (in-order LDS per wave).
    __builtin_amdgcn_wave_barrier();
  };

  vec8 ka[2][4], va_[8], kb2[2][4], vb2[8];
  int tile = tile0;
  if (tile < tile_end) load_tile(tile, ka, va_);
  while (tile < tile_end) {
    const int t1 = tile + kDvWaves;
    if (t1 < tile_end) load_tile(t1, kb2, vb2);
    step(tile, ka, va_);
    if (t1 >= tile_end) break;
    const int t2 = t1 + kDvWaves;
    if (t2 < tile_end) load_tile(t2, ka, va_);
    step(t1, kb2, vb2);
    tile = t2;
  }

  // The four waves' states -> one partial of the workgroup's split, through
  // the (now free) LDS: wave w's O^T block, maxima and sums.
  const float lt = rows4_sum(l);
  __syncthreads();  // every wave is done with its V buffer
  float* so = reinterpret_cast<float*>(dv_lds);        // [wave][16 columns][128 channels]
  float* sm = so + kDvWaves * 16 * HC_HEAD_DIM;         // [wave][16]
  float* sl = sm + kDvWaves * 16;                       // [wave][16]
#pragma unroll
  for (int db = 0; db < 8; ++db)
    *reinterpret_cast<f32x4*>(so + (wave * 16 + n16) * HC_HEAD_DIM + 16 * db + 4 * g4) = o[db];
  if (g4 == 0) {
    sm[wave * 16 + n16] = m;
    sl[wave * 16 + n16] = lt;
  }
  __syncthreads();
  // Thread x: column x / 16, channels 8 * (x % 16) + [0, 8).
  const int col = threadIdx.x >> 4, c0 = 8 * (threadIdx.x & 15);
  if (col >= d.ncols) return;
  float M = -INFINITY;
#pragma unroll
  for (int w = 0; w < kDvWaves; ++w) M = fmaxf(M, sm[w * 16 + col]);
  float wt[kDvWaves], L = 0.f;
#pragma unroll
  for (int w = 0; w < kDvWaves; ++w) {
    const float mw = sm[w * 16 + col];
    wt[w] = mw == -INFINITY ? 0.f : fast_exp2(mw - M);
    L = fmaf(sl[w * 16 + col], wt[w], L);
  }
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int w = 0; w < kDvWaves; ++w)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = fmaf(so[(w * 16 + col) * HC_HEAD_DIM + c0 + e], wt[w], acc[e]);
  const int cgi = col / a.Lq, cqi = col % a.Lq, chq = kvh * G + cgi;
  float* pp = a.part + (((int64_t)(b * a.Hq + chq) * a.Lq + cqi) * a.nsplit + split) * kPfPartStride;
  *reinterpret_cast<f32x4*>(pp + c0) = f32x4{acc[0], acc[1], acc[2], acc[3]};
  *reinterpret_cast<f32x4*>(pp + c0 + 4) = f32x4{acc[4], acc[5], acc[6], acc[7]};
  if (c0 == 0) {
    pp[HC_HEAD_DIM] = M;
    pp[HC_HEAD_DIM + 1] = L;
  }
}

// Split partials of one query -> its output row (and, for the last st_rows
// queries, its statistics): one workgroup per (batch, query head, query) of
// kMergeGroups x 128 threads, thread (group, d) summing channel d over the
// splits s = group (mod kMergeGroups).  The splits' maximum and weights
// 2^(m_s - M) are formed once, cooperatively, into LDS, so each thread's sum
// is a run of independent loads; the groups' sums are added in LDS.  Splits
// with no visible key (m = -inf) add nothing.
constexpr int kPfMaxSplits = 1024;
constexpr int kMergeGroups = 4;
constexpr int kMergeThreads = kMergeGroups * HC_HEAD_DIM;
template <typename T>
__global__ __launch_bounds__(kMergeThreads) void prefill_merge_kernel(const PfArgs a) {
  __shared__ float s_w[kPfMaxSplits];
  __shared__ float s_red[kMergeThreads / 64];
  __shared__ float s_acc[kMergeGroups][HC_HEAD_DIM];
  const int64_t qx = blockIdx.x;  // (b * Hq + hq) * Lq + qi
  const int qi = (int)(qx % a.Lq);
  const int bh = (int)(qx / a.Lq);
  const int hq = bh % a.Hq, b = bh / a.Hq;
  const float* pp = a.part + qx * a.nsplit * kPfPartStride;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int d = tid % HC_HEAD_DIM, grp = tid / HC_HEAD_DIM;
  constexpr int nw = kMergeThreads / 64;
  float mloc = -INFINITY;
  for (int s = tid; s < a.nsplit; s += kMergeThreads) mloc = fmaxf(mloc, pp[s * kPfPartStride + HC_HEAD_DIM]);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) mloc = fmaxf(mloc, __shfl_xor(mloc, off, 64));
  if (lane == 0) s_red[wv] = mloc;
  __syncthreads();
  float M = -INFINITY;
#pragma unroll
  for (int w = 0; w < nw; ++w) M = fmaxf(M, s_red[w]);
  __syncthreads();  // s_red is reused below
  float lloc = 0.f;
  for (int s = tid; s < a.nsplit; s += kMergeThreads) {
    const float ms = pp[s * kPfPartStride + HC_HEAD_DIM];
    const float e = ms == -INFINITY ? 0.f : fast_exp2(ms - M);
    s_w[s] = e;
    if (e > 0.f) lloc = fmaf(pp[s * kPfPartStride + HC_HEAD_DIM + 1], e, lloc);
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) lloc += __shfl_xor(lloc, off, 64);
  if (lane == 0) s_red[wv] = lloc;
  __syncthreads();
  float L = 0.f;
#pragma unroll
  for (int w = 0; w < nw; ++w) L += s_red[w];
  float acc = 0.f;
#pragma unroll 8
  for (int s = grp; s < a.nsplit; s += kMergeGroups) {
    const float e = s_w[s];
    const float x = pp[s * kPfPartStride + d];
    acc = e > 0.f ? fmaf(x, e, acc) : acc;
  }
  s_acc[grp][d] = acc;
  __syncthreads();
  if (grp != 0) return;
  float sum = 0.f;
#pragma unroll
  for (int g = 0; g < kMergeGroups; ++g) sum += s_acc[g][d];
  T* o = reinterpret_cast<T*>(a.out) + b * a.o_sb + hq * a.o_sh + (int64_t)qi * a.o_st;
  o[d] = Elem<T>::from_f32(sum / L);
  const int w = qi - (a.Lq - a.st_rows);
  if (a.st && w >= 0 && d == 0) {
    float* so = a.st + (((int64_t)b * a.Hq + hq) * a.st_rows + w) * 2;
    so[0] = M;
    so[1] = L;
  }
}

template <typename T>
int launch_prefill(const PfArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL((v_tiles_kernel<T>), dim3((unsigned)a.vt_tiles, (unsigned)a.rows), dim3(256), 0, stream, a);
  int rc = check_launch("hc_prefill_attn(v tiles)");
  if (rc) return rc;
  static std::once_flag once;
  static hipError_t attr = hipSuccess;
  std::call_once(once, [] {
    attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&prefill_attn_kernel<T, false>),
                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)pf_lds_bytes<T>());
    if (attr == hipSuccess)
      attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&prefill_attn_kernel<T, true>),
                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)pf_lds_bytes<T>());
  });
  if (attr != hipSuccess) return set_error(HC_ERR_HIP, "hc_prefill_attn: %s", hipGetErrorString(attr));
  const int64_t grid = (int64_t)a.rows * (a.Hq / a.Hkv) * a.nqb * a.nsplit;
  if (a.nsplit > 1)
    hipLaunchKernelGGL((prefill_attn_kernel<T, true>), dim3((unsigned)grid), dim3(kPfThreads), pf_lds_bytes<T>(),
                       stream, a);
  else
    hipLaunchKernelGGL((prefill_attn_kernel<T, false>), dim3((unsigned)grid), dim3(kPfThreads), pf_lds_bytes<T>(),
                       stream, a);
  if ((rc = check_launch("hc_prefill_attn"))) return rc;
  if (a.nsplit > 1) {
    const int64_t nq = (int64_t)(a.rows / a.Hkv) * a.Hq * a.Lq;
    hipLaunchKernelGGL((prefill_merge_kernel<T>), dim3((unsigned)nq), dim3(kMergeThreads), 0, stream, a);
    rc = check_launch("hc_prefill_attn(merge)");
  }
  return rc;
}

template <typename T>
int launch_decode_shaped(const DvArgs& d, hipStream_t stream) {
  static std::once_flag once;
  static hipError_t attr = hipSuccess;
  std::call_once(once, [] {
    attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&prefill_decode_kernel<T>),
                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)dv_lds_bytes<T>());
  });
  if (attr != hipSuccess) return set_error(HC_ERR_HIP, "hc_prefill_attn: %s", hipGetErrorString(attr));
  const int64_t grid = (int64_t)d.a.rows * d.a.nsplit;
  hipLaunchKernelGGL((prefill_decode_kernel<T>), dim3((unsigned)grid), dim3(kDvWaves * 64), dv_lds_bytes<T>(), stream,
                     d);
  int rc = check_launch("hc_prefill_attn(decode-shaped)");
  if (rc) return rc;
  const int64_t nq = (int64_t)(d.a.rows / d.a.Hkv) * d.a.Hq * d.a.Lq;
  hipLaunchKernelGGL((prefill_merge_kernel<T>), dim3((unsigned)nq), dim3(kMergeThreads), 0, stream, d.a);
  return check_launch("hc_prefill_attn(merge)");
}

// Resident workgroups of the decode-shaped kernel on the current device.
template <typename T>
int decode_shaped_slots() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  static std::mutex mu;
  static int cache[64];
  std::lock_guard<std::mutex> lock(mu);
  if (cache[dev] > 0) return cache[dev];
  const void* fn = reinterpret_cast<const void*>(&prefill_decode_kernel<T>);
  int per_cu = 0, cus = 0;
  if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)dv_lds_bytes<T>()) != hipSuccess)
    return 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kDvWaves * 64, dv_lds_bytes<T>()) != hipSuccess)
    return 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  cache[dev] = (per_cu > 0 ? per_cu : 1) * (cus > 0 ? cus : 1);
  return cache[dev];
}

// Workgroup splits of a decode-shaped call (0: not decode-shaped).  At most
// 16 (query head, query) columns per KV row and at least kDvMinTiles tiles
// of keys; each wave keeps at least kDvMinWaveTiles tiles; the grid aims at
// one resident round.
constexpr int kDvMinTiles = 32;
constexpr int kDvMinWaveTiles = 4;
int decode_shaped_splits(int dtype, int batch, int q_heads, int kv_heads, int q_len, int kv_len) {
  if (batch <= 0 || kv_heads <= 0 || q_heads <= 0 || q_heads % kv_heads) return 0;
  if ((q_heads / kv_heads) * q_len > 16) return 0;
  const int ntiles = (kv_len + HC_TILE - 1) / HC_TILE;
  if (ntiles < kDvMinTiles) return 0;
  const int slots = dtype == HC_DTYPE_F32 ? decode_shaped_slots<float>()
                    : dtype == HC_DTYPE_F16 ? decode_shaped_slots<_Float16>()
                                            : decode_shaped_slots<__bf16>();
  if (slots <= 0) return 0;
  const int rows = batch * kv_heads;
  const int by_slots = std::max(1, slots / rows);
  const int by_keys = std::max(1, ntiles / (kDvWaves * kDvMinWaveTiles));
  return std::min(std::min(by_slots, by_keys), kPfMaxSplits);
}

// Workgroups of the attention kernel resident on the current device at once
// (0 when the query fails), cached per device and element size.
template <typename T>
int prefill_slots() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  static std::mutex mu;
  static int cache[64];
  std::lock_guard<std::mutex> lock(mu);
  if (cache[dev] > 0) return cache[dev];
  int per_cu = 0, cus = 0;
  const void* fn = reinterpret_cast<const void*>(&prefill_attn_kernel<T, true>);
  if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)pf_lds_bytes<T>()) != hipSuccess)
    return 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kPfThreads, pf_lds_bytes<T>()) != hipSuccess)
    return 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  cache[dev] = (per_cu > 0 ? per_cu : 1) * (cus > 0 ? cus : 1);
  return cache[dev];
}

// Key splits for a launch: a split only pays where one query block per
// (row, query head) leaves most of the device idle over a long key range
// (decode-like and short-chunk calls).  Each split keeps at least
// kPfMinSplitIts iterations; the split grid aims at one resident round.
constexpr int kPfMinSplitIts = 8;
int prefill_nsplit(int dtype, int batch, int q_heads, int kv_heads, int q_len, int kv_len) {
  if (q_len > kPfBlockQ || batch <= 0 || q_heads <= 0 || kv_heads <= 0) return 1;
  const int slots = dtype == HC_DTYPE_F32 ? prefill_slots<float>()
                    : dtype == HC_DTYPE_F16 ? prefill_slots<_Float16>()
                                            : prefill_slots<__bf16>();
  const int64_t natural = (int64_t)batch * q_heads;  // one query block per (row, query head)
  if (slots <= 0 || 2 * natural > slots) return 1;
  const int nit = (kv_len + kPfKeys - 1) / kPfKeys;
  const int by_keys = nit / kPfMinSplitIts;
  const int by_slots = (int)(slots / natural);
  const int n = std::min(std::min(by_keys, by_slots), kPfMaxSplits);
  return n >= 2 ? n : 1;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// Tiles per row of the V tile buffer: kv_len rounded up to whole iterations.
int64_t v_tiles_per_row(int kv_len) {
  const int64_t it = ((int64_t)kv_len + kPfKeys - 1) / kPfKeys;
  return it * kPfTiles;
}

}  // namespace
}  // namespace hc

using namespace hc;

extern "C" size_t hc_prefill_workspace_size(int dtype, int batch, int kv_heads, int kv_len) {
  const int esz = dtype == HC_DTYPE_F32 ? 4 : 2;
  if (batch <= 0 || kv_heads <= 0 || kv_len <= 0) return 0;
  return (size_t)batch * kv_heads * v_tiles_per_row(kv_len) * HC_TILE_ELEMS * esz;
}

static size_t pf_align256(size_t x) { return (x + 255) / 256 * 256; }

// Split partials after the V tiles: [batch * q_heads * q_len][nsplit][kPfPartStride] floats.
static size_t pf_part_bytes(int batch, int q_heads, int q_len, int nsplit) {
  return nsplit > 1 ? (size_t)batch * q_heads * q_len * nsplit * kPfPartStride * sizeof(float) : 0;
}

extern "C" size_t hc_prefill_workspace_bytes(int dtype, int batch, int q_heads, int kv_heads, int q_len,
                                             int kv_len) {
  const size_t vt = hc_prefill_workspace_size(dtype, batch, kv_heads, kv_len);
  if (vt == 0 || q_heads <= 0 || q_len <= 0) return vt;
  const int dv = decode_shaped_splits(dtype, batch, q_heads, kv_heads, q_len, kv_len);
  if (dv > 0) return pf_align256(vt) + pf_part_bytes(batch, q_heads, q_len, dv);
  const int ns = prefill_nsplit(dtype, batch, q_heads, kv_heads, q_len, kv_len);
  return ns > 1 ? pf_align256(vt) + pf_part_bytes(batch, q_heads, q_len, ns) : vt;
}

static int prefill_entry(int dtype, const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                         const void* v, const int64_t* v_strides, void* out, const int64_t* out_strides, int batch,
                         int q_heads, int kv_heads, int q_len, int kv_len, float scale, void* workspace,
                         size_t workspace_bytes, int stat_rows, float* stat_out, void* stream);

extern "C" int hc_prefill_attn(int dtype, const void* q, const int64_t* q_strides, const void* k,
                               const int64_t* k_strides, const void* v, const int64_t* v_strides, void* out,
                               const int64_t* out_strides, int batch, int q_heads, int kv_heads, int q_len,
                               int kv_len, float scale, void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  return prefill_entry(dtype, q, q_strides, k, k_strides, v, v_strides, out, out_strides, batch, q_heads, kv_heads,
                       q_len, kv_len, scale, workspace, workspace_bytes, 0, nullptr, stream);
}

extern "C" int hc_prefill_attn_stats(int dtype, const void* q, const int64_t* q_strides, const void* k,
                                     const int64_t* k_strides, const void* v, const int64_t* v_strides, void* out,
                                     const int64_t* out_strides, int batch, int q_heads, int kv_heads, int q_len,
                                     int kv_len, float scale, void* workspace, size_t workspace_bytes, int stat_rows,
                                     float* stat_out, void* stream) {
  clear_error();
  if (stat_rows < 1 || stat_rows > q_len || !stat_out)
    return set_error(HC_ERR_INVALID, "hc_prefill_attn_stats: stat_rows=%d (q_len %d), stat_out %s", stat_rows, q_len,
                     stat_out ? "given" : "null");
  return prefill_entry(dtype, q, q_strides, k, k_strides, v, v_strides, out, out_strides, batch, q_heads, kv_heads,
                       q_len, kv_len, scale, workspace, workspace_bytes, stat_rows, stat_out, stream);
}

static int prefill_entry(int dtype, const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                         const void* v, const int64_t* v_strides, void* out, const int64_t* out_strides, int batch,
                         int q_heads, int kv_heads, int q_len, int kv_len, float scale, void* workspace,
                         size_t workspace_bytes, int stat_rows, float* stat_out, void* stream) {
  const int esz = dtype == HC_DTYPE_F32 ? 4 : (dtype == HC_DTYPE_BF16 || dtype == HC_DTYPE_F16) ? 2 : 0;
  if (esz == 0) return set_error(HC_ERR_INVALID, "hc_prefill_attn: unknown dtype %d", dtype);
  if (batch < 0 || q_heads <= 0 || kv_heads <= 0 || q_heads % kv_heads || q_len < 0 || kv_len < 0)
    return set_error(HC_ERR_INVALID, "hc_prefill_attn: batch=%d q_heads=%d kv_heads=%d q_len=%d kv_len=%d", batch,
                     q_heads, kv_heads, q_len, kv_len);
  if (q_len > kv_len)
    return set_error(HC_ERR_INVALID, "hc_prefill_attn: q_len %d exceeds kv_len %d (queries are the last keys)", q_len,
                     kv_len);
  if (batch == 0 || q_len == 0) return HC_OK;
  if (!q || !k || !v || !out || !q_strides || !k_strides || !v_strides || !out_strides)
    return set_error(HC_ERR_INVALID, "hc_prefill_attn: null pointer argument");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out))
    return set_error(HC_ERR_INVALID, "hc_prefill_attn: buffers must be 16-byte aligned");
  const int64_t* st[4] = {q_strides, k_strides, v_strides, out_strides};
  for (int i = 0; i < 4; ++i)
    for (int j = 0; j < 3; ++j)
      if (st[i][j] < 0 || (st[i][j] * esz) % 16)
        return set_error(HC_ERR_INVALID, "hc_prefill_attn: strides must be non-negative 16-byte multiples");
  const int64_t max_tok_stride = std::max(k_strides[2], v_strides[2]);
  if ((int64_t)kPfKeys * max_tok_stride * esz >= (int64_t)1 << 31)
    return set_error(HC_ERR_INVALID, "hc_prefill_attn: K/V token strides too large");
  if (!std::isfinite(scale) || !(scale > 0.f))
    return set_error(HC_ERR_INVALID, "hc_prefill_attn: scale must be finite and positive");
  const size_t need = hc_prefill_workspace_size(dtype, batch, kv_heads, kv_len);
  if (!workspace || workspace_bytes < need || !aligned16(workspace))
    return set_error(HC_ERR_INVALID, "hc_prefill_attn: workspace too small or unaligned (%zu < %zu bytes)",
                     workspace_bytes, need);
  PfArgs a;
  a.q = q;
  a.k = k;
  a.v = v;
  a.vt = workspace;
  a.out = out;
  a.q_sb = q_strides[0], a.q_sh = q_strides[1], a.q_st = q_strides[2];
  a.k_sb = k_strides[0], a.k_sh = k_strides[1], a.k_st = k_strides[2];
  a.v_sb = v_strides[0], a.v_sh = v_strides[1], a.v_st = v_strides[2];
  a.o_sb = out_strides[0], a.o_sh = out_strides[1], a.o_st = out_strides[2];
  a.Hq = q_heads;
  a.Hkv = kv_heads;
  a.Lq = q_len;
  a.Lk = kv_len;
  a.nqb = (q_len + kPfBlockQ - 1) / kPfBlockQ;
  a.vt_tiles = (int)v_tiles_per_row(kv_len);
  a.rows = batch * kv_heads;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.st = stat_out;
  a.st_rows = stat_rows;
  // A key split when it pays and the caller's workspace holds its partials
  // (hc_prefill_workspace_bytes); otherwise one pass over the keys.
  a.nsplit = 1;
  a.its = 1 << 30;
  a.part = nullptr;
  hipStream_t s = (hipStream_t)stream;
  // Decode-shaped calls: the packed-column kernel over natural-layout K/V.
  const int dv = decode_shaped_splits(dtype, batch, q_heads, kv_heads, q_len, kv_len);
  if (dv > 0 && workspace_bytes >= pf_align256(need) + pf_part_bytes(batch, q_heads, q_len, dv)) {
    DvArgs d;
    a.nsplit = dv;
    a.part = reinterpret_cast<float*>(reinterpret_cast<char*>(workspace) + pf_align256(need));
    d.a = a;
    d.ntiles = (kv_len + HC_TILE - 1) / HC_TILE;
    d.tps = (d.ntiles + dv - 1) / dv;
    d.ncols = (q_heads / kv_heads) * q_len;
    switch (dtype) {
      case HC_DTYPE_BF16: return launch_decode_shaped<__bf16>(d, s);
      case HC_DTYPE_F16: return launch_decode_shaped<_Float16>(d, s);
      default: return launch_decode_shaped<float>(d, s);
    }
  }
  const int ns = prefill_nsplit(dtype, batch, q_heads, kv_heads, q_len, kv_len);
  if (ns > 1 && workspace_bytes >= pf_align256(need) + pf_part_bytes(batch, q_heads, q_len, ns)) {
    const int nit = (kv_len + kPfKeys - 1) / kPfKeys;
    a.nsplit = ns;
    a.its = (nit + ns - 1) / ns;
    a.part = reinterpret_cast<float*>(reinterpret_cast<char*>(workspace) + pf_align256(need));
  }
  const int64_t grid = (int64_t)a.rows * (q_heads / kv_heads) * a.nqb * a.nsplit;
  if (grid > 0x7fffffffLL) return set_error(HC_ERR_INVALID, "hc_prefill_attn: grid too large");
  switch (dtype) {
    case HC_DTYPE_BF16: return launch_prefill<__bf16>(a, s);
    case HC_DTYPE_F16: return launch_prefill<_Float16>(a, s);
    default: return launch_prefill<float>(a, s);
  }
}
