// Writers and readers of the tiled ragged per-head KV store.
//
//   hc_gather_store  rows of a natural-layout [.., tokens, 128] source (device
//                    memory or a device-mapped host-pinned buffer) gathered by
//                    an index list into store slots [0, count) of a row.
//                    Serves the prefill keep-head copy
//                    (heterocache/cache_utils.py:914-937), the compressed-head
//                    gather + index_copy_ (heterocache/cache_utils.py:854-877)
//                    and the retrieval upload from the host tier
//                    (heterocache/cache_utils.py:1097-1123).
//   hc_append        one decode token per row at slot len[row], then len+1
//                    (heterocache/cache_utils.py:970-1005).
//   hc_store_read    unpack store slots [0, count) of rows back to natural
//                    layout (diagnostics and tests).
//   hc_gather_rows   natural-layout token rows picked by index lists, into a
//                    natural-layout destination (the baseline compressors'
//                    kept-token gathers, heterocache/kv_cluster.py).
//   hc_copy_rows     natural-layout token rows of selected heads copied to a
//                    natural-layout destination, typically the host-pinned
//                    full-KV tier (heterocache/cache_utils.py:939-967), by a
//                    capped number of workgroups so the copy runs at link
//                    speed beside compute instead of occupying the device.
#include <algorithm>

#include "hc_common.h"
#include "hc_internal.h"

namespace hc {

// A workgroup moves one 32-token tile of one job at a time through LDS:
// natural-layout 16-byte reads in, tile-permuted 16-byte writes out.  Work
// items (job, tile) are strided over the grid, so a host-sourced gather can
// run on a few workgroups: its reads wait on the host link, and a full grid
// would hold CU slots the decode kernel (sized to fill the device) needs.
template <typename T>
__global__ __launch_bounds__(256) void gather_store_kernel(
    const T* __restrict__ src_k, const T* __restrict__ src_v, const int64_t* __restrict__ src_off,
    int64_t src_tok_stride, int src_len, const int32_t* __restrict__ idx, const int64_t* __restrict__ idx_off,
    const int32_t* __restrict__ count, const int32_t* __restrict__ dst_row, T* __restrict__ kstore,
    T* __restrict__ vstore, const int64_t* __restrict__ row_tile_off, const int32_t* __restrict__ trigger,
    const int32_t* __restrict__ trig_of, int njobs, int tiles_per_job, const int64_t* __restrict__ src_k_addr,
    const int64_t* __restrict__ src_v_addr, int32_t* __restrict__ set_len) {
  __shared__ T sk[HC_TILE][HC_HEAD_DIM + 8];
  __shared__ T sv[HC_TILE][HC_HEAD_DIM + 8];
  const int64_t items = (int64_t)njobs * tiles_per_job;
  // set_len: each copied row's length becomes its count (workgroup 0; the
  // lengths are read only by later launches).
  if (set_len && blockIdx.x == 0)
    for (int j = threadIdx.x; j < njobs; j += blockDim.x)
      if (!trigger || trigger[trig_of ? trig_of[j] : 0] != 0) set_len[dst_row[j]] = count[j];
  const int lane = threadIdx.x & 63;
  // The workgroup's items are blockIdx.x + i * gridDim.x.  They are taken 64
  // at a time: lane i reads item i's trigger flag and count, and a ballot
  // keeps the live items, so gated-off and empty items cost one round trip
  // per 64 instead of one each (a small host-sourced grid walks many items).
  // Every wave computes the same mask, so all threads run the same items.
  for (int64_t base = blockIdx.x; base < items; base += (int64_t)gridDim.x * 64) {
  bool live = false;
  {
    const int64_t it = base + (int64_t)lane * gridDim.x;
    if (it < items) {
      const int jb = (int)(it / tiles_per_job);
      live = (!trigger || trigger[trig_of ? trig_of[jb] : 0] != 0) &&
             (int)(it % tiles_per_job) * HC_TILE < count[jb];
    }
  }
  uint64_t live_mask = __ballot(live);
  while (live_mask) {
  const int64_t item = base + (int64_t)__builtin_ctzll(live_mask) * gridDim.x;
  live_mask &= live_mask - 1;
  const int job = (int)(item / tiles_per_job);
  const int tile = (int)(item % tiles_per_job);
  const int n = count[job];
  const int tok0 = tile * HC_TILE;
  const int valid = min(HC_TILE, n - tok0);

  // Per-job source tensors (src_*_addr: device addresses, one per job) or
  // one base for all jobs.
  const T* bk = (src_k_addr ? reinterpret_cast<const T*>(src_k_addr[job]) : src_k) + src_off[job];
  const T* bv = (src_v_addr ? reinterpret_cast<const T*>(src_v_addr[job]) : src_v) + src_off[job];
  const int32_t* ix = idx ? idx + idx_off[job] : nullptr;
  // 32 tokens x 16 chunks of 8 elements, two chunks per thread.  All four
  // loads are issued before the first wait: a chunk past the item's last
  // token reads the last token's row again (in the source, not stored).
  static_assert(HC_TILE * 16 == 2 * 256, "two 8-element chunks per thread");
  typename Elem<T>::vec8 ra[2], rb[2];
  int pos[2];  // both positions first: an index read after the first row
               // loads would wait for them (the wait counter is in order)
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int t = min((threadIdx.x + 256 * q) >> 4, valid - 1);
    pos[q] = ix ? ix[tok0 + t] : tok0 + t;
  }
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int ch = (threadIdx.x + 256 * q) & 15;
    // Positions are clamped into the source like the reference's
    // clamp(max=L-1) before its gather (heterocache/cache_utils.py:852).
    const int64_t stok = ix ? (int64_t)min(max(pos[q], 0), src_len - 1) : (int64_t)pos[q];
    const int64_t off = stok * src_tok_stride + ch * 8;
    // Each source row is read once: streamed past L2 (the prefill
    // compression of a 128K Llama-3-8B layer, two gathers and the scorer,
    // 0.204 -> 0.200 ms).
    ra[q] = load8_stream_global<T>(bk + off);
    rb[q] = load8_stream_global<T>(bv + off);
  }
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int c = threadIdx.x + 256 * q;
    const int t = c >> 4, ch = c & 15;
    if (t < valid) {
      const typename Elem<T>::vec8 a = ra[q], b = rb[q];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if constexpr (sizeof(T) == 4) {
          sk[t][ch * 8 + e] = e < 4 ? a.lo[e] : a.hi[e - 4];
          sv[t][ch * 8 + e] = e < 4 ? b.lo[e] : b.hi[e - 4];
        } else {
          sk[t][ch * 8 + e] = a[e];
          sv[t][ch * 8 + e] = b[e];
        }
      }
    }
  }
  __syncthreads();

  const int64_t tile_base = (row_tile_off[dst_row[job]] + tile) * (int64_t)HC_TILE_ELEMS;
  T* kt = kstore + tile_base;
  T* vt = vstore + tile_base;
  for (int c = threadIdx.x; c < HC_TILE_ELEMS / 8; c += 256) {
    // K chunk c = ((h*4+s)*4+g)*16+m : token 16h+m, channels 32s+8g+[0,8).
    {
      const int m = c & 15, g = (c >> 4) & 3, s = (c >> 6) & 3, h = c >> 8;
      const int t = 16 * h + m;
      if (t < valid) {
        float v8[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) v8[e] = Elem<T>::to_f32(sk[t][32 * s + 8 * g + e]);
        *reinterpret_cast<typename Elem<T>::vec8*>(kt + c * 8) = pack8<T>(v8);
      }
    }
    // V chunk c = (mt*4+g)*16+nn : channel 16mt+nn, tokens 16*(i/4)+4g+i%4.
    {
      const int nn = c & 15, g = (c >> 4) & 3, mt = c >> 6;
      const int d = 16 * mt + nn;
      if (valid == HC_TILE) {
        float v8[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) v8[i] = Elem<T>::to_f32(sv[16 * (i >> 2) + 4 * g + (i & 3)][d]);
        *reinterpret_cast<typename Elem<T>::vec8*>(vt + c * 8) = pack8<T>(v8);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int t = 16 * (i >> 2) + 4 * g + (i & 3);
          if (t < valid) vt[c * 8 + i] = sv[t][d];
        }
      }
    }
  }
  __syncthreads();  // the next item refills the LDS tiles
  }
  }
}

// One wave per row: store the row's new token at slot len, then len += 1.
template <typename T>
__global__ __launch_bounds__(64) void append_kernel(const T* __restrict__ k_new, const T* __restrict__ v_new,
                                                    int64_t src_row_stride, T* __restrict__ kstore,
                                                    T* __restrict__ vstore, const int64_t* __restrict__ row_tile_off,
                                                    int32_t* __restrict__ row_len, const int32_t* __restrict__ row_cap,
                                                    int32_t* __restrict__ status) {
  const int row = blockIdx.x;
  const int len = row_len[row];
  if (len >= row_cap[row]) {
    if (threadIdx.x == 0 && status) atomicOr(status, 1);
    return;
  }
  const int tile = len / HC_TILE, t = len % HC_TILE;
  const int64_t base = (row_tile_off[row] + tile) * (int64_t)HC_TILE_ELEMS;
  const T* ks = k_new + (int64_t)row * src_row_stride;
  const T* vs = v_new + (int64_t)row * src_row_stride;
  for (int d = threadIdx.x; d < HC_HEAD_DIM; d += 64) {
    kstore[base + k_tile_offset(t, d)] = ks[d];
    vstore[base + v_tile_offset(t, d)] = vs[d];
  }
  __syncthreads();
  if (threadIdx.x == 0) row_len[row] = len + 1;
}

template <typename T>
__global__ __launch_bounds__(256) void store_read_kernel(const T* __restrict__ kstore, const T* __restrict__ vstore,
                                                         const int64_t* __restrict__ row_tile_off,
                                                         const int32_t* __restrict__ rows_sel, int count,
                                                         T* __restrict__ dst_k, T* __restrict__ dst_v) {
  const int j = blockIdx.y;
  const int row = rows_sel[j];
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= (int64_t)count * HC_HEAD_DIM) return;
  const int tok = (int)(e / HC_HEAD_DIM), d = (int)(e % HC_HEAD_DIM);
  const int64_t base = (row_tile_off[row] + tok / HC_TILE) * (int64_t)HC_TILE_ELEMS;
  dst_k[(int64_t)j * count * HC_HEAD_DIM + e] = kstore[base + k_tile_offset(tok % HC_TILE, d)];
  dst_v[(int64_t)j * count * HC_HEAD_DIM + e] = vstore[base + v_tile_offset(tok % HC_TILE, d)];
}

// Workgroups of a gather whose source is host memory read over the link.
constexpr int kHostGatherWorkgroups = 64;  // default cap of a host-sourced gather's grid

template <typename T>
static int launch_gather_store(const void* src_k, const void* src_v, const int64_t* src_off, int64_t src_tok_stride,
                               int src_len, const int32_t* idx, const int64_t* idx_off, const int32_t* count,
                               const int32_t* dst_row, void* kstore, void* vstore, const int64_t* row_tile_off,
                               int njobs, int max_count, const int32_t* trigger, const int32_t* trig_of,
                               bool host_src, int max_workgroups, hipStream_t s,
                               const int64_t* src_k_addr = nullptr, const int64_t* src_v_addr = nullptr,
                               int32_t* set_len = nullptr) {
  const int tiles = (max_count + HC_TILE - 1) / HC_TILE;
  const int64_t items = (int64_t)tiles * njobs;
  const int64_t cap = max_workgroups > 0 ? max_workgroups : (host_src ? kHostGatherWorkgroups : items);
  // At least one workgroup: with set_len a launch of no tiles still writes
  // the lengths.
  const unsigned grid = (unsigned)std::max<int64_t>(1, std::min<int64_t>(items, cap));
  hipLaunchKernelGGL((gather_store_kernel<T>), dim3(grid), dim3(256), 0, s, (const T*)src_k, (const T*)src_v, src_off,
                     src_tok_stride, src_len, idx, idx_off, count, dst_row, (T*)kstore, (T*)vstore, row_tile_off, trigger,
                     trig_of, njobs, tiles, src_k_addr, src_v_addr, set_len);
  return check_launch("hc_gather_store");
}

// Work item = (job, 32-token chunk); workgroups stride over the items, so a
// small grid streams any amount.  Rows are moved as 16-byte vectors.
constexpr int kCopyChunk = 32;

__global__ __launch_bounds__(256) void copy_rows_kernel(const uint8_t* __restrict__ src_k,
                                                       const uint8_t* __restrict__ src_v,
                                                       const int64_t* __restrict__ src_off, int64_t src_stride_b,
                                                       uint8_t* __restrict__ dst_k, uint8_t* __restrict__ dst_v,
                                                       const int64_t* __restrict__ dst_off, int64_t dst_stride_b,
                                                       const int32_t* __restrict__ count, int njobs,
                                                       int chunks_per_job, int vecs_per_row, int esz,
                                                       const int32_t* __restrict__ idx, int64_t idx_stride,
                                                       int src_len) {
  const int64_t items = (int64_t)njobs * chunks_per_job;
  for (int64_t item = blockIdx.x; item < items; item += gridDim.x) {
    const int job = (int)(item / chunks_per_job), chunk = (int)(item % chunks_per_job);
    const int t0 = chunk * kCopyChunk;
    const int valid = min(kCopyChunk, count[job] - t0);
    if (valid <= 0) continue;
    // Source token of destination token t: t itself, or idx[job][t] clamped
    // into [0, src_len) when an index list is given.
    const int32_t* ix = idx ? idx + (int64_t)job * idx_stride + t0 : nullptr;
    const int64_t so = (src_off[job] * esz) + (ix ? 0 : (int64_t)t0 * src_stride_b);
    const int64_t dofs = (dst_off[job] * esz) + (int64_t)t0 * dst_stride_b;
    const int n = valid * vecs_per_row;
    for (int c0 = threadIdx.x; c0 < n; c0 += 2 * 256) {
      // Two vectors of K and two of V in flight per thread.
      u32x4 a[2], b[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int c = c0 + u * 256;
        if (c < n) {
          const int r = c / vecs_per_row;
          const int64_t tok = ix ? (int64_t)min(max(ix[r], 0), src_len - 1) : r;
          const int64_t off = tok * src_stride_b + (c % vecs_per_row) * 16;
          a[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src_k + so + off));
          b[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src_v + so + off));
        }
      }
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int c = c0 + u * 256;
        if (c < n) {
          const int64_t off = (int64_t)(c / vecs_per_row) * dst_stride_b + (c % vecs_per_row) * 16;
          *reinterpret_cast<u32x4*>(dst_k + dofs + off) = a[u];
          *reinterpret_cast<u32x4*>(dst_v + dofs + off) = b[u];
        }
      }
    }
  }
}

// Translate a pointer into host-pinned memory to its device-mapped address.
static int map_host_ptr(const void* host, const void** dev) {
  void* d = nullptr;
  hipError_t e = hipHostGetDevicePointer(&d, const_cast<void*>(host), 0);
  if (e != hipSuccess)
    return set_error(HC_ERR_INVALID, "source is not device-mapped pinned host memory: %s", hipGetErrorString(e));
  *dev = d;
  return HC_OK;
}

}  // namespace hc

using namespace hc;

extern "C" int hc_gather_store(int dtype, const void* src_k, const void* src_v, int src_is_host,
                               const int64_t* src_off, int64_t src_tok_stride, int src_len, const int32_t* idx,
                               const int64_t* idx_off, const int32_t* count, const int32_t* dst_row, void* kstore,
                               void* vstore, const int64_t* row_tile_off, int njobs, int max_count,
                               const int32_t* trigger, const int32_t* trig_of, int max_workgroups, int32_t* set_len,
                               void* stream) {
  clear_error();
  if (njobs < 0 || max_count < 0 || njobs > 65535 || max_workgroups < 0)
    return set_error(HC_ERR_INVALID, "hc_gather_store: njobs=%d max_count=%d", njobs, max_count);
  if (njobs == 0) return HC_OK;
  if (max_count == 0 && !set_len) return HC_OK;
  if (src_len <= 0) return set_error(HC_ERR_INVALID, "hc_gather_store: src_len=%d", src_len);
  if (!idx && max_count > src_len)
    return set_error(HC_ERR_INVALID, "hc_gather_store: identity copy of %d tokens from a %d-token source", max_count,
                     src_len);
  if (!src_k || !src_v || !src_off || !count || !dst_row || !kstore || !vstore || !row_tile_off ||
      (idx && !idx_off))
    return set_error(HC_ERR_INVALID, "hc_gather_store: null pointer argument");
  if (src_tok_stride < HC_HEAD_DIM || (src_tok_stride % 8) != 0)
    return set_error(HC_ERR_INVALID, "hc_gather_store: token stride %lld must be >=128 and a multiple of 8",
                     (long long)src_tok_stride);
  const void* sk = src_k;
  const void* sv = src_v;
  if (src_is_host) {
    int rc = map_host_ptr(src_k, &sk);
    if (rc) return rc;
    rc = map_host_ptr(src_v, &sv);
    if (rc) return rc;
  }
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case HC_DTYPE_BF16:
      return launch_gather_store<__bf16>(sk, sv, src_off, src_tok_stride, src_len, idx, idx_off, count, dst_row, kstore,
                                         vstore, row_tile_off, njobs, max_count, trigger, trig_of, src_is_host != 0, max_workgroups, s,
                                         nullptr, nullptr, set_len);
    case HC_DTYPE_F16:
      return launch_gather_store<_Float16>(sk, sv, src_off, src_tok_stride, src_len, idx, idx_off, count, dst_row, kstore,
                                           vstore, row_tile_off, njobs, max_count, trigger, trig_of, src_is_host != 0, max_workgroups, s,
                                         nullptr, nullptr, set_len);
    case HC_DTYPE_F32:
      return launch_gather_store<float>(sk, sv, src_off, src_tok_stride, src_len, idx, idx_off, count, dst_row, kstore,
                                        vstore, row_tile_off, njobs, max_count, trigger, trig_of, src_is_host != 0, max_workgroups, s,
                                         nullptr, nullptr, set_len);
    default:
      return set_error(HC_ERR_INVALID, "hc_gather_store: unknown dtype %d", dtype);
  }
}

extern "C" int hc_gather_store_groups(int dtype, const void* src_k, const void* src_v, int src_is_host,
                                      const int64_t* src_off, const int64_t* group_tok_stride, int src_len,
                                      const int32_t* idx, const int64_t* idx_off, const int32_t* count,
                                      const int32_t* dst_row, void* kstore, void* vstore,
                                      const int64_t* row_tile_off, int ngroups, const int32_t* group_begin,
                                      const int32_t* group_max_count, const int32_t* trigger,
                                      const int32_t* trig_of, int max_workgroups, void* const* events,
                                      const int64_t* src_k_addr, const int64_t* src_v_addr, void* stream) {
  clear_error();
  if (ngroups < 0 || ngroups > 65535 || max_workgroups < 0)
    return set_error(HC_ERR_INVALID, "hc_gather_store_groups: ngroups=%d", ngroups);
  if (ngroups == 0) return HC_OK;
  if (!group_begin || !group_max_count || !group_tok_stride)
    return set_error(HC_ERR_INVALID, "hc_gather_store_groups: null group array");
  for (int g = 0; g < ngroups; ++g) {
    if (group_begin[g + 1] < group_begin[g] || group_begin[g] < 0 || group_max_count[g] < 0)
      return set_error(HC_ERR_INVALID, "hc_gather_store_groups: group %d spans jobs [%d, %d), max count %d", g,
                       group_begin[g], group_begin[g + 1], group_max_count[g]);
  }
  if (group_begin[ngroups] > 65535)
    return set_error(HC_ERR_INVALID, "hc_gather_store_groups: %d jobs", group_begin[ngroups]);
  // Every group is validated before anything is launched, so an invalid
  // group leaves no earlier group half done.
  for (int g = 0; g < ngroups; ++g) {
    const int nj = group_begin[g + 1] - group_begin[g];
    if (nj == 0 || group_max_count[g] == 0) continue;
    if (src_len <= 0) return set_error(HC_ERR_INVALID, "hc_gather_store_groups: src_len=%d", src_len);
    if (!idx && group_max_count[g] > src_len)
      return set_error(HC_ERR_INVALID, "hc_gather_store_groups: identity copy of %d tokens from a %d-token source",
                       group_max_count[g], src_len);
    if (group_tok_stride[g] < HC_HEAD_DIM || (group_tok_stride[g] % 8) != 0)
      return set_error(HC_ERR_INVALID, "hc_gather_store_groups: group %d token stride %lld", g,
                       (long long)group_tok_stride[g]);
  }
  const bool by_addr = src_k_addr != nullptr;
  if ((src_k_addr == nullptr) != (src_v_addr == nullptr))
    return set_error(HC_ERR_INVALID, "hc_gather_store_groups: give both per-job address tables or neither");
  if (by_addr && src_is_host)
    return set_error(HC_ERR_INVALID, "hc_gather_store_groups: per-job addresses are device addresses");
  if ((!by_addr && (!src_k || !src_v)) || !src_off || !count || !dst_row || !kstore || !vstore ||
      !row_tile_off || (idx && !idx_off))
    return set_error(HC_ERR_INVALID, "hc_gather_store_groups: null pointer argument");
  const void* sk = src_k;
  const void* sv = src_v;
  if (src_is_host) {
    int rc = map_host_ptr(src_k, &sk);
    if (rc) return rc;
    rc = map_host_ptr(src_v, &sv);
    if (rc) return rc;
  }
  hipStream_t s = (hipStream_t)stream;
  for (int g = 0; g < ngroups; ++g) {
    const int b0 = group_begin[g], nj = group_begin[g + 1] - b0;
    if (nj > 0 && group_max_count[g] > 0) {
      const int64_t* so = src_off + b0;
      const int64_t* io = idx ? idx_off + b0 : nullptr;
      const int32_t* cn = count + b0;
      const int32_t* dr = dst_row + b0;
      const int32_t* to = trig_of ? trig_of + b0 : nullptr;
      const int64_t* ka = by_addr ? src_k_addr + b0 : nullptr;
      const int64_t* va = by_addr ? src_v_addr + b0 : nullptr;
      int rc;
      switch (dtype) {
        case HC_DTYPE_BF16:
          rc = launch_gather_store<__bf16>(sk, sv, so, group_tok_stride[g], src_len, idx, io, cn, dr, kstore, vstore,
                                           row_tile_off, nj, group_max_count[g], trigger, to, src_is_host != 0,
                                           max_workgroups, s, ka, va);
          break;
        case HC_DTYPE_F16:
          rc = launch_gather_store<_Float16>(sk, sv, so, group_tok_stride[g], src_len, idx, io, cn, dr, kstore,
                                             vstore, row_tile_off, nj, group_max_count[g], trigger, to,
                                             src_is_host != 0, max_workgroups, s, ka, va);
          break;
        case HC_DTYPE_F32:
          rc = launch_gather_store<float>(sk, sv, so, group_tok_stride[g], src_len, idx, io, cn, dr, kstore, vstore,
                                          row_tile_off, nj, group_max_count[g], trigger, to, src_is_host != 0,
                                          max_workgroups, s, ka, va);
          break;
        default:
          return set_error(HC_ERR_INVALID, "hc_gather_store_groups: unknown dtype %d", dtype);
      }
      if (rc) return rc;
    }
    if (events && events[g]) {
      const hipError_t e = hipEventRecord((hipEvent_t)events[g], s);
      if (e != hipSuccess)
        return set_error(HC_ERR_HIP, "hc_gather_store_groups: event of group %d: %s", g, hipGetErrorString(e));
    }
  }
  return HC_OK;
}

extern "C" int hc_append(int dtype, const void* k_new, const void* v_new, int64_t src_row_stride, void* kstore,
                         void* vstore, const int64_t* row_tile_off, int32_t* row_len, const int32_t* row_cap,
                         int rows, int32_t* status, void* stream) {
  clear_error();
  if (rows < 0) return set_error(HC_ERR_INVALID, "hc_append: rows=%d", rows);
  if (rows == 0) return HC_OK;
  if (!k_new || !v_new || !kstore || !vstore || !row_tile_off || !row_len || !row_cap)
    return set_error(HC_ERR_INVALID, "hc_append: null pointer argument");
  if (src_row_stride < HC_HEAD_DIM)
    return set_error(HC_ERR_INVALID, "hc_append: row stride %lld < 128", (long long)src_row_stride);
  hipStream_t s = (hipStream_t)stream;
#define HC_APPEND(T)                                                                                            \
  hipLaunchKernelGGL((append_kernel<T>), dim3(rows), dim3(64), 0, s, (const T*)k_new, (const T*)v_new,          \
                     src_row_stride, (T*)kstore, (T*)vstore, row_tile_off, row_len, row_cap, status);           \
  return check_launch("hc_append");
  switch (dtype) {
    case HC_DTYPE_BF16: { HC_APPEND(__bf16) }
    case HC_DTYPE_F16: { HC_APPEND(_Float16) }
    case HC_DTYPE_F32: { HC_APPEND(float) }
    default:
      return set_error(HC_ERR_INVALID, "hc_append: unknown dtype %d", dtype);
  }
#undef HC_APPEND
}

extern "C" int hc_store_read(int dtype, const void* kstore, const void* vstore, const int64_t* row_tile_off,
                             const int32_t* rows_sel, int nrows, int count, void* dst_k, void* dst_v, void* stream) {
  clear_error();
  if (nrows < 0 || count < 0 || nrows > 65535) return set_error(HC_ERR_INVALID, "hc_store_read: bad sizes");
  if (nrows == 0 || count == 0) return HC_OK;
  if (!kstore || !vstore || !row_tile_off || !rows_sel || !dst_k || !dst_v)
    return set_error(HC_ERR_INVALID, "hc_store_read: null pointer argument");
  hipStream_t s = (hipStream_t)stream;
  dim3 grid((unsigned)(((int64_t)count * HC_HEAD_DIM + 255) / 256), nrows);
#define HC_READ(T)                                                                                         \
  hipLaunchKernelGGL((store_read_kernel<T>), grid, dim3(256), 0, s, (const T*)kstore, (const T*)vstore,    \
                     row_tile_off, rows_sel, count, (T*)dst_k, (T*)dst_v);                                 \
  return check_launch("hc_store_read");
  switch (dtype) {
    case HC_DTYPE_BF16: { HC_READ(__bf16) }
    case HC_DTYPE_F16: { HC_READ(_Float16) }
    case HC_DTYPE_F32: { HC_READ(float) }
    default:
      return set_error(HC_ERR_INVALID, "hc_store_read: unknown dtype %d", dtype);
  }
#undef HC_READ
}

extern "C" int hc_copy_rows(int dtype, const void* src_k, const void* src_v, const int64_t* src_off,
                            int64_t src_tok_stride, void* dst_k, void* dst_v, int dst_is_host, const int64_t* dst_off,
                            int64_t dst_tok_stride, const int32_t* count, int njobs, int max_count,
                            int max_workgroups, void* stream) {
  clear_error();
  const int esz = dtype == HC_DTYPE_F32 ? 4 : (dtype == HC_DTYPE_BF16 || dtype == HC_DTYPE_F16) ? 2 : 0;
  if (esz == 0) return set_error(HC_ERR_INVALID, "hc_copy_rows: unknown dtype %d", dtype);
  if (njobs < 0 || max_count < 0 || max_workgroups < 1)
    return set_error(HC_ERR_INVALID, "hc_copy_rows: njobs=%d max_count=%d max_workgroups=%d", njobs, max_count,
                     max_workgroups);
  if (njobs == 0 || max_count == 0) return HC_OK;
  if (!src_k || !src_v || !src_off || !dst_k || !dst_v || !dst_off || !count)
    return set_error(HC_ERR_INVALID, "hc_copy_rows: null pointer argument");
  if (src_tok_stride < HC_HEAD_DIM || dst_tok_stride < HC_HEAD_DIM || (src_tok_stride * esz) % 16 ||
      (dst_tok_stride * esz) % 16)
    return set_error(HC_ERR_INVALID, "hc_copy_rows: token strides must be >= 128 elements and 16-byte multiples");
  if (((uintptr_t)src_k | (uintptr_t)src_v | (uintptr_t)dst_k | (uintptr_t)dst_v) % 16)
    return set_error(HC_ERR_INVALID, "hc_copy_rows: buffers must be 16-byte aligned");
  void* dk = dst_k;
  void* dv = dst_v;
  if (dst_is_host) {
    const void* m = nullptr;
    int rc = map_host_ptr(dst_k, &m);
    if (rc) return rc;
    dk = const_cast<void*>(m);
    rc = map_host_ptr(dst_v, &m);
    if (rc) return rc;
    dv = const_cast<void*>(m);
  }
  const int chunks = (max_count + kCopyChunk - 1) / kCopyChunk;
  const int64_t items = (int64_t)njobs * chunks;
  const unsigned grid = (unsigned)std::min<int64_t>(items, max_workgroups);
  hipLaunchKernelGGL(copy_rows_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream, (const uint8_t*)src_k,
                     (const uint8_t*)src_v, src_off, src_tok_stride * esz, (uint8_t*)dk, (uint8_t*)dv, dst_off,
                     dst_tok_stride * esz, count, njobs, chunks, HC_HEAD_DIM * esz / 16, esz, nullptr, 0, 0);
  return check_launch("hc_copy_rows");
}

extern "C" int hc_gather_rows(int dtype, const void* src_k, const void* src_v, const int64_t* src_off,
                              int64_t src_tok_stride, int src_len, const int32_t* idx, int64_t idx_stride,
                              void* dst_k, void* dst_v, const int64_t* dst_off, int64_t dst_tok_stride,
                              const int32_t* count, int njobs, int max_count, void* stream) {
  clear_error();
  const int esz = dtype == HC_DTYPE_F32 ? 4 : (dtype == HC_DTYPE_BF16 || dtype == HC_DTYPE_F16) ? 2 : 0;
  if (esz == 0) return set_error(HC_ERR_INVALID, "hc_gather_rows: unknown dtype %d", dtype);
  if (njobs < 0 || max_count < 0 || src_len < 0 || idx_stride < 0)
    return set_error(HC_ERR_INVALID, "hc_gather_rows: njobs=%d max_count=%d src_len=%d", njobs, max_count, src_len);
  if (njobs == 0 || max_count == 0) return HC_OK;
  if (src_len == 0) return set_error(HC_ERR_INVALID, "hc_gather_rows: empty source");
  if (!src_k || !src_v || !src_off || !idx || !dst_k || !dst_v || !dst_off || !count)
    return set_error(HC_ERR_INVALID, "hc_gather_rows: null pointer argument");
  if (idx_stride < max_count) return set_error(HC_ERR_INVALID, "hc_gather_rows: idx_stride below max_count");
  if (src_tok_stride < HC_HEAD_DIM || dst_tok_stride < HC_HEAD_DIM || (src_tok_stride * esz) % 16 ||
      (dst_tok_stride * esz) % 16)
    return set_error(HC_ERR_INVALID, "hc_gather_rows: token strides must be >= 128 elements and 16-byte multiples");
  if (((uintptr_t)src_k | (uintptr_t)src_v | (uintptr_t)dst_k | (uintptr_t)dst_v) % 16)
    return set_error(HC_ERR_INVALID, "hc_gather_rows: buffers must be 16-byte aligned");
  const int chunks = (max_count + kCopyChunk - 1) / kCopyChunk;
  const int64_t items = (int64_t)njobs * chunks;
  const unsigned grid = (unsigned)std::min<int64_t>(items, 65535);
  hipLaunchKernelGGL(copy_rows_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream, (const uint8_t*)src_k,
                     (const uint8_t*)src_v, src_off, src_tok_stride * esz, (uint8_t*)dst_k, (uint8_t*)dst_v, dst_off,
                     dst_tok_stride * esz, count, njobs, chunks, HC_HEAD_DIM * esz / 16, esz, idx, idx_stride,
                     src_len);
  return check_launch("hc_gather_rows");
}
