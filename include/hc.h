/*
 * libhc — C ABI of the MI355X compressed-KV attention path.
 *
 * Every entry point takes plain pointers and sizes, launches asynchronously
 * on the given HIP stream (passed as void*, NULL = default stream), never
 * allocates device memory, never synchronises the host and never throws.
 * The return value is HC_OK (0) or a negative hc_status; hc_last_error()
 * returns a thread-local message describing the last failure.
 *
 * KV store geometry shared by all calls (see heterocache_amd/csrc/hc_common.h):
 *   kstore / vstore : one buffer per layer, 32-token x 128-channel tiles,
 *                     tile-permuted so each MFMA operand is one 16-byte load.
 *   row_tile_off    : int64 [rows], first tile of row r = b*Hkv + h.
 *   row_len         : int32 [rows], tokens held by row r (device resident).
 *   row_cap         : int32 [rows], capacity of row r in tokens (tile multiple).
 * dtype codes: HC_DTYPE_F32, HC_DTYPE_F16, HC_DTYPE_BF16; head_dim is 128.
 */
#ifndef HC_H_
#define HC_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HC_ABI_VERSION 1

enum hc_status {
  HC_OK = 0,
  HC_ERR_INVALID = -1,  /* bad shape, pointer or size */
  HC_ERR_CAPACITY = -2, /* a row would exceed its capacity ("Layer i OOM.") */
  HC_ERR_HIP = -3,      /* the HIP runtime reported an error */
};

enum hc_dtype { HC_DTYPE_F32 = 0, HC_DTYPE_F16 = 1, HC_DTYPE_BF16 = 2 };

/* Thread-local description of the last error (empty string after success). */
const char* hc_last_error(void);
int hc_version(void);
int hc_tile_tokens(void);
int hc_head_dim(void);

/*
 * Decode attention over the ragged per-head store, GQA group of `group`
 * query heads per row, no causal mask:
 *   out[r, g, :] = softmax(scale * q[r, g, :] . K_r^T) V_r   over len[r] tokens
 * (zeros for an empty row).  q, out: [rows, group, 128] contiguous, dtype.
 * Replaces flash_attn_with_kvcache(q_in, k_pool, v_pool, cache_seqlens,
 * block_table, causal=False) at heterocache/llama_model.py:382-389 and
 * heterocache/qwen_model.py:194-201.
 *
 * row_order (optional): permutation of the rows giving the order in which
 * their chunks are scheduled (longest first is fastest).
 * k_new/v_new (optional, [rows, 128]): fused decode append -- the new token
 * is attended at slot row_len[r], stored there, and every row_len advances by
 * one when the launch completes (the append of heterocache/cache_utils.py:
 * 970-1005 and the attention in one launch).
 * num_parts: hc_decode_num_parts() of the lengths the launch attends
 * (row_len, +1 with k_new).  workspace: at least
 * hc_decode_workspace_size(rows, group, num_parts) bytes, zero-filled before
 * its first use; each completed launch leaves its counters at zero again, so
 * one workspace serves any sequence of launches on one stream (launches that
 * overlap in time need separate workspaces).
 */
int hc_decode_attn(int dtype, const void* q, void* kstore, void* vstore, const int64_t* row_tile_off, int32_t* row_len,
                   const int32_t* row_order, int rows, int group, float scale, const void* k_new, const void* v_new,
                   void* out, void* workspace, size_t workspace_bytes, int64_t num_parts, int tiles_per_wave,
                   void* stream);
int64_t hc_decode_num_parts(const int32_t* host_row_len, int rows, int tiles_per_wave);
size_t hc_decode_workspace_size(int rows, int group, int64_t num_parts);

/*
 * Gather natural-layout rows into store slots [0, count[j]) of row dst_row[j]:
 *   store[dst_row[j]][i] = src[src_off[j] + idx[idx_off[j] + i] * src_tok_stride]
 * (idx == NULL copies source tokens 0..count-1; indices are clamped into
 * [0, src_len) like the reference's clamp before its gather).  With src_is_host != 0 the
 * sources are host-pinned, device-mapped buffers read over the host link.
 * When trigger != NULL the call does nothing unless *trigger != 0 (device).
 * Replaces the keep-head index_copy_ (heterocache/cache_utils.py:914-937),
 * the compressed-head gather + index_copy_ (heterocache/cache_utils.py:854-877)
 * and the retrieval index_select + copy_ (heterocache/cache_utils.py:1097-1123).
 */
int hc_gather_store(int dtype, const void* src_k, const void* src_v, int src_is_host, const int64_t* src_off,
                    int64_t src_tok_stride, int src_len, const int32_t* idx, const int64_t* idx_off, const int32_t* count,
                    const int32_t* dst_row, void* kstore, void* vstore, const int64_t* row_tile_off, int njobs,
                    int max_count, const int32_t* trigger, void* stream);

/*
 * Append one token per row at slot row_len[r], then row_len[r] += 1.
 * k_new/v_new row r starts at r * src_row_stride elements.  A full row is left
 * unchanged and sets bit 0 of *status (device, optional).
 * Replaces the decode branch of HeteroCache.update
 * (heterocache/cache_utils.py:970-1005).
 */
int hc_append(int dtype, const void* k_new, const void* v_new, int64_t src_row_stride, void* kstore, void* vstore,
              const int64_t* row_tile_off, int32_t* row_len, const int32_t* row_cap, int rows, int32_t* status,
              void* stream);

/*
 * Unpack slots [0, count) of rows rows_sel[0..nrows) to natural layout
 * dst_k/dst_v [nrows, count, 128].  Counterpart of
 * HeteroCache._get_physical_content (heterocache/cache_utils.py:768-780).
 */
int hc_store_read(int dtype, const void* kstore, const void* vstore, const int64_t* row_tile_off,
                  const int32_t* rows_sel, int nrows, int count, void* dst_k, void* dst_v, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* HC_H_ */
