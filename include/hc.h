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

#define HC_ABI_VERSION 2

enum hc_status {
  HC_OK = 0,
  HC_ERR_INVALID = -1,  /* bad shape, pointer or size */
  HC_ERR_CAPACITY = -2, /* a row would exceed its capacity ("Layer i OOM.") */
  HC_ERR_HIP = -3,      /* the HIP runtime reported an error */
};

enum hc_dtype { HC_DTYPE_F32 = 0, HC_DTYPE_F16 = 1, HC_DTYPE_BF16 = 2 };

/* Thread-local description of the last error (empty string after success). */
const char* hc_last_error(void);

/*
 * Read the device status word that hc_append and hc_decode_attn raise when a
 * row is at capacity: waits for `stream`, stores the word in *value (optional),
 * zeroes it when `clear` is set, and returns HC_ERR_CAPACITY when bit 0 is
 * set (HC_OK otherwise).  The one call that synchronises the host; it exists
 * so that launches replayed from a HIP graph, which no host check precedes,
 * still surface the reference's pool exhaustion ("Layer i OOM.",
 * heterocache/cache_utils.py:988-990) as a typed error.
 */
int hc_read_status(int32_t* status, int clear, int32_t* value, void* stream);

/*
 * No counterpart in the reference: a measurement aid for the roofline of
 * the HBM-bound kernels.  Reads `bytes` (a multiple of 16, 16-byte aligned)
 * from device memory with nontemporal 16-byte loads, one in flight per
 * thread, over workgroups_per_cu * (compute units) workgroups of 256 threads
 * (8 read fastest on MI355X), and discards them (sink, one float, is
 * written only when the sum equals one arbitrary value, -1.2345e-37, so the
 * loads are kept; a zero-filled buffer never writes it).  The time of a
 * call over a buffer larger than the last-level cache is the part's
 * streaming-read ceiling, against which a kernel's achieved bandwidth can be
 * set beside the data-sheet peak.
 */
int hc_stream_read(const void* src, size_t bytes, float* sink, int workgroups_per_cu, void* stream);
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
 * is attended at slot row_len[r], stored there, and row_len[r] advances by
 * one when the launch completes (the append of heterocache/cache_utils.py:
 * 970-1005 and the attention in one launch).  row_cap is required with a
 * fused append: a row with row_len[r] >= row_cap[r] is left unchanged (no
 * store, no advance), its output is NaN and bit 0 of *status is set (status
 * optional) -- the device-side form of the reference's "Layer i OOM."
 * (heterocache/cache_utils.py:988-990); hc_read_status turns it into
 * HC_ERR_CAPACITY.
 * chunk_tiles: 32-token tiles per workgroup (each row is cut into chunks of
 * this many tiles; the 4 waves of a workgroup split a chunk evenly);
 * hc_decode_chunk_tiles() picks the value that fills the device in one
 * resident round for the given lengths.
 * num_parts: hc_decode_num_parts(lengths, rows, chunk_tiles) of the lengths
 * the launch attends (row_len, +1 with k_new); a larger value (surplus
 * workgroups exit) lets a captured graph replay while the lengths grow.  If
 * the grid it sizes is smaller than the device lengths need, every row's
 * output is NaN and nothing is stored or advanced.
 * workspace: at least hc_decode_workspace_size(rows, group, num_parts) bytes;
 * every field is written before it is read within one call, so it needs no
 * initialisation, and one workspace serves any sequence of launches on one
 * stream (launches that overlap in time need separate workspaces).
 */
int hc_decode_attn(int dtype, const void* q, void* kstore, void* vstore, const int64_t* row_tile_off, int32_t* row_len,
                   const int32_t* row_cap, const int32_t* row_order, int rows, int group, float scale,
                   const void* k_new, const void* v_new, void* out, void* workspace, size_t workspace_bytes,
                   int64_t num_parts, int chunk_tiles, int32_t* status, void* stream);
/*
 * hc_decode_attn that also reports, for every row r and query head g, the
 * softmax statistics of the row's first stat_len attended tokens: with
 * s_t = scale * log2(e) * q[r, g, :] . k_t (base-2 scores; with stat_flags
 * HC_SCORE_ROUND_BF16 / HC_SCORE_ROUND_F16 the reference's cast chain
 * s_t = round(round(q . k_t) * scale) * log2(e), rounding to that type, as
 * hc_score's flags do -- the attention output itself never rounds),
 *   stat_out[r * stat_row_stride + g * stat_head_stride + 0] = M (a bound of
 *     max_t s_t over t < stat_len; -inf when no token lies below stat_len),
 *   stat_out[... + 1] = sum over t < stat_len of exp2(s_t - M),
 * both float32, NaN for a row flagged at capacity or by an undersized grid.
 * Tokens at or beyond stat_len (the decode tokens after a prompt of
 * stat_len) are attended but left out.  The pivot drift check
 * (heterocache/cache_utils.py:1030-1047: softmax of the buffered decode
 * queries over a pivot's prefill keys) needs exactly these normalisers; with
 * them hc_score_given_stats forms its probabilities in one pass over the
 * keys.  Arguments otherwise as hc_decode_attn (same workspace size).
 */
int hc_decode_attn_stats(int dtype, const void* q, void* kstore, void* vstore, const int64_t* row_tile_off,
                         int32_t* row_len, const int32_t* row_cap, const int32_t* row_order, int rows, int group,
                         float scale, const void* k_new, const void* v_new, void* out, void* workspace,
                         size_t workspace_bytes, int64_t num_parts, int chunk_tiles, int32_t* status, int stat_len,
                         float* stat_out, int64_t stat_row_stride, int64_t stat_head_stride, int stat_flags,
                         void* stream);
/*
 * hc_decode_attn without a caller workspace, for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc); it has no counterpart in the reference.  Arguments and
 * results are those of hc_decode_attn; the split-K partials live in a 16 MiB
 * device array of the library (one per device, held until the process ends,
 * its address resolved on the first call made on that device -- make that
 * first call outside graph capture).  Launches whose
 * hc_decode_workspace_size(rows, group, num_parts) exceeds 16 MiB are
 * rejected with HC_ERR_INVALID.  Every call on a device shares that device's
 * array: calls that overlap in time on one device (two streams, or two
 * threads) race and must be serialised by the caller.  The array needs no
 * clearing between calls.  The call allocates and frees nothing.
 */
int hc_decode_attn_noalloc(int dtype, const void* q, void* kstore, void* vstore, const int64_t* row_tile_off,
                           int32_t* row_len, const int32_t* row_cap, const int32_t* row_order, int rows, int group,
                           float scale, const void* k_new, const void* v_new, void* out, int64_t num_parts,
                           int chunk_tiles, int32_t* status, void* stream);

/* Workgroups (chunks) of one hc_decode_attn launch over these lengths. */
int64_t hc_decode_num_parts(const int32_t* host_row_len, int rows, int chunk_tiles);
/* chunk_tiles for hc_decode_attn: the smallest chunk (at least 4 tiles)
 * whose grid fits the current device's resident workgroup slots for this
 * dtype and group; from 24 tiles up it is rounded up to a multiple of 4 so
 * the workgroup's four waves stream equal shares (one chunk per row when
 * even the smallest does not fit); negative
 * hc_status on error.  No counterpart in the reference (flash-attn chooses
 * its split internally). */
int hc_decode_chunk_tiles(int dtype, const int32_t* host_row_len, int rows, int group);
size_t hc_decode_workspace_size(int rows, int group, int64_t num_parts);

/*
 * Gather natural-layout rows into store slots [0, count[j]) of row dst_row[j]:
 *   store[dst_row[j]][i] = src[src_off[j] + idx[idx_off[j] + i] * src_tok_stride]
 * (idx == NULL copies source tokens 0..count-1; indices are clamped into
 * [0, src_len) like the reference's clamp before its gather).  With src_is_host != 0 the
 * sources are host-pinned, device-mapped buffers read over the host link.
 * When trigger != NULL job j is skipped unless trigger[trig_of ? trig_of[j] : 0]
 * != 0 (device flags; one launch can serve several gated groups of jobs).
 * max_workgroups caps the grid, whose workgroups stride over the (job,
 * 32-token tile) items (0: one workgroup per item from device memory, 64
 * from host memory -- a host-sourced gather waits on the link, and beside a
 * decode launch that fills the device its workgroups take slots the decode
 * kernel needs).  set_len (optional, int32 per store row): the length of
 * every copied row dst_row[j] becomes count[j] (gated like the copy), so a
 * prefill store needs no separate length update.
 * Replaces the keep-head index_copy_ (heterocache/cache_utils.py:914-937),
 * the compressed-head gather + index_copy_ (heterocache/cache_utils.py:854-877)
 * and the retrieval index_select + copy_ (heterocache/cache_utils.py:1097-1123).
 */
int hc_gather_store(int dtype, const void* src_k, const void* src_v, int src_is_host, const int64_t* src_off,
                    int64_t src_tok_stride, int src_len, const int32_t* idx, const int64_t* idx_off, const int32_t* count,
                    const int32_t* dst_row, void* kstore, void* vstore, const int64_t* row_tile_off, int njobs,
                    int max_count, const int32_t* trigger, const int32_t* trig_of, int max_workgroups,
                    int32_t* set_len, void* stream);

/*
 * hc_gather_store over jobs split into ngroups consecutive groups (host
 * arrays: group_begin[ngroups + 1] job boundaries, group_max_count[ngroups],
 * group_tok_stride[ngroups] source token stride of each group): one gather
 * launch per group on `stream`, each followed by hipEventRecord(events[g])
 * when events (host array of hipEvent_t, entries may be NULL) is given --
 * also for an empty group -- so a consumer of group g's rows waits for that
 * group alone.  Device arrays are indexed by global job as in
 * hc_gather_store; trig_of keeps global trigger indices.  All groups are
 * validated before the first launch.  src_k_addr / src_v_addr (device
 * int64 arrays, one address per job, or both NULL): each job's source
 * tensor base in device memory, to which src_off[j] is added -- so one
 * launch gathers from several tensors (each layer's prefill K/V) -- in
 * place of src_k / src_v.  Serves the retrieval of one drift
 * check, one group per layer: the reference copies each satellite's rows
 * with its own H2D copy_ on the default stream before the next step
 * (heterocache/cache_utils.py:1097-1123); here each layer's next attention
 * waits only for its own satellites' rows.
 */
int hc_gather_store_groups(int dtype, const void* src_k, const void* src_v, int src_is_host, const int64_t* src_off,
                           const int64_t* group_tok_stride, int src_len, const int32_t* idx, const int64_t* idx_off,
                           const int32_t* count, const int32_t* dst_row, void* kstore, void* vstore,
                           const int64_t* row_tile_off, int ngroups, const int32_t* group_begin,
                           const int32_t* group_max_count, const int32_t* trigger, const int32_t* trig_of,
                           int max_workgroups, void* const* events, const int64_t* src_k_addr,
                           const int64_t* src_v_addr, void* stream);

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

/*
 * Copy token rows [0, count[j]) (128 channels each) of K and V between two
 * natural layouts:
 *   dst[dst_off[j] + t*dst_tok_stride + c] = src[src_off[j] + t*src_tok_stride + c]
 * (offsets and strides in elements; rows 16-byte aligned).  With
 * dst_is_host != 0 the destination is host-pinned memory written through its
 * device mapping.  At most max_workgroups workgroups stride over the work, so
 * a copy to the host link can run beside compute without occupying the
 * device.  Replaces the D2H copy of the satellite heads' full K/V into the
 * pinned tier (heterocache/cache_utils.py:939-967).
 */
int hc_copy_rows(int dtype, const void* src_k, const void* src_v, const int64_t* src_off, int64_t src_tok_stride,
                 void* dst_k, void* dst_v, int dst_is_host, const int64_t* dst_off, int64_t dst_tok_stride,
                 const int32_t* count, int njobs, int max_count, int max_workgroups, void* stream);

/*
 * Causal prefill attention (flash-attention forward), head_dim 128:
 *   out[b, i, hq, :] = sum_t softmax_t(scale * q[b, hq, i] . k[b, hq/G, t]) v[b, hq/G, t],
 *   t <= kv_len - q_len + i,  G = q_heads / kv_heads.
 * The queries are the last q_len of the kv_len positions (bottom-right causal
 * alignment), so the same call serves a whole prompt (q_len == kv_len) and a
 * chunk of a chunked prefill over the keys staged so far.  Each of q, k, v and
 * out is addressed as base + b*strides[0] + h*strides[1] + t*strides[2] + c
 * (element strides, 16-byte multiples; channels contiguous), so the
 * projections' [B, T, H, 128] layout is read without a copy; scale > 0.  Arithmetic: MFMA
 * on the input type, fp32 accumulation and softmax, probabilities rounded to
 * the input type for the P.V product.  Replaces the flash-attn prefill call
 * of LlamaAttention / Qwen2Attention (heterocache/llama_model.py:353-361,
 * through transformers' flash_attention_forward).
 */
int hc_prefill_attn(int dtype, const void* q, const int64_t* q_strides, const void* k, const int64_t* k_strides,
                    const void* v, const int64_t* v_strides, void* out, const int64_t* out_strides, int batch,
                    int q_heads, int kv_heads, int q_len, int kv_len, float scale, void* workspace,
                    size_t workspace_bytes, void* stream);

/*
 * hc_prefill_attn that also reports the softmax statistics of the last
 * stat_rows queries of every (batch, query head), 1 <= stat_rows <= q_len:
 *   stat_out[((b*q_heads + hq)*stat_rows + w)*2 + 0] = M,
 *   stat_out[((b*q_heads + hq)*stat_rows + w)*2 + 1] = L,
 * for query i = q_len - stat_rows + w over its visible keys, with
 * max_t s_t - 8 <= M <= max_t s_t for the scaled base-2 scores
 * s_t = scale * log2(e) * q_i . k_t and L = sum_t exp2(s_t - M), so
 * softmax_t = exp2(s_t - (M + log2 L)).  These are the normalisers of the
 * observation-window softmax the prefill scorers recompute over the same
 * keys (HeteroCache.prefill_select and init_coefficient,
 * heterocache/cache_utils.py:807-829 and :1158-1187; SnapKV,
 * heterocache/kv_cluster.py:165-185), which then need one key pass
 * (hc_score_with_stats).  The attention output is bit-identical to
 * hc_prefill_attn's.
 */
int hc_prefill_attn_stats(int dtype, const void* q, const int64_t* q_strides, const void* k,
                          const int64_t* k_strides, const void* v, const int64_t* v_strides, void* out,
                          const int64_t* out_strides, int batch, int q_heads, int kv_heads, int q_len, int kv_len,
                          float scale, void* workspace, size_t workspace_bytes, int stat_rows, float* stat_out,
                          void* stream);

/* Device workspace bytes hc_prefill_attn needs (V re-laid out in 32-token
 * tiles, written and read within the call: no initialisation). */
size_t hc_prefill_workspace_size(int dtype, int batch, int kv_heads, int kv_len);

/* Workspace bytes that also hold the split partials of a short call: where
 * one block of at most 128 queries per (batch, query head) would leave most
 * of the current device idle over a long key range (decode-like steps of
 * the baseline caches, a short last chunk of a chunked prefill), a
 * workspace of this size lets hc_prefill_attn / hc_prefill_attn_stats split
 * the keys across workgroups and merge the partials (flash-decoding style;
 * calls with at most 16 query heads x queries per KV row pack them into one
 * MFMA column block and read K and V in their natural layout).
 * With hc_prefill_workspace_size bytes the call runs unsplit.  The split
 * changes the fp32 summation order, not the result's tolerance.  No
 * reference counterpart: flash-attn picks its own split inside
 * (heterocache/llama_model.py:353-361 and transformers' attention call for
 * the baseline caches). */
size_t hc_prefill_workspace_bytes(int dtype, int batch, int q_heads, int kv_heads, int q_len, int kv_len);

/*
 * Gather token rows by index between natural layouts:
 *   dst[dst_off[j] + t*dst_tok_stride + c] = src[src_off[j] + i*src_tok_stride + c],
 *   i = clamp(idx[j*idx_stride + t], 0, src_len - 1),  t < count[j]
 * (offsets and strides in elements; rows 16-byte aligned).  Replaces the
 * kept-token `gather` + `cat` of the baseline compressors (PyramidKV, SnapKV,
 * H2O, StreamingLLM: heterocache/kv_cluster.py:101-106 and :130-135,
 * :192-197, :448-449, :517-522).
 */
int hc_gather_rows(int dtype, const void* src_k, const void* src_v, const int64_t* src_off, int64_t src_tok_stride,
                   int src_len, const int32_t* idx, int64_t idx_stride, void* dst_k, void* dst_v,
                   const int64_t* dst_off, int64_t dst_tok_stride, const int32_t* count, int njobs, int max_count,
                   void* stream);

/*
 * Head-analysis pooling (offline head classification):
 *   out[b*heads_out + h][t] = avg_pool_k(mean_{g<group} attn[b*batch_stride + (h*group + g)*head_stride + t])
 * for t < span; zero padding kernel/2, divisor kernel (odd kernel).  With
 * 16-bit input the group mean is rounded to the input type.  Replaces the
 * GQA mean + last-row sum + avg_pool1d of get_head_topk_exact
 * (tools/get_cluster.py:13-56); the top-k that follows is hc_select_topk and
 * the overlap ratios hc_set_bits + hc_overlap_count.
 */
int hc_head_pool(int dtype, const void* attn, int64_t batch_stride, int64_t head_stride, int batch, int heads_out,
                 int group, int span, int kernel, float* out, void* stream);

/* hc_score flags */
#define HC_SCORE_CAUSAL_WINDOW 1 /* window row w sees keys t <= L - W + w (kv_cluster.py:169-175) */
#define HC_SCORE_SUM_WINDOW 2    /* sum probabilities over the W rows of a query head (kv_cluster.py:178) */
#define HC_SCORE_ROUND_BF16 4    /* reproduce the reference's casts to bfloat16 */
#define HC_SCORE_ROUND_F16 8     /* reproduce the reference's casts to float16 */
#define HC_SCORE_ACCUMULATE 16   /* add the call's scores into `scores` instead of overwriting them */

/*
 * Pooled observation-window scores, maxed over the GQA group:
 *   S[j][w'][t] = max_g pool_k( sum_w softmax_t(scale * q_{j,g,w} . k_{j,t} + mask) ),  t < span
 * (no sum, w' = w, without HC_SCORE_SUM_WINDOW).  Query row (g, w) of job j is
 * q + q_off[j] + g*q_head_stride + w*q_row_stride (128 contiguous elements).
 * Keys: natural layout, token t of job j at k + k_off[j] + t*k_tok_stride; or,
 * when row_tile_off != NULL, slots [0, seq_len) of store row k_row[j] of the
 * tiled store k (read in place).  pooling: 0 = avg_pool1d (zero padding,
 * divisor kernel), 1 = max_pool1d (-inf padding); odd kernel, padding kernel/2.
 * scores: [njobs][W' ][span] float32.  hist (optional, fewer than 32 query
 * rows, no accumulation): per output row (job, w') 4096 uint32 bins counting
 * the scores by the top 12 bits of their order-preserving keys -- the
 * first digit hc_drift_select selects on; the call zeroes it first.
 * Replaces the scoring op sequences of HeteroCache.prefill_select
 * (heterocache/cache_utils.py:807-829), init_coefficient (:1158-1187),
 * decode_select (:1030-1057) and SnapKVCluster.update_kv
 * (heterocache/kv_cluster.py:165-185).
 */
int hc_score(int dtype, const void* q, const int64_t* q_off, int64_t q_head_stride, int64_t q_row_stride,
             const void* k, const int64_t* k_off, int64_t k_tok_stride, const int64_t* row_tile_off,
             const int32_t* k_row, int njobs, int seq_len, int group, int window, int flags, int span, int pooling,
             int kernel, float scale, float* scores, void* workspace, size_t workspace_bytes, uint32_t* hist,
             void* stream);
size_t hc_score_workspace_size(int njobs, int seq_len, int group, int window, int flags);

/*
 * hc_score with every query row's softmax statistics given, in the uncast
 * float32 form (no rounding flag): the probability and pooling passes alone,
 * so the keys are read once.  Arguments as hc_score's, plus the statistics
 * (M, L) of row r = g*window + w of job j (M bounds the scaled base-2 scores,
 * L = sum_t exp2(s_t - M) over the row's visible keys, as
 * hc_prefill_attn_stats and hc_decode_attn_stats report them) at
 *   stats + base + 2r                              (stat_head_stride == 0)
 *   stats + base + g*stat_head_stride + 2w         (otherwise, >= 2*window)
 * with base = stat_off ? stat_off[j] : 2*group*window*j.  Workspace: at least
 * njobs * W' * group * span floats (hc_score_workspace_size suffices).
 * Replaces the same scoring op sequences as hc_score (prefill_select,
 * heterocache/cache_utils.py:807-829; init_coefficient, :1158-1187; SnapKV,
 * heterocache/kv_cluster.py:165-185) when the prefill attention has already
 * formed the softmax normalisers.
 */
int hc_score_with_stats(int dtype, const void* q, const int64_t* q_off, int64_t q_head_stride, int64_t q_row_stride,
                        const void* k, const int64_t* k_off, int64_t k_tok_stride, const int64_t* row_tile_off,
                        const int32_t* k_row, int njobs, int seq_len, int group, int window, int flags, int span,
                        int pooling, int kernel, float scale, const float* stats, const int64_t* stat_off,
                        int64_t stat_head_stride, float* scores, void* workspace, size_t workspace_bytes,
                        void* stream);

/*
 * hc_score's pivot drift scoring in one pass over the keys, given every query
 * row's softmax statistics (heterocache/cache_utils.py:1030-1057): for job j,
 * query row r = g*window + w (query q + q_off[j] + g*q_head_stride +
 * w*q_row_stride) and key t < seq_len of store row k_row[j] (read in place
 * through row_tile_off),
 *   p[r][t] = exp2(s - (M + log2 L)),  s = scale * log2(e) * q . k_t,
 *   (M, L) = stats[stat_off[j] + 2r], stats[stat_off[j] + 2r + 1]
 * (as hc_decode_attn_stats reports them; L = 0 gives p = 0), and
 *   scores[j][w][t] = max_g pool(p[g*window + w])[t]
 * with avg (pooling 0, zero padding, divided by kernel) or max (pooling 1)
 * pooling of width kernel in {1, 3, 5, 7, 9}; group*window < 32.  flags
 * HC_SCORE_ROUND_BF16 / HC_SCORE_ROUND_F16 (or 0): hc_score's cast chain,
 * s = round(round(q . k_t) * scale) * log2(e), p = round(exp2(s - M) / L),
 * the pooled value rounded before the max, with (M, L) of that chain
 * (hc_decode_attn_stats under the same flag).  No statistics pass and no
 * stored logits: the keys are read once.  No workspace; scores is
 * [njobs][window][seq_len] float32 (hc_drift_select builds the score
 * histograms itself when given none).
 */
int hc_score_given_stats(int dtype, const void* q, const int64_t* q_off, int64_t q_head_stride,
                         int64_t q_row_stride, const void* kstore, const int64_t* row_tile_off, const int32_t* k_row,
                         int njobs, int seq_len, int group, int window, int flags, int pooling, int kernel,
                         float scale, const float* stats, const int64_t* stat_off, float* scores, void* stream);

/*
 * CAKE layer scoring, CAKECluster.update_kv (heterocache/kv_cluster.py:284-315).
 * Job j = b*kv_heads + h holds query heads h*group .. h*group+group-1; query
 * row (g, w) is q + q_off[j] + g*q_head_stride + w*q_row_stride, w < window
 * (the last `window` positions), and key t is k + k_off[j] + t*k_tok_stride.
 * p = softmax over the seq_len keys of scale * q.k with the window causally
 * masked (row w sees t <= seq_len - window + w), cast to the model dtype
 * under HC_SCORE_ROUND_BF16 / _F16 (the only flags accepted).  Over the
 * positions t < span = seq_len - window:
 *   scores[j][t] = max_g avg_pool1d_5(mean_w p + gamma * var_w p)
 *     (unbiased variance over the window rows; casts where the reference
 *     casts: mean, var, gamma*var, their sum, the pooled value);
 *   stats_out[0] = -sum p log(p + 1e-10) over every row and t < span;
 *   stats_out[1] = sum of var_w p over batch, then heads, then t (cast after
 *     each stage, as var.sum(0).sum(0).sum(0));
 *   stats_out[2] = stats_out[0] * stats_out[1], or 0 when either is NaN.
 * window: a positive multiple of 16 below seq_len; group*window <= 256
 * (<= 128 for float32).  stats_out: 3 floats in device memory.
 */
int hc_cake_score(int dtype, const void* q, const int64_t* q_off, int64_t q_head_stride, int64_t q_row_stride,
                  const void* k, const int64_t* k_off, int64_t k_tok_stride, int batch, int kv_heads, int seq_len,
                  int group, int window, int flags, float scale, float gamma, float* scores, float* stats_out,
                  void* workspace, size_t workspace_bytes, void* stream);
size_t hc_cake_workspace_size(int batch, int kv_heads, int seq_len, int group, int window);

/*
 * Per-job top-k kept set in ascending position order.  Job j keeps the
 * cap[j] positions of scores[j*score_stride + t], t < span, ranked by (score
 * descending, position ascending); with window > 0 it keeps cap[j] - window of
 * them and appends positions span .. span+window-1.  Writes idx[j*idx_stride
 * + i] (at most idx_stride entries per job) and counts[j] (optional).
 * Replaces topk -> mask -> sort of heterocache/cache_utils.py:831-851, the
 * SnapKV topk + window concat of heterocache/kv_cluster.py:187-197 and the
 * drift / retrieval topk of heterocache/cache_utils.py:1060-1061, 1090-1093.
 * key_bits (0 = 32): the scores are non-negative and their float32 bit
 * patterns end in 32 - key_bits zero bits (scores rounded to bfloat16: 16;
 * to float16: 19, the reference's cast chain), so a radix pass per 8 of the
 * leading key_bits suffices; the result is the one of 32.  A wrong hint
 * ranks scores that differ only in the ignored bits as ties.
 */
int hc_select_topk(const float* scores, int64_t score_stride, int njobs, int span, const int32_t* caps, int window,
                   int32_t* idx, int64_t idx_stride, int32_t* counts, void* hist, size_t hist_bytes, void* scratch,
                   size_t scratch_bytes, int key_bits, void* stream);
/* hist: hc_select_hist_size(njobs) bytes, zero-filled before its first use;
 * every completed call leaves it zeroed again (calls on one stream may share
 * it).  scratch: hc_select_scratch_size(njobs, span) bytes, no initialisation. */
size_t hc_select_hist_size(int njobs);
size_t hc_select_scratch_size(int njobs, int span);

/*
 * Position lists -> bitmasks: set j (words uint32 words at bits + j*words) is
 * cleared and then holds the first counts[j] (or fixed_count) positions of
 * list row r = (row_of ? row_of[j] : j), idx + r*idx_stride (row_of lets the
 * sets take their lists from a selection's rows in another order, without a
 * reordering copy).  With trigger != NULL set j is left untouched unless
 * trigger[trig_of ? trig_of[j] : j] != 0.  Holds the pivot reference sets of
 * heterocache/cache_utils.py:1189-1190 (prefill) and :1082 (update on drift).
 */
int hc_set_bits(const int32_t* idx, int64_t idx_stride, const int32_t* counts, int fixed_count, int nsets,
                uint32_t* bits, int64_t words, int nbits, const int32_t* trigger, const int32_t* trig_of,
                const int64_t* row_of, void* stream);

/*
 * out[j] = |{ idx[j*idx_stride + i] : i < count } ∩ set(ref_of ? ref_of[j] : j)|.
 * The searchsorted overlap of heterocache/cache_utils.py:1063-1073.
 */
int hc_overlap_count(const int32_t* idx, int64_t idx_stride, int count, int nlists, const uint32_t* bits,
                     int64_t words, int nbits, const int32_t* ref_of, int32_t* out, void* stream);

/*
 * The whole drift decision of a group of pivot rows from their step scores,
 * without index lists.  Row j of nsets (j = leader * batch + b) holds `steps`
 * score rows scores[(j*steps + s)*score_stride + t], t < span; caps[j*steps +
 * s] (= K) is the size of each step's top set, ranked by (score descending,
 * position ascending).  Computes overlap[j*steps + s] = |top_K(j, s) ∩ set j|
 * against the bitmask sets (set j: `words` uint32 words at bits + j*words)
 * straight from each step's threshold, then trigger[leader] as
 * hc_drift_decide does (batch mean of count / K, median over the steps, <
 * threshold), and finally, for every set whose leader triggered
 * (trigger[trig_of[j]]), rewrites set j as top_K of its last step.  Replaces
 * the topk + sort + searchsorted + median + set update of
 * heterocache/cache_utils.py:1059-1082 without writing the K-long index
 * lists.  hist: the score histograms hc_score built for these rows (its
 * `hist` output, [nsets*steps][4096]), or NULL to have them built here with
 * one more pass over the scores; from them one pass over the scores counts
 * the overlap above each row's threshold bin and collects the bin's
 * positions, and a per-row radix over those candidates fixes the exact
 * threshold and tie cut (ties of the threshold: lowest positions first).
 * scratch: hc_drift_scratch_size(nsets*steps, span) bytes, no
 * initialisation.
 */
int hc_drift_select(const float* scores, int64_t score_stride, int nsets, int steps, int batch, int span,
                    const int32_t* caps, int K, uint32_t* bits, int64_t words, const int32_t* trig_of, int nlead,
                    double threshold, int32_t* overlap, int32_t* trigger, const uint32_t* hist, void* scratch,
                    size_t scratch_bytes, void* stream);
size_t hc_drift_scratch_size(int njobs, int span);

/*
 * counts: [npiv][batch][steps] overlap counts of top-K sets.  Per pivot:
 * overlap[s] = mean_b(count/K) (float32), median over steps as
 * statistics.median defines it, trigger = median < threshold
 * (heterocache/cache_utils.py:1073-1080).  overlap and median are optional.
 */
int hc_drift_decide(const int32_t* counts, int npiv, int batch, int steps, int K, double threshold, float* overlap,
                    double* median, int32_t* trigger, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* HC_H_ */
