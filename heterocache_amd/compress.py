"""Prefill compression and pivot scoring on libhc kernels.

Host-side composition of hc_score / hc_select_topk / hc_gather_store into the
reference's operations:

  last_query_scores   pooled last-query attention per KV head
                      (heterocache/cache_utils.py:807-829, :1158-1187)
  window_scores       SnapKV observation-window scores
                      (heterocache/kv_cluster.py:165-185), generalised to a
                      GQA group (max over the group)
  cake_scores         CAKE mean + gamma * variance scores with the layer's
                      entropy and variance sums (heterocache/kv_cluster.py:284-315)
  pivot_step_scores   buffered decode queries vs a pivot's prefill keys read
                      in place from the store (heterocache/cache_utils.py:1030-1057)
  select_kept         per-head budget top-k in ascending order
                      (heterocache/cache_utils.py:831-851)
"""
import math

import torch

from . import _lib, ops

ROUND_FLAGS = {None: 0, torch.float32: 0, torch.bfloat16: _lib.HC_SCORE_ROUND_BF16,
               torch.float16: _lib.HC_SCORE_ROUND_F16}
# Leading bits of the float32 pattern a score rounded to that dtype can set
# (bfloat16: sign, exponent and 7 mantissa bits; float16: its 10 mantissa
# bits below the float32 exponent): hc_select_topk's key_bits.
KEY_BITS = {None: 0, torch.float32: 0, torch.bfloat16: 16, torch.float16: 19}


def _check_qk(q, k):
    if q.dim() != 4 or k.dim() != 4 or q.shape[-1] != 128 or k.shape[-1] != 128:
        raise ValueError("q and k must be [B, heads, seq, 128]")
    if q.stride(-1) != 1 or k.stride(-1) != 1:
        raise ValueError("q and k need a unit channel stride")
    if q.shape[0] != k.shape[0]:
        raise ValueError("q and k batch sizes differ")


def _dev_i64(vals, device):
    return ops.to_device(list(vals), device, torch.int64)


# Per-job element offsets depend only on shapes and strides, not on the data:
# they are built and copied to the device once per layout.
_OFFSETS = {}
_OFFSETS_MAX = 256


def _job_offsets(key, device, build):
    """(q_off, k_off) int64 device tensors for a layout key, built by build()."""
    key = (str(device),) + key
    hit = _OFFSETS.get(key)
    if hit is None:
        if len(_OFFSETS) >= _OFFSETS_MAX:
            _OFFSETS.clear()
        q_off, k_off = build()
        hit = _OFFSETS[key] = (_dev_i64(q_off, device), _dev_i64(k_off, device))
    return hit


def window_scores(q, k, kv_heads, group, window, pooling="avgpool", kernel=5, window_keep=False, causal=True,
                  round_dtype=None, scale=None, stream=None, stats=None):
    """Scores [B * len(kv_heads), span] of the last `window` query positions.

    q: [B, Hq, Lq, 128]; k: [B, Hkv, L, 128] (post-RoPE, any strides with unit
    channel stride).  Query heads h*group .. h*group+group-1 score kv head h.
    window_keep=True scores only [0, L - window) (SnapKV); otherwise [0, L).
    round_dtype reproduces the reference's casts to that dtype.
    stats: the softmax statistics [B, Hq, Ws, 2] (Ws >= window) that
    ops.prefill_attn reported for the last Ws queries of this q over this k;
    given them, the scorer reads the keys once (uncast scores only, and the
    window must see causally, as the attention did, unless it is one row).
    """
    _check_qk(q, k)
    B, Hq, Lq, _ = q.shape
    L = k.shape[2]
    if window > Lq:
        raise ValueError("window longer than the query sequence")
    scale = 1.0 / math.sqrt(128) if scale is None else scale
    kv_heads = tuple(kv_heads)

    def build():
        q_off = [b * q.stride(0) + h * group * q.stride(1) + (Lq - window) * q.stride(2)
                 for b in range(B) for h in kv_heads]
        k_off = [b * k.stride(0) + h * k.stride(1) for b in range(B) for h in kv_heads]
        return q_off, k_off
    q_off, k_off = _job_offsets(("window", B, kv_heads, group, window, Lq, q.stride()[:3], k.stride()[:2]),
                                q.device, build)
    flags = ROUND_FLAGS[round_dtype] | _lib.HC_SCORE_SUM_WINDOW
    if causal:
        flags |= _lib.HC_SCORE_CAUSAL_WINDOW
    span = L - window if window_keep else L
    if stats is not None:
        if ROUND_FLAGS[round_dtype]:
            raise ValueError("attention statistics are of uncast logits: no round_dtype with stats")
        if not causal and window > 1:
            raise ValueError("attention statistics describe a causal window")
        Ws = stats.shape[2]
        if stats.shape[:2] != (B, Hq) or Ws < window or stats.shape[3] != 2 or not stats.is_contiguous():
            raise ValueError(f"stats must be a contiguous [{B}, {Hq}, >= {window}, 2] tensor")
        stat_off = _job_offsets(("window_stats", B, kv_heads, group, window, Hq, Ws), q.device,
                                lambda: ([((b * Hq + h * group) * Ws + Ws - window) * 2 for b in range(B)
                                          for h in kv_heads], [0]))[0]
        out = ops.score_with_stats(q, q_off, q.stride(1), q.stride(2), k, k_off, k.stride(2), L, group, window, span,
                                   pooling, kernel, scale, stats, stat_off=stat_off, stat_head_stride=2 * Ws,
                                   flags=flags, stream=stream)
        return out.view(q_off.numel(), span)
    out = ops.score(q, q_off, q.stride(1), q.stride(2), k, k_off, k.stride(2), L, group, window, span, pooling, kernel,
                    scale, flags=flags, stream=stream)
    return out.view(q_off.numel(), span)


def cake_scores(q, k, window, gamma=200.0, round_dtype=None, scale=None, stream=None):
    """CAKE heavy-hitter scores [B * Hkv, L - window] and the device triple
    (entropy, variance sum, preference) of one layer
    (heterocache/kv_cluster.py:284-315).

    q: [B, Hq, Lq, 128] (the last `window` positions are the observation
    window); k: [B, Hkv, L, 128], not repeated: query heads h*G .. h*G+G-1
    score kv head h.
    """
    _check_qk(q, k)
    B, Hq, Lq, _ = q.shape
    Hkv, L = k.shape[1], k.shape[2]
    if Hq % Hkv:
        raise ValueError(f"{Hq} query heads do not group over {Hkv} kv heads")
    if window > Lq:
        raise ValueError("window longer than the query sequence")
    group = Hq // Hkv
    scale = 1.0 / math.sqrt(128) if scale is None else scale
    def build():
        q_off = [b * q.stride(0) + h * group * q.stride(1) + (Lq - window) * q.stride(2)
                 for b in range(B) for h in range(Hkv)]
        k_off = [b * k.stride(0) + h * k.stride(1) for b in range(B) for h in range(Hkv)]
        return q_off, k_off
    q_off, k_off = _job_offsets(("cake", B, Hkv, group, window, Lq, q.stride()[:3], k.stride()[:2]), q.device, build)
    return ops.cake_score(q, q_off, q.stride(1), q.stride(2), k, k_off, k.stride(2), B, Hkv, L, group, window, scale,
                          gamma, flags=ROUND_FLAGS[round_dtype], stream=stream)


def last_query_scores(q, k, kv_heads, group, pooling="avgpool", kernel=5, round_dtype=None, scale=None, stream=None,
                      stats=None):
    """Pooled last-query attention per KV head, max over its query group
    (stats: as for window_scores; the last row is used)."""
    return window_scores(q, k, kv_heads, group, 1, pooling, kernel, window_keep=False, causal=False,
                         round_dtype=round_dtype, scale=scale, stream=stream, stats=stats)


def pivot_step_metadata(q_steps, store, rows, heads, group):
    """Device offset tensors of pivot_step_scores for a fixed pivot set."""
    B = q_steps.shape[0]
    hkv = store.rows // B
    q_off = [(r // hkv) * q_steps.stride(0) + h * group * q_steps.stride(1) for r, h in zip(rows, heads)]
    return _dev_i64(q_off, q_steps.device), ops.to_device(list(rows), q_steps.device, torch.int32)


def pivot_step_scores(q_steps, store, rows, heads, group, seq_len, pooling="avgpool", kernel=5, round_dtype=None,
                      scale=None, stream=None, metadata=None, hist=None):
    """Scores [len(rows), S, seq_len] of S buffered decode queries per pivot
    (and, into `hist`, their first-digit key histograms; see ops.score).

    q_steps: [B, Hq, S, 128]; rows[j] is the store row of pivot j (batch
    b_j = rows[j] // Hkv) whose query heads are heads[j]*group + g.  Keys are
    the pivot's store slots [0, seq_len), read in place.
    """
    B, Hq, S, D = q_steps.shape
    if D != 128 or q_steps.stride(-1) != 1:
        raise ValueError("q_steps must be [B, Hq, S, 128] with unit channel stride")
    scale = 1.0 / math.sqrt(128) if scale is None else scale
    q_off, k_row = metadata if metadata is not None else pivot_step_metadata(q_steps, store, rows, heads, group)
    flags = ROUND_FLAGS[round_dtype]
    out = ops.score(q_steps, q_off, q_steps.stride(1), q_steps.stride(2), store.k, None, 0,
                    seq_len, group, S, seq_len, pooling, kernel, scale, flags=flags,
                    row_tile_off=store.row_tile_off, k_row=k_row, hist=hist, stream=stream)
    return out.view(q_off.numel(), S, seq_len)


def select_kept(scores, caps, window=0, max_cap=None, stream=None, round_dtype=None):
    """Ascending kept positions [jobs, max_cap (+window)] and counts [jobs].

    scores: [jobs, span] float32 (span excludes a force-kept window).
    caps: per-job budgets (python ints or an int32 device tensor).
    round_dtype: the dtype the scores were rounded to by the reference's
    cast chain (non-negative scores; the selection then runs fewer radix
    passes, with the same result).
    """
    jobs, span = scores.shape
    if not torch.is_tensor(caps):
        caps_list = [int(c) for c in caps]
        caps = ops.to_device(caps_list, scores.device, torch.int32)
        if max_cap is None:
            max_cap = max(caps_list) if caps_list else 0
    width = max(1, min(max_cap if max_cap is not None else span + window, span + window))
    idx = torch.empty((jobs, width), dtype=torch.int32, device=scores.device)
    idx, counts = ops.select_topk(scores, caps, span, window=window, idx=idx, stream=stream,
                                  key_bits=KEY_BITS.get(round_dtype, 0))
    return idx, counts
