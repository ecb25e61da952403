"""Numpy restatement of HeteroCache's compressed-KV attention path (oracle).

TEST INFRASTRUCTURE ONLY -- imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the product.

Conventions: arrays are numpy; a "row" is one (batch, kv-head) pair, row =
b * Hkv + h; tensors follow the reference's [B, heads, seq, d] layout.

Tie-break (stated, the reference's torch.topk order on its GPU is
implementation defined): among equal scores the LOWER token index ranks
first.  Every selection here is "sort by (-score, index), take the first k".

Pinning of each function (beyond its own formula) -- tests/test_oracle.py:
  get_compress_len / prefill_caps / capacity_f64  hand vectors from the
      reference's numbers (49629 @128K, 2048 @config-0, f32-vs-f64 edge).
  softmax / pooling / group max   torch.nn.functional (softmax, avg_pool1d,
      max_pool1d) on random inputs, and closed forms (uniform scores).
  topk_select                     brute force over all subsets on tiny
      inputs; torch.topk on distinct scores.
  topk_set                        equals the sorted topk_indices list on
      random, heavily tied and edge-case (k = 0, k >= n) inputs.
  window_scores                   reduces to last_query_scores at W=1 and to
      snapkv_update_kv at G=1 (the two reference functions it generalises).
  decode_attention                float64 closed form vs torch SDPA; a
      one-token row returns V exactly; uniform keys give the mean of V.
  softmax_lse2                    scipy.special.logsumexp / ln 2 on random
      rows; n equal keys give s + log2(n); stat_len cuts the keys.
  drift_check                     overlap of identical sets is 1, of disjoint
      sets is 0; statistics.median.
  retrieval_indices               ascending-prefix rule on a hand example.
  reorder_plan                    the committed Llama-3.1-8B head JSON, layer
      23 (leader order quirk) worked out by hand.
  cake_layer_scores               at gamma 0 and G = 1, W * hh equals
      window_scores (SnapKV avgpool-5); uniform keys against closed forms
      (statistics.variance, the entropy of 1/n rows, zero-padded pooling
      edges); the group max of two one-head calls.
  cake_adjust_budgets             hand vectors (clip + spread, truncation,
      negative difference) and sum == total on random budgets.
  cake_prefill                    final kept set of every layer = top-(min of
      its budgets over the prompt) of its own scores; budgets sum to the total.
"""
import math
import statistics

import numpy as np

HEAD_DIM = 128


# --------------------------------------------------------------------------
# a1, a2: budgets
# --------------------------------------------------------------------------
def get_compress_len(compression_ratio, full_heads, ori_len, num_kv_heads):
    """heterocache/cache_utils.py:15-16 (float64, truncation toward zero)."""
    return int((compression_ratio * num_kv_heads - full_heads) * ori_len / (num_kv_heads - full_heads))


def prefill_caps(base, ratios, seq_len):
    """Per-head prefill budget, float32 product then truncation, clamped to L.

    heterocache/cache_utils.py:793-799: caps = (base * ratios_f32).int();
    keep_lens = clamp(caps, max=L).
    """
    r = np.asarray(ratios, dtype=np.float32)
    caps = (np.float32(base) * r).astype(np.float32)
    caps = np.trunc(caps).astype(np.int64)
    return np.minimum(caps, seq_len)


def capacity_f64(base, ratio, seq_len):
    """Float64 budget used for pool sizing and retrieval lengths.

    heterocache/cache_utils.py:714-718 and :1084-1087: min(int(base*ratio), L).
    """
    return max(min(int(base * ratio), seq_len), 0)


# --------------------------------------------------------------------------
# dtype emulation
# --------------------------------------------------------------------------
def round_bf16(x):
    """Round float32 values to bfloat16 (round-to-nearest-even), as float32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32).reshape(x.shape)


def round_to(x, io_dtype):
    """Round to the model dtype ('bfloat16' / 'float16'); None keeps float32."""
    x = np.asarray(x, dtype=np.float32)
    if io_dtype is None or io_dtype == "float32":
        return x
    if io_dtype == "bfloat16":
        return round_bf16(x)
    if io_dtype == "float16":
        return x.astype(np.float16).astype(np.float32)
    raise ValueError(io_dtype)


# --------------------------------------------------------------------------
# scoring primitives
# --------------------------------------------------------------------------
def softmax_f32(logits, axis=-1):
    """nn.functional.softmax(x, dtype=float32): evaluated in float64, rounded."""
    z = np.asarray(logits, dtype=np.float64)
    m = np.max(z, axis=axis, keepdims=True)
    e = np.exp(z - m)
    return (e / np.sum(e, axis=axis, keepdims=True)).astype(np.float32)


def pool1d(x, kind, kernel):
    """F.avg_pool1d / F.max_pool1d with padding=kernel//2, stride 1 (last axis).

    avg: zero padding, divisor = kernel (count_include_pad=True).
    max: -inf padding.  Only odd kernels keep the length (reference uses 5, 7).
    """
    if kernel % 2 != 1:
        raise ValueError("pooling kernel must be odd")
    x = np.asarray(x, dtype=np.float64)
    p = kernel // 2
    L = x.shape[-1]
    pad_val = 0.0 if kind == "avgpool" else -np.inf
    xp = np.full(x.shape[:-1] + (L + 2 * p,), pad_val, dtype=np.float64)
    xp[..., p:p + L] = x
    win = np.stack([xp[..., j:j + L] for j in range(kernel)], axis=0)
    if kind == "avgpool":
        return (win.sum(axis=0) / kernel).astype(np.float32)
    if kind == "maxpool":
        return win.max(axis=0).astype(np.float32)
    raise ValueError(f"Pooling method not supported: {kind}")


def last_query_scores(q_last, k, pooling, kernel, io_dtype=None, scale=None):
    """Pooled last-query attention, max over the query group.

    heterocache/cache_utils.py:807-829 (prefill_select) and :1158-1187
    (init_coefficient):  w = softmax_f32(q.K^T/sqrt(d)).to(dtype);
    pool_k(w); max over the G query heads of each kv head.
    q_last: [n_kv, G, d]; k: [n_kv, L, d] -> scores [n_kv, L] (float32).
    """
    q_last = np.asarray(q_last, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    d = q_last.shape[-1]
    return _pooled_group_max(np.einsum("hgd,hld->hgl", q_last, k), d, pooling, kernel, io_dtype, scale)


def _pooled_group_max(dots, d, pooling, kernel, io_dtype, scale):
    """The steps of last_query_scores after the dot products q.k
    (dots [n, G, L] float64): scale and casts, softmax_f32, pooling, max
    over the group."""
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    if io_dtype not in (None, "float32"):
        logits = round_to(round_to(dots, io_dtype) * np.float32(scale), io_dtype)
    else:
        logits = (dots * scale).astype(np.float32)
    w = round_to(softmax_f32(logits), io_dtype)
    w = round_to(pool1d(w, pooling, kernel), io_dtype)
    return w.max(axis=1)


def window_scores(q_win, k, pooling, kernel, window_keep, io_dtype=None, scale=None):
    """Observation-window score, generalising the reference's two scorers.

    S_h[t] = max_g pool_k( sum_w softmax_t(q_{g,w}.k_t/sqrt(d) + causal) )
    q_win: [n_kv, G, W, d], the last W query positions; k: [n_kv, L, d].
    The window's own W keys are causally masked (query w sees key L-W+j only
    for j <= w), kv_cluster.py:169-175.  With window_keep the scored span is
    [0, L-W) (kv_cluster.py:178) -- at G=1 this is SnapKVCluster.update_kv's
    score (heterocache/kv_cluster.py:155-185).  Without it the span is [0, L)
    and at W=1 this is last_query_scores (heterocache/cache_utils.py:807-829).
    The window sum of a cast softmax is rounded once (ATen reductions
    accumulate in float32).  Returns [n_kv, span] float32.
    """
    q_win = np.asarray(q_win, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    n_kv, G, W, d = q_win.shape
    L = k.shape[1]
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    logits = np.einsum("hgwd,hld->hgwl", q_win, k)
    if io_dtype not in (None, "float32"):
        logits = round_to(round_to(logits, io_dtype) * np.float32(scale), io_dtype).astype(np.float64)
    else:
        logits = (logits * scale).astype(np.float32).astype(np.float64)
    # causal mask inside the window: query w may see window key j <= w.
    for w in range(W):
        logits[:, :, w, L - W + w + 1:] = -np.inf
    p = round_to(softmax_f32(logits), io_dtype)
    span = L - W if window_keep else L
    s = round_to(p[..., :span].astype(np.float64).sum(axis=2), io_dtype)
    s = round_to(pool1d(s, pooling, kernel), io_dtype)
    return s.max(axis=1)


def snapkv_update_kv(key_states, query_states, value_states, window_size, compression_ratio, pooling, kernel,
                     num_key_value_groups, io_dtype=None):
    """SnapKVCluster.update_kv, heterocache/kv_cluster.py:155-199.

    key/query/value: [B, H, L, d] (keys already repeated per query head).
    Returns compressed (key, value) [B, H, cap, d].
    """
    B, H, L, d = query_states.shape
    cap = max(int(compression_ratio * L / num_key_value_groups), 2)
    if cap > L:
        return key_states, value_states
    W = window_size
    ks, vs = [], []
    for b in range(B):
        kb, vb = [], []
        for h in range(H):
            s = window_scores(query_states[b, h][None, None, -W:], key_states[b, h][None], pooling, kernel,
                              window_keep=True, io_dtype=io_dtype)[0]
            top = topk_indices(s, cap - W)  # reference order: descending score
            kb.append(np.concatenate([key_states[b, h, :L - W][top], key_states[b, h, L - W:]], axis=0))
            vb.append(np.concatenate([value_states[b, h, :L - W][top], value_states[b, h, L - W:]], axis=0))
        ks.append(np.stack(kb))
        vs.append(np.stack(vb))
    return np.stack(ks), np.stack(vs)


def pyramidkv_layer_capacity(max_capacity_prompt, q_len, window, beta, num_hidden_layers, layer_idx):
    """Kept tokens before the window of PyramidKVCluster.update_kv, or None
    when the prompt stays uncompressed (heterocache/kv_cluster.py:61-79,
    :84, :97, :126).  Python floor division as the reference."""
    cap, W = max_capacity_prompt, window
    min_num = (cap - W) // beta
    max_num = (cap - W) * 2 - min_num
    if max_num >= q_len - W:
        max_num = q_len - W
        min_num = (cap - W) * 2 - max_num
    steps = (max_num - min_num) // (num_hidden_layers - 1)
    if q_len < cap:
        return None
    if q_len < (cap - W) * 2:
        return cap - W
    return max_num - layer_idx * steps


def pyramidkv_update_kv(key_states, query_states, value_states, window_size, compression_ratio, pooling, kernel,
                        num_key_value_groups, num_hidden_layers, layer_idx, beta=20, io_dtype=None):
    """PyramidKVCluster.update_kv, heterocache/kv_cluster.py:55-136: the
    SnapKV score with a per-layer capacity.  Returns compressed (key, value)
    [B, H, keep + W, d] in the reference's order (top-k by descending score,
    then the window)."""
    B, H, L, d = query_states.shape
    cap = int(compression_ratio * L / num_key_value_groups)
    keep = pyramidkv_layer_capacity(cap, L, window_size, beta, num_hidden_layers, layer_idx)
    if keep is None:
        return key_states, value_states
    W = window_size
    ks, vs = [], []
    for b in range(B):
        kb, vb = [], []
        for h in range(H):
            sc = window_scores(query_states[b, h][None, None, -W:], key_states[b, h][None], pooling, kernel,
                               window_keep=True, io_dtype=io_dtype)[0]
            top = topk_indices(sc, keep)
            kb.append(np.concatenate([key_states[b, h, :L - W][top], key_states[b, h, L - W:]], axis=0))
            vb.append(np.concatenate([value_states[b, h, :L - W][top], value_states[b, h, L - W:]], axis=0))
        ks.append(np.stack(kb))
        vs.append(np.stack(vb))
    return np.stack(ks), np.stack(vs)


def h2o_scores(query_states, key_states, scale=None):
    """Heavy-hitter score of H2OKVCluster.update_kv (heterocache/kv_cluster.py:
    406-440): softmax over all keys of every query position (no mask), summed
    over the query positions.  [B, H, L] float64."""
    q = np.asarray(query_states, dtype=np.float64)
    k = np.asarray(key_states, dtype=np.float64)
    scale = 1.0 / math.sqrt(q.shape[-1]) if scale is None else scale
    z = scale * np.einsum("bhid,bhtd->bhit", q, k)
    z -= z.max(axis=-1, keepdims=True)
    p = np.exp(z)
    p /= p.sum(axis=-1, keepdims=True)
    return p.sum(axis=2)


def h2o_update_kv(key_states, query_states, value_states, compression_ratio, num_key_value_groups):
    """H2OKVCluster.update_kv (heterocache/kv_cluster.py:397-450): the top
    capacity keys by heavy-hitter score, no window.  Returns (key, value, kept
    index lists [B, H, cap] in descending score order)."""
    B, H, L, d = query_states.shape
    cap = max(int(compression_ratio * L / num_key_value_groups), 2)
    if cap > L:
        return key_states, value_states, None
    sc = h2o_scores(query_states, key_states)
    top = np.stack([np.stack([topk_indices(sc[b, h], cap) for h in range(H)]) for b in range(B)])
    k = np.take_along_axis(np.asarray(key_states), top[..., None], axis=2)
    v = np.take_along_axis(np.asarray(value_states), top[..., None], axis=2)
    return k, v, top


def streamingllm_update_kv(key_states, value_states, compression_ratio, sink=4):
    """StreamingLLMKVCluster.update_kv (heterocache/kv_cluster.py:500-523):
    the first `sink` tokens and the last max(int(r L), 5) - 4 tokens."""
    L = key_states.shape[2]
    recent = max(int(compression_ratio * L), 5) - 4
    if recent > L:
        return key_states, value_states
    keep = np.concatenate([np.arange(sink), np.arange(L - recent, L)])
    return key_states[:, :, keep], value_states[:, :, keep]


def cake_layer_scores(query_states, key_states, window, gamma=200.0, io_dtype=None, scale=None):
    """Scoring of CAKECluster.update_kv for one layer (heterocache/kv_cluster.py:284-315).

    query_states [B, Hq, L, d]; key_states [B, Hkv, L, d], repeated over the
    query group for the logits (:290-292).  p = softmax_f32 of the last W
    query rows against all L keys, the window causally masked, cast to
    io_dtype (:293-303).  Over the positions t < L - W:
      entropy = -sum p log(p + 1e-10)                       (:220-224, :305)
      var     = unbiased variance over the W rows (cast); var_sum =
                var.sum(0) .sum(0) .sum(0), cast after each stage  (:307)
      pref    = entropy * var_sum, 0.0 when either is NaN   (:308-313)
      hh      = max over a kv head's query heads of
                avg_pool5(cast(cast(mean) + cast(gamma * var)))  (:317-324)
    Returns (hh [B, Hkv, L - W] float32, entropy, var_sum, pref).
    """
    q = np.asarray(query_states, dtype=np.float64)
    k = np.asarray(key_states, dtype=np.float64)
    B, Hq, L, d = q.shape
    Hkv = k.shape[1]
    G, W = Hq // Hkv, window
    span = L - W
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    logits = np.einsum("bhwd,bhld->bhwl", q[:, :, L - W:], np.repeat(k, G, axis=1))
    if io_dtype not in (None, "float32"):
        logits = round_to(round_to(logits, io_dtype) * np.float32(scale), io_dtype).astype(np.float64)
    else:
        logits = (logits * scale).astype(np.float32).astype(np.float64)
    for w in range(W):
        logits[:, :, w, L - W + w + 1:] = -np.inf
    p = round_to(softmax_f32(logits), io_dtype)[..., :span]          # float32 values
    p64 = p.astype(np.float64)
    entropy = -float(np.sum(p64 * np.log((p + np.float32(1e-10)).astype(np.float64))))
    mean = round_to(p64.mean(axis=2), io_dtype).astype(np.float64)   # [B, Hq, span]
    var = round_to(p64.var(axis=2, ddof=1), io_dtype).astype(np.float64)
    score = round_to(mean + round_to(gamma * var, io_dtype), io_dtype)
    pooled = round_to(pool1d(score, "avgpool", 5), io_dtype)
    hh = pooled.reshape(B, Hkv, G, span).max(axis=2)
    vs = round_to(var.sum(axis=0), io_dtype).astype(np.float64)      # over the batch
    vs = round_to(vs.sum(axis=0), io_dtype).astype(np.float64)       # over the heads
    var_sum = float(round_to(vs.sum(), io_dtype).reshape(-1)[0])
    entropy = float(np.float32(entropy))
    pref = 0.0 if (math.isnan(entropy) or math.isnan(var_sum)) else float(np.float32(entropy) * np.float32(var_sum))
    return hh, entropy, var_sum, pref


def cake_adjust_budgets(budget_list, total_budget, seq_len):
    """CAKECluster.adjust_budgets (heterocache/kv_cluster.py:225-271).

    Budgets truncate toward zero and are clipped at seq_len; the clipped
    excess is spread evenly over the layers still below seq_len (the
    remainder one each to the first of them).  The difference to
    total_budget is then spread the same way: added over the layers below
    seq_len, or taken from the layers above 1.
    """
    b = np.array(budget_list, dtype=np.int64)
    excess = int(np.maximum(b - seq_len, 0).sum())
    b = np.minimum(b, seq_len)
    if excess > 0:
        open_ = np.flatnonzero(b < seq_len)
        if open_.size:
            b[open_] += excess // open_.size
            b[open_[:excess % open_.size]] += 1
    diff = int(total_budget - b.sum())
    if diff != 0:
        open_ = np.flatnonzero(b < seq_len) if diff > 0 else np.flatnonzero(b > 1)
        if open_.size:
            step, rem = divmod(abs(diff), open_.size)
            sign = 1 if diff > 0 else -1
            b[open_] += sign * step
            b[open_[:rem]] += sign
    return [int(x) for x in b]


def cake_prefill(layers, compression_ratio, window, num_layers, gamma=200.0, io_dtype=None):
    """CAKECache + CAKECluster over one prompt, layer by layer
    (heterocache/kv_cluster.py:273-379, heterocache/cache_utils.py:277-373).

    layers: [(query_states [B, Hq, L, d], key_states [B, Hkv, L, d]), ...] in
    layer order.  After scoring layer l the total budget
    (cap - W) * num_layers is split over layers 0..l in proportion to their
    preference scores (float32, as the reference's numpy values), adjusted,
    and every layer 0..l is evicted again to its budget: top-k of its
    current scores (descending, ties to the lower position), window kept.
    Returns None when the prompt stays whole (cap > L), else
    (kept, budgets, prefs): kept[l] [B, Hkv, budget_l] int64 positions in
    the reference's order (window positions L-W.. follow), budgets[l] the
    final layer_budget entries, prefs the float32 preference scores.
    """
    L = layers[0][0].shape[2]
    W = window
    cap = max(int(compression_ratio * L), 2)
    if cap > L:
        return None
    total = (cap - W) * num_layers
    prefs, scores, kept, budgets = [], [], [], []
    for q, k in layers:
        hh, _, _, pref = cake_layer_scores(q, k, W, gamma, io_dtype)
        B, Hkv, span = hh.shape
        prefs.append(np.float32(pref))
        scores.append(hh)
        kept.append(np.broadcast_to(np.arange(span), (B, Hkv, span)).copy())
        budgets.append(cap - W)
        tot = sum(prefs)
        split = cake_adjust_budgets([p / tot * total for p in prefs], total, L - W)
        for i, bud in enumerate(split):
            bud = min(bud, L - W)
            n = min(bud, scores[i].shape[-1])
            top = np.stack([np.stack([topk_indices(scores[i][b, h], n) for h in range(Hkv)]) for b in range(B)])
            scores[i] = np.take_along_axis(scores[i], top, axis=-1)
            kept[i] = np.take_along_axis(kept[i], top, axis=-1)
            budgets[i] = bud
    return kept, budgets, prefs


def head_topk_sets(attn, num_q_heads, num_kv_heads, max_length, topk, io_dtype=None):
    """get_head_topk_exact, tools/get_cluster.py:13-56: the last query row of
    each (KV) head -- its query group averaged when the map holds the query
    heads of a GQA model -- limited to max_length, avg-pooled (k = min(5, n),
    zero padding k//2, divisor k) and its top-k position set.  attn:
    [B, heads, rows, seq] (or [B, heads, seq]).  Returns sets[h][b] (python
    sets) and the head count."""
    a = np.asarray(attn, dtype=np.float32)
    if a.ndim == 3:
        a = a[:, :, None]
    B, Hs, R, S = a.shape
    if num_q_heads != num_kv_heads and Hs == num_q_heads:
        G = num_q_heads // num_kv_heads
        a = a.reshape(B, num_kv_heads, G, R, S).mean(axis=2, dtype=np.float32)
        if io_dtype is not None:
            a = round_to(a, io_dtype)
    H = a.shape[1]
    sets = [[set() for _ in range(B)] for _ in range(H)]
    n = min(max_length, S)
    for h in range(H):
        vec = a[:, h, -1, :n]
        if vec.shape[-1] == 0:
            continue
        k = min(5, vec.shape[-1])
        pooled = pool1d(vec.astype(np.float32), "avgpool", k).astype(np.float32)
        kk = min(topk, vec.shape[-1])
        if kk == 0:
            continue
        for b in range(B):
            sets[h][b] = set(topk_indices(pooled[b], kk).tolist())
    return sets, H


def overlap_ratio(set_a, set_b, topk):
    """calculate_overlap_ratio, tools/get_cluster.py:58-66."""
    if not set_a or not set_b:
        return 0.0
    return len(set_a & set_b) / (len(set_a) if set_a else topk)


def star_clusters_greedy(adjacency, heads):
    """find_star_clusters_greedy, tools/get_cluster.py:70-110."""
    unassigned = set(heads)
    clusters, assigned = {}, set()
    while unassigned:
        cands = [(len(adjacency.get(n, set()) & unassigned), n, adjacency.get(n, set()) & unassigned)
                 for n in unassigned]
        cands.sort(key=lambda x: (-x[0], x[1]))
        degree, leader, members = cands[0]
        if degree == 0:
            break
        clusters[leader] = sorted(members)
        unassigned.remove(leader)
        assigned.add(leader)
        for m in members:
            unassigned.remove(m)
            assigned.add(m)
    return clusters, assigned


def head_analysis(maps, num_layers, num_q_heads, num_kv_heads, topk, max_length, stable_threshold, sim_threshold,
                  decode_step):
    """analyze_combined_heads, tools/get_cluster.py:113-330, on maps[layer][step]
    -> [B, heads, rows, seq] arrays.  Returns the JSON dict (relations keyed by
    int head; json.dumps turns them into the reference's string keys)."""
    type_map = {"anchor": 1, "volatile": 2, "pivot": 3, "satellite": 4}
    total = num_q_heads
    cls = [[0] * total for _ in range(num_layers)]
    alloc = [[-1.0] * total for _ in range(num_layers)]
    rel = [{} for _ in range(num_layers)]
    counts = {k: 0 for k in type_map}
    steps = sorted({s for per in maps.values() for s in per})
    prefill, decode = steps[0], steps[1:]
    spatial = decode_step if decode_step in steps else steps[-1]
    for layer in range(num_layers):
        if layer not in maps or prefill not in maps[layer]:
            continue
        base, H = head_topk_sets(maps[layer][prefill], num_q_heads, num_kv_heads, max_length, topk)
        B = len(base[0])
        if H != total and layer == 0:
            cls = [[0] * H for _ in range(num_layers)]
            alloc = [[-1.0] * H for _ in range(num_layers)]
        history = {h: [] for h in range(H)}
        for step in decode:
            if step not in maps[layer]:
                continue
            cur, _ = head_topk_sets(maps[layer][step], num_q_heads, num_kv_heads, max_length, topk)
            for h in range(H):
                ovs = [overlap_ratio(base[h][b], cur[h][b], topk) for b in range(B)]
                history[h].append(sum(ovs) / len(ovs))
        med, dyn = {}, {}
        for h in range(H):
            if not history[h]:
                dyn[h], med[h] = "volatile", 0.0
            else:
                med[h] = float(np.median(history[h]))
                dyn[h] = "volatile" if med[h] < stable_threshold else "anchor"
        adj = {}
        if spatial in maps[layer]:
            sp, _ = head_topk_sets(maps[layer][spatial], num_q_heads, num_kv_heads, max_length, topk)
            for i in range(H):
                for j in range(H):
                    if i == j:
                        continue
                    sim = sum(overlap_ratio(sp[i][b], sp[j][b], topk) for b in range(B)) / B
                    if sim >= sim_threshold:
                        adj.setdefault(i, set()).add(j)
        clusters, assigned = star_clusters_greedy(adj, list(range(H)))
        rel[layer] = clusters
        for h in range(H):
            alloc[layer][h] = med[h]
            if h in clusters:
                cls[layer][h] = type_map["pivot"]
                counts["pivot"] += 1
                alloc[layer][h] = -1.0
            elif h in assigned:
                cls[layer][h] = type_map["satellite"]
                counts["satellite"] += 1
            elif dyn[h] == "anchor":
                cls[layer][h] = type_map["anchor"]
                counts["anchor"] += 1
            else:
                cls[layer][h] = type_map["volatile"]
                counts["volatile"] += 1
                alloc[layer][h] = -1.0
    targets = [v for row in alloc for v in row if v > -0.5]
    inv_total = sum(1.0 / (v + 1e-6) for v in targets)
    if targets and inv_total > 1e-9:
        for r in range(len(alloc)):
            for c in range(len(alloc[r])):
                if alloc[r][c] > -0.5:
                    alloc[r][c] = (1.0 / (alloc[r][c] + 1e-6)) / inv_total * len(targets)
    return {"meta": {"type_map": type_map, "counts": counts}, "classification_matrix": cls,
            "allocation_matrix": alloc, "leader_member_relations": rel}


# --------------------------------------------------------------------------
# selection
# --------------------------------------------------------------------------
def topk_indices(scores, k):
    """Indices of the k largest scores, descending, ties -> lower index first.

    Stands in for torch.topk(k, sorted=True) (heterocache/cache_utils.py:832,
    :1061, :1092, :1189) under the stated tie-break.
    """
    s = np.asarray(scores)
    order = np.argsort(-s.astype(np.float64), kind="stable")
    return order[:k].astype(np.int64)


def topk_set(scores, k):
    """The positions topk_indices(scores, k) selects, ascending, in linear
    time: every score above the k-th largest value, then the lowest
    positions among the scores equal to it (the same tie rule).  The drift
    check and the retrieval take their sets this way; `scores` holds no NaN."""
    s = np.asarray(scores, dtype=np.float64)
    n = s.size
    if k <= 0:
        return np.empty(0, dtype=np.int64)
    if k >= n:
        return np.arange(n, dtype=np.int64)
    tau = np.partition(s, n - k)[n - k]
    above = np.flatnonzero(s > tau)
    tied = np.flatnonzero(s == tau)[:k - above.size]
    return np.sort(np.concatenate([above, tied])).astype(np.int64)


def topk_select(scores, cap):
    """Kept token set of one head, ascending positions.

    heterocache/cache_utils.py:831-851: topk(max cap) -> mask rank >= cap_h
    -> ascending sort.  The first cap_h entries of the sorted top-max_k list
    are the head's own top-cap_h, so the result is sort(topk(cap_h)).
    """
    return np.sort(topk_indices(scores, cap))


def select_with_window(scores, cap, seq_len, window):
    """Budget cap with the last `window` tokens force-kept (SnapKV style).

    heterocache/kv_cluster.py:187-197: topk(cap - W) over [0, L-W) plus the
    window.  Returned ascending (the store keeps temporal order,
    heterocache/cache_utils.py:782-786).
    """
    if cap >= seq_len:
        return np.arange(seq_len, dtype=np.int64)
    body = topk_select(scores[:seq_len - window], max(cap - window, 0))
    return np.concatenate([body, np.arange(seq_len - window, seq_len, dtype=np.int64)])


# --------------------------------------------------------------------------
# a10: decode attention
# --------------------------------------------------------------------------
def decode_attention(q, ks, vs, scale=None):
    """softmax(scale * q K^T) V per row, float64 closed form.

    Stands in for flash_attn_with_kvcache(..., causal=False)
    (heterocache/llama_model.py:382-389).  q: [rows, G, d]; ks/vs: lists of
    [len_r, d] arrays.  Returns [rows, G, d] float64 (zeros for empty rows).
    """
    q = np.asarray(q, dtype=np.float64)
    rows, G, d = q.shape
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    out = np.zeros((rows, G, d), dtype=np.float64)
    for r in range(rows):
        k = np.asarray(ks[r], dtype=np.float64)
        v = np.asarray(vs[r], dtype=np.float64)
        if k.shape[0] == 0:
            continue
        z = scale * (q[r] @ k.T)
        z -= z.max(axis=-1, keepdims=True)
        p = np.exp(z)
        p /= p.sum(axis=-1, keepdims=True)
        out[r] = p @ v
    return out


def softmax_lse2(q, ks, stat_len, scale=None, io_dtype=None):
    """Base-2 log-normaliser of every (row, query head) softmax over the
    row's first stat_len keys, float64.

    The drift check's probabilities (heterocache/cache_utils.py:1037-1043,
    softmax(q K^T / sqrt(d), dtype=float32) over a pivot's prefill keys) are
    exp2(s_t - lse2) with s_t = scale * log2(e) * q.k_t and
    lse2 = log2(sum_t exp2(s_t)); hc_decode_attn_stats reports lse2 as a
    (bound M, sum of exp2(s_t - M)) pair.  io_dtype ('bfloat16' /
    'float16'): the logits of the reference's casts instead, as
    _pooled_group_max forms them, s_t = log2(e) * round(round(q.k_t) * scale).
    q: [rows, G, d]; ks: list of [len_r, d].  Returns [rows, G] (-inf for a
    row with no key below stat_len).
    """
    q = np.asarray(q, dtype=np.float64)
    rows, G, d = q.shape
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    out = np.full((rows, G), -np.inf)
    for r in range(rows):
        k = np.asarray(ks[r], dtype=np.float64)[:stat_len]
        if k.shape[0] == 0:
            continue
        if io_dtype not in (None, "float32"):
            logits = round_to(round_to(q[r] @ k.T, io_dtype) * np.float32(scale), io_dtype)
            s2 = math.log2(math.e) * logits.astype(np.float64)
        else:
            s2 = scale * math.log2(math.e) * (q[r] @ k.T)
        m = s2.max(axis=-1, keepdims=True)
        out[r] = m[:, 0] + np.log2(np.exp2(s2 - m).sum(axis=-1))
    return out


def prefill_attention(q, k, v, scale=None):
    """Causal prefill attention, float64 closed form.

    Stands in for the flash-attn prefill call of LlamaAttention
    (heterocache/llama_model.py:353-361, transformers' flash_attention_forward
    with causal=True).  q: [B, Hq, Lq, d]; k, v: [B, Hkv, Lk, d] with
    Lq <= Lk; query i sits at position Lk - Lq + i and sees keys t <= that
    position (flash-attn's bottom-right alignment).  Query head h reads KV
    head h // (Hq // Hkv).  Returns [B, Lq, Hq, d] float64.
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    B, Hq, Lq, d = q.shape
    Hkv, Lk = k.shape[1], k.shape[2]
    G = Hq // Hkv
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    visible = np.arange(Lk)[None, :] <= (Lk - Lq + np.arange(Lq))[:, None]
    out = np.zeros((B, Lq, Hq, d), dtype=np.float64)
    for b in range(B):
        for h in range(Hq):
            z = scale * (q[b, h] @ k[b, h // G].T)
            z = np.where(visible, z, -np.inf)
            z -= z.max(axis=-1, keepdims=True)
            p = np.exp(z)
            p /= p.sum(axis=-1, keepdims=True)
            out[b, :, h] = p @ v[b, h // G]
    return out


# --------------------------------------------------------------------------
# a12, a13: pivot drift and retrieval
# --------------------------------------------------------------------------
def pivot_step_scores(q_steps, k_prefill, pooling, kernel, io_dtype=None, scale=None):
    """Scores of the buffered decode queries against a pivot's prefill keys.

    heterocache/cache_utils.py:1030-1057: logits of every (query head g,
    step s) -> softmax_f32 -> cast -> pool -> max over g.
    q_steps: [G, S, d]; k_prefill: [L, d] -> [S, L] float32.
    """
    q = np.asarray(q_steps, dtype=np.float64)
    G, S, d = q.shape
    k = np.asarray(k_prefill, dtype=np.float64)
    # Every (step, head) row against the same keys: one product, then the
    # per-step steps of last_query_scores.
    dots = (q.transpose(1, 0, 2).reshape(S * G, d) @ k.T).reshape(S, G, -1)
    return _pooled_group_max(dots, d, pooling, kernel, io_dtype, scale)


def drift_check(step_scores, ref_set, base_len, threshold):
    """Top-K overlap of each buffered step with the reference set, median.

    heterocache/cache_utils.py:1059-1080.  step_scores: [B, S, L];
    ref_set: [B, K] indices.  overlap_s = mean_b |topK_s ∩ ref_b| / K;
    coefficient = statistics.median(overlap); trigger = coefficient < thr.
    Returns (overlaps [S], median, trigger, cur_last [B, K] (topK of the last
    step, ascending)).
    """
    B, S, L = step_scores.shape
    overl = np.zeros((B, S), dtype=np.float64)
    cur_last = []
    for b in range(B):
        ref = np.zeros(L, dtype=bool)
        ref[np.asarray(ref_set[b], dtype=np.int64)] = True
        for s in range(S):
            cur = topk_set(step_scores[b, s], base_len)
            overl[b, s] = np.float32(np.count_nonzero(ref[cur])) / np.float32(base_len)
            if s == S - 1:
                cur_last.append(cur)
    overlaps = overl.astype(np.float32).mean(axis=0, dtype=np.float32)
    med = statistics.median([float(x) for x in overlaps])
    return overlaps, med, med < threshold, np.stack(cur_last)


def retrieval_lengths(base_len, member_ratios, seq_len, topk=None, use_f32=True):
    """Tokens retrieved into each satellite, heterocache/cache_utils.py:1084-1087.

    The reference uses float64 min(int(base*ratio), L); with use_f32 the
    float32 prefill cap is used instead so the write never passes the
    prefill region.  topk (the north-star retrieval size) caps every length.
    """
    if use_f32:
        lens = prefill_caps(base_len, member_ratios, seq_len).tolist()
    else:
        lens = [capacity_f64(base_len, r, seq_len) for r in member_ratios]
    if topk is not None:
        lens = [min(n, topk) for n in lens]
    return [int(n) for n in lens]


def retrieval_indices(last_step_scores, lengths):
    """Ascending top-max(len) list; member m takes its first len_m entries.

    heterocache/cache_utils.py:1090-1105 (per batch row; the reference's
    squeeze() makes the B=1 case the defined one).
    """
    mk = max(lengths) if lengths else 0
    idx = topk_set(last_step_scores, mk)
    return [idx[:n] for n in lengths]


# --------------------------------------------------------------------------
# a14: head order and derived lists
# --------------------------------------------------------------------------
SORT_PRIORITY = {1: 0, 4: 1, 2: 2, 3: 3}


def reorder_plan(classification, relations):
    """Head permutation and derived lists of one layer.

    heterocache/utils.py:101-116 (stable sort anchor, satellite, volatile,
    pivot) and :300-343 (derived lists, relations remapped in the original
    dict order, members sorted).
    Returns dict(perm, compress, select, update, keep, relations).
    """
    perm = [i for i, _ in sorted(enumerate(classification), key=lambda x: SORT_PRIORITY.get(x[1], 99))]
    cls = [classification[i] for i in perm]
    o2n = {old: new for new, old in enumerate(perm)}
    rel = {}
    for leader, members in relations.items():
        if int(leader) in o2n:
            rel[str(o2n[int(leader)])] = sorted(o2n[m] for m in members if m in o2n)
    return {
        "perm": perm,
        "compress": cls.count(1) + cls.count(4),
        "select": [i for i, x in enumerate(cls) if x == 3],
        "update": [i for i, x in enumerate(cls) if x == 4],
        "keep": [i for i, x in enumerate(cls) if x in (2, 3)],
        "relations": rel,
    }


def allocation_ratios(stabilities):
    """Inverse-stability allocation, tools/get_cluster.py:276-307.

    stabilities: list of per-layer lists, -1 for full-KV heads.  Targets get
    ratio = (1/(s+1e-6)) / sum(1/(s'+1e-6)) * n_targets (mean exactly 1).
    """
    targets = [s for row in stabilities for s in row if s > -0.5]
    n = len(targets)
    tot = sum(1.0 / (s + 1e-6) for s in targets)
    out = []
    for row in stabilities:
        out.append([((1.0 / (s + 1e-6)) / tot * n) if s > -0.5 else -1.0 for s in row])
    return out


# --------------------------------------------------------------------------
# End-to-end cache flow (one layer at a time), numpy
# --------------------------------------------------------------------------
class CacheOracle:
    """HeteroCache's per-layer flow on numpy arrays.

    Follows heterocache/cache_utils.py:884-1005 (update), :1149-1190
    (init_coefficient), :782-882 (prefill_select), :1007-1147
    (decode_select) and heterocache/llama_model.py:368-401 /
    heterocache/qwen_model.py:176-211 (decode order).  `data` is the
    augmented head record (derived lists in reordered head indices).  Defaults
    match the device build: float32 retrieval lengths and each pivot compared
    with its own reference set (quirks=True: the reference's float64 lengths
    and relation-order set indexing).

    Rows live in buffers sized for `max_gen` decode tokens, so long contexts
    append without copying; rows[layer][r] is [K view, V view] of the row's
    current tokens.

    score_hook(kind, layer, head, scores) -> scores, when given, sees every
    score array the flow ranks before it is ranked and returns the array the
    selection then uses: kind "prefill" (head h, [L] for one batch row --
    called once per (b, h) in batch-major order), "pivot" (pivot head, [L]
    per batch row), "drift" (leader head, [B, S, L]).  A test can record the
    oracle's own scores there and substitute a device's, so that the flow's
    integer logic (top-k and its tie rule, overlaps, medians, triggers,
    ascending prefixes, slot writes) is checked exactly on the device's
    scores while the scores themselves are compared within a tolerance.  A
    hook with a true `replaces_drift` attribute is called with scores None
    for "drift" and returns the [B, S, L] scores outright, so the oracle
    does not score the step queries itself.
    """

    def __init__(self, data, batch, q_heads, kv_heads, num_layers, ratio, threshold, decode_step, pooling, kernel,
                 retrieval_topk=None, quirks=False, select_before_attention=False, max_gen=64, score_hook=None,
                 io_dtype=None):
        self.data = data
        self.B, self.Hq, self.Hkv, self.NL = batch, q_heads, kv_heads, num_layers
        self.G = q_heads // kv_heads
        self.ratio, self.threshold, self.S = ratio, threshold, decode_step
        self.pooling, self.kernel = pooling, kernel
        self.topk, self.quirks, self.select_first = retrieval_topk, quirks, select_before_attention
        self.max_gen = max_gen
        self.score_hook = score_hook
        self.io_dtype = io_dtype    # the reference's casts of scores to the model dtype ("bfloat16", ...)
        self.full_heads = data["meta"]["counts"]["volatile"] + data["meta"]["counts"]["pivot"]
        self.rows = {}      # layer -> list over b*Hkv+h of [K, V] views [len, 128]
        self._buf = {}      # layer -> list over rows of (K, V) buffers [len + max_gen, 128]
        self.tier = {}      # layer -> (K, V) [B, Hkv, L, 128]
        self.ref = {}       # layer -> {leader: [set per b]}
        self.qbuf = {}
        self.base = None
        self.L = None
        self.triggers = []  # (layer, leader, triggered) per check
        self.medians = []   # (layer, leader, median) per check

    def _scores(self, kind, layer, head, scores):
        return scores if self.score_hook is None else self.score_hook(kind, layer, head, scores)

    def _set_row(self, layer, r, k_rows, v_rows):
        n, d = k_rows.shape
        kb = np.zeros((n + self.max_gen, d), dtype=k_rows.dtype)
        vb = np.zeros((n + self.max_gen, d), dtype=v_rows.dtype)
        kb[:n] = k_rows
        vb[:n] = v_rows
        self._buf[layer][r] = (kb, vb)
        self.rows[layer][r] = [kb[:n], vb[:n]]

    def prefill(self, layer, q, k, v):
        B, Hkv, L, _ = k.shape
        if self.base is None:
            self.L = L
            self.base = get_compress_len(self.ratio, self.full_heads, L, Hkv * self.NL)
        keep = set(self.data["need_to_keep_counts"][layer])
        n_c = self.data["need_to_compress_counts"][layer]
        caps = prefill_caps(self.base, self.data["allocation_matrix"][layer][:n_c], L)
        self.rows[layer] = [None] * (B * Hkv)
        self._buf[layer] = [None] * (B * Hkv)
        empty = np.zeros((0, k.shape[-1]), k.dtype)
        for b in range(B):
            for h in range(Hkv):
                r = b * Hkv + h
                if h in keep:
                    self._set_row(layer, r, k[b, h], v[b, h])
                elif h < n_c:
                    s = last_query_scores(q[b, h * self.G:(h + 1) * self.G, -1][None], k[b, h][None], self.pooling,
                                          self.kernel, io_dtype=self.io_dtype)[0]
                    s = self._scores("prefill", layer, h, s)
                    sel = topk_select(s, int(caps[h]))
                    self._set_row(layer, r, k[b, h][sel], v[b, h][sel])
                else:
                    self._set_row(layer, r, empty, empty)
        self.tier[layer] = (k, v)
        pivots = list(self.data["need_to_select_counts"][layer])
        rel = self.data["leader_member_relations"][layer]
        K = min(self.base, L)
        sets = {}
        for p in pivots:
            sets[p] = []
            for b in range(B):
                s = last_query_scores(q[b, p * self.G:(p + 1) * self.G, -1][None], k[b, p][None], self.pooling,
                                      self.kernel, io_dtype=self.io_dtype)[0]
                sets[p].append(set(topk_indices(self._scores("pivot", layer, p, s), K).tolist()))
        ref = {}
        for i, leader in enumerate(int(x) for x in rel):
            src = pivots[min(i, len(pivots) - 1)] if self.quirks else leader
            ref[leader] = sets[src]
        self.ref[layer] = ref
        self.qbuf[layer] = []

    def decode(self, layer, q, k_new, v_new, attend=True):
        """One decode step of one layer; returns attention output [B, Hq, 128]
        (float64), or None with attend=False (the step's append and selection
        still happen)."""
        B, Hkv = self.B, self.Hkv
        for b in range(B):
            for h in range(Hkv):
                r = b * Hkv + h
                kb, vb = self._buf[layer][r]
                n = len(self.rows[layer][r][0])
                if n >= len(kb):
                    raise RuntimeError(f"Layer {layer} OOM.")
                kb[n] = k_new[b, h, 0]
                vb[n] = v_new[b, h, 0]
                self.rows[layer][r] = [kb[:n + 1], vb[:n + 1]]
        if self.select_first:
            self._select(layer, q)
        out = None
        if attend:
            qa = q[:, :, 0].reshape(B * Hkv, self.G, -1)
            out = decode_attention(qa, [r[0] for r in self.rows[layer]], [r[1] for r in self.rows[layer]])
            out = out.reshape(B, self.Hq, -1)
        if not self.select_first:
            self._select(layer, q)
        return out

    def _select(self, layer, q):
        self.qbuf[layer].append(q[:, :, 0])
        if len(self.qbuf[layer]) < self.S:
            return
        qs = np.stack(self.qbuf[layer], axis=2)  # [B, Hq, S, d]
        self.qbuf[layer] = []
        rel = self.data["leader_member_relations"][layer]
        K = min(self.base, self.L)
        alloc = self.data["allocation_matrix"][layer]
        kt, vt = self.tier[layer]
        for leader_s, members in rel.items():
            leader = int(leader_s)
            if not members:
                continue
            if getattr(self.score_hook, "replaces_drift", False):
                # The hook supplies the step scores itself (a device's), and
                # the oracle's own float64 scoring of the step queries is
                # skipped: a long run replays the integer flow at every check.
                sc = np.asarray(self.score_hook("drift", layer, leader, None))
            else:
                sc = np.stack([pivot_step_scores(qs[b, leader * self.G:(leader + 1) * self.G],
                                                 self.rows[layer][b * self.Hkv + leader][0][:self.L], self.pooling,
                                                 self.kernel, io_dtype=self.io_dtype) for b in range(self.B)])
                sc = self._scores("drift", layer, leader, sc)
            ref = [np.fromiter(s, dtype=np.int64, count=len(s)) for s in self.ref[layer][leader]]
            _, med, trig, cur_last = drift_check(sc, ref, K, self.threshold)
            self.triggers.append((layer, leader, bool(trig)))
            self.medians.append((layer, leader, med))
            if not trig:
                continue
            self.ref[layer][leader] = [set(c.tolist()) for c in cur_last]
            lens = retrieval_lengths(self.base, [alloc[m] for m in members], self.L, topk=self.topk,
                                     use_f32=not self.quirks)
            for b in range(self.B):
                idxs = retrieval_indices(sc[b, -1], lens)
                for m, ix in zip(members, idxs):
                    if len(ix) == 0:
                        continue
                    r = self.rows[layer][b * self.Hkv + m]
                    r[0][:len(ix)] = kt[b, m][ix]
                    r[1][:len(ix)] = vt[b, m][ix]
