"""Baseline KV compressors on the libhc kernels.

Drop-ins for the compressors of heterocache/kv_cluster.py that HeteroCache is
compared against: same class names, constructor arguments, `reset` and
`update_kv(key_states, query_states, value_states, attention_mask,
num_key_value_groups)` contract (keys and values arrive repeated per query
head, as the reference's callers pass them; the result is the compressed
[B, H, kept, 128] pair).  Scoring runs in hc_score, selection in
hc_select_topk and the kept-row copy in hc_gather_rows.

One deliberate difference: the reference gathers kept rows in top-k order
(descending score, ties implementation-defined); these return them in
ascending position order, the order a causal cache holds them in.  Attention
over the result is the same, as it does not depend on key order; the kept
position sets are identical (tests compare sets and rows).

CAKECluster keeps the reference's calling convention, which differs from
the others: update_kv takes the cache first, scores the layer with
hc_cake_score (keys not repeated: a kv head's query group is scored
against it directly) and evicts every layer scored so far to its share of
the total budget, in place in the cache.
"""
import math

import numpy as np
import torch

from . import _lib, compress, ops


def _round_dtype(dtype, round_scores):
    return dtype if round_scores and dtype in (torch.bfloat16, torch.float16) else None


def _window_keep(key_states, query_states, value_states, window, keep, kernel, pooling, round_scores):
    """Kept rows of SnapKV-style scoring: the top `keep` positions of
    [0, L - window) by pooled window score, ascending, then the window."""
    B, H, L, D = query_states.shape
    scores = compress.window_scores(query_states, key_states, range(H), 1, window, pooling, kernel,
                                    window_keep=True, causal=True,
                                    round_dtype=_round_dtype(query_states.dtype, round_scores))
    # hc_select_topk's cap counts the force-kept window.
    idx, counts = compress.select_kept(scores, [keep + window] * (B * H), window=window, max_cap=keep + window)
    return ops.gather_rows(key_states, value_states, idx, counts)


class SnapKVCluster:
    """heterocache/kv_cluster.py:138-199."""

    def __init__(self, window_size=64, compression_ratio=0.5, kernel_size=5, pooling="avgpool", round_scores=True):
        self.window_size = window_size
        self.compression_ratio = compression_ratio
        self.kernel_size = kernel_size
        self.pooling = pooling
        self.round_scores = round_scores

    def reset(self, window_size=64, max_capacity_prompt=256 + 64, kernel_size=5, pooling="avgpool"):
        self.window_size = window_size
        self.max_capacity_prompt = max_capacity_prompt
        assert self.max_capacity_prompt - self.window_size > 0
        self.kernel_size = kernel_size
        self.pooling = pooling

    def update_kv(self, key_states, query_states, value_states, attention_mask, num_key_value_groups):
        assert key_states.shape[-2] == query_states.shape[-2]
        q_len = query_states.shape[-2]
        if not hasattr(self, "max_capacity_prompt"):
            self.max_capacity_prompt = max(int(self.compression_ratio * q_len / num_key_value_groups), 2)
        if self.max_capacity_prompt > q_len:
            return key_states, value_states
        keep = self.max_capacity_prompt - self.window_size
        if keep < 0:
            raise ValueError(f"capacity {self.max_capacity_prompt} is below the window {self.window_size}")
        return _window_keep(key_states, query_states, value_states, self.window_size, keep, self.kernel_size,
                            self.pooling, self.round_scores)


class PyramidKVCluster:
    """heterocache/kv_cluster.py:31-136: SnapKV scoring with a per-layer
    capacity that shrinks linearly from the first layer to the last."""

    def __init__(self, num_hidden_layers=32, window_size=64, compression_ratio=0.5, kernel_size=5,
                 pooling="avgpool", beta=20, num_layers=80, layer_idx=None, merge=None, round_scores=True):
        self.layer_idx = layer_idx
        self.num_hidden_layers = num_hidden_layers
        self.steps = -1
        self.beta = beta
        self.window_size = window_size
        self.compression_ratio = compression_ratio
        self.kernel_size = kernel_size
        self.pooling = pooling
        self.merge = merge
        self.round_scores = round_scores

    def reset(self, window_size=64, max_capacity_prompt=256 + 64, kernel_size=5, pooling="avgpool", merge=None):
        self.window_size = window_size
        self.max_capacity_prompt = max_capacity_prompt
        assert self.max_capacity_prompt - self.window_size > 0
        self.kernel_size = kernel_size
        self.pooling = pooling
        self.merge = merge

    def layer_capacity(self, q_len):
        """Tokens kept (before the window) by this layer at prompt length q_len,
        or None when the prompt is left uncompressed (kv_cluster.py:61-79)."""
        W = self.window_size
        cap = self.max_capacity_prompt
        min_num = (cap - W) // self.beta
        max_num = (cap - W) * 2 - min_num
        if max_num >= q_len - W:
            max_num = q_len - W
            min_num = (cap - W) * 2 - max_num
        steps = (max_num - min_num) // (self.num_hidden_layers - 1)
        if q_len < cap:
            return None
        if q_len < (cap - W) * 2:
            return cap - W
        return max_num - self.layer_idx * steps

    def update_kv(self, key_states, query_states, value_states, attention_mask, num_key_value_groups):
        assert key_states.shape[-2] == query_states.shape[-2]
        q_len = query_states.shape[-2]
        if not hasattr(self, "max_capacity_prompt"):
            self.max_capacity_prompt = int(self.compression_ratio * key_states.shape[-2] / num_key_value_groups)
        keep = self.layer_capacity(q_len)
        if keep is None:
            return key_states, value_states
        if keep < 0:
            raise ValueError(f"layer {self.layer_idx}: negative capacity {keep}")
        return _window_keep(key_states, query_states, value_states, self.window_size, keep, self.kernel_size,
                            self.pooling, self.round_scores)


class H2OKVCluster:
    """heterocache/kv_cluster.py:381-480: heavy hitters by the attention every
    prompt position pays each key (softmax over all keys, no mask, float32),
    summed over all query positions; the top capacity keys are kept."""

    # Query rows per hc_score call: the scorer holds at most 256 rows of a
    # 16-bit type, 128 of float32.
    QUERY_CHUNK = {torch.float32: 128}

    def __init__(self, window_size=64, compression_ratio=0.5, kernel_size=5, pooling="avgpool", merge=None):
        self.window_size = window_size
        self.compression_ratio = compression_ratio
        self.kernel_size = kernel_size
        self.pooling = pooling
        self.merge = merge

    def reset(self, window_size=64, max_capacity_prompt=256 + 64, kernel_size=5, pooling="avgpool", merge=None):
        self.window_size = window_size
        self.max_capacity_prompt = max_capacity_prompt
        assert self.max_capacity_prompt - self.window_size > 0
        self.kernel_size = kernel_size
        self.pooling = pooling
        self.merge = merge

    def heavy_hitter_scores(self, key_states, query_states):
        """[B*H, L] float32: sum over every query position of its softmax row."""
        B, H, L, D = query_states.shape
        scores = torch.empty((B * H, 1, L), dtype=torch.float32, device=query_states.device)
        k_off = ops.to_device([b * key_states.stride(0) + h * key_states.stride(1) for b in range(B) for h in range(H)],
                              query_states.device, torch.int64)
        base = [b * query_states.stride(0) + h * query_states.stride(1) for b in range(B) for h in range(H)]
        flags = _lib.HC_SCORE_SUM_WINDOW
        chunk = self.QUERY_CHUNK.get(query_states.dtype, 256)
        # Row blocks: full chunks, then the tail split into a multiple of 16
        # and powers of two (the window sizes a summed scorer call takes).
        blocks, s = [], 0
        while L - s >= chunk:
            blocks.append((s, chunk))
            s += chunk
        tail = L - s
        for w in ([tail // 16 * 16] if tail >= 16 else []) + [b for b in (8, 4, 2, 1) if tail % 16 & b]:
            blocks.append((s, w))
            s += w
        # Every block's query offsets in one host-to-device copy.
        q_offs = ops.to_device(np.asarray([[o + s * query_states.stride(2) for o in base] for s, _ in blocks],
                                          dtype=np.int64), query_states.device)
        for i, (s, w) in enumerate(blocks):
            ops.score(query_states, q_offs[i], query_states.stride(1), query_states.stride(2), key_states, k_off,
                      key_states.stride(2), L, 1, w, L, "avgpool", 1, 1.0 / math.sqrt(D),
                      flags=flags | (_lib.HC_SCORE_ACCUMULATE if s else 0), out=scores)
        return scores.view(B * H, L)

    def update_kv(self, key_states, query_states, value_states, attention_mask, num_key_value_groups):
        assert key_states.shape[-2] == query_states.shape[-2]
        B, H, q_len, D = query_states.shape
        if not hasattr(self, "max_capacity_prompt"):
            self.max_capacity_prompt = max(int(self.compression_ratio * key_states.shape[-2] / num_key_value_groups),
                                           2)
        if self.max_capacity_prompt > q_len:
            return key_states, value_states
        cap = self.max_capacity_prompt
        scores = self.heavy_hitter_scores(key_states, query_states)
        idx, counts = compress.select_kept(scores, [cap] * (B * H), max_cap=cap)
        return ops.gather_rows(key_states, value_states, idx, counts)


class StreamingLLMKVCluster:
    """heterocache/kv_cluster.py:482-523: the first four (sink) tokens plus the
    most recent ones."""

    SINK_TOKENS = 4

    def __init__(self, window_size=64, compression_ratio=0.5, kernel_size=5, pooling="avgpool", merge=None):
        self.window_size = window_size
        self.compression_ratio = compression_ratio
        self.kernel_size = kernel_size
        self.pooling = pooling
        self.merge = merge

    def reset(self, window_size=64, max_capacity_prompt=256 + 64, kernel_size=5, pooling="avgpool", merge=None):
        self.window_size = window_size
        self.max_capacity_prompt = max_capacity_prompt
        assert self.max_capacity_prompt - self.window_size > 0
        self.kernel_size = kernel_size
        self.pooling = pooling
        self.merge = merge

    def update_kv(self, key_states, query_states, value_states, attention_mask, num_key_value_groups):
        assert key_states.shape[-2] == query_states.shape[-2]
        B, H, q_len, D = query_states.shape
        if not hasattr(self, "max_capacity_prompt"):
            self.max_capacity_prompt = max(int(self.compression_ratio * key_states.shape[-2]), 5) - self.SINK_TOKENS
            self.sink_token = self.SINK_TOKENS
        if self.max_capacity_prompt > q_len:
            return key_states, value_states
        recent = self.max_capacity_prompt
        keep = np.concatenate([np.arange(self.sink_token), np.arange(q_len - recent, q_len)]).astype(np.int32)
        idx = ops.to_device(np.tile(keep, (B * H, 1)), key_states.device)
        return ops.gather_rows(key_states, value_states, idx, len(keep))


class CAKECluster:
    """heterocache/kv_cluster.py:201-379: layer budgets in proportion to a
    preference score (entropy times variance of the window's attention), and
    per-layer eviction by mean + gamma * variance of the window attention.

    Each layer's prompt is scored once (hc_cake_score: heavy-hitter scores,
    entropy, variance sum); after layer l the total budget
    (capacity - window) * num_layers is split over layers 0..l and every one
    of them is evicted to its share (hc_select_topk over its current scores,
    hc_gather_rows of its cached rows).  Kept rows stay in position order.
    """

    def __init__(self, window_size=64, compression_ratio=0.5, kernel_size=5, pooling="avgpool", round_scores=True):
        self.window_size = window_size
        self.compression_ratio = compression_ratio
        self.kernel_size = kernel_size
        self.pooling = pooling
        self.round_scores = round_scores
        self.tau1 = 1
        self.tau2 = 1
        self.gamma = 200.0

    def reset(self, window_size=64, max_capacity_prompt=256 + 64, kernel_size=5, pooling="avgpool"):
        self.window_size = window_size
        self.max_capacity_prompt = max_capacity_prompt
        assert self.max_capacity_prompt - self.window_size > 0
        self.kernel_size = kernel_size
        self.pooling = pooling

    def adjust_budgets(self, budget_list, total_budget, seq_len, layer_nums):
        """Integer layer budgets (heterocache/kv_cluster.py:225-271): truncate,
        clip at seq_len and spread the clipped excess evenly over the layers
        below seq_len (remainder one each to the first of them); then spread
        the difference to total_budget the same way, adding over the layers
        below seq_len or taking from the layers above 1."""
        budgets = [int(x) for x in budget_list]

        def spread(amount, members, sign):
            per, rem = divmod(amount, len(members))
            for n, i in enumerate(members):
                budgets[i] += sign * (per + (1 if n < rem else 0))

        excess = sum(max(x - seq_len, 0) for x in budgets)
        budgets = [min(x, seq_len) for x in budgets]
        below = [i for i, x in enumerate(budgets) if x < seq_len]
        if excess > 0 and below:
            spread(excess, below, 1)
        diff = total_budget - sum(budgets)
        if diff > 0:
            members = [i for i, x in enumerate(budgets) if x < seq_len]
        else:
            members = [i for i, x in enumerate(budgets) if x > 1]
        if diff != 0 and members:
            spread(abs(diff), members, 1 if diff > 0 else -1)
        return budgets

    def preference(self, entropy, variance):
        """entropy**(1/tau1) * variance**(1/tau2) in float32, 0 when either
        is NaN (heterocache/kv_cluster.py:305-313)."""
        entropy, variance = np.float32(entropy), np.float32(variance)
        if np.isnan(entropy) or np.isnan(variance):
            return np.float32(0.0)
        return np.float32(entropy ** np.float32(1 / self.tau1) * variance ** np.float32(1 / self.tau2))

    def update_kv(self, past_key_values, key_states, query_states, value_states, attention_mask, num_key_value_groups):
        assert key_states.shape[-2] == query_states.shape[-2]
        B, H, q_len, D = query_states.shape
        if not hasattr(self, "max_capacity_prompt"):
            self.max_capacity_prompt = max(int(self.compression_ratio * q_len), 2)
            self.total_size = (self.max_capacity_prompt - self.window_size) * past_key_values.num_layers
        if self.max_capacity_prompt > q_len:
            return key_states, value_states
        W = self.window_size
        if self.max_capacity_prompt < W or q_len <= W:
            raise ValueError(f"capacity {self.max_capacity_prompt} / prompt {q_len} leave no room beside the "
                             f"window {W}")
        hh, stats = compress.cake_scores(query_states, key_states, W, gamma=self.gamma,
                                         round_dtype=_round_dtype(query_states.dtype, self.round_scores))
        entropy, variance, _ = stats.cpu().numpy()
        past_key_values.pref_scores.append(self.preference(entropy, variance))
        past_key_values.evict_scores.append(hh.view(B, key_states.shape[1], q_len - W))
        past_key_values.layer_budget.append(self.max_capacity_prompt - W)
        prefs = past_key_values.pref_scores
        total_pref = sum(prefs)
        if total_pref == 0:
            # Every preference is 0 (NaN statistics): the reference divides
            # 0 by 0; split the total evenly instead.
            shares = [np.float32(self.total_size / len(prefs))] * len(prefs)
        else:
            shares = [p / total_pref * self.total_size for p in prefs]
        budgets = self.adjust_budgets(shares, self.total_size, q_len - W, past_key_values.num_layers)
        for layer_idx, budget in enumerate(budgets):
            budget = min(budget, q_len - W)
            self.evcit_layer_kvcache(past_key_values, layer_idx, budget)
            past_key_values.layer_budget[layer_idx] = budget

    def evcit_layer_kvcache(self, past_key_values, layer_idx, budget):
        """Keep the top `budget` rows of the layer by its current scores
        plus the window (heterocache/kv_cluster.py:351-379; the name is the
        reference's)."""
        scores = past_key_values.evict_scores[layer_idx]
        B, Hkv, n = scores.shape
        budget = min(budget, n)
        if budget < 0:
            raise ValueError(f"negative budget {budget} for layer {layer_idx}")
        if budget == n:
            return past_key_values
        W = self.window_size
        flat = scores.reshape(B * Hkv, n)
        # Budgets filled on the device: a host list would cost a blocking copy per eviction.
        caps = torch.full((B * Hkv,), budget + W, dtype=torch.int32, device=flat.device)
        idx, counts = compress.select_kept(flat, caps, window=W, max_cap=budget + W)
        k, v = ops.gather_rows(past_key_values.key_cache[layer_idx], past_key_values.value_cache[layer_idx], idx,
                               counts)
        past_key_values.key_cache[layer_idx] = k
        past_key_values.value_cache[layer_idx] = v
        past_key_values.evict_scores[layer_idx] = torch.gather(flat, 1, idx[:, :budget].long()).view(B, Hkv, budget)
        return past_key_values

    evict_layer_kvcache = evcit_layer_kvcache
