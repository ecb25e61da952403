"""Seeded synthetic workloads for the compressed-KV attention path.

There are no checkpoints or datasets here, so every workload is synthetic:
a head-classification record in the reference's JSON schema
(tools/get_cluster.py:313-321: meta / classification_matrix /
allocation_matrix / leader_member_relations) and the per-row budgets it
implies at a given context length and compression ratio.
"""
import numpy as np

ANCHOR, VOLATILE, PIVOT, SATELLITE = 1, 2, 3, 4
TYPE_MAP = {"anchor": ANCHOR, "volatile": VOLATILE, "pivot": PIVOT, "satellite": SATELLITE}


def get_compress_len(compression_ratio, full_heads, ori_len, num_kv_heads):
    """Base budget, heterocache/cache_utils.py:15-16 (float64, truncated)."""
    return int((compression_ratio * num_kv_heads - full_heads) * ori_len / (num_kv_heads - full_heads))


def inverse_stability_allocation(stability):
    """Allocation ratios from per-head stabilities (-1 marks full-KV heads).

    Follows tools/get_cluster.py:276-307: ratio = (1/(s+1e-6)) / sum(1/(s'+1e-6))
    * n_targets over every anchor and satellite head of the model, so the
    ratios average exactly 1.
    """
    eps = 1e-6
    targets = [s for row in stability for s in row if s > -0.5]
    n = len(targets)
    total = sum(1.0 / (s + eps) for s in targets)
    out = []
    for row in stability:
        out.append([(1.0 / (s + eps)) / total * n if s > -0.5 else -1.0 for s in row])
    return out


def synthetic_head_json(num_layers, num_kv_heads, seed, singleton_volatile=0.25, stability_range=(0.3, 0.95)):
    """Head classification with seeded clusters of 1-4 heads per layer.

    A cluster of one head is an anchor (or, with probability
    `singleton_volatile`, a volatile head); a larger cluster has one pivot
    and satellites.  Stabilities are uniform in `stability_range`.
    """
    rng = np.random.default_rng(seed)
    cls, stab, rel = [], [], []
    counts = {"anchor": 0, "volatile": 0, "pivot": 0, "satellite": 0}
    for _ in range(num_layers):
        perm = rng.permutation(num_kv_heads).tolist()
        types = [0] * num_kv_heads
        layer_rel = {}
        i = 0
        while i < num_kv_heads:
            size = int(rng.integers(1, 5))
            group = perm[i:i + size]
            i += size
            if len(group) == 1:
                t = VOLATILE if rng.random() < singleton_volatile else ANCHOR
                types[group[0]] = t
                counts["volatile" if t == VOLATILE else "anchor"] += 1
            else:
                types[group[0]] = PIVOT
                counts["pivot"] += 1
                for m in group[1:]:
                    types[m] = SATELLITE
                    counts["satellite"] += 1
                layer_rel[str(group[0])] = sorted(group[1:])
        s = [float(rng.uniform(*stability_range)) if t in (ANCHOR, SATELLITE) else -1.0 for t in types]
        cls.append(types)
        stab.append(s)
        rel.append(layer_rel)
    return {
        "meta": {"type_map": dict(TYPE_MAP), "counts": counts},
        "classification_matrix": cls,
        "allocation_matrix": inverse_stability_allocation(stab),
        "leader_member_relations": rel,
    }


def full_head_count(data):
    return data["meta"]["counts"]["volatile"] + data["meta"]["counts"]["pivot"]


def row_budgets(data, layer, seq_len, compression_ratio, num_layers, num_kv_heads, batch=1):
    """Prefill length of every row (b, h) of one layer (before any reorder).

    Full-KV heads (volatile, pivot) keep all seq_len tokens; compressed heads
    keep min(trunc(f32(base) * f32(ratio)), seq_len)
    (heterocache/cache_utils.py:793-799).
    """
    base = get_compress_len(compression_ratio, full_head_count(data), seq_len, num_kv_heads * num_layers)
    types = data["classification_matrix"][layer]
    alloc = np.asarray(data["allocation_matrix"][layer], dtype=np.float32)
    out = []
    for h in range(num_kv_heads):
        if types[h] in (VOLATILE, PIVOT):
            out.append(seq_len)
        else:
            out.append(int(min(np.trunc(np.float32(base) * alloc[h]), seq_len)))
    return np.tile(np.asarray(out, dtype=np.int64), batch), base


def config0_inputs(seed=1000, seq_len=4096, q_heads=32, kv_heads=8, window=32, outlier_channels=4,
                   outlier_scale=8.0, sinks=4, compression_ratio=0.5, weights=(0.5, 1.5)):
    """One Llama-3-8B-shape layer for the CPU-runnable reference case.

    float32 q [1, Hq, L, 128] (the last `window` rows are the observation
    window), K/V [1, Hkv, L, 128] ~ N(0, 1) with `outlier_channels` seeded
    channels per head scaled by `outlier_scale`; positions [0, sinks) hold
    attention-sink keys equal to twice the mean window query of the head's
    group.  A seeded half of the KV heads gets allocation weight weights[0],
    the rest weights[1]; budgets are the float32 caps of
    get_compress_len(ratio, 0, L, Hkv) times the weight.  One decode step of
    fresh q / k / v follows.
    """
    rng = np.random.default_rng(seed)
    d, G = 128, q_heads // kv_heads
    q = rng.standard_normal((1, q_heads, seq_len, d)).astype(np.float32)
    k = rng.standard_normal((1, kv_heads, seq_len, d)).astype(np.float32)
    v = rng.standard_normal((1, kv_heads, seq_len, d)).astype(np.float32)
    for h in range(kv_heads):
        ch = rng.choice(d, outlier_channels, replace=False)
        k[0, h][:, ch] *= outlier_scale
        v[0, h][:, ch] *= outlier_scale
        k[0, h, :sinks] = 2.0 * q[0, h * G:(h + 1) * G, seq_len - window:].mean(axis=(0, 1))
    perm = rng.permutation(kv_heads)
    alloc = np.empty(kv_heads)
    alloc[perm[:kv_heads // 2]] = weights[0]
    alloc[perm[kv_heads // 2:]] = weights[1]
    base = get_compress_len(compression_ratio, 0, seq_len, kv_heads)
    caps = np.minimum(np.trunc(np.float32(base) * alloc.astype(np.float32)).astype(np.int64), seq_len)
    return {"q": q, "k": k, "v": v, "caps": caps, "alloc": alloc, "base": base, "window": window,
            "q_dec": rng.standard_normal((1, q_heads, 1, d)).astype(np.float32),
            "k_dec": rng.standard_normal((1, kv_heads, 1, d)).astype(np.float32),
            "v_dec": rng.standard_normal((1, kv_heads, 1, d)).astype(np.float32)}
