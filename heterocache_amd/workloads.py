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


def synthetic_head_json(num_layers, num_kv_heads, seed, singleton_volatile=0.25, stability_range=(0.3, 0.95),
                        max_full=None):
    """Head classification with seeded clusters of 1-4 heads per layer.

    A cluster of one head is an anchor (or, with probability
    `singleton_volatile`, a volatile head); a larger cluster has one pivot
    and satellites.  Stabilities are uniform in `stability_range`.
    max_full caps the model-wide count of full-KV heads (volatile + pivot):
    once it is reached, singletons become anchors and larger clusters split
    into anchors, so a low compression ratio keeps a positive base budget
    (get_compress_len needs ratio * heads > full heads).
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
            full_left = max_full is None or counts["volatile"] + counts["pivot"] < max_full
            if len(group) == 1 or not full_left:
                for hd in group:
                    t = VOLATILE if (full_left and rng.random() < singleton_volatile) else ANCHOR
                    types[hd] = t
                    counts["volatile" if t == VOLATILE else "anchor"] += 1
                    full_left = max_full is None or counts["volatile"] + counts["pivot"] < max_full
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


# ---------------------------------------------------------------------------
# Decode workloads with planted attention structure (device-side, seeded)
# ---------------------------------------------------------------------------
def _unit(x):
    return x / x.norm(dim=-1, keepdim=True)


def _orthogonal_unit(torch, gen, u, device):
    """Random unit vectors orthogonal to the unit rows of u (same shape)."""
    v = torch.randn(u.shape, generator=gen, device=device)
    v = v - (v * u).sum(-1, keepdim=True) * u
    return _unit(v)


class NeedleWorkload:
    """Llama-shaped layers at a long context with 16 planted needle keys and
    step queries that drift on a schedule, so drift checks at threshold 0.5
    trigger naturally.

    Per query head, q = sqrt(d) * (a * u + sqrt(1 - a^2) * v): u is the unit
    needle direction of the query head's KV head, v a unit direction
    orthogonal to it.  Keys and values are N(0, 1), so a query's logit
    q.k / sqrt(d) is N(0, 1) over ordinary keys; a needle key is
    (sigma / a) * u + N(0, 1) noise, which puts its expected logit at +sigma
    standard deviations with every step query.  v follows the decode
    windows of `decode_step` steps: window 0 keeps the prefill query's
    direction, a fresh direction starts at every odd window and is kept by
    the even window after it, and each step perturbs it by `noise` -- so the
    pooled top sets stay put across a window and its successor and jump at
    odd windows (overlap about the budget fraction, below 0.5).

    Everything is generated on `device` from seeded torch generators; one
    layer at a time (layer(i)) so a 32-layer 128K model never holds more
    than one layer of inputs.
    """

    def __init__(self, seq_len, kv_heads=8, group=4, head_dim=128, steps=20, decode_step=5, seed=1002, needles=16,
                 sigma=6.0, affinity=0.2, noise=0.05, device="cuda", dtype=None):
        import torch
        self.torch = torch
        self.L, self.Hkv, self.G, self.d = seq_len, kv_heads, group, head_dim
        self.steps, self.S, self.seed = steps, decode_step, seed
        self.nneedle, self.sigma, self.a, self.noise = needles, sigma, affinity, noise
        self.device = torch.device(device)
        self.dtype = dtype or torch.bfloat16

    def _gen(self, layer, salt):
        g = self.torch.Generator(device=self.device)
        g.manual_seed(self.seed * 1_000_003 + layer * 7919 + salt)
        return g

    def needle_positions(self, layer):
        g = self.torch.Generator().manual_seed(self.seed * 31 + layer)
        return self.torch.randperm(self.L, generator=g)[:self.nneedle].sort().values

    def direction_index(self, step):
        """Query direction of a decode step: 0 in window 0, then a new one at
        every odd window (kept by the even window that follows)."""
        return (step // self.S + 1) // 2

    def layer(self, layer):
        """Prefill K/V [1, Hkv, L, d], the last prefill query [1, Hq, 1, d],
        decode queries [steps, 1, Hq, 1, d] and new K/V [steps, 1, Hkv, 1, d]."""
        torch, dev, d = self.torch, self.device, self.d
        Hq = self.Hkv * self.G
        g = self._gen(layer, 0)
        k = torch.randn((1, self.Hkv, self.L, d), generator=g, device=dev)
        v = torch.randn((1, self.Hkv, self.L, d), generator=g, device=dev)
        u = _unit(torch.randn((self.Hkv, d), generator=g, device=dev))
        pos = self.needle_positions(layer).to(dev)
        c = self.sigma / self.a
        k[0, :, pos] = c * u[:, None, :] + torch.randn((self.Hkv, len(pos), d), generator=g, device=dev)
        uq = u.repeat_interleave(self.G, dim=0)                       # [Hq, d]
        ndir = self.direction_index(self.steps - 1) + 1
        dirs = [_orthogonal_unit(torch, g, uq, dev) for _ in range(ndir)]
        b = (1.0 - self.a ** 2) ** 0.5

        def query(vdir):
            return (d ** 0.5) * (self.a * uq + b * vdir)

        q_last = query(dirs[0]).view(1, Hq, 1, d)
        qs = []
        for t in range(self.steps):
            w = dirs[self.direction_index(t)]
            w = _unit(w + self.noise * _orthogonal_unit(torch, g, uq, dev))
            qs.append(query(w).view(1, Hq, 1, d))
        kn = torch.randn((self.steps, 1, self.Hkv, 1, d), generator=g, device=dev)
        vn = torch.randn((self.steps, 1, self.Hkv, 1, d), generator=g, device=dev)
        cast = lambda x: x.to(self.dtype)
        return {"k": cast(k), "v": cast(v), "q_last": cast(q_last), "q_steps": cast(torch.stack(qs)),
                "k_new": cast(kn), "v_new": cast(vn), "needles": pos}


class BlockDriftWorkload:
    """Llama-shaped layers whose attention drifts to a new block of 8
    high-affinity key positions every `period` decode steps.

    Per query head, q = sqrt(d) * (alpha * w_b + sqrt(1 - alpha^2) * v):
    w_b is the unit direction of the sum of the 8 keys of block b (block
    b = step // period, block 0 for the prefill's last query) of the query
    head's KV head, so those keys score about alpha * |k|^2 / |sum| ~ 4 alpha
    standard deviations above the ordinary N(0, 1) logits; v is a unit
    direction of the query head, perturbed by `noise` each step.  Queries of
    one block keep their top sets, a new block moves them (a drift the
    threshold-0.5 check catches).  Block starts are seeded, non-overlapping.
    """

    def __init__(self, seq_len, kv_heads=8, group=4, head_dim=128, steps=20, period=200, seed=1004, block=8,
                 alpha=0.9, noise=0.05, device="cuda", dtype=None):
        import torch
        self.torch = torch
        self.L, self.Hkv, self.G, self.d = seq_len, kv_heads, group, head_dim
        self.steps, self.period, self.seed, self.block = steps, period, seed, block
        self.alpha, self.noise = alpha, noise
        self.device = torch.device(device)
        self.dtype = dtype or torch.bfloat16

    def block_starts(self, layer):
        nb = (self.steps - 1) // self.period + 1
        g = self.torch.Generator().manual_seed(self.seed * 37 + layer)
        slots = self.torch.randperm(self.L // self.block, generator=g)[:nb]
        return (slots * self.block).tolist()

    def prefill(self, layer):
        """Prefill K/V [1, Hkv, L, d] in the workload dtype."""
        torch, dev = self.torch, self.device
        g = torch.Generator(device=dev)
        g.manual_seed(self.seed * 1_000_003 + layer * 7919)
        k = torch.randn((1, self.Hkv, self.L, self.d), generator=g, device=dev).to(self.dtype)
        v = torch.randn((1, self.Hkv, self.L, self.d), generator=g, device=dev).to(self.dtype)
        return k, v

    def queries(self, layer, k):
        """The last prefill query [1, Hq, 1, d], decode queries [steps, 1, Hq,
        1, d] and new K/V [steps, 1, Hkv, 1, d] for this layer's prefill keys."""
        torch, dev, d = self.torch, self.device, self.d
        Hq = self.Hkv * self.G
        g = torch.Generator(device=dev)
        g.manual_seed(self.seed * 1_000_003 + layer * 7919 + 1)
        starts = self.block_starts(layer)
        w = []
        for s0 in starts:
            sums = k[0, :, s0:s0 + self.block].float().sum(dim=1)        # [Hkv, d]
            w.append(_unit(sums).repeat_interleave(self.G, dim=0))       # [Hq, d]
        base = _unit(torch.randn((Hq, d), generator=g, device=dev))
        b = (1.0 - self.alpha ** 2) ** 0.5

        def query(blk, vdir):
            vdir = _unit(vdir - (vdir * w[blk]).sum(-1, keepdim=True) * w[blk])
            return (d ** 0.5) * (self.alpha * w[blk] + b * vdir)

        q_last = query(0, base).view(1, Hq, 1, d)
        qs = []
        for t in range(self.steps):
            vt = base + self.noise * torch.randn((Hq, d), generator=g, device=dev)
            qs.append(query(t // self.period, vt).view(1, Hq, 1, d))
        kn = torch.randn((self.steps, 1, self.Hkv, 1, d), generator=g, device=dev)
        vn = torch.randn((self.steps, 1, self.Hkv, 1, d), generator=g, device=dev)
        cast = lambda x: x.to(self.dtype)
        return {"q_last": cast(q_last), "q_steps": cast(torch.stack(qs)), "k_new": cast(kn), "v_new": cast(vn),
                "blocks": starts}
