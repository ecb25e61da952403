"""Head-classification JSON producer on the libhc kernels.

Counterpart of tools/get_cluster.py (analyze_combined_heads, :113-330): from
saved attention maps of one prefill step and several decode steps per layer,
classify every (KV) head as anchor, volatile, pivot or satellite and write
the JSON that HeteroCache consumes (schema :313-321).

Per layer:
  * each map's last query row, averaged over a KV head's query group and
    avg-pooled (k = 5), gives the head's top-k position set
    (get_head_topk_exact, :13-56): hc_head_pool, then hc_select_topk;
  * temporal stability: per decode step, |prefill set ∩ step set| / |prefill
    set| averaged over the batch; the median over steps decides anchor (>=
    stable_threshold) or volatile (:210-241): hc_set_bits + hc_overlap_count;
  * spatial similarity at the target step: the same ratio between every pair
    of heads, averaged over the batch; pairs at or above sim_threshold are
    edges (:243-258): hc_set_bits + hc_overlap_count;
  * greedy star clustering: repeatedly the unassigned head with the most
    unassigned neighbours (lowest index on ties) leads its neighbours
    (find_star_clusters_greedy, :70-110), on the host;
  * allocation ratios: inverse median score over the anchor and satellite
    heads, normalised to a mean of one (:286-307), on the host.

Inputs are tensors (``maps[layer][step] -> [B, heads, rows, seq]``) or a
directory of the reference's ``attn_weights_{layer}_{step}.pt`` files, read
with torch.load(weights_only=True).

The maps themselves come from a calibration generate() (tools/get_weights.py:
30-212): collect_maps runs greedy generation through the patched attention
with an AttentionRecorder attached, which keeps each layer's last query row
of attention probabilities at the prefill and at every decode step (the only
row the classification reads), computed by hc_score, instead of saving whole
[B, heads, q_len, kv_len] maps.
"""
import glob
import os
import pathlib

import numpy as np
import torch

from . import _lib, compress, ops

TYPE_MAP = {"anchor": 1, "volatile": 2, "pivot": 3, "satellite": 4}
POOL_KERNEL = 5


def head_topk_sets(attn, num_q_heads, num_kv_heads, max_length, topk):
    """Top-k position sets of every (batch, head) of one attention map.

    attn: [B, heads, rows, seq] (or [B, heads, seq]) device tensor; when it
    holds num_q_heads heads of a GQA model the query group of each KV head is
    averaged.  Returns (idx int32 [B*H, max(k, 1)] ascending, k, H, span)
    with k = min(topk, span) entries per set.
    """
    lib = _lib.load()
    if attn.dim() == 3:
        attn = attn.unsqueeze(2)
    B, Hs, R, S = attn.shape
    if num_q_heads != num_kv_heads and Hs == num_q_heads:
        group, H = num_q_heads // num_kv_heads, num_kv_heads
    else:
        group, H = 1, Hs
    span = min(max_length, S)
    if attn.stride(-1) != 1:
        attn = attn.contiguous()
    last = attn[:, :, R - 1]
    k = min(topk, span)
    idx = torch.empty((B * H, max(k, 1)), dtype=torch.int32, device=attn.device)
    if k > 0:
        pooled = torch.empty((B * H, span), dtype=torch.float32, device=attn.device)
        kernel = min(POOL_KERNEL, span)
        _lib.check(lib.hc_head_pool(ops.dtype_code(attn.dtype), ops._ptr(last), attn.stride(0), attn.stride(1), B, H,
                                    group, span, kernel, ops._ptr(pooled), ops._stream(None, attn)))
        caps = torch.full((B * H,), k, dtype=torch.int32, device=attn.device)
        ops.select_topk(pooled, caps, span, idx=idx)
    return idx, k, H, span


def _intersections(lists, k, sets, nbits, ref_of):
    """|lists[p][:k] ∩ sets[ref_of[p]][:k]| per list p (sets become bitmasks)."""
    dev = lists.device
    words = max((nbits + 31) // 32, 1)
    bits = torch.zeros((sets.shape[0], words), dtype=torch.int32, device=dev)
    ops.set_bits(sets, None, bits, nbits, fixed_count=k)
    ref = ops.to_device(np.asarray(ref_of, dtype=np.int32), dev)
    return ops.overlap_count(lists, k, bits, nbits, ref_of=ref).cpu().numpy()


def _star_clusters(adjacency, num_heads):
    """find_star_clusters_greedy (tools/get_cluster.py:70-110)."""
    unassigned = set(range(num_heads))
    clusters, assigned = {}, set()
    while unassigned:
        cands = sorted(((len(adjacency.get(n, set()) & unassigned), n) for n in unassigned),
                       key=lambda c: (-c[0], c[1]))
        degree, leader = cands[0]
        if degree == 0:
            break
        members = sorted(adjacency[leader] & unassigned)
        clusters[leader] = members
        unassigned.discard(leader)
        assigned.add(leader)
        for m in members:
            unassigned.discard(m)
            assigned.add(m)
    return clusters, assigned


def analyze(maps, num_layers, num_q_heads, num_kv_heads, topk=1024, max_length=5000, stable_threshold=0.5,
            sim_threshold=0.5, decode_step=5000):
    """The head-analysis JSON (a dict) from maps[layer][step] -> attention map."""
    total = num_q_heads
    classification = [[0] * total for _ in range(num_layers)]
    allocation = [[-1.0] * total for _ in range(num_layers)]
    relations = [{} for _ in range(num_layers)]
    counts_by_type = {k: 0 for k in TYPE_MAP}
    steps = sorted({s for per in maps.values() for s in per})
    if not steps:
        raise ValueError("no attention maps")
    prefill_step, decode_steps = steps[0], steps[1:]
    spatial_step = decode_step if decode_step in steps else steps[-1]
    for layer in range(num_layers):
        per = maps.get(layer)
        if per is None or prefill_step not in per:
            continue
        base, kb, H, span0 = head_topk_sets(per[prefill_step], num_q_heads, num_kv_heads, max_length, topk)
        B = base.shape[0] // H
        if H != total and layer == 0:
            classification = [[0] * H for _ in range(num_layers)]
            allocation = [[-1.0] * H for _ in range(num_layers)]
        history = [[] for _ in range(H)]
        for step in decode_steps:
            if step not in per:
                continue
            cur, kc, _, span1 = head_topk_sets(per[step], num_q_heads, num_kv_heads, max_length, topk)
            if kb == 0 or kc == 0:  # an empty set overlaps nothing (get_cluster.py:58-66)
                ratios = np.zeros((B, H))
            else:
                # |base ∩ cur| / |base|; both sets hold k_cur and k_base positions
                inter = _intersections(cur, kc, base, max(span0, span1), list(range(B * H)))
                ratios = inter.reshape(B, H) / kb
            for h in range(H):
                history[h].append(float(sum(ratios[:, h]) / B))
        median = [float(np.median(h)) if h else 0.0 for h in history]
        dyn = ["volatile" if (not history[h] or median[h] < stable_threshold) else "anchor" for h in range(H)]
        adjacency = {}
        if spatial_step in per:
            sp, ks, _, span2 = head_topk_sets(per[spatial_step], num_q_heads, num_kv_heads, max_length, topk)
            sims = np.zeros((H, H))
            if ks > 0:
                for off in range(1, H):
                    # list p = (b, i) against the set of head j = (i + off) % H
                    ref_of = [b * H + (i + off) % H for b in range(B) for i in range(H)]
                    inter = _intersections(sp, ks, sp, span2, ref_of).reshape(B, H)
                    for i in range(H):
                        sims[i, (i + off) % H] = float(sum(inter[:, i] / ks)) / B
            for i in range(H):
                for j in range(H):
                    if i != j and sims[i, j] >= sim_threshold:
                        adjacency.setdefault(i, set()).add(j)
        clusters, assigned = _star_clusters(adjacency, H)
        relations[layer] = clusters
        for h in range(H):
            allocation[layer][h] = median[h]
            if h in clusters:
                classification[layer][h] = TYPE_MAP["pivot"]
                counts_by_type["pivot"] += 1
                allocation[layer][h] = -1.0
            elif h in assigned:
                classification[layer][h] = TYPE_MAP["satellite"]
                counts_by_type["satellite"] += 1
            elif dyn[h] == "anchor":
                classification[layer][h] = TYPE_MAP["anchor"]
                counts_by_type["anchor"] += 1
            else:
                classification[layer][h] = TYPE_MAP["volatile"]
                counts_by_type["volatile"] += 1
                allocation[layer][h] = -1.0
    targets = [v for row in allocation for v in row if v > -0.5]
    eps = 1e-6
    inv_total = sum(1.0 / (v + eps) for v in targets)
    if targets and inv_total > 1e-9:
        for r in range(len(allocation)):
            for c in range(len(allocation[r])):
                v = allocation[r][c]
                if v > -0.5:
                    allocation[r][c] = (1.0 / (v + eps)) / inv_total * len(targets)
    return {"meta": {"type_map": dict(TYPE_MAP), "counts": counts_by_type},
            "classification_matrix": classification, "allocation_matrix": allocation,
            "leader_member_relations": relations}


def load_maps(tensor_save_dir, device="cuda"):
    """maps[layer][step] from attn_weights_{layer}_{step}.pt files (weights only)."""
    maps = {}
    for f in glob.glob(os.path.join(tensor_save_dir, "attn_weights_*_*.pt")):
        parts = pathlib.Path(f).stem.split("_")
        try:
            layer, step = int(parts[2]), int(parts[3])
        except (IndexError, ValueError):
            continue
        maps.setdefault(layer, {})[step] = torch.load(f, map_location="cpu", weights_only=True).to(device)
    return maps


class AttentionRecorder:
    """Attention observer of the patched attention: per layer and forward,
    the last query row's probabilities softmax(scale * q_last . K^T) over all
    kv_len keys, [B, Hq, 1, kv_len] in the model dtype (the reference casts
    its float32 softmax to the model dtype, tools/get_weights.py:53-55),
    stored as maps[layer][kv_len].  With save_dir each map is also written
    as the reference's attn_weights_{layer}_{kv_len}.pt.

    hc_score computes it: one job per (batch, query head) against its KV
    head's keys, window 1, pooling kernel 1 (the identity), with the
    reference's casts of the logits and probabilities in 16-bit models."""

    def __init__(self, save_dir=None):
        self.maps = {}
        self.save_dir = save_dir
        if save_dir:
            os.makedirs(save_dir, exist_ok=True)

    def __call__(self, layer_idx, query_states, key_states, attention_mask, scaling):
        q, k = query_states, key_states
        B, Hq, Lq, _ = q.shape
        Hkv, L = k.shape[1], k.shape[2]
        if attention_mask is not None and attention_mask.dim() == 4:
            last = attention_mask[..., -1, :L]
            hidden = ~last if last.dtype == torch.bool else last != 0
            if bool(hidden.any()):
                raise NotImplementedError("attention recording takes unpadded batches (the last row sees every key)")
        G = Hq // Hkv
        q_off = [b * q.stride(0) + h * q.stride(1) + (Lq - 1) * q.stride(2) for b in range(B) for h in range(Hq)]
        k_off = [b * k.stride(0) + (h // G) * k.stride(1) for b in range(B) for h in range(Hq)]
        dev = q.device
        probs = ops.score(q, ops.to_device(q_off, dev, torch.int64), q.stride(1), q.stride(2), k,
                          ops.to_device(k_off, dev, torch.int64), k.stride(2), L, 1, 1, L, "avgpool", 1,
                          float(scaling), flags=compress.ROUND_FLAGS.get(q.dtype, 0))
        m = probs.view(B, Hq, 1, L).to(q.dtype)
        self.maps.setdefault(layer_idx, {})[L] = m
        if self.save_dir:
            torch.save(m.cpu(), os.path.join(self.save_dir, f"attn_weights_{layer_idx}_{L}.pt"))


def collect_maps(model, input_ids, max_new_tokens, attention_mask=None, save_dir=None):
    """Calibration run (tools/get_weights.py:140-212): greedy generate() of
    max_new_tokens on a model built under utils.install_attention_patch(),
    with a plain cache, recording the attention maps.  Returns (maps, the
    generated ids); maps[layer] has one entry per forward, keyed by kv_len
    (the prompt length, then one more per decode step)."""
    from . import llama_model
    rec = AttentionRecorder(save_dir)
    llama_model.ATTENTION_OBSERVERS.append(rec)
    try:
        with torch.no_grad():
            out = model.generate(input_ids, attention_mask=attention_mask, max_new_tokens=max_new_tokens,
                                 do_sample=False)
    finally:
        llama_model.ATTENTION_OBSERVERS.remove(rec)
    return rec.maps, out
