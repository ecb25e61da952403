"""PyTorch-CPU restatement of the reference's op sequence on one layer.

TEST INFRASTRUCTURE ONLY -- imported by tests/ and bench.py's cpu_baseline
leg, never by the product.  It is the CPU baseline: the reference's own
torch op sequence run on the host cores, for the single-layer case the
reference can run on a CPU (a Llama-3-8B layer in float32 at 4096 tokens):

  score_select  SnapKV-style observation-window scoring, as
                SnapKVCluster.update_kv issues it (heterocache/kv_cluster.py:
                165-185: matmul of the last W queries with the keys, additive
                causal mask inside the window, softmax in float32, sum over the
                window, max_pool1d), then the max over each KV head's query
                group and per-head top-(cap - W) with the window appended,
                sorted ascending (heterocache/cache_utils.py:831-851,
                heterocache/kv_cluster.py:187-197);
  gather        the kept K/V rows (heterocache/cache_utils.py:852-877);
  decode        the new token appended to every row and attention of the
                group's queries over it, softmax(q.K^T / sqrt(d)).V -- the
                closed form of the flash_attn_with_kvcache call of
                heterocache/llama_model.py:368-401.

The scores are pinned against the numpy oracle (window_scores) and the
decode output against its float64 closed form (tests/test_oracle.py).
"""
import math
import os
import statistics
import time

import torch
import torch.nn.functional as F


def score_select(q_win, k, caps, window, kernel):
    """q_win [Hkv, G, W, d], k [Hkv, L, d] float32, caps per KV head ->
    (scores [Hkv, L - W], kept positions per head, ascending)."""
    Hkv, G, W, d = q_win.shape
    L = k.shape[1]
    logits = torch.matmul(q_win, k.transpose(1, 2).unsqueeze(1)) / math.sqrt(d)   # [Hkv, G, W, L]
    mask = torch.full((W, W), torch.finfo(logits.dtype).min)
    cond = torch.arange(W)
    mask.masked_fill_(cond < (cond + 1).view(W, 1), 0)
    logits[..., L - W:] += mask
    p = F.softmax(logits, dim=-1, dtype=torch.float32)
    s = p[..., :L - W].sum(dim=-2)                                                # [Hkv, G, L - W]
    s = F.max_pool1d(s, kernel_size=kernel, padding=kernel // 2, stride=1)
    s = s.max(dim=1).values                                                       # [Hkv, L - W]
    tail = torch.arange(L - W, L)
    kept = [torch.cat([torch.sort(s[h].topk(int(caps[h]) - W).indices).values, tail]) for h in range(Hkv)]
    return s, kept


def gather(k, v, kept):
    """Kept rows of every KV head: lists of [cap_h, d] K and V."""
    return [k[h].index_select(0, ix) for h, ix in enumerate(kept)], [v[h].index_select(0, ix) for h, ix in enumerate(kept)]


def decode(q, ks, vs, k_new, v_new):
    """q [Hkv, G, d], rows ks/vs [n_h, d], new token k_new/v_new [Hkv, d]:
    append, then softmax(q.K^T / sqrt(d)).V per row -> [Hkv, G, d]."""
    d = q.shape[-1]
    out = []
    for h in range(q.shape[0]):
        kh = torch.cat([ks[h], k_new[h:h + 1]])
        vh = torch.cat([vs[h], v_new[h:h + 1]])
        w = torch.softmax(torch.matmul(q[h], kh.t()) / math.sqrt(d), dim=-1)
        out.append(torch.matmul(w, vh))
    return torch.stack(out)


def config0_tensors(c):
    """Torch tensors of a workloads.config0_inputs() case."""
    Hkv = c["k"].shape[1]
    Hq, L, d = c["q"].shape[1], c["q"].shape[2], c["q"].shape[3]
    G, W = Hq // Hkv, c["window"]
    q_win = torch.as_tensor(c["q"][0, :, L - W:]).reshape(Hkv, G, W, d).contiguous()
    return {"q_win": q_win, "k": torch.as_tensor(c["k"][0]), "v": torch.as_tensor(c["v"][0]),
            "caps": [int(x) for x in c["caps"]], "window": W,
            "q_dec": torch.as_tensor(c["q_dec"][0, :, 0]).reshape(Hkv, G, d).contiguous(),
            "k_dec": torch.as_tensor(c["k_dec"][0, :, 0]), "v_dec": torch.as_tensor(c["v_dec"][0, :, 0])}


def host_description():
    """Cores this process may use, the machine's count, and the CPU model."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        nproc = len(os.sched_getaffinity(0))
    except AttributeError:
        nproc = os.cpu_count() or 1
    return {"nproc": nproc, "cpu_count": os.cpu_count(), "model": model}


def time_stages(t, threads, runs=20, warmup=3, kernel=7):
    """Median µs per stage of the config-0 layer over `runs` timed runs after
    `warmup` untimed ones, with `threads` intra-op threads."""
    old = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        times = {"score_pool_topk": [], "gather": [], "decode": []}
        for i in range(warmup + runs):
            t0 = time.perf_counter()
            _, kept = score_select(t["q_win"], t["k"], t["caps"], t["window"], kernel)
            t1 = time.perf_counter()
            ks, vs = gather(t["k"], t["v"], kept)
            t2 = time.perf_counter()
            decode(t["q_dec"], ks, vs, t["k_dec"], t["v_dec"])
            t3 = time.perf_counter()
            if i >= warmup:
                times["score_pool_topk"].append((t1 - t0) * 1e6)
                times["gather"].append((t2 - t1) * 1e6)
                times["decode"].append((t3 - t2) * 1e6)
        med = {k: statistics.median(v) for k, v in times.items()}
        rows = sum(c + 1 for c in t["caps"])
        d = t["k"].shape[-1]
        med["decode_bytes"] = rows * d * 4 * 2           # float32 K and V of every row, new token included
        med["decode_gbs"] = med["decode_bytes"] / (med["decode"] * 1e-6) / 1e9
        return med
    finally:
        torch.set_num_threads(old)
