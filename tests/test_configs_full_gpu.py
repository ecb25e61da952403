"""The reference's configurations at their own sizes through HeteroCache,
checked against the oracle stage by stage.

At 128K-224K positions the float32 device scores and the oracle's float64
scores can swap neighbours at a budget boundary, so end-to-end equality of
kept sets is not a property either side can promise.  Each test therefore
checks two things:

* the scores each stage ranks (prefill selection, pivot reference sets,
  drift steps) against the oracle's own float64 scores, within 2e-4
  relative;
* the oracle's whole integer flow -- top-k with its tie rule, reference
  sets, overlaps, medians, triggers, retrieval prefixes, slot writes --
  run on the device's own scores (CacheOracle's score hook), which must
  reproduce the device's stores bit for bit, its triggers exactly, and its
  attention outputs within 2e-2 (bf16) of the float64 closed form.

The drift decisions are also recomputed from the oracle's own scores; the
workloads put every median at least 0.05 away from the 0.5 threshold, so
both agree.
"""
import json
import os

import numpy as np
import pytest
import torch

from heterocache_amd import utils, workloads
from heterocache_amd.cache_utils import HeteroCache, HeteroCacheConfig
from oracle import hc_oracle as O
from tests.gpu_util import as_np

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "head_analysis_llama-3.1-8b-instruct.json")
SCORE_RTOL = 2e-4
ATTN_TOL = 2e-2


def llama_json():
    raw = json.load(open(GOLDEN))
    return utils.augment_head_data(raw, [utils.head_permutation(r) for r in raw["classification_matrix"]])


def rel_err(got, ref):
    got, ref = np.asarray(got, dtype=np.float64), np.asarray(ref, dtype=np.float64)
    return float(np.max(np.abs(got - ref) / np.maximum(np.abs(ref), 1e-30)))


class Recorder:
    """HeteroCache observer: host copies of what the checked layers rank
    (batch row 0), and every check's trigger flags for all layers."""

    def __init__(self, layers):
        self.layers = set(layers)
        self.prefill, self.pivots = {}, {}
        self.drift = {}       # (layer, leader) -> list of [S, L] score arrays, one per check
        self.checks = []      # per check: {(layer, leader): triggered}

    def __call__(self, event, **kw):
        if event == "prefill_select" and kw["layer"] in self.layers:
            self.prefill[kw["layer"]] = (list(kw["rows"]), as_np(kw["scores"]))
        elif event == "pivot_sets" and kw["layer"] in self.layers:
            self.pivots[kw["layer"]] = (list(kw["pivots"]), as_np(kw["scores"]))
        elif event == "drift_check":
            trig = kw["trigger"].cpu().numpy()
            trig_of = kw["trig_of"].cpu().numpy()
            flags = {}
            for j, (layer, head, b) in enumerate(kw["row_ids"]):
                if b == 0:
                    flags[(layer, head)] = bool(trig[trig_of[j]])
                if b == 0 and layer in self.layers:
                    self.drift.setdefault((layer, head), []).append(as_np(kw["scores"][j]))
            self.checks.append(flags)


class DeviceScores:
    """CacheOracle score hook: substitutes the device's scores (batch 1)
    and records the oracle's own scores' error and drift decisions."""

    def __init__(self, rec, threshold):
        self.rec, self.thr = rec, threshold
        self.orc = None
        self.err = []          # (kind, layer, head, relative error)
        self.own = []          # (layer, leader, own median, own trigger, device-score median)

    def __call__(self, kind, layer, head, s):
        if kind == "prefill":
            rows, sc = self.rec.prefill[layer]
            dev = sc[rows.index(head)]
        elif kind == "pivot":
            pivots, sc = self.rec.pivots[layer]
            dev = sc[pivots.index(head)]
        else:
            dev = self.rec.drift[(layer, head)].pop(0)[None]
            K = min(self.orc.base, self.orc.L)
            ref = [sorted(x) for x in self.orc.ref[layer][head]]
            _, own_med, own_trig, _ = O.drift_check(s, ref, K, self.thr)
            _, dev_med, _, _ = O.drift_check(dev, ref, K, self.thr)
            self.own.append((layer, head, own_med, bool(own_trig), dev_med))
        self.err.append((kind, layer, head, rel_err(dev, s)))
        return dev


def check_stores(cache, orc, layers, B, Hkv):
    for layer in layers:
        store = cache.stores[layer]
        for r in range(B * Hkv):
            n = int(store.host_len[r])
            ok, ov = orc.rows[layer][r]
            assert n == len(ok), (layer, r)
            ks, vs = store.read_rows([r], n)
            assert np.array_equal(as_np(ks[0]), ok) and np.array_equal(as_np(vs[0]), ov), (layer, r)


def check_ref_sets(cache, orc, layers, L):
    """Device reference bitmasks (relation order, batch 1) equal the oracle's sets."""
    for layer in layers:
        st = cache._drift[layer]
        bits = st.ref_bits.cpu().numpy().view(np.uint32)
        for i, leader in enumerate(st.leaders):
            w = bits[i]
            pos = np.nonzero((w[np.arange(L) >> 5] >> (np.arange(L) & 31)) & 1)[0]
            assert set(pos.tolist()) == orc.ref[layer][leader][0], (layer, leader)


def test_config2_needles_128k_llama_json(dev):
    """Config 2: Llama-3-8B shape at 131072 tokens, all 32 layers with the
    reference's head JSON (33 pivots, 196 satellites), full-KV tier in
    host-pinned memory, 16 needle keys at +6 sigma, drift check every 5
    steps at threshold 0.5, top-1024 retrieval, 20 decode steps (4 checks).
    The step queries keep their direction in checks 1 and 3 and take a new
    one in checks 2 and 4, so every leader of every layer triggers exactly
    at checks 2 and 4.  Layers 0 and 23 (two leaders, relation order not
    ascending) are checked against the oracle stage by stage."""
    L, Hkv, G, D, NL, S, steps = 131072, 8, 4, 128, 32, 5, 20
    checked = [0, 23]
    data = llama_json()
    rec = Recorder(checked)
    cfg = HeteroCacheConfig(data, compression_ratio=0.5, stable_threshold=0.5, real_offload=True,
                            max_gen_len=steps + 4, decode_step=S, pooling="avgpool", kernel_size=5,
                            num_attn_heads=Hkv * G, num_kv_heads=Hkv, num_layers=NL, retrieval_topk=1024,
                            tier_placement="host", round_scores=False)
    cache = HeteroCache(cfg)
    cache.observer = rec
    wl = workloads.NeedleWorkload(L, kv_heads=Hkv, group=G, steps=steps, decode_step=S, seed=1002, device=dev)
    hook = DeviceScores(rec, 0.5)
    orc = O.CacheOracle(data, 1, Hkv * G, Hkv, NL, 0.5, 0.5, S, "avgpool", 5, retrieval_topk=1024,
                        max_gen=steps + 4, score_hook=hook)
    hook.orc = orc
    step_inputs, needles = {}, {}
    for layer in range(NL):
        x = wl.layer(layer)
        k, v = cache.update(x["k"], x["v"], layer)
        cache.init_coefficient(x["q_last"], k, layer)
        cache.prefill_select(x["q_last"], k, v, layer)
        if layer in checked:
            orc.prefill(layer, as_np(x["q_last"]), as_np(x["k"]), as_np(x["v"]))
            needles[layer] = x["needles"].cpu().numpy()
        step_inputs[layer] = (x["q_steps"], x["k_new"], x["v_new"])
        del x, k, v
    assert orc.base == cache.base_compress_len == 49629
    for t in range(steps):
        outs = {}
        for layer in range(NL):
            q, kn, vn = (a[t] for a in step_inputs[layer])
            cache.update(kn, vn, layer)
            o = cache.decode_attention(q, layer)
            cache.decode_select(q, layer)
            if layer in checked:
                outs[layer] = o
        for layer in checked:
            q, kn, vn = (as_np(a[t]) for a in step_inputs[layer])
            ref = orc.decode(layer, q, kn, vn)
            err = np.abs(as_np(outs[layer]).reshape(1, Hkv * G, D) - ref).max()
            assert err <= ATTN_TOL, f"step {t} layer {layer}: max-abs {err}"
    torch.cuda.synchronize()
    # Natural triggers: every leader of every layer, at checks 2 and 4 only.
    assert len(rec.checks) == steps // S
    for c, flags in enumerate(rec.checks):
        assert len(flags) == 33
        assert all(f == (c % 2 == 1) for f in flags.values()), (c, flags)
    # The checked layers' triggers equal the oracle's decisions ...
    dev_trig = [(l, h, rec.checks[c][(l, h)]) for c in range(len(rec.checks)) for l in checked
                for h in cache._drift[l].leaders]
    assert sorted(dev_trig) == sorted(orc.triggers)
    # ... and those the oracle takes on its own float64 scores, with margin.
    for layer, leader, own_med, own_trig, dev_med in hook.own:
        assert abs(own_med - 0.5) >= 0.05 and abs(dev_med - own_med) < 5e-3
    assert [t for *_, t, _ in hook.own] == [t for _, _, t in orc.triggers]
    assert max(e for *_, e in hook.err) <= SCORE_RTOL
    check_stores(cache, orc, checked, 1, Hkv)
    check_ref_sets(cache, orc, checked, L)
    # Retrieval brought every needle into satellites that took >= 128 tokens.
    alloc = data["allocation_matrix"]
    for layer in checked:
        tier_k = orc.tier[layer][0][0]
        for leader, members in data["leader_member_relations"][layer].items():
            for m in members:
                n = min(int(O.prefill_caps(orc.base, [alloc[layer][m]], L)[0]), 1024)
                if n < 128:
                    continue
                rows_k = orc.rows[layer][m][0][:n]
                for p in needles[layer]:
                    assert (rows_k == tier_k[m, p]).all(axis=1).any(), (layer, m, p)


def f16_steps(got, ref):
    """|got - ref| in units of the float16 spacing at ref (2^-24 below the
    normal range, where the cast chain's small probabilities live)."""
    got, ref = np.asarray(got, dtype=np.float64), np.asarray(ref, dtype=np.float64)
    sp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
    return np.abs(got - ref) / sp


class CastChainScores(DeviceScores):
    """DeviceScores for the reference's float16 cast chain: also records,
    per scored head, how far the device scores sit from the oracle's cast
    chain in float16 steps."""

    def __init__(self, rec, threshold):
        super().__init__(rec, threshold)
        self.steps = []        # (kind, layer, head, max steps, positions off by more than one step, positions)

    def __call__(self, kind, layer, head, s):
        dev = super().__call__(kind, layer, head, s)
        st = f16_steps(dev, s)
        self.steps.append((kind, layer, head, float(st.max()), int((st > 1.0).sum()), int(st.size)))
        return dev


def test_config2_reference_cast_chain_fp16_128k(dev):
    """Config 2 in the reference's own arithmetic: a float16 model (the
    reference's load dtype) with round_scores=True, i.e. logits rounded to
    float16, scaled and rounded again, float32 softmax rounded to float16,
    pooled and rounded (heterocache/cache_utils.py:814-819, 1037-1043,
    1167-1175).  131072 tokens, all 32 layers with the reference's head
    JSON, needle queries, drift check every 5 steps at threshold 0.5,
    top-1024 retrieval, 20 steps (4 checks: every leader triggers at checks
    2 and 4).  Layers 0 and 23 are checked stage by stage:

    * every score the device ranks (prefill selection, pivot sets, drift
      steps) equals the oracle's float16 cast chain to within two float16
      steps at the score's magnitude (subnormal spacing below 2^-14), and
      all but a few in a million within one.  Two is what the chain allows
      for a probability one step off (the float32 softmax arithmetic): it
      moves the average of 5 by at most 8/5 steps of the average, since
      steps are powers of two;
    * the oracle's integer flow on the device scores -- where the cast
      chain ties massively, the lowest position first -- reproduces the
      triggers, reference sets and stores bit for bit;
    * attention is within 2e-2 of the float64 closed form."""
    L, Hkv, G, D, NL, S, steps = 131072, 8, 4, 128, 32, 5, 20
    checked = [0, 23]
    data = llama_json()
    rec = Recorder(checked)
    cfg = HeteroCacheConfig(data, compression_ratio=0.5, stable_threshold=0.5, real_offload=True,
                            max_gen_len=steps + 4, decode_step=S, pooling="avgpool", kernel_size=5,
                            num_attn_heads=Hkv * G, num_kv_heads=Hkv, num_layers=NL, retrieval_topk=1024,
                            round_scores=True)
    cache = HeteroCache(cfg)
    cache.observer = rec
    wl = workloads.NeedleWorkload(L, kv_heads=Hkv, group=G, steps=steps, decode_step=S, seed=1002, device=dev,
                                  dtype=torch.float16)
    hook = CastChainScores(rec, 0.5)
    orc = O.CacheOracle(data, 1, Hkv * G, Hkv, NL, 0.5, 0.5, S, "avgpool", 5, retrieval_topk=1024,
                        max_gen=steps + 4, score_hook=hook, io_dtype="float16")
    hook.orc = orc
    step_inputs = {}
    for layer in range(NL):
        x = wl.layer(layer)
        k, v = cache.update(x["k"], x["v"], layer)
        cache.init_coefficient(x["q_last"], k, layer)
        cache.prefill_select(x["q_last"], k, v, layer)
        if layer in checked:
            orc.prefill(layer, as_np(x["q_last"]), as_np(x["k"]), as_np(x["v"]))
        step_inputs[layer] = (x["q_steps"], x["k_new"], x["v_new"])
        del x, k, v
    assert orc.base == cache.base_compress_len == 49629
    assert cache.one_pass_checks == 0
    for t in range(steps):
        outs = {}
        for layer in range(NL):
            q, kn, vn = (a[t] for a in step_inputs[layer])
            cache.update(kn, vn, layer)
            o = cache.decode_attention(q, layer)
            cache.decode_select(q, layer)
            if layer in checked:
                outs[layer] = o
        for layer in checked:
            q, kn, vn = (as_np(a[t]) for a in step_inputs[layer])
            ref = orc.decode(layer, q, kn, vn)
            err = np.abs(as_np(outs[layer]).reshape(1, Hkv * G, D) - ref).max()
            assert err <= ATTN_TOL, f"step {t} layer {layer}: max-abs {err}"
    torch.cuda.synchronize()
    assert len(rec.checks) == steps // S
    # Every check scored in one pass, from the float16 cast chain's
    # statistics that the decode launches reported.
    assert cache.one_pass_checks >= steps // S
    for c, flags in enumerate(rec.checks):
        assert len(flags) == 33
        assert all(f == (c % 2 == 1) for f in flags.values()), (c, flags)
    dev_trig = [(l, h, rec.checks[c][(l, h)]) for c in range(len(rec.checks)) for l in checked
                for h in cache._drift[l].leaders]
    assert sorted(dev_trig) == sorted(orc.triggers)
    kinds = sorted({k for k, *_ in hook.steps})
    assert kinds == ["drift", "pivot", "prefill"], kinds
    worst = max(hook.steps, key=lambda x: x[3])
    off = sum(x[4] for x in hook.steps)
    total = sum(x[5] for x in hook.steps)
    print(f"cast chain: {len(hook.steps)} score rows, {total} scores, worst {worst[3]:.2f} float16 steps "
          f"({worst[:3]}), {off} beyond one step")
    check_stores(cache, orc, checked, 1, Hkv)
    check_ref_sets(cache, orc, checked, L)
    assert worst[3] <= 2.0, worst
    assert off <= total * 1e-5, (off, total)


class ReplayDriftScores(DeviceScores):
    """DeviceScores whose drift scores replace the oracle's outright: the
    oracle skips its own float64 scoring of the step queries, so a long run
    can replay the integer flow on the device's scores at every check."""
    replaces_drift = True

    def __call__(self, kind, layer, head, s):
        if kind == "drift":
            return self.rec.drift[(layer, head)].pop(0)[None]
        return super().__call__(kind, layer, head, s)


def test_config2_needles_128k_all_1000_steps(dev):
    """Config 2 for its whole run: 1000 decode steps at 131072 tokens, all
    32 layers with the reference's head JSON, the full-KV tier in
    host-pinned memory, the default configuration (bfloat16, the
    reference's cast chain), drift check every 5 steps at threshold 0.5 and
    top-1024 retrieval: 200 checks, every leader of every layer triggering
    at every second one (100 retrievals per leader).

    * Every check's trigger flags, for all 33 leaders, follow the needle
      workload's schedule.
    * Layer 23 (two leaders, relation order not ascending) is replayed by
      the oracle's integer flow on the device's own scores at every check
      (top-k with its tie rule, overlaps, medians, triggers, ascending
      prefixes, slot writes): the triggers match check by check, and after
      the 1000 steps its stores and reference sets are bit for bit the
      oracle's.
    * Its attention is within 2e-2 of the float64 closed form at sampled
      steps: the first, the two after the first retrieval, and steps in the
      middle and at the end of the run."""
    L, Hkv, G, D, NL, S, steps = 131072, 8, 4, 128, 32, 5, 1000
    lc = 23
    data = llama_json()
    rec = Recorder([lc])
    cfg = HeteroCacheConfig(data, compression_ratio=0.5, stable_threshold=0.5, real_offload=True,
                            max_gen_len=steps + 4, decode_step=S, pooling="avgpool", kernel_size=5,
                            num_attn_heads=Hkv * G, num_kv_heads=Hkv, num_layers=NL, retrieval_topk=1024,
                            tier_placement="host")
    cache = HeteroCache(cfg)
    assert cache.round_scores
    cache.observer = rec
    wl = workloads.NeedleWorkload(L, kv_heads=Hkv, group=G, steps=steps, decode_step=S, seed=1002, device=dev)
    hook = ReplayDriftScores(rec, 0.5)
    orc = O.CacheOracle(data, 1, Hkv * G, Hkv, NL, 0.5, 0.5, S, "avgpool", 5, retrieval_topk=1024,
                        max_gen=steps + 4, score_hook=hook)
    hook.orc = orc
    step_inputs = {}
    for layer in range(NL):
        x = wl.layer(layer)
        k, v = cache.update(x["k"], x["v"], layer)
        cache.init_coefficient(x["q_last"], k, layer)
        cache.prefill_select(x["q_last"], k, v, layer)
        if layer == lc:
            orc.prefill(layer, as_np(x["q_last"]), as_np(x["k"]), as_np(x["v"]))
        step_inputs[layer] = (x["q_steps"], x["k_new"], x["v_new"])
        del x, k, v
    assert cache.tier_mode == "host"
    sampled = {0, 10, 11, 500, 999}
    for t in range(steps):
        out = None
        for layer in range(NL):
            q, kn, vn = (a[t] for a in step_inputs[layer])
            cache.update(kn, vn, layer)
            o = cache.decode_attention(q, layer)
            cache.decode_select(q, layer)
            if layer == lc:
                out = o
        q, kn, vn = (as_np(a[t]) for a in step_inputs[lc])
        ref = orc.decode(lc, q, kn, vn, attend=t in sampled)
        if ref is not None:
            err = np.abs(as_np(out).reshape(1, Hkv * G, D) - ref).max()
            assert err <= ATTN_TOL, f"step {t}: max-abs {err}"
    torch.cuda.synchronize()
    assert len(rec.checks) == steps // S
    for c, flags in enumerate(rec.checks):
        assert len(flags) == 33
        assert all(f == (c % 2 == 1) for f in flags.values()), (c, flags)
    assert not any(rec.drift.values())  # every recorded check was replayed
    dev_trig = [(lc, h, rec.checks[c][(lc, h)]) for c in range(len(rec.checks)) for h in cache._drift[lc].leaders]
    assert dev_trig == orc.triggers
    assert sum(t for *_, t in orc.triggers) == len(cache._drift[lc].leaders) * steps // S // 2
    check_stores(cache, orc, [lc], 1, Hkv)
    check_ref_sets(cache, orc, [lc], L)


def test_config4_chunked_224k_then_drift_block(dev):
    """Config 4: Llama-3-8B shape at 229376 tokens, all 32 layers with the
    reference's head JSON.  An 8K-chunked prefill (chunks fed layer by
    layer, in model order) leaves every store, length and reference set
    identical to a single-shot prefill of the same K/V.  Then 205 decode
    steps on the chunked cache (full-KV tier in host-pinned memory,
    top-1024 retrieval) with attention drifting to a new block of 8 keys
    at step 200: no leader triggers in the 40 checks inside the first block,
    every leader triggers at the check after the boundary.  Layer 23 is
    checked against the oracle stage by stage (attention at sampled
    steps)."""
    L, Hkv, G, D, NL, S, steps, chunk = 229376, 8, 4, 128, 32, 5, 205, 8192
    checked = [23]
    data = llama_json()
    rec = Recorder(checked)

    def make(host_tier):
        cfg = HeteroCacheConfig(data, compression_ratio=0.5, stable_threshold=0.5, real_offload=host_tier,
                                max_gen_len=steps + 4, decode_step=S, pooling="avgpool", kernel_size=5,
                                num_attn_heads=Hkv * G, num_kv_heads=Hkv, num_layers=NL, retrieval_topk=1024,
                                tier_placement="host", round_scores=False)
        return HeteroCache(cfg)

    whole, chunked = make(False), make(True)
    chunked.begin_prefill(L)
    chunked.observer = rec
    wl = workloads.BlockDriftWorkload(L, kv_heads=Hkv, group=G, steps=steps, period=200, seed=1004, device=dev)
    kv, step_inputs = {}, {}
    for layer in range(NL):
        k, v = wl.prefill(layer)
        x = wl.queries(layer, k)
        kv[layer] = (k, v)
        step_inputs[layer] = (x["q_last"], x["q_steps"], x["k_new"], x["v_new"])
        kc, vc = whole.update(k, v, layer)
        whole.init_coefficient(x["q_last"], kc, layer)
        whole.prefill_select(x["q_last"], kc, vc, layer)
    filler = torch.zeros((1, Hkv * G, 1, D), dtype=torch.bfloat16, device=dev)
    for s in range(0, L, chunk):
        e = min(s + chunk, L)
        for layer in range(NL):
            k, v = kv[layer]
            q = step_inputs[layer][0] if e == L else filler
            kc, vc = chunked.update(k[:, :, s:e], v[:, :, s:e], layer, {"query_states": q})
            assert kc.shape[2] == e
            chunked.init_coefficient(q, kc, layer)
            chunked.prefill_select(q, kc, vc, layer)
            assert chunked.prefill_pending(layer) == (e < L)
    torch.cuda.synchronize()
    assert whole.base_compress_len == chunked.base_compress_len == 86851
    assert torch.equal(whole._ref_bits_all, chunked._ref_bits_all)
    for a, b in zip(whole.stores, chunked.stores):
        assert a.host_len.tolist() == b.host_len.tolist() and torch.equal(a.row_len, b.row_len)
        for r in range(a.rows):  # written slots only (the arenas are not cleared)
            n = int(a.host_len[r])
            ka, va = a.read_rows([r], n)
            kb, vb = b.read_rows([r], n)
            assert torch.equal(ka, kb) and torch.equal(va, vb), (a.layer_idx, r)
    del whole
    hook = DeviceScores(rec, 0.5)
    orc = O.CacheOracle(data, 1, Hkv * G, Hkv, NL, 0.5, 0.5, S, "avgpool", 5, retrieval_topk=1024,
                        max_gen=steps + 4, score_hook=hook)
    hook.orc = orc
    for layer in checked:
        orc.prefill(layer, as_np(step_inputs[layer][0]), as_np(kv[layer][0]), as_np(kv[layer][1]))
    kv.clear()
    attend_at = {0, 1, 100, 199, 200, 201, 204}
    for t in range(steps):
        outs = {}
        for layer in range(NL):
            _, qs, kn, vn = step_inputs[layer]
            chunked.update(kn[t], vn[t], layer)
            o = chunked.decode_attention(qs[t], layer)
            chunked.decode_select(qs[t], layer)
            if layer in checked:
                outs[layer] = o
        for layer in checked:
            _, qs, kn, vn = step_inputs[layer]
            ref = orc.decode(layer, as_np(qs[t]), as_np(kn[t]), as_np(vn[t]), attend=t in attend_at)
            if ref is not None:
                err = np.abs(as_np(outs[layer]).reshape(1, Hkv * G, D) - ref).max()
                assert err <= ATTN_TOL, f"step {t} layer {layer}: max-abs {err}"
    torch.cuda.synchronize()
    assert len(rec.checks) == steps // S == 41
    for c, flags in enumerate(rec.checks):
        assert len(flags) == 33
        assert all(f == (c == 40) for f in flags.values()), (c, [k for k, f in flags.items() if f != (c == 40)])
    dev_trig = [(l, h, rec.checks[c][(l, h)]) for c in range(len(rec.checks)) for l in checked
                for h in chunked._drift[l].leaders]
    assert sorted(dev_trig) == sorted(orc.triggers)
    for layer, leader, own_med, own_trig, dev_med in hook.own:
        assert abs(own_med - 0.5) >= 0.05 and abs(dev_med - own_med) < 5e-3
    assert [t for *_, t, _ in hook.own] == [t for _, _, t in orc.triggers]
    assert max(e for *_, e in hook.err) <= SCORE_RTOL
    check_stores(chunked, orc, checked, 1, Hkv)
    check_ref_sets(chunked, orc, checked, L)


def test_config4_224k_all_2000_steps(dev):
    """Config 4's decode run in full: 229376 tokens, all 32 layers with the
    reference's head JSON, the default configuration (bfloat16, the
    reference's cast chain), full-KV tier in host-pinned memory, top-1024
    retrieval, and 2000 decode steps whose attention moves to a new block of
    8 keys every 200 steps: of the 400 checks exactly the 9 after a block
    change trigger, each for all 33 leaders.  Layer 23 is replayed by the
    oracle's integer flow on the device's scores at every check: triggers
    check by check, stores and reference sets bit for bit after the run,
    attention within 2e-2 of float64 at sampled steps.  (The chunked
    prefill's equality with a single-shot one is the 205-step test's.)"""
    L, Hkv, G, D, NL, S, steps, period = 229376, 8, 4, 128, 32, 5, 2000, 200
    lc = 23
    data = llama_json()
    rec = Recorder([lc])
    cfg = HeteroCacheConfig(data, compression_ratio=0.5, stable_threshold=0.5, real_offload=True,
                            max_gen_len=steps + 4, decode_step=S, pooling="avgpool", kernel_size=5,
                            num_attn_heads=Hkv * G, num_kv_heads=Hkv, num_layers=NL, retrieval_topk=1024,
                            tier_placement="host")
    cache = HeteroCache(cfg)
    assert cache.round_scores
    cache.observer = rec
    wl = workloads.BlockDriftWorkload(L, kv_heads=Hkv, group=G, steps=steps, period=period, seed=1004, device=dev)
    hook = ReplayDriftScores(rec, 0.5)
    orc = O.CacheOracle(data, 1, Hkv * G, Hkv, NL, 0.5, 0.5, S, "avgpool", 5, retrieval_topk=1024,
                        max_gen=steps + 4, score_hook=hook)
    hook.orc = orc
    step_inputs = {}
    for layer in range(NL):
        k, v = wl.prefill(layer)
        x = wl.queries(layer, k)
        kc, vc = cache.update(k, v, layer)
        cache.init_coefficient(x["q_last"], kc, layer)
        cache.prefill_select(x["q_last"], kc, vc, layer)
        if layer == lc:
            orc.prefill(layer, as_np(x["q_last"]), as_np(k), as_np(v))
        step_inputs[layer] = (x["q_steps"], x["k_new"], x["v_new"])
        del k, v, kc, vc, x
    assert cache.tier_mode == "host" and cache.base_compress_len == orc.base == 86851
    sampled = {0, 200, 201, 1000, 1800, 1999}
    for t in range(steps):
        out = None
        for layer in range(NL):
            q, kn, vn = (a[t] for a in step_inputs[layer])
            cache.update(kn, vn, layer)
            o = cache.decode_attention(q, layer)
            cache.decode_select(q, layer)
            if layer == lc:
                out = o
        q, kn, vn = (as_np(a[t]) for a in step_inputs[lc])
        ref = orc.decode(lc, q, kn, vn, attend=t in sampled)
        if ref is not None:
            err = np.abs(as_np(out).reshape(1, Hkv * G, D) - ref).max()
            assert err <= ATTN_TOL, f"step {t}: max-abs {err}"
    torch.cuda.synchronize()
    assert len(rec.checks) == steps // S == 400
    change = {c for c in range(400) if c > 0 and (c * S) % period == 0}
    assert len(change) == 9
    for c, flags in enumerate(rec.checks):
        assert len(flags) == 33
        assert all(f == (c in change) for f in flags.values()), (c, [k for k, f in flags.items() if f != (c in change)])
    assert not any(rec.drift.values())  # every recorded check was replayed
    dev_trig = [(lc, h, rec.checks[c][(lc, h)]) for c in range(len(rec.checks)) for h in cache._drift[lc].leaders]
    assert dev_trig == orc.triggers
    check_stores(cache, orc, [lc], 1, Hkv)
    check_ref_sets(cache, orc, [lc], L)


@pytest.mark.parametrize("ctx", [16384, 32768, 49152, 65536])
def test_config3_qwen_sequence_full_context(dev, ctx):
    """Config 3, one sequence of the ragged batch per run (the reference's
    cache is defined for batch 1, so each sequence is checked against a
    batch-1 oracle run): Qwen2.5-7B shape (28 layers, 4 KV heads, GQA 7),
    ratio 0.25, synthetic head JSON with at most 14 full heads, top-512
    retrieval, drift check every 5 steps at threshold 0.5, Qwen order
    (select before attention, so a retrieval is attended in its own step).
    10 decode steps: every leader keeps its set at the first check and
    triggers at the second.  The first layer with a satellite is checked
    against the oracle stage by stage."""
    Hkv, G, D, NL, S, steps = 4, 7, 128, 28, 5, 10
    raw = workloads.synthetic_head_json(NL, Hkv, 1003, max_full=14)
    data = utils.augment_head_data(raw, [utils.head_permutation(r) for r in raw["classification_matrix"]])
    checked = [next(l for l in range(NL) if any(data["leader_member_relations"][l].values()))]
    rec = Recorder(checked)
    cfg = HeteroCacheConfig(data, compression_ratio=0.25, stable_threshold=0.5, real_offload=True,
                            max_gen_len=steps + 4, decode_step=S, pooling="avgpool", kernel_size=5,
                            num_attn_heads=Hkv * G, num_kv_heads=Hkv, num_layers=NL, retrieval_topk=512,
                            round_scores=False)
    cache = HeteroCache(cfg)
    cache.observer = rec
    wl = workloads.NeedleWorkload(ctx, kv_heads=Hkv, group=G, steps=steps, decode_step=S, seed=1003 + ctx, device=dev)
    hook = DeviceScores(rec, 0.5)
    orc = O.CacheOracle(data, 1, Hkv * G, Hkv, NL, 0.25, 0.5, S, "avgpool", 5, retrieval_topk=512,
                        select_before_attention=True, max_gen=steps + 4, score_hook=hook)
    hook.orc = orc
    step_inputs = {}
    for layer in range(NL):
        x = wl.layer(layer)
        k, v = cache.update(x["k"], x["v"], layer)
        cache.init_coefficient(x["q_last"], k, layer)
        cache.prefill_select(x["q_last"], k, v, layer)
        if layer in checked:
            orc.prefill(layer, as_np(x["q_last"]), as_np(x["k"]), as_np(x["v"]))
        step_inputs[layer] = (x["q_steps"], x["k_new"], x["v_new"])
        del x, k, v
    F = data["meta"]["counts"]["volatile"] + data["meta"]["counts"]["pivot"]
    assert cache.base_compress_len == orc.base == workloads.get_compress_len(0.25, F, ctx, Hkv * NL) > 0
    for t in range(steps):
        outs = {}
        for layer in range(NL):
            q, kn, vn = (a[t] for a in step_inputs[layer])
            cache.update(kn, vn, layer)
            cache.decode_select(q, layer)
            o = cache.decode_attention(q, layer)
            if layer in checked:
                outs[layer] = o
        for layer in checked:
            q, kn, vn = (as_np(a[t]) for a in step_inputs[layer])
            ref = orc.decode(layer, q, kn, vn)
            err = np.abs(as_np(outs[layer]).reshape(1, Hkv * G, D) - ref).max()
            assert err <= ATTN_TOL, f"step {t} layer {layer}: max-abs {err}"
    torch.cuda.synchronize()
    nlead = sum(len(r) for r in data["leader_member_relations"])
    # Qwen order checks layer by layer: group each leader's flags over the checks.
    flags = {}
    for f in rec.checks:
        for key, val in f.items():
            flags.setdefault(key, []).append(val)
    assert len(flags) == nlead and all(v == [False, True] for v in flags.values()), flags
    dev_trig = [(l, h, flags[(l, h)][c]) for c in range(2) for l in checked for h in cache._drift[l].leaders]
    assert sorted(dev_trig) == sorted(orc.triggers)
    for layer, leader, own_med, own_trig, dev_med in hook.own:
        assert abs(own_med - 0.5) >= 0.05 and abs(dev_med - own_med) < 5e-3
    assert [t for *_, t, _ in hook.own] == [t for _, _, t in orc.triggers]
    assert max(e for *_, e in hook.err) <= SCORE_RTOL
    check_stores(cache, orc, checked, 1, Hkv)
    check_ref_sets(cache, orc, checked, ctx)


def test_config3_qwen_64k_200_steps_default_configuration(dev):
    """Config 3's longest sequence (65536 tokens) over 200 decode steps in the
    default configuration (bfloat16, the reference's cast chain), Qwen order
    (select before attention), top-512 retrieval every 5 steps: 40 checks,
    every leader triggering at every second one.  The first layer with a
    satellite is replayed by the oracle's integer flow on the device's
    scores at every check; its stores and reference sets are bit for bit
    the oracle's after the run, and its attention is within 2e-2 of float64
    at sampled steps (a retrieval is attended in its own step here)."""
    ctx, Hkv, G, D, NL, S, steps = 65536, 4, 7, 128, 28, 5, 200
    raw = workloads.synthetic_head_json(NL, Hkv, 1003, max_full=14)
    data = utils.augment_head_data(raw, [utils.head_permutation(r) for r in raw["classification_matrix"]])
    lc = next(l for l in range(NL) if any(data["leader_member_relations"][l].values()))
    rec = Recorder([lc])
    cfg = HeteroCacheConfig(data, compression_ratio=0.25, stable_threshold=0.5, real_offload=True,
                            max_gen_len=steps + 4, decode_step=S, pooling="avgpool", kernel_size=5,
                            num_attn_heads=Hkv * G, num_kv_heads=Hkv, num_layers=NL, retrieval_topk=512)
    cache = HeteroCache(cfg)
    assert cache.round_scores
    cache.observer = rec
    wl = workloads.NeedleWorkload(ctx, kv_heads=Hkv, group=G, steps=steps, decode_step=S, seed=1003 + ctx, device=dev)
    hook = ReplayDriftScores(rec, 0.5)
    orc = O.CacheOracle(data, 1, Hkv * G, Hkv, NL, 0.25, 0.5, S, "avgpool", 5, retrieval_topk=512,
                        select_before_attention=True, max_gen=steps + 4, score_hook=hook)
    hook.orc = orc
    step_inputs = {}
    for layer in range(NL):
        x = wl.layer(layer)
        k, v = cache.update(x["k"], x["v"], layer)
        cache.init_coefficient(x["q_last"], k, layer)
        cache.prefill_select(x["q_last"], k, v, layer)
        if layer == lc:
            orc.prefill(layer, as_np(x["q_last"]), as_np(x["k"]), as_np(x["v"]))
        step_inputs[layer] = (x["q_steps"], x["k_new"], x["v_new"])
        del x, k, v
    sampled = {0, 9, 10, 100, 199}
    for t in range(steps):
        out = None
        for layer in range(NL):
            q, kn, vn = (a[t] for a in step_inputs[layer])
            cache.update(kn, vn, layer)
            cache.decode_select(q, layer)
            o = cache.decode_attention(q, layer)
            if layer == lc:
                out = o
        q, kn, vn = (as_np(a[t]) for a in step_inputs[lc])
        ref = orc.decode(lc, q, kn, vn, attend=t in sampled)
        if ref is not None:
            err = np.abs(as_np(out).reshape(1, Hkv * G, D) - ref).max()
            assert err <= ATTN_TOL, f"step {t}: max-abs {err}"
    torch.cuda.synchronize()
    nlead = sum(len(r) for r in data["leader_member_relations"])
    flags = {}
    for f in rec.checks:
        for key, val in f.items():
            flags.setdefault(key, []).append(val)
    pattern = [c % 2 == 1 for c in range(steps // S)]
    assert len(flags) == nlead and all(v == pattern for v in flags.values())
    assert not any(rec.drift.values())
    dev_trig = [(lc, h, flags[(lc, h)][c]) for c in range(steps // S) for h in cache._drift[lc].leaders]
    assert dev_trig == orc.triggers
    check_stores(cache, orc, [lc], 1, Hkv)
    check_ref_sets(cache, orc, [lc], ctx)


def _sdpa_repeated_kv(module, query, key, value, attention_mask, dropout=0.0, scaling=None, is_causal=None,
                      **kwargs):
    """transformers attention function for the float32 stock reference:
    K/V repeated to the query heads, then PyTorch SDPA with the causal flag
    (transformers' own SDPA path passes grouped K/V, which only SDPA's math
    kernel takes; at 32K in float32 its score matrix does not fit)."""
    import torch.nn.functional as F
    if attention_mask is not None:
        raise ValueError("the float32 reference runs without an attention mask")
    rep = query.shape[1] // key.shape[1]
    key = key.repeat_interleave(rep, dim=1)
    value = value.repeat_interleave(rep, dim=1)
    out = F.scaled_dot_product_attention(query, key, value, is_causal=query.shape[2] > 1, scale=scaling)
    return out.transpose(1, 2).contiguous(), None


def _llama8b_config(max_pos, attn="sdpa"):
    from transformers import LlamaConfig
    return LlamaConfig(vocab_size=128256, hidden_size=4096, intermediate_size=14336, num_hidden_layers=32,
                       num_attention_heads=32, num_key_value_heads=8, head_dim=128, max_position_embeddings=max_pos,
                       rope_theta=500000.0, attn_implementation=attn)


def test_config1_llama8b_32k_generate(dev):
    """Config 1: the 32-layer Llama-3-8B shape (random init, vocab 128256) on
    a 32768-token prompt of seeded random ids, 256 greedy tokens.

    * Keep-all budgets (one anchor keeping the whole prompt, every other head
      full) in float32: the patched model's generate() under HeteroCache
      returns the stock transformers model's tokens (SDPA attention,
      DynamicCache), and its per-step logits agree within 1e-3 relative.
      (In bf16 a random-init 32-layer model turns rounding into logit
      differences of several percent -- transformers' own eager and SDPA
      paths differ by about 9 % -- so greedy tokens cannot pin equivalence
      there.)
    * Compressed, bf16, as the configuration specifies: ratio 0.5 with the
      seeded synthetic clusters of 1-4 heads, drift checks every 5 steps;
      layer 17's decode attention at steps 0, 127 and 254 equals the float64
      closed form over its store rows and the appended token (<= 2e-2), and
      every row's length advances by one per generated token."""
    from transformers import LlamaForCausalLM
    L, new, D = 32768, 256, 128
    cfg = _llama8b_config(L + new + 8)
    ids = torch.randint(0, 128256, (1, L), generator=torch.Generator().manual_seed(1001)).to(dev)
    def greedy(model, cache):
        """Greedy decoding by plain forwards, without an attention mask."""
        toks, logits = [], []
        with torch.no_grad():
            o = model(ids, past_key_values=cache, use_cache=True, logits_to_keep=1)
            for _ in range(new):
                lg = o.logits[:, -1].float()
                logits.append(lg)
                toks.append(lg.argmax(-1))
                o = model(toks[-1].view(1, 1), past_key_values=o.past_key_values, use_cache=True)
        return torch.stack(toks, 1), torch.cat(logits)

    from transformers import AttentionInterface
    AttentionInterface.register("sdpa_repeated_kv", _sdpa_repeated_kv)
    torch.manual_seed(0)
    with torch.device(dev):
        stock = LlamaForCausalLM(_llama8b_config(L + new + 8, "sdpa_repeated_kv")).eval()
    ref_toks, ref_logits = greedy(stock, None)
    weights = stock.state_dict()
    del stock
    torch.cuda.empty_cache()
    keep_all = {"meta": {"type_map": dict(workloads.TYPE_MAP),
                         "counts": {"anchor": 1, "volatile": 255, "pivot": 0, "satellite": 0}},
                "classification_matrix": [[1] + [2] * 7] + [[2] * 8 for _ in range(31)],
                "allocation_matrix": [[1.0] + [-1.0] * 7] + [[-1.0] * 8 for _ in range(31)],
                "leader_member_relations": [{} for _ in range(32)]}
    with utils.install_attention_patch():
        with torch.device(dev):
            model = LlamaForCausalLM(cfg).eval()
    model.load_state_dict(weights)
    perms = utils.reorder_model_weights_by_classification(model, keep_all)
    cc = utils.build_cache_config(model, utils.augment_head_data(keep_all, perms), compression_ratio=1.0,
                                  max_gen_len=new + 8)
    toks, logits = greedy(model, HeteroCache(cc))
    assert torch.equal(toks, ref_toks)
    rel = ((logits - ref_logits).norm(dim=-1) / ref_logits.norm(dim=-1)).max().item()
    assert rel <= 1e-3, rel
    del model, toks, logits, ref_toks, ref_logits
    torch.cuda.empty_cache()

    # Compressed bf16 run of the configuration.
    raw = workloads.synthetic_head_json(32, 8, 1001)
    with utils.install_attention_patch():
        with torch.device(dev):
            model = LlamaForCausalLM(cfg).to(torch.bfloat16).eval()
    model.load_state_dict({k: v.to(torch.bfloat16) for k, v in weights.items()})
    del weights
    perms = utils.reorder_model_weights_by_classification(model, raw)
    data = utils.augment_head_data(raw, perms)
    cc = utils.build_cache_config(model, data, compression_ratio=0.5, max_gen_len=new + 8, decode_step=5)
    utils.attach_cache(model, cc)
    sampled, at, errs, caches = 17, {0, 127, new - 2}, [], []   # decode forwards are steps 0 .. new - 2
    orig_attn, orig_init = HeteroCache.decode_attention, HeteroCache.__init__
    calls = {"n": 0}

    def spy_init(self, c):
        orig_init(self, c)
        caches.append(self)

    def spy_attn(self, query_states, layer_idx, out=None):
        if layer_idx != sampled:
            return orig_attn(self, query_states, layer_idx, out)
        step = calls["n"]
        calls["n"] += 1
        if step not in at:
            return orig_attn(self, query_states, layer_idx, out)
        torch.cuda.synchronize()   # retrieval gathers on the side stream included
        store = self.stores[layer_idx]
        kn, vn = self._pending[layer_idx]
        rows = range(store.rows)
        ks = [np.concatenate([as_np(store.read_rows([r], int(store.host_len[r]))[0][0]), as_np(kn[0, r])])
              for r in rows]
        vs = [np.concatenate([as_np(store.read_rows([r], int(store.host_len[r]))[1][0]), as_np(vn[0, r])])
              for r in rows]
        o = orig_attn(self, query_states, layer_idx, out)
        qq = as_np(query_states).reshape(store.rows, -1, D)
        errs.append(float(np.abs(as_np(o).reshape(store.rows, -1, D) - O.decode_attention(qq, ks, vs)).max()))
        return o

    HeteroCache.decode_attention, HeteroCache.__init__ = spy_attn, spy_init
    try:
        with torch.no_grad():
            seq = model.generate(ids, max_new_tokens=new, do_sample=False)
    finally:
        HeteroCache.decode_attention, HeteroCache.__init__ = orig_attn, orig_init
    torch.cuda.synchronize()
    assert seq.shape == (1, L + new)
    assert len(errs) == 3 and max(errs) <= ATTN_TOL, errs
    cache = caches[-1]
    assert sum(len(r) for r in data["leader_member_relations"]) > 0
    # 255 decode forwards after the prefill (the last token is not fed back):
    # keep heads hold the prompt, compressed heads their float32 budget.
    for layer in range(32):
        n_c = data["need_to_compress_counts"][layer]
        caps = O.prefill_caps(cache.base_compress_len, data["allocation_matrix"][layer][:n_c], L)
        keep = set(data["need_to_keep_counts"][layer])
        expect = [(L if h in keep else int(caps[h])) + new - 1 for h in range(8)]
        assert cache.stores[layer].row_len.tolist() == expect, layer
