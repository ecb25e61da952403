"""HeteroCache end to end (prefill, decode, drift, retrieval) vs CacheOracle.

Two layers, GQA 4, one batch row.  Decode steps 0-4 repeat the last prefill
query (pivot overlap 1.0: no retrieval); steps 5-9 use fresh random queries
(overlap ~ K/L ~ 0.33 < 0.5: retrieval).  Every step's attention output is
compared with the oracle (1e-4 float32, 2e-2 bf16); trigger decisions and the
final store rows (copies: bit-exact) are compared too.  Llama order, Qwen
order (select before attention), retrieval top-k and the reference-quirk
mode are covered.
"""
import math

import numpy as np
import pytest
import torch

from heterocache_amd import ops, workloads
from heterocache_amd.cache_utils import HeteroCache, HeteroCacheConfig
from heterocache_amd.utils import augment_head_data, head_permutation
from oracle import hc_oracle as O
from tests.gpu_util import as_np

pytestmark = pytest.mark.gpu

CLASSES = [[1, 4, 4, 1, 2, 3, 4, 1],   # layer 0: one volatile, one pivot
           [4, 4, 3, 1, 1, 4, 3, 4]]   # layer 1: two pivots, relations not in ascending order
RELATIONS = [{"5": [1, 2, 6]}, {"6": [0, 1], "2": [5, 7]}]


def head_data(seed=0):
    rng = np.random.default_rng(seed)
    stab = [[float(rng.uniform(0.3, 0.9)) if t in (1, 4) else -1.0 for t in row] for row in CLASSES]
    counts = {"anchor": 0, "volatile": 0, "pivot": 0, "satellite": 0}
    names = {1: "anchor", 2: "volatile", 3: "pivot", 4: "satellite"}
    for row in CLASSES:
        for t in row:
            counts[names[t]] += 1
    raw = {"meta": {"type_map": dict(workloads.TYPE_MAP), "counts": counts},
           "classification_matrix": [list(r) for r in CLASSES],
           "allocation_matrix": workloads.inverse_stability_allocation(stab),
           "leader_member_relations": [dict(r) for r in RELATIONS]}
    perms = [head_permutation(r) for r in CLASSES]
    return augment_head_data(raw, perms)


def run(dev, dtype, select_first=False, topk=None, quirks=False, L=2048, steps=10, batched=True, groups=1,
        chunks=None, tier="host", overlap=False, stream="auto", one_pass=True, budget=None, expect_tier=None):
    """tier: "host" / "device" / "auto" placement of the full-KV tier, or
    "prefill" (real_offload=False: the prefill K/V kept as the tier); with
    "auto", budget is tier_device_budget and expect_tier the placement it
    must choose.  overlap: batched checks on the side stream
    (overlap_drift_check).  stream: retrieval_stream.  one_pass:
    one_pass_drift_check.  The prefill runs as the model's attention runs it
    (prefill_stat_rows asks for no statistics at window_size 1)."""
    torch.manual_seed(0)
    B, Hq, Hkv, NL, D = 1, 32, 8, 2, 128
    data = head_data()
    cfg = HeteroCacheConfig(data=data, compression_ratio=0.5, stable_threshold=0.5, real_offload=tier != "prefill",
                            max_gen_len=steps + 4, decode_step=5, pooling="avgpool", kernel_size=5,
                            num_attn_heads=Hq, num_kv_heads=Hkv, num_layers=NL, retrieval_topk=topk,
                            reference_quirks=quirks, batched_drift_check=batched, drift_check_groups=groups,
                            tier_placement="host" if tier == "prefill" else tier, overlap_drift_check=overlap,
                            round_scores=False, retrieval_stream=stream, one_pass_drift_check=one_pass,
                            tier_device_budget=budget)
    cache = HeteroCache(cfg)
    if chunks is not None:
        cache.begin_prefill(L)

    def select(qc, kc, vc, layer):
        st = None
        W = cache.prefill_stat_rows(qc, layer)
        if W:
            st = torch.empty((B, Hq, W, 2), dtype=torch.float32, device=dev)
            ops.prefill_attn(qc, kc, vc, 1 / math.sqrt(D), stat_out=st)
        cache.init_coefficient(qc, kc, layer, stats=st)
        cache.prefill_select(qc, kc, vc, layer, stats=st)
    orc = O.CacheOracle(data, B, Hq, Hkv, NL, 0.5, 0.5, 5, "avgpool", 5, retrieval_topk=topk, quirks=quirks,
                        select_before_attention=select_first)
    g = torch.Generator().manual_seed(1)
    last_q = []
    for layer in range(NL):
        q = torch.randn((B, Hq, L, D), generator=g).to(dtype).to(dev)
        k = torch.randn((B, Hkv, L, D), generator=g).to(dtype).to(dev)
        v = torch.randn((B, Hkv, L, D), generator=g).to(dtype).to(dev)
        if chunks is None:
            kc, vc = cache.update(k, v, layer)
            select(q, kc, vc, layer)
        else:  # chunked prefill: the oracle still sees the whole prompt
            bounds = np.cumsum([0] + list(chunks))
            assert bounds[-1] == L
            for s, e in zip(bounds[:-1], bounds[1:]):
                qc = q[:, :, s:e]
                kc, vc = cache.update(k[:, :, s:e], v[:, :, s:e], layer, {"query_states": qc})
                assert kc.shape[2] == e
                select(qc, kc, vc, layer)
                assert cache.prefill_pending(layer) == (e < L)
        orc.prefill(layer, as_np(q), as_np(k), as_np(v))
        last_q.append(q[:, :, -1:].clone())
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    triggers = []
    for step in range(steps):
        for layer in range(NL):
            q = last_q[layer] if step < 5 else torch.randn((B, Hq, 1, D), generator=g).to(dtype).to(dev)
            kn = torch.randn((B, Hkv, 1, D), generator=g).to(dtype).to(dev)
            vn = torch.randn((B, Hkv, 1, D), generator=g).to(dtype).to(dev)
            cache.update(kn, vn, layer)
            if select_first:
                cache.decode_select(q, layer)
            out = cache.decode_attention(q, layer)
            if not select_first:
                cache.decode_select(q, layer)
            ref = orc.decode(layer, as_np(q), as_np(kn), as_np(vn))
            err = np.abs(as_np(out).reshape(B, Hq, D) - ref).max()
            assert err <= tol, f"step {step} layer {layer}: max-abs {err}"
        if (step + 1) % 5 == 0:
            # A deferred (batched) check has run once the last layer is done
            # (on the side stream when overlapped: wait for every stream).
            torch.cuda.synchronize()
            for layer in range(NL):
                st = cache._drift[layer]
                for i, leader in enumerate(st.leaders):
                    triggers.append((layer, leader, bool(st.trigger[i].item())))
    torch.cuda.synchronize()
    assert cache.tier_mode == (expect_tier or tier)
    # Batched checks in Llama order score in one pass from the statistics the
    # decode launches reported (every cycle, the first included).
    one_pass = one_pass and batched and not select_first
    assert cache.one_pass_checks == ((steps // 5) * groups if one_pass else 0)
    assert cache.attn_stats_layers == 0
    assert triggers == orc.triggers
    for layer in range(NL):
        store = cache.stores[layer]
        for r in range(B * Hkv):
            n = int(store.host_len[r])
            ks, vs = store.read_rows([r], n)
            ok, ov = orc.rows[layer][r]
            assert n == len(ok), (layer, r)
            assert np.array_equal(as_np(ks[0]), ok) and np.array_equal(as_np(vs[0]), ov), (layer, r)
    return triggers


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_llama_order(dev, dtype):
    trig = run(dev, dtype)
    # First check: overlap 1.0 everywhere; second: every leader retrieves.
    assert [t for _, _, t in trig] == [False] * 3 + [True] * 3


def test_llama_order_two_check_groups(dev):
    """Each layer's check as its own batched group (the second group's
    leaders start past the first global leader)."""
    trig = run(dev, torch.float32, groups=2)
    assert [t for _, _, t in trig] == [False] * 3 + [True] * 3


@pytest.mark.parametrize("groups,tier", [(1, "device"), (2, "device"), (1, "host")])
def test_llama_order_overlapped_checks(dev, groups, tier):
    """Batched checks and their retrieval on the side stream, overlapping the
    other layers' attention (overlap_drift_check): every output, trigger and
    store equals the oracle's, as on the main stream."""
    trig = run(dev, torch.float32, groups=groups, tier=tier, overlap=True)
    assert [t for _, _, t in trig] == [False] * 3 + [True] * 3


def test_llama_order_layer_by_layer_checks(dev):
    """The per-layer check path (batched_drift_check=False) gives the same
    outputs, triggers and stores."""
    trig = run(dev, torch.float32, batched=False)
    assert [t for _, _, t in trig] == [False] * 3 + [True] * 3


def test_qwen_order_select_before_attention(dev):
    run(dev, torch.float32, select_first=True)


@pytest.mark.parametrize("tier", ["device", "prefill"])
@pytest.mark.parametrize("select_first", [False, True])
def test_tier_placements(dev, tier, select_first):
    """The full-KV tier in an HBM arena, or (real_offload=False) the prefill
    K/V kept as is: same outputs, triggers and stores as the oracle, in both
    step orders (the batched check retrieves every layer of its group in
    one gather from the arena)."""
    trig = run(dev, torch.float32, select_first=select_first, topk=64, tier=tier)
    assert [t for _, _, t in trig] == [False] * 3 + [True] * 3


@pytest.mark.parametrize("tier,stream", [("device", "side"), ("host", "main")])
def test_retrieval_stream_choices(dev, tier, stream):
    """The retrieval gathers on the stream the default does not pick for the
    tier (per-layer gathers and events on the side stream for the HBM tier,
    one gather on the check's stream for the host tier): same outputs,
    triggers and stores."""
    trig = run(dev, torch.float32, topk=64, tier=tier, stream=stream)
    assert [t for _, _, t in trig] == [False] * 3 + [True] * 3


def test_two_pass_drift_check(dev):
    """one_pass_drift_check=False: the batched checks take the statistics
    pass with stored logits (no decode-reported statistics); same outputs,
    triggers and stores."""
    trig = run(dev, torch.float32, one_pass=False)
    assert [t for _, _, t in trig] == [False] * 3 + [True] * 3


@pytest.mark.parametrize("budget,expect", [(1, "host"), (1 << 40, "device")])
def test_auto_tier_placement_follows_the_budget(dev, budget, expect):
    """tier_placement="auto": the tier goes to HBM when the model's whole
    tier fits tier_device_budget bytes, to pinned host memory otherwise."""
    run(dev, torch.float32, topk=64, tier="auto", budget=budget, expect_tier=expect)


def test_retrieval_topk(dev):
    run(dev, torch.float32, topk=64)


def test_reference_quirks(dev):
    run(dev, torch.float32, quirks=True)


@pytest.mark.parametrize("chunks", [[700, 700, 648], [1024, 1023, 1]])
def test_chunked_prefill_equals_single_shot(dev, chunks):
    """A prefill staged in chunks (the last one a single token in the second
    case) selects, stores and decodes exactly as the single-shot oracle."""
    trig = run(dev, torch.float32, chunks=chunks)
    assert [t for _, _, t in trig] == [False] * 3 + [True] * 3


def test_chunked_prefill_with_observation_window_equals_single_shot(dev):
    """window_size = 8 with a last chunk shorter than the window: the kept
    query rows span two chunks; stores, reference sets and one decode step
    equal the single-shot cache's bit for bit."""
    torch.manual_seed(0)
    B, Hq, Hkv, NL, D, L = 1, 32, 8, 2, 128, 1500
    data = head_data()

    def make():
        cfg = HeteroCacheConfig(data=data, compression_ratio=0.5, stable_threshold=0.5, real_offload=True,
                                max_gen_len=4, decode_step=5, pooling="maxpool", kernel_size=7,
                                num_attn_heads=Hq, num_kv_heads=Hkv, num_layers=NL, window_size=8,
                                round_scores=False)
        return HeteroCache(cfg)

    g = torch.Generator().manual_seed(9)
    qs = [torch.randn((B, Hq, L, D), generator=g).to(dev) for _ in range(NL)]
    ks = [torch.randn((B, Hkv, L, D), generator=g).to(dev) for _ in range(NL)]
    vs = [torch.randn((B, Hkv, L, D), generator=g).to(dev) for _ in range(NL)]
    whole, chunked = make(), make()
    chunked.begin_prefill(L)
    for layer in range(NL):
        kc, vc = whole.update(ks[layer], vs[layer], layer)
        whole.init_coefficient(qs[layer], kc, layer)
        whole.prefill_select(qs[layer], kc, vc, layer)
        for s, e in ((0, 745), (745, 1497), (1497, 1500)):
            qc = qs[layer][:, :, s:e]
            kc, vc = chunked.update(ks[layer][:, :, s:e], vs[layer][:, :, s:e], layer, {"query_states": qc})
            chunked.init_coefficient(qc, kc, layer)
            chunked.prefill_select(qc, kc, vc, layer)
    q1 = torch.randn((B, Hq, 1, D), generator=g).to(dev)
    k1 = torch.randn((B, Hkv, 1, D), generator=g).to(dev)
    v1 = torch.randn((B, Hkv, 1, D), generator=g).to(dev)
    outs = []
    for cache in (whole, chunked):
        o = []
        for layer in range(NL):
            cache.update(k1, v1, layer)
            o.append(cache.decode_attention(q1, layer))
        outs.append(torch.stack(o))
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
    for layer in range(NL):
        a, b = whole.stores[layer], chunked.stores[layer]
        assert a.host_len.tolist() == b.host_len.tolist()
        for r in range(B * Hkv):
            n = int(a.host_len[r])
            ka, va = a.read_rows([r], n)
            kb, vb = b.read_rows([r], n)
            assert torch.equal(ka, kb) and torch.equal(va, vb), (layer, r)
        if whole._drift[layer].ref_bits is not None:
            assert torch.equal(whole._drift[layer].ref_bits, chunked._drift[layer].ref_bits)


@pytest.mark.parametrize("one_pass", [True, False])
@pytest.mark.parametrize("dtype,io,step", [(torch.bfloat16, "bfloat16", 2.0 ** -7), (torch.float16, "float16", 2.0 ** -10)])
def test_reference_cast_chain(dev, dtype, io, step, one_pass):
    """round_scores=True (the reference's casts of logits, probabilities and
    pooled scores to the model dtype) on a bfloat16 model and on a float16
    one (the reference's load dtype), the drift checks in one pass over the
    pivot keys: the device scores equal the oracle's
    cast chain to within one step of that dtype; the oracle's
    integer flow run on the device scores reproduces the
    triggers and the stores bit for bit, and the attention outputs match
    the float64 closed form.  The cast scores tie massively, so this also
    exercises the lowest-position tie rule of every selection.  one_pass
    False: the checks take the two-pass scorer (statistics pass with stored
    logits) instead."""
    from tests.test_configs_full_gpu import DeviceScores, Recorder
    B, Hq, Hkv, NL, D, L, steps = 1, 32, 8, 2, 128, 2048, 10
    data = head_data()
    cfg = HeteroCacheConfig(data=data, compression_ratio=0.5, stable_threshold=0.5, real_offload=True,
                            max_gen_len=steps + 4, decode_step=5, pooling="avgpool", kernel_size=5,
                            num_attn_heads=Hq, num_kv_heads=Hkv, num_layers=NL, round_scores=True,
                            one_pass_drift_check=one_pass)
    cache = HeteroCache(cfg)
    rec = Recorder(range(NL))
    cache.observer = rec
    hook = DeviceScores(rec, 0.5)
    orc = O.CacheOracle(data, B, Hq, Hkv, NL, 0.5, 0.5, 5, "avgpool", 5, score_hook=hook, io_dtype=io)
    hook.orc = orc
    g = torch.Generator().manual_seed(3)
    last_q = []
    for layer in range(NL):
        q = torch.randn((B, Hq, 1, D), generator=g).to(dtype).to(dev)
        k = torch.randn((B, Hkv, L, D), generator=g).to(dtype).to(dev)
        v = torch.randn((B, Hkv, L, D), generator=g).to(dtype).to(dev)
        kc, vc = cache.update(k, v, layer)
        cache.init_coefficient(q, kc, layer)
        cache.prefill_select(q, kc, vc, layer)
        orc.prefill(layer, as_np(q), as_np(k), as_np(v))
        last_q.append(q)
    for step in range(steps):
        outs = []
        for layer in range(NL):
            q = last_q[layer] if step < 5 else torch.randn((B, Hq, 1, D), generator=g).to(dtype).to(dev)
            kn = torch.randn((B, Hkv, 1, D), generator=g).to(dtype).to(dev)
            vn = torch.randn((B, Hkv, 1, D), generator=g).to(dtype).to(dev)
            cache.update(kn, vn, layer)
            outs.append((cache.decode_attention(q, layer), q, kn, vn))
            cache.decode_select(q, layer)
        # The device checks this step's layers after the last one; the oracle follows.
        for layer, (out, q, kn, vn) in enumerate(outs):
            ref = orc.decode(layer, as_np(q), as_np(kn), as_np(vn))
            assert np.abs(as_np(out).reshape(B, Hq, D) - ref).max() <= 2e-2
    torch.cuda.synchronize()
    # With one_pass, both checks scored in one pass, from the cast chain's
    # statistics that the decode launches reported.
    assert cache.one_pass_checks == (steps // 5 if one_pass else 0)
    flags = [(l, h, c[(l, h)]) for c in rec.checks for l in range(NL) for h in cache._drift[l].leaders]
    assert flags == orc.triggers and [f for *_, f in flags] == [False] * 3 + [True] * 3
    assert max(e for *_, e in hook.err) <= step * 1.01
    for layer in range(NL):
        store = cache.stores[layer]
        for r in range(B * Hkv):
            n = int(store.host_len[r])
            ks, vs = store.read_rows([r], n)
            ok, ov = orc.rows[layer][r]
            assert n == len(ok) and np.array_equal(as_np(ks[0]), ok) and np.array_equal(as_np(vs[0]), ov)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_observation_window_from_attention_statistics(dev, dtype):
    """window_size = 32 (128 query rows per KV head): prefill_select scores
    from the prefill attention's statistics (one key pass) as the patched
    attention hands them over.  The scores are within 2e-5 of the two-pass
    scorer's on the same inputs and within 2e-4 of the oracle's window
    scores, and the two caches' stores are identical on this seed."""
    B, Hq, Hkv, NL, D, L, W = 1, 32, 8, 2, 128, 3000, 32
    data = head_data()
    seen = {}

    def make(tag):
        cfg = HeteroCacheConfig(data=data, compression_ratio=0.5, stable_threshold=0.5, real_offload=True,
                                max_gen_len=4, decode_step=5, pooling="maxpool", kernel_size=7,
                                num_attn_heads=Hq, num_kv_heads=Hkv, num_layers=NL, window_size=W,
                                attention_stats_scoring=tag == "stats", round_scores=False)
        cache = HeteroCache(cfg)
        cache.observer = lambda event, **kw: seen.setdefault((tag, event, kw.get("layer")), kw.get("scores"))
        return cache

    g = torch.Generator().manual_seed(21)
    qs = [torch.randn((B, Hq, L, D), generator=g).to(dtype).to(dev) for _ in range(NL)]
    ks = [torch.randn((B, Hkv, L, D), generator=g).to(dtype).to(dev) for _ in range(NL)]
    vs = [torch.randn((B, Hkv, L, D), generator=g).to(dtype).to(dev) for _ in range(NL)]
    caches = {"stats": make("stats"), "two_pass": make("two_pass")}
    for tag, cache in caches.items():
        for layer in range(NL):
            kc, vc = cache.update(ks[layer], vs[layer], layer)
            st = None
            n = cache.prefill_stat_rows(qs[layer], layer)
            assert n == (W if tag == "stats" else 0)
            if n:
                st = torch.empty((B, Hq, n, 2), dtype=torch.float32, device=dev)
                ops.prefill_attn(qs[layer], kc, vc, 1 / math.sqrt(D), stat_out=st)
            cache.init_coefficient(qs[layer], kc, layer, stats=st)
            cache.prefill_select(qs[layer], kc, vc, layer, stats=st)
    torch.cuda.synchronize()
    assert caches["stats"].attn_stats_layers == NL and caches["two_pass"].attn_stats_layers == 0
    G = Hq // Hkv
    for layer in range(NL):
        s1 = as_np(seen[("stats", "prefill_select", layer)])
        s0 = as_np(seen[("two_pass", "prefill_select", layer)])
        assert np.abs(s1 - s0).max() / np.abs(s0).max() < 2e-5
        qn, kn = as_np(qs[layer]), as_np(ks[layer])
        n_c = data["need_to_compress_counts"][layer]
        ref = O.window_scores(np.stack([qn[0, h * G:(h + 1) * G, -W:] for h in range(n_c)]), kn[0, :n_c], "maxpool",
                              7, window_keep=True)
        assert np.abs(s1 - ref).max() / np.abs(ref).max() < 2e-4
        a, b = caches["stats"].stores[layer], caches["two_pass"].stores[layer]
        assert np.array_equal(a.host_len, b.host_len)
        for r in range(B * Hkv):
            m = int(a.host_len[r])
            ka, va = a.read_rows([r], m)
            kb, vb = b.read_rows([r], m)
            assert torch.equal(ka, kb) and torch.equal(va, vb), (layer, r)
