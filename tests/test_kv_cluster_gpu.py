"""Baseline compressors (SnapKV, PyramidKV, H2O, StreamingLLM, CAKE) on the
libhc kernels vs the oracle's restatements of heterocache/kv_cluster.py.

Keys and values arrive repeated per query head, as the reference's callers
pass them (CAKE: one row per KV head, as its cache holds them).  Channel 127 of V holds each token's position, so the kept
positions are read back from the gathered rows.  Kept sets must equal the
oracle's except inside the tie band around the budget threshold (float32
noise, or one bf16 ulp with the reference's casts); gathered rows are exact
copies.  The reference returns kept rows in top-k order, these in ascending
position order (attention over them is the same).
"""
import numpy as np
import pytest
import torch

from heterocache_amd import kv_cluster
from oracle import hc_oracle as O
from tests.gpu_util import as_np

pytestmark = pytest.mark.gpu


def _inputs(dev, B, H, L, seed, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, L, 128, generator=g)
    k = torch.randn(B, H, L, 128, generator=g)
    k[..., :4] *= 4
    v = torch.randn(B, H, L, 128, generator=g)
    v[..., 127] = torch.arange(L, dtype=torch.float32)
    if dtype != torch.float32:
        q, k = q.to(dtype), k.to(dtype)
        v = v.to(dtype)
        v[..., 127] = 0  # positions are only exact in float32; read them from K instead
    return q.to(dev), k.to(dev), v.to(dev)


def _positions(kout, vout, kin):
    """Kept positions per (b, h), ascending, from the gathered rows."""
    if vout.dtype == torch.float32:
        return as_np(vout[..., 127]).astype(np.int64)
    # Match K rows back to the source (rows are exact copies).
    kin_np, kout_np = as_np(kin), as_np(kout)
    B, H = kin.shape[:2]
    pos = np.zeros(kout.shape[:3], dtype=np.int64)
    for b in range(B):
        for h in range(H):
            lookup = {kin_np[b, h, t].tobytes(): t for t in range(kin.shape[2])}
            pos[b, h] = [lookup[r.tobytes()] for r in kout_np[b, h]]
    return pos


def _check_kept(got, ref, body_scores, keep, tol):
    """got/ref: kept positions of one head (ref in any order)."""
    assert len(got) == len(ref)
    assert np.all(np.diff(got) > 0), "positions must be ascending"
    diff = set(got.tolist()).symmetric_difference(np.asarray(ref).tolist())
    if not diff:
        return
    tau = np.sort(body_scores)[::-1][keep - 1]
    assert all(abs(body_scores[t] - tau) <= tol(tau) for t in diff), sorted(diff)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_snapkv_cluster(dev, dtype):
    B, H, L, W, G = 1, 8, 1024, 32, 4
    print(f"snapkv dtype={dtype}", flush=True)
    q, k, v = _inputs(dev, B, H, L, 31, dtype)
    cl = kv_cluster.SnapKVCluster(window_size=W, compression_ratio=0.5, kernel_size=7, pooling="maxpool")
    ko, vo = cl.update_kv(k, q, v, None, G)
    torch.cuda.synchronize()
    cap = max(int(0.5 * L / G), 2)
    assert ko.shape == (B, H, cap, 128)
    io = {torch.float32: None, torch.bfloat16: "bfloat16", torch.float16: "float16"}[dtype]
    pos = _positions(ko, vo, k)
    qn, kn = as_np(q), as_np(k)
    for h in range(H):
        s = O.window_scores(qn[0, h][None, None, -W:], kn[0, h][None], "maxpool", 7, window_keep=True, io_dtype=io)[0]
        ref = O.select_with_window(s, cap, L, W)
        tol = (lambda tau: 1e-5 * abs(tau)) if io is None else (lambda tau: abs(tau) * 2.0 ** -7)
        _check_kept(pos[0, h], ref, s, cap - W, tol)
        assert pos[0, h, -W:].tolist() == list(range(L - W, L))
        assert torch.equal(ko[0, h], k[0, h, torch.as_tensor(pos[0, h], device=dev)])


@pytest.mark.parametrize("layer", [0, 5, 31])
def test_pyramidkv_cluster(dev, layer):
    B, H, L, W, G, NL = 2, 4, 2048, 32, 4, 32
    print(f"pyramidkv layer={layer}", flush=True)
    q, k, v = _inputs(dev, B, H, L, 40 + layer)
    cl = kv_cluster.PyramidKVCluster(num_hidden_layers=NL, window_size=W, compression_ratio=0.5, kernel_size=5,
                                     pooling="avgpool", layer_idx=layer)
    ko, vo = cl.update_kv(k, q, v, None, G)
    torch.cuda.synchronize()
    keep = O.pyramidkv_layer_capacity(int(0.5 * L / G), L, W, 20, NL, layer)
    assert ko.shape == (B, H, keep + W, 128)
    pos = _positions(ko, vo, k)
    qn, kn = as_np(q), as_np(k)
    for b in range(B):
        for h in range(H):
            s = O.window_scores(qn[b, h][None, None, -W:], kn[b, h][None], "avgpool", 5, window_keep=True)[0]
            ref = np.concatenate([O.topk_indices(s, keep), np.arange(L - W, L)])
            _check_kept(pos[b, h], ref, s, keep, lambda tau: 1e-5 * abs(tau))


def test_h2o_cluster(dev):
    """530 float32 query rows: four 128-row scorer calls (probability pass),
    then 16- and 2-row ones (logit-store pass), accumulated into one score
    row."""
    B, H, L, G = 1, 4, 530, 2
    print("h2o", flush=True)
    q, k, v = _inputs(dev, B, H, L, 50)
    cl = kv_cluster.H2OKVCluster(compression_ratio=0.5)
    scores = cl.heavy_hitter_scores(k, q)
    ko, vo = cl.update_kv(k, q, v, None, G)
    torch.cuda.synchronize()
    ref_s = O.h2o_scores(as_np(q), as_np(k))
    got_s = as_np(scores).reshape(B, H, L)
    assert np.max(np.abs(got_s - ref_s) / np.maximum(np.abs(ref_s), 1e-6)) < 2e-4
    cap = max(int(0.5 * L / G), 2)
    assert ko.shape == (B, H, cap, 128)
    _, _, top = O.h2o_update_kv(as_np(k), as_np(q), as_np(v), 0.5, G)
    pos = _positions(ko, vo, k)
    for h in range(H):
        _check_kept(pos[0, h], top[0, h], ref_s[0, h], cap, lambda tau: 1e-5 * abs(tau))


def test_streamingllm_cluster(dev):
    B, H, L = 2, 3, 1000
    q, k, v = _inputs(dev, B, H, L, 60)
    ko, vo = kv_cluster.StreamingLLMKVCluster(compression_ratio=0.3).update_kv(k, q, v, None, 1)
    torch.cuda.synchronize()
    rk, rv = O.streamingllm_update_kv(as_np(k), as_np(v), 0.3)
    assert np.array_equal(as_np(ko), rk) and np.array_equal(as_np(vo), rv)


def test_short_prompts_stay_uncompressed(dev):
    q, k, v = _inputs(dev, 1, 2, 40, 70)
    for cl in (kv_cluster.SnapKVCluster(window_size=8, compression_ratio=2.0),
               kv_cluster.H2OKVCluster(compression_ratio=2.0),
               kv_cluster.StreamingLLMKVCluster(compression_ratio=2.0)):
        ko, vo = cl.update_kv(k, q, v, None, 1)
        assert ko is k and vo is v


@pytest.mark.parametrize("dtype,Hq,Hkv", [(torch.float32, 4, 2), (torch.bfloat16, 4, 2), (torch.bfloat16, 7, 1),
                                         (torch.float16, 4, 2)])
def test_cake_scores(dev, dtype, Hq, Hkv):
    """hc_cake_score vs the oracle: heavy-hitter scores, entropy, variance sum
    and preference of one layer (keys not repeated; bf16 with the
    reference's casts: agreement to about one bf16 ulp)."""
    from heterocache_amd import compress
    g = torch.Generator().manual_seed(21)
    B, L, W = 2, 700, 32
    q = torch.randn(B, Hq, L, 128, generator=g).to(dtype)
    k = torch.randn(B, Hkv, L, 128, generator=g)
    k[..., :4] *= 4
    k = k.to(dtype)
    io = {torch.float32: None, torch.bfloat16: "bfloat16", torch.float16: "float16"}[dtype]
    hh, stats = compress.cake_scores(q.to(dev), k.to(dev), W, round_dtype=None if io is None else dtype)
    ref_hh, ent, var_sum, pref = O.cake_layer_scores(q.float().numpy(), k.float().numpy(), W, io_dtype=io)
    got = as_np(hh).reshape(B, Hkv, L - W)
    st = as_np(stats).astype(np.float64)
    if io is None:
        np.testing.assert_allclose(got, ref_hh, rtol=1e-4, atol=1e-8)
        tol = 1e-4
    elif io == "bfloat16":
        np.testing.assert_allclose(got, ref_hh, rtol=1.6e-2, atol=1e-6)
        tol = 1e-2
    else:  # float16: ulp 2^-11 relative, but subnormals below 6e-5 (the probabilities of a 700-key row)
        np.testing.assert_allclose(got, ref_hh, rtol=4e-3, atol=2e-7)
        tol = 2e-3
    assert st[0] == pytest.approx(ent, rel=tol)
    assert st[1] == pytest.approx(var_sum, rel=tol)
    assert st[2] == pytest.approx(pref, rel=2 * tol)


def test_cake_cache_prefill_matches_oracle(dev):
    """Three layers through CAKECache.update: layer budgets equal the
    oracle's, every layer keeps the oracle's positions (tie band aside) plus
    the window, in position order, as exact row copies; the prefill
    attention sees the whole prompt."""
    from heterocache_amd.cache_utils import CAKECache, CompressionCacheConfig
    B, Hq, Hkv, L, W, NL, ratio = 1, 4, 2, 600, 32, 3, 0.3
    cache = CAKECache(CompressionCacheConfig(window_size=W, compression_ratio=ratio, num_attn_heads=Hq,
                                             num_kv_heads=Hkv, num_layers=NL))
    layers = []
    for layer in range(NL):
        g = torch.Generator().manual_seed(30 + layer)
        q = torch.randn(B, Hq, L, 128, generator=g)
        k = torch.randn(B, Hkv, L, 128, generator=g)
        k[..., :4] *= 4
        v = torch.randn(B, Hkv, L, 128, generator=g)
        v[..., 127] = torch.arange(L, dtype=torch.float32)
        layers.append((q.numpy(), k.numpy()))
        ko, vo = cache.update(k.to(dev), v.to(dev), layer,
                              {"query_states": q.to(dev), "num_key_value_groups": Hq // Hkv, "attention_mask": None})
        assert ko.shape == (B, Hkv, L, 128)
    kept, budgets, prefs = O.cake_prefill(layers, ratio, W, NL)
    assert cache.layer_budget == budgets
    np.testing.assert_allclose(np.array(cache.pref_scores, np.float64), np.array(prefs, np.float64), rtol=1e-3)
    for layer in range(NL):
        hh, _, _, _ = O.cake_layer_scores(*layers[layer], W)
        pos = as_np(cache.value_cache[layer][..., 127]).astype(np.int64)
        n = kept[layer].shape[-1]
        assert pos.shape == (B, Hkv, n + W)
        for h in range(Hkv):
            got = pos[0, h]
            np.testing.assert_array_equal(got[n:], np.arange(L - W, L))
            _check_kept(got[:n], kept[layer][0, h], hh[0, h], n, lambda tau: 1e-4 * abs(tau) + 1e-9)
            np.testing.assert_array_equal(as_np(cache.key_cache[layer][0, h]), layers[layer][1][0, h][got])
