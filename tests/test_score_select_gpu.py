"""hc_score and hc_select_topk against the oracle.

Scores: float32 chain within rtol 2e-4 of the float64-evaluated oracle on the
same (dtype-rounded) inputs; bf16 cast chain within one bf16 ulp with >= 97%
exact.  Selection: bit-exact against the oracle's (-score, index) ranking on
the SAME score array (ties included).  End to end (GPU scores -> GPU
selection vs oracle scores -> oracle selection): identical except for
positions whose oracle score lies within 1e-5 (relative) of the budget
threshold.
"""
import math

import numpy as np
import pytest
import torch

from heterocache_amd import compress, ops
from heterocache_amd.store import KVStore
from oracle import hc_oracle as O
from tests.gpu_util import TORCH_DT, as_np

pytestmark = pytest.mark.gpu


def qk(dev, B, Hq, Hkv, Lq, L, dtype, seed, strided=True, sinks=False):
    g = torch.Generator().manual_seed(seed)
    if strided:  # the projection layout: [B, L, H, d].transpose(1, 2)
        q = torch.randn((B, Lq, Hq, 128), generator=g).to(dtype).to(dev).transpose(1, 2)
        k = torch.randn((B, L, Hkv, 128), generator=g).to(dtype).to(dev).transpose(1, 2)
    else:
        q = torch.randn((B, Hq, Lq, 128), generator=g).to(dtype).to(dev)
        k = torch.randn((B, Hkv, L, 128), generator=g).to(dtype).to(dev)
    if sinks:
        k = k.clone()
        k[:, :, :4] = 2 * q[:, ::Hq // Hkv, -1:].mean(dim=2, keepdim=True)[:, :Hkv].to(dtype)
    return q, k


def rel_err(a, b):
    return np.abs(a - b).max() / max(np.abs(b).max(), 1e-30)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
@pytest.mark.parametrize("pooling,kernel", [("avgpool", 5), ("maxpool", 7)])
def test_last_query_scores(dev, dtype, pooling, kernel):
    B, Hq, Hkv, L = 1, 32, 8, 3000
    q, k = qk(dev, B, Hq, Hkv, L, L, dtype, 1, sinks=True)
    heads = [0, 1, 2, 5, 7]
    s = compress.last_query_scores(q, k, heads, 4, pooling, kernel)
    qn, kn = as_np(q), as_np(k)
    ref = O.last_query_scores(np.stack([qn[0, h * 4:(h + 1) * 4, -1] for h in heads]), kn[0, heads], pooling, kernel)
    assert s.shape == (len(heads), L)
    assert rel_err(as_np(s), ref) < 2e-4


def test_last_query_scores_batch_and_gqa7(dev):
    B, Hq, Hkv, L = 2, 28, 4, 1500
    q, k = qk(dev, B, Hq, Hkv, L, L, torch.bfloat16, 2)
    s = compress.last_query_scores(q, k, range(Hkv), 7, "avgpool", 5)
    qn, kn = as_np(q), as_np(k)
    for b in range(B):
        ref = O.last_query_scores(np.stack([qn[b, h * 7:(h + 1) * 7, -1] for h in range(Hkv)]), kn[b], "avgpool", 5)
        assert rel_err(as_np(s[b * Hkv:(b + 1) * Hkv]), ref) < 2e-4


@pytest.mark.parametrize("G,W", [(4, 32), (1, 32), (4, 16), (2, 8), (4, 4)])
def test_snapkv_window_scores(dev, G, W):
    B, Hkv, L = 1, 3, 2000
    q, k = qk(dev, B, Hkv * G, Hkv, L, L, torch.float32, 3)
    s = compress.window_scores(q, k, range(Hkv), G, W, "maxpool", 7, window_keep=True)
    qn, kn = as_np(q), as_np(k)
    qw = np.stack([qn[0, h * G:(h + 1) * G, -W:] for h in range(Hkv)])
    ref = O.window_scores(qw, kn[0], "maxpool", 7, window_keep=True)
    assert s.shape == (Hkv, L - W)
    assert rel_err(as_np(s), ref) < 2e-4


def test_bf16_cast_chain(dev):
    B, Hq, Hkv, L = 1, 32, 8, 4096
    q, k = qk(dev, B, Hq, Hkv, L, L, torch.bfloat16, 4)
    s = as_np(compress.last_query_scores(q, k, range(Hkv), 4, "avgpool", 5, round_dtype=torch.bfloat16))
    qn, kn = as_np(q), as_np(k)
    ref = O.last_query_scores(np.stack([qn[0, h * 4:(h + 1) * 4, -1] for h in range(Hkv)]), kn[0], "avgpool", 5,
                              io_dtype="bfloat16")
    assert np.array_equal(s, O.round_bf16(s)), "scores must be bf16 values"
    rel = np.abs(s - ref) / np.maximum(np.abs(ref), 1e-30)
    assert rel.max() <= 2.0 ** -7 + 1e-9
    assert (s == ref).mean() >= 0.97


def test_pivot_step_scores_read_store_in_place(dev):
    B, Hq, Hkv, L, S, G = 1, 32, 8, 2500, 5, 4
    q, k = qk(dev, B, Hq, Hkv, 1, L, torch.bfloat16, 5, strided=False)
    steps = torch.randn((B, Hq, S, 128), generator=torch.Generator().manual_seed(6)).to(torch.bfloat16).to(dev)
    store = KVStore([L + 64] * Hkv, torch.bfloat16, dev)
    store.write_rows(k, k, [(0, h) for h in range(Hkv)], list(range(Hkv)), [L] * Hkv)
    pivots = [6, 7]
    s = compress.pivot_step_scores(steps, store, pivots, pivots, G, L, "avgpool", 5)
    sn, kn = as_np(steps), as_np(k)
    for j, h in enumerate(pivots):
        ref = O.pivot_step_scores(sn[0, h * G:(h + 1) * G], kn[0, h], "avgpool", 5)
        assert rel_err(as_np(s[j]), ref) < 2e-4


@pytest.mark.parametrize("L,pooling,kernel", [(4099, "avgpool", 7), (4099, "maxpool", 5), (300, "avgpool", 1),
                                               (1000, "maxpool", 9), (131072, "avgpool", 7)])
def test_score_given_stats(dev, L, pooling, kernel):
    """hc_score_given_stats: drift scores of S buffered queries per pivot in
    one key pass, (a) with the oracle's float64 normalisers as the statistics
    and (b) with the statistics the decode launches of the S steps reported
    (hc_decode_attn_stats over the prompt of L keys): both within 2e-4 of the
    oracle's scores, and (b) within 1e-5 of the two-pass scorer's."""
    from heterocache_amd import ops
    B, Hq, Hkv, S, G = 2, 16, 4, 5, 4
    rng = np.random.default_rng(L + kernel)
    k = torch.as_tensor(rng.standard_normal((B, Hkv, L, 128)), dtype=torch.float32)
    k[..., :4] *= 5
    k = k.to(torch.bfloat16).to(dev)
    steps = torch.as_tensor(rng.standard_normal((B, Hq, S, 128)), dtype=torch.float32).to(torch.bfloat16).to(dev)
    store = KVStore([L + 64] * (B * Hkv), torch.bfloat16, dev)
    store.write_rows(k, k, [(b, h) for b in range(B) for h in range(Hkv)], list(range(B * Hkv)), [L] * (B * Hkv))
    pivots = [(0, 1), (0, 3), (1, 0), (1, 3)]
    rows = [b * Hkv + h for b, h in pivots]
    q_off, k_row = compress.pivot_step_metadata(steps, store, rows, [h for _, h in pivots], G)
    scale = 1 / math.sqrt(128)
    sn, kn = as_np(steps), as_np(k)
    refs = [O.pivot_step_scores(sn[b, h * G:(h + 1) * G], kn[b, h], pooling, kernel) for b, h in pivots]
    # (a) the oracle's normalisers: M = lse2, L = 1.
    st = np.zeros((len(pivots), G * S, 2), dtype=np.float32)
    for j, (b, h) in enumerate(pivots):
        qr = sn[b, h * G:(h + 1) * G].reshape(1, G * S, 128)  # rows g*S + w
        st[j, :, 0] = O.softmax_lse2(qr, [kn[b, h]], L, scale)[0]
        st[j, :, 1] = 1.0
    stats = torch.tensor(st).to(dev)
    st_off = torch.arange(len(pivots), dtype=torch.int64, device=dev) * (G * S * 2)
    got = ops.score_given_stats(steps, q_off, steps.stride(1), steps.stride(2), store.k, store.row_tile_off, k_row,
                                L, G, S, pooling, kernel, scale, stats, st_off)
    for j in range(len(pivots)):
        assert rel_err(as_np(got[j]), refs[j]) < 2e-4, j
    # (b) statistics from the S decode launches over the stored prompt.
    dstats = torch.full((B * Hkv, G, S, 2), float("nan"), dtype=torch.float32, device=dev)
    for w in range(S):
        qw = steps[:, :, w].reshape(B * Hkv, G, 128).contiguous()
        store.attend(qw, scale, stat_len=L, stat_out=dstats[:, :, w])
    st_off = torch.tensor(rows, dtype=torch.int64, device=dev) * (G * S * 2)
    got2 = ops.score_given_stats(steps, q_off, steps.stride(1), steps.stride(2), store.k, store.row_tile_off, k_row,
                                 L, G, S, pooling, kernel, scale, dstats, st_off)
    two_pass = compress.pivot_step_scores(steps, store, rows, [h for _, h in pivots], G, L, pooling, kernel)
    torch.cuda.synchronize()
    for j in range(len(pivots)):
        assert rel_err(as_np(got2[j]), refs[j]) < 2e-4, j
        assert rel_err(as_np(got2[j]), as_np(two_pass[j])) < 1e-5, j


@pytest.mark.parametrize("dt,L,pooling,kernel", [("bf16", 4099, "avgpool", 5), ("f16", 4099, "maxpool", 7),
                                                  ("f16", 131072, "avgpool", 5), ("bf16", 300, "avgpool", 1)])
def test_score_given_stats_cast_chain(dev, dt, L, pooling, kernel):
    """hc_score_given_stats under the reference's cast chain (flags
    HC_SCORE_ROUND_*), with the statistics the S decode launches reported
    under the same flag: every score within two steps of the model dtype of
    the oracle's cast-chain scores and of the two-pass cast-chain scorer's
    (the statistics' summation order may move a probability, and then its
    pooled value, across a rounding boundary), and over 99 % of them equal
    to the two-pass scores."""
    B, Hq, Hkv, S, G = 1, 16, 4, 5, 4
    tdt = TORCH_DT[dt]
    io = {"bf16": "bfloat16", "f16": "float16"}[dt]
    flags = compress.ROUND_FLAGS[tdt]
    rng = np.random.default_rng(L + kernel + 7)
    k = torch.as_tensor(rng.standard_normal((B, Hkv, L, 128)), dtype=torch.float32)
    k[..., :4] *= 5
    k = k.to(tdt).to(dev)
    steps = torch.as_tensor(rng.standard_normal((B, Hq, S, 128)), dtype=torch.float32).to(tdt).to(dev)
    store = KVStore([L + 64] * (B * Hkv), tdt, dev)
    store.write_rows(k, k, [(0, h) for h in range(Hkv)], list(range(Hkv)), [L] * Hkv)
    pivots = [1, 3]
    q_off, k_row = compress.pivot_step_metadata(steps, store, pivots, pivots, G)
    scale = 1 / math.sqrt(128)
    dstats = torch.full((B * Hkv, G, S, 2), float("nan"), dtype=torch.float32, device=dev)
    for w in range(S):
        qw = steps[:, :, w].reshape(B * Hkv, G, 128).contiguous()
        store.attend(qw, scale, stat_len=L, stat_out=dstats[:, :, w], stat_flags=flags)
    st_off = torch.tensor(pivots, dtype=torch.int64, device=dev) * (G * S * 2)
    got = ops.score_given_stats(steps, q_off, steps.stride(1), steps.stride(2), store.k, store.row_tile_off, k_row,
                                L, G, S, pooling, kernel, scale, dstats, st_off, flags=flags)
    two_pass = compress.pivot_step_scores(steps, store, pivots, pivots, G, L, pooling, kernel, round_dtype=tdt)
    torch.cuda.synchronize()
    sn, kn = as_np(steps), as_np(k)
    for j, h in enumerate(pivots):
        g, t = as_np(got[j]), as_np(two_pass[j])
        ref = O.pivot_step_scores(sn[0, h * G:(h + 1) * G], kn[0, h], pooling, kernel, io_dtype=io)
        tol = 2 * dtype_spacing(ref, dt)
        assert np.all(np.abs(g - ref) <= tol), (j, (np.abs(g - ref) / tol).max())
        assert np.all(np.abs(g - t) <= tol), (j, (np.abs(g - t) / tol).max())
        assert np.mean(g == t) > 0.99, (j, np.mean(g == t))


def dtype_spacing(x, dt):
    """Step of the model dtype at |x| (float16: its subnormal step near 0)."""
    x = np.abs(np.asarray(x, dtype=np.float64))
    if dt == "f16":
        return np.spacing(x.astype(np.float16)).astype(np.float64)
    e = np.floor(np.log2(np.maximum(x, 2.0 ** -126)))
    return 2.0 ** (e - 7)


# -- selection --------------------------------------------------------------------
def check_select(scores_np, caps, window, idx, counts):
    span = scores_np.shape[1]
    for j, cap in enumerate(caps):
        if window:
            body = O.topk_select(scores_np[j], min(max(cap - window, 0), span))
            ref = np.concatenate([body, np.arange(span, span + window)])
        else:
            ref = O.topk_select(scores_np[j], min(cap, span))
        assert counts[j] == len(ref), (j, counts[j], len(ref))
        assert np.array_equal(idx[j, :len(ref)], ref), f"job {j}: kept set differs"


@pytest.mark.parametrize("quant", [None, 1e-3, 0.25])
def test_select_bit_exact_with_ties(dev, quant):
    rng = np.random.default_rng(7)
    span = 10007
    s = rng.random((6, span)).astype(np.float32)
    if quant:  # heavy ties
        s = (np.round(s / quant) * quant).astype(np.float32)
    s[0, 100:200] = 0.0
    caps = [0, 1, 37, 5000, span, span + 5]
    st = torch.tensor(s).to(dev)
    idx, counts = compress.select_kept(st, caps)
    check_select(s, caps, 0, as_np(idx).astype(np.int64), as_np(counts).astype(np.int64))


def test_select_window_mode(dev):
    rng = np.random.default_rng(8)
    span, W = 4000, 32
    s = rng.random((3, span)).astype(np.float32)
    caps = [W, 1000, span + W]
    idx, counts = compress.select_kept(torch.tensor(s).to(dev), caps, window=W)
    check_select(s, caps, W, as_np(idx).astype(np.int64), as_np(counts).astype(np.int64))


def test_select_all_equal_scores(dev):
    s = np.full((2, 3000), 0.125, np.float32)
    idx, counts = compress.select_kept(torch.tensor(s).to(dev), [1500, 7])
    assert as_np(idx)[0, :1500].tolist() == list(range(1500))
    assert as_np(idx)[1, :7].tolist() == list(range(7))


def test_end_to_end_indices_outside_tie_band(dev):
    """GPU scores + GPU selection vs oracle scores + oracle selection."""
    B, Hq, Hkv, L = 1, 32, 8, 4096
    q, k = qk(dev, B, Hq, Hkv, L, L, torch.float32, 9, sinks=True)
    caps = [1024, 3072, 1024, 3072, 1024, 1024, 3072, 3072]
    s = compress.last_query_scores(q, k, range(Hkv), 4, "maxpool", 7)
    idx, counts = compress.select_kept(s, caps)
    qn, kn = as_np(q), as_np(k)
    ref_s = O.last_query_scores(np.stack([qn[0, h * 4:(h + 1) * 4, -1] for h in range(Hkv)]), kn[0], "maxpool", 7)
    idx, counts = idx.cpu().numpy(), counts.cpu().numpy()
    for h in range(Hkv):
        got = set(idx[h, :counts[h]].tolist())
        ref = O.topk_select(ref_s[h], caps[h])
        tau = np.sort(ref_s[h])[::-1][caps[h] - 1]
        diff = got.symmetric_difference(ref.tolist())
        band = [t for t in diff if abs(ref_s[h][t] - tau) > 1e-5 * abs(tau)]
        assert not band, f"head {h}: {len(band)} positions differ outside the tie band"
        assert len(diff) <= 0.01 * caps[h]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("B,Hkv,G,W,Ws,heads", [(1, 3, 4, 32, 32, (0, 1, 2)), (2, 4, 4, 32, 64, (1, 3)),
                                                (1, 2, 7, 32, 32, (0, 1)), (1, 2, 1, 16, 16, (0, 1)),
                                                (2, 2, 2, 8, 8, (1,))])
def test_window_scores_with_attention_stats(dev, dtype, B, Hkv, G, W, Ws, heads):
    """Window scores and last-query scores with the prefill attention's
    statistics (one key pass) against the oracle (2e-4) and against the
    two-pass scorer on the same inputs (2e-5)."""
    from heterocache_amd import ops
    L = 2500
    if dtype == torch.float32 and G * W > 128:
        pytest.skip("float32 scoring holds at most 128 query rows")
    print(f"window scores with stats dtype={dtype} B={B} Hkv={Hkv} G={G} W={W} Ws={Ws} heads={heads}", flush=True)
    q, k = qk(dev, B, Hkv * G, Hkv, L, L, dtype, 11 + G + W, sinks=True)
    v = torch.randn(k.shape, generator=torch.Generator().manual_seed(12)).to(dtype).to(dev)
    scale = 1 / math.sqrt(128)
    st = torch.full((B, Hkv * G, Ws, 2), float("nan"), dtype=torch.float32, device=dev)
    ops.prefill_attn(q, k, v, scale, stat_out=st)
    s1 = compress.window_scores(q, k, heads, G, W, "maxpool", 7, window_keep=True, stats=st)
    s0 = compress.window_scores(q, k, heads, G, W, "maxpool", 7, window_keep=True)
    l1 = compress.last_query_scores(q, k, heads, G, "avgpool", 5, stats=st)
    l0 = compress.last_query_scores(q, k, heads, G, "avgpool", 5)
    torch.cuda.synchronize()
    qn, kn = as_np(q), as_np(k)
    for b in range(B):
        for j, h in enumerate(heads):
            r = b * len(heads) + j
            ref = O.window_scores(qn[b, h * G:(h + 1) * G, -W:][None], kn[b, h][None], "maxpool", 7,
                                  window_keep=True)[0]
            assert rel_err(as_np(s1[r]), ref) < 2e-4, (b, h)
            lref = O.last_query_scores(qn[b, h * G:(h + 1) * G, -1][None], kn[b, h][None], "avgpool", 5)[0]
            assert rel_err(as_np(l1[r]), lref) < 2e-4, (b, h)
    assert rel_err(as_np(s1), as_np(s0)) < 2e-5
    assert rel_err(as_np(l1), as_np(l0)) < 2e-5


def test_window_scores_with_stats_rejects_rounding(dev):
    q, k = qk(dev, 1, 4, 1, 64, 64, torch.bfloat16, 3)
    st = torch.zeros((1, 4, 32, 2), dtype=torch.float32, device=dev)
    with pytest.raises(ValueError):
        compress.window_scores(q, k, [0], 4, 32, "maxpool", 7, window_keep=True, round_dtype=torch.bfloat16, stats=st)
    with pytest.raises(ValueError):
        compress.window_scores(q, k, [0], 4, 32, "maxpool", 7, causal=False, stats=st)


def test_window_scores_with_attention_stats_128k(dev):
    """At the full 128K context (8 KV heads, GQA 4, W = 32, bf16): scores
    from the attention's statistics against the two-pass scorer (2e-5) for
    every head, and against the oracle for one head (2e-4)."""
    from heterocache_amd import ops
    B, Hkv, G, W, L = 1, 8, 4, 32, 131072
    print(f"window scores with stats at L={L}", flush=True)
    g = torch.Generator().manual_seed(5)
    q = torch.randn((B, Hkv * G, W, 128), generator=g).to(torch.bfloat16).to(dev)
    k = torch.randn((B, Hkv, L, 128), generator=g).to(torch.bfloat16).to(dev)
    v = torch.randn((B, Hkv, L, 128), generator=g).to(torch.bfloat16).to(dev)
    st = torch.full((B, Hkv * G, W, 2), float("nan"), dtype=torch.float32, device=dev)
    ops.prefill_attn(q, k, v, 1 / math.sqrt(128), stat_out=st)
    s1 = compress.window_scores(q, k, range(Hkv), G, W, "maxpool", 7, window_keep=True, stats=st)
    s0 = compress.window_scores(q, k, range(Hkv), G, W, "maxpool", 7, window_keep=True)
    torch.cuda.synchronize()
    assert s1.shape == (Hkv, L - W)
    assert rel_err(as_np(s1), as_np(s0)) < 2e-5
    h = 5
    qn, kn = as_np(q[0, h * G:(h + 1) * G]), as_np(k[0, h])
    ref = O.window_scores(qn[None], kn[None], "maxpool", 7, window_keep=True)[0]
    assert rel_err(as_np(s1[h]), ref) < 2e-4


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_select_with_key_bits_equals_all_passes(dev, dt):
    """hc_select_topk's key_bits for scores rounded by the cast chain (16 for
    bfloat16, 19 for float16: two and three radix passes instead of four):
    the kept sets and counts are the four-pass ones, also where most scores
    tie (a handful of distinct values) and where the budget cuts inside a
    tie run, and they match the oracle's ranking."""
    rng = np.random.default_rng(7)
    jobs, span = 6, 40000
    base = rng.random((jobs, span)) ** 3
    base[1] = rng.integers(0, 4, span) / 7.0          # four distinct values
    base[2] = 0.25                                     # all equal
    base[3, ::3] = 0.0                                 # zeros among the rest
    s = torch.tensor(base, dtype=torch.float32).to(dt).to(torch.float32).to(dev)
    caps = torch.tensor([1000, 12345, 777, 39999, 1, 20000], dtype=torch.int32, device=dev)
    a_idx, a_cnt = ops.select_topk(s, caps, span, idx=torch.empty((jobs, span), dtype=torch.int32, device=dev))
    b_idx, b_cnt = ops.select_topk(s, caps, span, idx=torch.empty((jobs, span), dtype=torch.int32, device=dev),
                                   key_bits=compress.KEY_BITS[dt])
    torch.cuda.synchronize()
    assert torch.equal(a_cnt, b_cnt)
    sn = s.cpu().numpy()
    for j in range(jobs):
        n = int(a_cnt[j])
        assert torch.equal(a_idx[j, :n], b_idx[j, :n]), j
        want = np.sort(O.topk_select(sn[j], int(caps[j])))
        assert np.array_equal(b_idx[j, :n].cpu().numpy(), want), j
