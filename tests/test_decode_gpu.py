"""Decode attention (hc_decode_attn) vs the float64 closed form of the oracle.

Parity bar: max-abs <= 2e-2 (bf16), 1e-2 (fp16), 1e-4 (fp32).
"""
import ctypes
import math

import numpy as np
import pytest
import torch

from heterocache_amd.store import KVStore
from oracle import hc_oracle as O
from tests.gpu_util import ATTN_TOL, TORCH_DT, as_np, fill_store

pytestmark = pytest.mark.gpu


def run_case(dev, dt, lens, G, seed, chunk_tiles=16, extra_cap=0, scale=None, outliers=False):
    rng = np.random.default_rng(seed)
    tdt = TORCH_DT[dt]
    ks = [torch.as_tensor(rng.standard_normal((L, 128)), dtype=torch.float32) for L in lens]
    vs = [torch.as_tensor(rng.standard_normal((L, 128)), dtype=torch.float32) for L in lens]
    if outliers:  # a few large channels and one dominant token per row
        for k in ks:
            k[:, :4] *= 8
            if k.shape[0] > 3:
                k[3] *= 3
    q = torch.as_tensor(rng.standard_normal((len(lens), G, 128)), dtype=torch.float32)
    store = KVStore([L + extra_cap for L in lens], tdt, dev)
    fill_store(store, [k.to(dev) for k in ks], [v.to(dev) for v in vs], dev)
    qd = q.to(tdt).to(dev)
    scale = 1.0 / math.sqrt(128) if scale is None else scale
    out = store.attend(qd, scale, chunk_tiles=chunk_tiles)
    torch.cuda.synchronize()
    # The oracle sees exactly the values the device holds.
    ref = O.decode_attention(as_np(qd), [as_np(k.to(tdt)) for k in ks], [as_np(v.to(tdt)) for v in vs], scale)
    err = np.abs(as_np(out) - ref).max() if out.numel() else 0.0
    return err, out


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
def test_ragged_rows_gqa4(dev, dt):
    lens = [1, 31, 32, 33, 100, 1000, 4097, 255]
    err, _ = run_case(dev, dt, lens, 4, seed=11)
    assert err <= ATTN_TOL[dt], err


@pytest.mark.parametrize("G", [1, 2, 7, 8, 16])
def test_group_sizes(dev, G):
    err, _ = run_case(dev, "bf16", [77, 513, 2048, 3], G, seed=100 + G)
    assert err <= ATTN_TOL["bf16"], err


@pytest.mark.parametrize("chunk", [1, 3, 4, 5, 8, 30, 64, None])
def test_chunking_is_invisible(dev, chunk):
    """Any chunk size (including ones that leave waves idle or split unevenly)
    and the automatic choice give the same attention."""
    err, _ = run_case(dev, "f32", [5000, 17, 1024], 4, seed=7, chunk_tiles=chunk)
    assert err <= ATTN_TOL["f32"], err


def test_empty_row_gives_zeros(dev):
    err, out = run_case(dev, "bf16", [0, 50, 0, 7], 4, seed=3)
    assert err <= ATTN_TOL["bf16"]
    assert torch.count_nonzero(out[0]) == 0 and torch.count_nonzero(out[2]) == 0


def test_outliers_and_sinks(dev):
    err, _ = run_case(dev, "bf16", [4096, 1500], 4, seed=5, outliers=True)
    assert err <= ATTN_TOL["bf16"], err
    err, _ = run_case(dev, "f32", [4096, 1500], 4, seed=5, outliers=True)
    assert err <= ATTN_TOL["f32"], err


def test_stale_tail_does_not_leak(dev):
    """Slots past len hold other data (here: NaN); the kernel must mask them."""
    lens = [45, 70]
    rng = np.random.default_rng(9)
    store = KVStore([128, 128], torch.bfloat16, dev)
    store.k.fill_(float("nan"))
    store.v.fill_(float("nan"))
    ks = [torch.as_tensor(rng.standard_normal((L, 128)), dtype=torch.float32).to(dev) for L in lens]
    vs = [torch.as_tensor(rng.standard_normal((L, 128)), dtype=torch.float32).to(dev) for L in lens]
    fill_store(store, ks, vs, dev)
    q = torch.as_tensor(rng.standard_normal((2, 4, 128)), dtype=torch.float32).to(torch.bfloat16).to(dev)
    out = store.attend(q, 1 / math.sqrt(128))
    ref = O.decode_attention(as_np(q), [as_np(k.bfloat16()) for k in ks], [as_np(v.bfloat16()) for v in vs])
    assert np.isfinite(as_np(out)).all()
    assert np.abs(as_np(out) - ref).max() <= ATTN_TOL["bf16"]


def test_matches_torch_sdpa_fp32(dev):
    """Independent check against torch's own attention in float32."""
    rng = np.random.default_rng(21)
    L, G = 3000, 4
    k = torch.as_tensor(rng.standard_normal((L, 128)), dtype=torch.float32).to(dev)
    v = torch.as_tensor(rng.standard_normal((L, 128)), dtype=torch.float32).to(dev)
    q = torch.as_tensor(rng.standard_normal((1, G, 128)), dtype=torch.float32).to(dev)
    store = KVStore([L], torch.float32, dev)
    fill_store(store, [k], [v], dev)
    out = store.attend(q, 1 / math.sqrt(128))
    ref = torch.softmax((q[0] @ k.T) / math.sqrt(128), dim=-1) @ v
    assert (out[0] - ref).abs().max().item() <= 1e-4


@pytest.mark.parametrize("dt", ["bf16", "f32"])
def test_fused_append_matches_oracle_over_steps(dev, dt):
    """attend(k_new=...) matches the oracle and append-then-attend step after
    step (the fused path folds the new token in after the stored tiles, so
    the two agree to the attention tolerance, not bitwise); the stores end
    up bit-identical."""
    lens = [0, 1, 31, 32, 63, 100, 1023, 1024, 2500, 4096]
    steps, G = 6, 4
    tdt = TORCH_DT[dt]
    rng = np.random.default_rng(77)
    ks = [torch.as_tensor(rng.standard_normal((L, 128)), dtype=torch.float32).to(tdt).to(dev) for L in lens]
    vs = [torch.as_tensor(rng.standard_normal((L, 128)), dtype=torch.float32).to(tdt).to(dev) for L in lens]
    a = KVStore([L + steps for L in lens], tdt, dev)
    b = KVStore([L + steps for L in lens], tdt, dev)
    fill_store(a, ks, vs, dev)
    fill_store(b, ks, vs, dev)
    hist_k = [as_np(k) for k in ks]
    hist_v = [as_np(v) for v in vs]
    scale = 1 / math.sqrt(128)
    for s in range(steps):
        kn = torch.as_tensor(rng.standard_normal((len(lens), 128)), dtype=torch.float32).to(tdt).to(dev)
        vn = torch.as_tensor(rng.standard_normal((len(lens), 128)), dtype=torch.float32).to(tdt).to(dev)
        q = torch.as_tensor(rng.standard_normal((len(lens), G, 128)), dtype=torch.float32).to(tdt).to(dev)
        a.append(kn, vn)
        oa = a.attend(q, scale)
        ob = b.attend(q, scale, k_new=kn, v_new=vn)
        torch.cuda.synchronize()
        for r in range(len(lens)):
            hist_k[r] = np.concatenate([hist_k[r], as_np(kn[r:r + 1])])
            hist_v[r] = np.concatenate([hist_v[r], as_np(vn[r:r + 1])])
        ref = O.decode_attention(as_np(q), hist_k, hist_v, scale)
        assert np.abs(as_np(ob) - ref).max() <= ATTN_TOL[dt]
        assert np.abs(as_np(oa) - ref).max() <= ATTN_TOL[dt]
        assert (oa.float() - ob.float()).abs().max().item() <= ATTN_TOL[dt], f"step {s}: fused vs append+attend"
    assert b.row_len.tolist() == [L + steps for L in lens]
    assert b.host_len.tolist() == [L + steps for L in lens]
    for r in range(len(lens)):
        ka, va = a.read_rows([r], lens[r] + steps)
        kb, vb = b.read_rows([r], lens[r] + steps)
        assert torch.equal(ka, kb) and torch.equal(va, vb)


@pytest.mark.parametrize("G", [1, 4, 7, 16])
def test_merge_folds_parts_beyond_the_register_batch(dev, G):
    """A row of 547 parts: the merge folds its first 128 parts from registers
    and the rest in its online loop, for several group sizes."""
    err, _ = run_case(dev, "bf16", [70000, 300], G, seed=31 + G, chunk_tiles=4)
    assert err <= ATTN_TOL["bf16"], err


@pytest.mark.parametrize("dt,io_dtype", [("bf16", None), ("f32", None), ("bf16", "bfloat16"), ("f16", "float16")])
@pytest.mark.parametrize("chunk", [4, None])
def test_softmax_stats_below_stat_len(dev, dt, io_dtype, chunk):
    """hc_decode_attn_stats: for every row and query head, M + log2(L) is the
    float64 base-2 log-normaliser over the row's first stat_len attended
    tokens (tile-aligned and not, beyond every row, with and without a fused
    append whose new token lies above or below stat_len); the attention
    output is the plain call's, bit for bit.  With a rounding flag, the
    normaliser of the reference's cast chain of the logits (the oracle's
    io_dtype form)."""
    from heterocache_amd import compress
    lens, G = [5000, 3000, 40, 0, 2055], 4
    flags = compress.ROUND_FLAGS[TORCH_DT[dt]] if io_dtype else 0
    tdt = TORCH_DT[dt]
    rng = np.random.default_rng(17)
    ks = [torch.as_tensor(rng.standard_normal((L, 128)), dtype=torch.float32).to(tdt) for L in lens]
    vs = [torch.as_tensor(rng.standard_normal((L, 128)), dtype=torch.float32).to(tdt) for L in lens]
    for k in ks:
        k[:, :4] *= 6  # outlier channels: wide score range
    q = torch.as_tensor(rng.standard_normal((len(lens), G, 128)), dtype=torch.float32).to(tdt).to(dev)
    kn = torch.as_tensor(rng.standard_normal((len(lens), 128)), dtype=torch.float32).to(tdt).to(dev)
    vn = torch.as_tensor(rng.standard_normal((len(lens), 128)), dtype=torch.float32).to(tdt).to(dev)
    scale = 1 / math.sqrt(128)
    for stat_len in (1000, 2048, 2056, 4100, 100000):
        for append in (False, True):
            a = KVStore([L + 4 for L in lens], tdt, dev)
            b = KVStore([L + 4 for L in lens], tdt, dev)
            for st in (a, b):
                fill_store(st, [k.to(dev) for k in ks], [v.to(dev) for v in vs], dev)
            stats = torch.full((len(lens), G, 2), 7.0, dtype=torch.float32, device=dev)
            extra = dict(k_new=kn, v_new=vn) if append else {}
            oa = a.attend(q, scale, chunk_tiles=chunk, stat_len=stat_len, stat_out=stats, stat_flags=flags,
                          **extra).clone()
            ob = b.attend(q, scale, chunk_tiles=chunk, **extra)
            torch.cuda.synchronize()
            assert torch.equal(oa, ob), (stat_len, append)
            keys = [as_np(torch.cat([k.to(dev), kn[r:r + 1]]) if append else k) for r, k in enumerate(ks)]
            ref = O.softmax_lse2(as_np(q), keys, stat_len, scale, io_dtype=io_dtype)
            st = stats.cpu().numpy().astype(np.float64)
            with np.errstate(divide="ignore"):
                got = st[..., 0] + np.log2(st[..., 1])
            empty = np.isinf(ref)
            assert np.all(st[empty][:, 0] == -np.inf) and np.all(st[empty][:, 1] == 0), (stat_len, append)
            err = np.abs(got[~empty] - ref[~empty]).max()
            assert err <= 2e-5 * max(1.0, np.abs(ref[~empty]).max()), (stat_len, append, err)


def test_row_order_does_not_change_results(dev):
    lens = [300, 5000, 64, 2049]
    rng = np.random.default_rng(4)
    ks = [torch.as_tensor(rng.standard_normal((L, 128)), dtype=torch.float32).to(dev) for L in lens]
    vs = [torch.as_tensor(rng.standard_normal((L, 128)), dtype=torch.float32).to(dev) for L in lens]
    st = KVStore(lens, torch.float32, dev)
    fill_store(st, ks, vs, dev)
    q = torch.as_tensor(rng.standard_normal((4, 4, 128)), dtype=torch.float32).to(dev)
    o1 = st.attend(q, 0.1).clone()
    st.row_order = torch.tensor([2, 0, 3, 1], dtype=torch.int32, device=dev)
    o2 = st.attend(q, 0.1)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)


def test_auto_chunk_fits_one_round(dev):
    """hc_decode_chunk_tiles: at least one tile per wave; below 24 tiles
    minimal (one tile less would need more workgroups); from 24 tiles whole
    tiles per wave (a multiple of 4) and minimal among those; one chunk per
    row when rows alone exceed the device's slots; an error for a bad
    dtype."""
    from heterocache_amd import _lib, ops
    seen = set()
    for lens in ([131072] * 4 + [65536] * 4, [5000, 17, 1024], [0, 3], [200_000] * 3 + [10] * 5,
                 [16384, 2048, 4096, 6144] * 4):
        c = ops.decode_chunk_tiles(lens, 4, torch.bfloat16)
        assert c >= 4
        step = 4 if c >= 24 else 1
        seen.add(step)
        assert c % step == 0
        if c > 4:
            assert ops.decode_num_parts(lens, c - step) > ops.decode_num_parts(lens, c)
    assert seen == {1, 4}, "both regimes covered"
    many = [4096] * 20000
    assert ops.decode_chunk_tiles(many, 4, torch.bfloat16) == 128
    lens = np.asarray([10], dtype=np.int32)
    assert _lib.load().hc_decode_chunk_tiles(9, lens.ctypes.data_as(ctypes.c_void_p), 1, 4) == _lib.HC_ERR_INVALID


def test_graph_replays_match_eager_steps(dev):
    """The decode step (fused append + attention over two stores) captured
    in a HIP graph with fixed chunk sizes and grids sized for the lengths
    the last replay reaches: each of several replays, with new inputs
    written eagerly in between, equals the same step run eagerly with the
    same chunk sizes (bitwise), and the stores end up identical."""
    from heterocache_amd import _lib, ops
    steps, G = 5, 4
    lens = [[0, 31, 700, 5000, 33], [1, 1024, 12000, 64, 2047]]
    tdt = torch.bfloat16
    rng = np.random.default_rng(91)
    graph_stores, eager_stores = [], []
    for ls in lens:
        ks = [torch.as_tensor(rng.standard_normal((L, 128)), dtype=torch.float32).to(tdt).to(dev) for L in ls]
        vs = [torch.as_tensor(rng.standard_normal((L, 128)), dtype=torch.float32).to(tdt).to(dev) for L in ls]
        for group in (graph_stores, eager_stores):
            st = KVStore([L + steps for L in ls], tdt, dev)
            fill_store(st, ks, vs, dev)
            group.append(st)
    rows = len(lens[0])
    q = torch.zeros((2, rows, G, 128), dtype=tdt, device=dev)
    kn = torch.zeros((2, rows, 128), dtype=tdt, device=dev)
    vn = torch.zeros_like(kn)
    out_g = torch.empty((2, rows, G, 128), dtype=tdt, device=dev)
    out_e = torch.empty_like(out_g)
    scale = 1 / math.sqrt(128)
    cts = [ops.decode_chunk_tiles(st.host_len + 1, G, tdt) for st in graph_stores]
    parts = [ops.decode_num_parts(st.host_len + steps, ct) for st, ct in zip(graph_stores, cts)]
    ws = torch.empty(max(_lib.load().hc_decode_workspace_size(rows, G, n) for n in parts), dtype=torch.uint8,
                     device=dev)
    len0 = [st.host_len.astype(np.int64).copy() for st in graph_stores]
    graph = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        for i, st in enumerate(graph_stores):
            st.attend(q[i], scale, out=out_g[i], k_new=kn[i], v_new=vn[i], chunk_tiles=cts[i], num_parts=parts[i],
                      workspace=ws)
    for s in range(steps):
        q.copy_(torch.as_tensor(rng.standard_normal(tuple(q.shape)), dtype=torch.float32).to(tdt))
        kn.copy_(torch.as_tensor(rng.standard_normal(tuple(kn.shape)), dtype=torch.float32).to(tdt))
        vn.copy_(torch.as_tensor(rng.standard_normal(tuple(vn.shape)), dtype=torch.float32).to(tdt))
        graph.replay()
        for i, st in enumerate(eager_stores):
            st.attend(q[i], scale, out=out_e[i], k_new=kn[i], v_new=vn[i], chunk_tiles=cts[i])
        torch.cuda.synchronize()
        assert torch.equal(out_g, out_e), f"replay {s}"
        assert not torch.isnan(out_g.float()).any()
    for st, l0, ref in zip(graph_stores, len0, eager_stores):
        st.sync_host_lengths(l0 + steps)
        assert st.row_len.tolist() == ref.row_len.tolist() == (l0 + steps).tolist()
        for r in range(rows):
            ka, va = st.read_rows([r], int(l0[r]) + steps)
            kb, vb = ref.read_rows([r], int(l0[r]) + steps)
            assert torch.equal(ka, kb) and torch.equal(va, vb)


def _abi_decode(lib, ops, store, q, out, ws, parts, chunk, kn=None, vn=None, status=None):
    """hc_decode_attn through the C ABI (no host-side capacity or grid check)."""
    return lib.hc_decode_attn(ops.dtype_code(q.dtype), q.data_ptr(), store.k.data_ptr(), store.v.data_ptr(),
                              store.row_tile_off.data_ptr(), store.row_len.data_ptr(), store.row_cap.data_ptr(),
                              store.row_order.data_ptr(), q.shape[0], q.shape[1], 1 / math.sqrt(128),
                              kn.data_ptr() if kn is not None else None, vn.data_ptr() if vn is not None else None,
                              out.data_ptr(), ws.data_ptr(), ws.numel(), parts, chunk,
                              status.data_ptr() if status is not None else None,
                              torch.cuda.current_stream().cuda_stream)


def _store_snapshot(store):
    return [tuple(t.clone() for t in store.read_rows([r], int(store.host_cap[r]))) for r in range(store.rows)]


def test_undersized_grid_gives_nan_rows(dev):
    """hc_decode_attn called (through the C ABI, which the Python wrapper
    would refuse) with fewer workgroups than the lengths need, into a
    workspace a valid launch over the same rows has just filled: every row
    comes out NaN (no stale partial of the earlier launch is merged), the
    fused append stores nothing and no length advances."""
    from heterocache_amd import _lib, ops
    lens, G = [5000, 3000, 40], 4
    rng = np.random.default_rng(5)
    ks = [torch.as_tensor(rng.standard_normal((L, 128)), dtype=torch.float32).to(dev) for L in lens]
    vs = [torch.as_tensor(rng.standard_normal((L, 128)), dtype=torch.float32).to(dev) for L in lens]
    store = KVStore([L + 8 for L in lens], torch.bfloat16, dev)
    fill_store(store, ks, vs, dev)
    q = torch.randn((len(lens), G, 128), device=dev).to(torch.bfloat16)
    kn = torch.randn((len(lens), 128), device=dev).to(torch.bfloat16)
    vn = torch.randn((len(lens), 128), device=dev).to(torch.bfloat16)
    chunk = 4
    need = ops.decode_num_parts(store.host_len + 1, chunk)
    small = 10
    assert need > small
    lib = _lib.load()
    ws = torch.zeros(lib.hc_decode_workspace_size(len(lens), G, need), dtype=torch.uint8, device=dev)
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    # A valid launch (no append) leaves finite partials and row info in ws.
    out = torch.zeros_like(q)
    assert _abi_decode(lib, ops, store, q, out, ws, need, chunk) == 0
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    before = _store_snapshot(store)
    out = torch.zeros_like(q)
    assert _abi_decode(lib, ops, store, q, out, ws, small, chunk, kn, vn, status) == 0
    torch.cuda.synchronize()
    assert torch.isnan(out.float()).all()
    assert store.row_len.tolist() == lens
    assert status.item() == 0
    after = _store_snapshot(store)
    for (ka, va), (kb, vb) in zip(before, after):
        assert torch.equal(ka, kb) and torch.equal(va, vb)


def test_fused_append_at_capacity_sets_status(dev):
    """A row at capacity (not the last row of the buffer) under a fused
    append, launched without the host check (as a graph replay would): the
    row is unchanged and comes out NaN, the status word is set, the other
    rows append and attend normally and their neighbours' tiles are
    untouched; KVStore.check_status raises the reference's "Layer i OOM."
    and clears the word."""
    from heterocache_amd import _lib, ops
    caps, G = [64, 96, 40], 4
    lens = [64, 50, 39]          # row 0 is full; row 1 follows it in the buffer
    rng = np.random.default_rng(11)
    ks = [torch.as_tensor(rng.standard_normal((L, 128)), dtype=torch.float32).to(dev) for L in lens]
    vs = [torch.as_tensor(rng.standard_normal((L, 128)), dtype=torch.float32).to(dev) for L in lens]
    store = KVStore(caps, torch.float32, dev, layer_idx=7)
    fill_store(store, ks, vs, dev)
    q = torch.randn((3, G, 128), device=dev)
    kn = torch.randn((3, 128), device=dev)
    vn = torch.randn((3, 128), device=dev)
    before = _store_snapshot(store)
    out = ops.decode_attn(q, store.k, store.v, store.row_tile_off, store.row_len, store.host_len + 0, 1 / math.sqrt(128),
                          row_order=store.row_order, k_new=kn, v_new=vn, row_cap=store.row_cap, status=store.status)
    torch.cuda.synchronize()
    assert store.row_len.tolist() == [64, 51, 40]
    assert store.status.item() == 1
    o = as_np(out)
    assert np.isnan(o[0]).all()
    kk = [np.concatenate([as_np(ks[r]), as_np(kn[r:r + 1])]) for r in (1, 2)]
    vv = [np.concatenate([as_np(vs[r]), as_np(vn[r:r + 1])]) for r in (1, 2)]
    ref = O.decode_attention(as_np(q[1:]), kk, vv)
    assert np.abs(o[1:] - ref).max() <= 1e-4
    after = _store_snapshot(store)
    assert torch.equal(before[0][0], after[0][0]) and torch.equal(before[0][1], after[0][1])
    for r in (1, 2):
        n = lens[r]
        assert torch.equal(before[r][0][0, :n], after[r][0][0, :n])
        assert torch.equal(after[r][0][0, n], kn[r]) and torch.equal(after[r][1][0, n], vn[r])
        assert torch.equal(before[r][0][0, n + 1:], after[r][0][0, n + 1:])
    with pytest.raises(RuntimeError, match="Layer 7 OOM."):
        store.check_status()
    assert store.status.item() == 0
    store.check_status()  # cleared


def test_graph_replay_past_capacity_raises_oom(dev):
    """A captured decode step replayed past a row's capacity: replays up to
    the capacity match eager steps, the replay past it leaves that row (the
    first of three) unchanged and NaN, and check_status raises."""
    from heterocache_amd import _lib, ops
    caps, lens, G = [64, 96, 96], [62, 60, 33], 4   # capacities are whole 32-token tiles
    rng = np.random.default_rng(12)
    ks = [torch.as_tensor(rng.standard_normal((L, 128)), dtype=torch.float32).to(dev) for L in lens]
    vs = [torch.as_tensor(rng.standard_normal((L, 128)), dtype=torch.float32).to(dev) for L in lens]
    gst, est = (KVStore(caps, torch.bfloat16, dev, layer_idx=3) for _ in range(2))
    for st in (gst, est):
        fill_store(st, ks, vs, dev)
    q = torch.randn((3, G, 128), device=dev).to(torch.bfloat16)
    kn = torch.randn((3, 128), device=dev).to(torch.bfloat16)
    vn = torch.randn((3, 128), device=dev).to(torch.bfloat16)
    ct = 4
    parts = ops.decode_num_parts(np.asarray(caps) + 1, ct)
    lib = _lib.load()
    ws = torch.empty(lib.hc_decode_workspace_size(3, G, parts), dtype=torch.uint8, device=dev)
    out_g = torch.empty_like(q)
    out_e = torch.empty_like(q)
    graph = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        gst.attend(q, 1 / math.sqrt(128), out=out_g, k_new=kn, v_new=vn, chunk_tiles=ct, num_parts=parts, workspace=ws)
    for s in range(2):       # row 0 goes 62 -> 63 -> 64 (its capacity)
        graph.replay()
        est.attend(q, 1 / math.sqrt(128), out=out_e, k_new=kn, v_new=vn, chunk_tiles=ct)
        torch.cuda.synchronize()
        assert torch.equal(out_g, out_e), s
    gst.check_status()
    snap = _store_snapshot(gst)
    graph.replay()           # row 0 is full now
    torch.cuda.synchronize()
    assert gst.row_len.tolist() == [64, 63, 36]
    assert torch.isnan(out_g[0].float()).all() and torch.isfinite(out_g[1:].float()).all()
    after = _store_snapshot(gst)
    assert torch.equal(snap[0][0], after[0][0]) and torch.equal(snap[0][1], after[0][1])
    with pytest.raises(RuntimeError, match="Layer 3 OOM."):
        gst.check_status()
