"""Tiled KV store writers/readers: bit-exact against plain indexing.

Covers the prefill keep-head copy, the indexed (compressed-head / retrieval)
gather from device and from host-pinned memory, partial-tile writes that
must preserve existing slots, decode append and the capacity error.
"""
import numpy as np
import pytest
import torch

from heterocache_amd.store import KVStore

pytestmark = pytest.mark.gpu


def rand(shape, dtype, dev, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    return torch.randn(shape, generator=g).to(dtype).to(dev)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_identity_copy_roundtrip(dev, dtype):
    B, H, L = 2, 3, 200
    k = rand((B, H, L, 128), dtype, dev, 1)
    v = rand((B, H, L, 128), dtype, dev, 2)
    store = KVStore([L + 50] * (B * H), dtype, dev)
    jobs = [(b, h) for b in range(B) for h in range(H)]
    store.write_rows(k, v, jobs, list(range(B * H)), [L] * (B * H))
    rk, rv = store.read_rows(list(range(B * H)), L)
    assert torch.equal(rk, k.reshape(B * H, L, 128))
    assert torch.equal(rv, v.reshape(B * H, L, 128))
    assert store.row_len.tolist() == [L] * (B * H)


def test_strided_projection_source(dev):
    """K as produced by proj(x).view(B, L, H, d).transpose(1, 2) (non-contiguous)."""
    B, H, L = 1, 8, 77
    x = rand((B, L, H * 128), torch.bfloat16, dev, 3)
    k = x.view(B, L, H, 128).transpose(1, 2)
    store = KVStore([L] * H, torch.bfloat16, dev)
    store.write_rows(k, k, [(0, h) for h in range(H)], list(range(H)), [L] * H)
    rk, _ = store.read_rows(list(range(H)), L)
    assert torch.equal(rk, k[0])


@pytest.mark.parametrize("host", [False, True])
def test_indexed_gather(dev, host):
    B, H, L = 1, 4, 1000
    k = rand((B, H, L, 128), torch.bfloat16, dev, 4)
    v = rand((B, H, L, 128), torch.bfloat16, dev, 5)
    if host:
        kh = torch.empty(k.shape, dtype=k.dtype, pin_memory=True)
        vh = torch.empty(v.shape, dtype=v.dtype, pin_memory=True)
        kh.copy_(k.cpu())
        vh.copy_(v.cpu())
        src_k, src_v = kh, vh
    else:
        src_k, src_v = k, v
    rng = np.random.default_rng(0)
    counts = [300, 1, 33, 0]
    M = max(counts)
    idx = np.zeros((H, M), dtype=np.int32)
    for h in range(H):
        idx[h, :counts[h]] = np.sort(rng.choice(L, counts[h], replace=False))
    store = KVStore([512] * H, torch.bfloat16, dev)
    store.write_rows(src_k, src_v, [(0, h) for h in range(H)], list(range(H)), counts,
                     idx=torch.as_tensor(idx).to(dev), src_is_host=host)
    torch.cuda.synchronize()
    for h in range(H):
        n = counts[h]
        if n == 0:
            continue
        rk, rv = store.read_rows([h], n)
        sel = torch.as_tensor(idx[h, :n], dtype=torch.long, device=dev)
        assert torch.equal(rk[0], k[0, h].index_select(0, sel))
        assert torch.equal(rv[0], v[0, h].index_select(0, sel))


def test_partial_tile_write_preserves_tail(dev):
    L = 100
    k = rand((1, 1, L, 128), torch.bfloat16, dev, 6)
    v = rand((1, 1, L, 128), torch.bfloat16, dev, 7)
    k2 = rand((1, 1, L, 128), torch.bfloat16, dev, 8)
    v2 = rand((1, 1, L, 128), torch.bfloat16, dev, 9)
    store = KVStore([L], torch.bfloat16, dev)
    store.write_rows(k, v, [(0, 0)], [0], [L])
    idx = torch.arange(40, dtype=torch.int32, device=dev).view(1, 40) * 2
    store.write_rows(k2, v2, [(0, 0)], [0], [40], idx=idx, set_len=False)
    rk, rv = store.read_rows([0], L)
    sel = idx[0].long()
    assert torch.equal(rk[0, :40], k2[0, 0].index_select(0, sel))
    assert torch.equal(rv[0, :40], v2[0, 0].index_select(0, sel))
    assert torch.equal(rk[0, 40:], k[0, 0, 40:])
    assert torch.equal(rv[0, 40:], v[0, 0, 40:])
    assert store.host_len.tolist() == [L]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_append_sequence(dev, dtype):
    rows, L0, steps = 5, [0, 31, 32, 63, 100], 40
    store = KVStore([L + steps for L in L0], dtype, dev)
    base_k = rand((1, rows, max(L0), 128), dtype, dev, 10)
    base_v = rand((1, rows, max(L0), 128), dtype, dev, 11)
    store.write_rows(base_k, base_v, [(0, r) for r in range(rows)], list(range(rows)), L0)
    new_k = rand((steps, rows, 128), dtype, dev, 12)
    new_v = rand((steps, rows, 128), dtype, dev, 13)
    for s in range(steps):
        store.append(new_k[s], new_v[s])
    torch.cuda.synchronize()
    assert store.row_len.tolist() == [L + steps for L in L0]
    assert store.host_len.tolist() == [L + steps for L in L0]
    for r in range(rows):
        n = L0[r] + steps
        rk, rv = store.read_rows([r], n)
        exp_k = torch.cat([base_k[0, r, :L0[r]], new_k[:, r]])
        exp_v = torch.cat([base_v[0, r, :L0[r]], new_v[:, r]])
        assert torch.equal(rk[0], exp_k)
        assert torch.equal(rv[0], exp_v)
    assert store.status.item() == 0


def test_append_capacity_error(dev):
    store = KVStore([32, 64], torch.bfloat16, dev)
    store.set_lengths([32, 10])
    kn = torch.zeros((2, 128), dtype=torch.bfloat16, device=dev)
    with pytest.raises(RuntimeError, match="OOM"):
        store.append(kn, kn)
    assert store.host_len.tolist() == [32, 10]


@pytest.mark.parametrize("to_host", [False, True])
def test_copy_rows_strided_source_small_grid(dev, to_host):
    """hc_copy_rows: selected heads of a transposed-view source into another
    layout (device or host-pinned), bit-exact, with a grid smaller than the
    work and counts below the length."""
    from heterocache_amd import ops
    B, H, L = 2, 5, 700
    g = torch.Generator().manual_seed(21)
    k = torch.randn((B, L, H, 128), generator=g).to(torch.bfloat16).to(dev).transpose(1, 2)
    v = torch.randn((B, L, H, 128), generator=g).to(torch.bfloat16).to(dev).transpose(1, 2)
    shape = (B, 3, L, 128)
    if to_host:
        dk = torch.zeros(shape, dtype=torch.bfloat16).pin_memory()
        dv = torch.zeros(shape, dtype=torch.bfloat16).pin_memory()
    else:
        dk = torch.zeros(shape, dtype=torch.bfloat16, device=dev)
        dv = torch.zeros(shape, dtype=torch.bfloat16, device=dev)
    src = [(0, 4), (1, 1), (0, 0), (1, 3)]
    dst = [(1, 2), (0, 0), (0, 1), (1, 0)]
    counts = [L, 33, 1, 650]
    side = torch.cuda.Stream()
    ops.copy_rows(k, v, src, dk, dv, dst, counts, dst_is_host=to_host, max_workgroups=3, stream=side)
    torch.cuda.synchronize()
    dk, dv = dk.cpu(), dv.cpu()
    kc, vc = k.cpu(), v.cpu()
    for (b, h), (b2, h2), n in zip(src, dst, counts):
        assert torch.equal(dk[b2, h2, :n], kc[b, h, :n]) and torch.equal(dv[b2, h2, :n], vc[b, h, :n])
        assert not dk[b2, h2, n:].any()
    ek = torch.zeros(shape, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError, match="count exceeds"):
        ops.copy_rows(k, v, [(0, 0)], ek, ek.clone(), [(0, 0)], [L + 1])


@pytest.mark.parametrize("host", [False, True])
def test_gather_groups_match_one_gather_and_record_each_event(dev, host):
    """hc_gather_store_groups: jobs in four groups (one of them empty, one
    whose leader did not trigger, one with a 2x token stride over an
    interleaved source) give the same store, bit for bit, as one
    hc_gather_store per group, and every group's event is recorded on the
    gather stream -- also the empty group's."""
    from heterocache_amd import ops
    L, D = 700, 128
    dt = torch.bfloat16
    base_k = rand((2 * L * D * 4,), dt, dev, 11)
    base_v = rand((2 * L * D * 4,), dt, dev, 12)
    if host:
        src_k = torch.empty(base_k.shape, dtype=dt, pin_memory=True)
        src_v = torch.empty(base_v.shape, dtype=dt, pin_memory=True)
        src_k.copy_(base_k.cpu())
        src_v.copy_(base_v.cpu())
    else:
        src_k, src_v = base_k, base_v
    rng = np.random.default_rng(5)
    # Groups: [0, 3) stride 128, [3, 3) empty, [3, 5) stride 256 (interleaved), [5, 7) gated off.
    begin = np.array([0, 3, 3, 5, 7], dtype=np.int32)
    strides = np.array([D, D, 2 * D, D], dtype=np.int64)
    counts = np.array([300, 1, 33, 64, 200, 90, 17], dtype=np.int32)
    src_off = np.array([0, L * D, 2 * L * D, 3 * L * D, 3 * L * D + D, 5 * L * D, 6 * L * D], dtype=np.int64)
    trig_of = np.array([0, 0, 0, 1, 1, 2, 2], dtype=np.int32)
    trigger = torch.tensor([1, 1, 0], dtype=torch.int32, device=dev)
    M = int(counts.max())
    idx = np.zeros((len(counts), M), dtype=np.int32)
    for j, n in enumerate(counts):
        idx[j, :n] = np.sort(rng.choice(L, n, replace=False))
    idx_d = torch.as_tensor(idx).to(dev)
    idx_off = torch.as_tensor(np.arange(len(counts)) * M, dtype=torch.int64).to(dev)
    a = KVStore([512] * len(counts), dt, dev)
    b = KVStore([512] * len(counts), dt, dev)
    dst = torch.arange(len(counts), dtype=torch.int32, device=dev)
    cnt = torch.as_tensor(counts).to(dev)
    so = torch.as_tensor(src_off).to(dev)
    to = torch.as_tensor(trig_of).to(dev)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    events = [torch.cuda.Event() for _ in range(4)]
    for ev in events:
        ev.record(side)
    gmax = [int(counts[begin[g]:begin[g + 1]].max()) if begin[g + 1] > begin[g] else 0 for g in range(4)]
    ops.gather_store_groups(src_k, src_v, so, strides, L, idx_d, idx_off, cnt, dst, a.k, a.v, a.row_tile_off,
                            begin, gmax, events, src_is_host=host, trigger=trigger, trig_of=to, stream=side)
    for g in range(4):
        b0, b1 = begin[g], begin[g + 1]
        if b1 > b0:
            ops.gather_store(src_k, src_v, so[b0:b1], int(strides[g]), L, idx_d, idx_off[b0:b1], cnt[b0:b1],
                             dst[b0:b1], b.k, b.v, b.row_tile_off, gmax[g], src_is_host=host, trigger=trigger,
                             trig_of=to[b0:b1])
    torch.cuda.current_stream().wait_event(events[-1])
    torch.cuda.synchronize()
    assert all(ev.query() for ev in events)
    for j, n in enumerate(counts):
        ka, va = a.read_rows([j], int(n))
        kb, vb = b.read_rows([j], int(n))
        assert torch.equal(ka, kb) and torch.equal(va, vb), j
        if trig_of[j] == 2:   # gated off: the store keeps its (zero) slots
            assert not ka.any()
        else:
            g = int(np.searchsorted(begin, j, side="right") - 1)
            sel = torch.as_tensor(src_off[j] + idx[j, :n].astype(np.int64) * strides[g], device=dev)
            rows = sel[:, None] + torch.arange(D, device=dev)[None, :]
            assert torch.equal(ka[0], base_k[rows]) and torch.equal(va[0], base_v[rows]), j


def test_gather_groups_from_per_job_tensors(dev):
    """hc_gather_store_groups with per-job source addresses: jobs read two
    separate [1, H, L, 128] tensors (one a strided projection view) in one
    launch (one token stride), each row bit for bit the rows indexed."""
    from heterocache_amd import ops
    L, D, H = 500, 128, 3
    dt = torch.bfloat16
    x = rand((1, L, H * D), dt, dev, 23)
    kb = x.view(1, L, H, D).transpose(1, 2)          # token stride H * 128, as the projections give
    y = rand((1, L, H * D), dt, dev, 24)
    vb = y.view(1, L, H, D).transpose(1, 2)
    # A second pair of tensors with the same (projection) token stride.
    ka = rand((1, L, H * D), dt, dev, 25).view(1, L, H, D).transpose(1, 2)
    va = rand((1, L, H * D), dt, dev, 26).view(1, L, H, D).transpose(1, 2)
    rng = np.random.default_rng(9)
    srcs = [(ka, va, 1), (kb, vb, 2), (kb, vb, 0)]
    counts = np.array([77, 200, 5], dtype=np.int32)
    M = int(counts.max())
    idx = np.zeros((3, M), dtype=np.int32)
    for j, n in enumerate(counts):
        idx[j, :n] = np.sort(rng.choice(L, n, replace=False))
    idx_d = torch.as_tensor(idx).to(dev)
    idx_off = torch.as_tensor(np.arange(3) * M, dtype=torch.int64).to(dev)
    src_off = torch.as_tensor([k.stride(1) * h for k, _, h in srcs], dtype=torch.int64).to(dev)
    k_addr = torch.as_tensor([k.data_ptr() for k, _, _ in srcs], dtype=torch.int64).to(dev)
    v_addr = torch.as_tensor([v.data_ptr() for _, v, _ in srcs], dtype=torch.int64).to(dev)
    st = KVStore([256] * 3, dt, dev)
    cnt = torch.as_tensor(counts).to(dev)
    dst = torch.arange(3, dtype=torch.int32, device=dev)
    ops.gather_store_groups(ka, va, src_off, np.array([H * D], dtype=np.int64), L, idx_d, idx_off, cnt, dst,
                            st.k, st.v, st.row_tile_off, np.array([0, 3], dtype=np.int32), [M], [None],
                            src_k_addr=k_addr, src_v_addr=v_addr)
    torch.cuda.synchronize()
    for j, (k, v, h) in enumerate(srcs):
        n = int(counts[j])
        rk, rv = st.read_rows([j], n)
        sel = torch.as_tensor(idx[j, :n], dtype=torch.long, device=dev)
        assert torch.equal(rk[0], k[0, h].index_select(0, sel)) and torch.equal(rv[0], v[0, h].index_select(0, sel)), j


def test_stream_read_reads_and_leaves_the_sink(dev):
    """hc_stream_read (the bench's read-ceiling measurement): over a
    zero-filled buffer it leaves the sink alone, and it refuses a size that
    is not a multiple of 16 bytes and an out-of-range workgroup count."""
    from heterocache_amd import _lib, ops
    buf = torch.zeros(1 << 20, dtype=torch.float32, device=dev)
    sink = torch.full((1,), 7.0, dtype=torch.float32, device=dev)
    ops.stream_read(buf, sink=sink)
    ops.stream_read(buf, workgroups_per_cu=1, sink=sink)
    torch.cuda.synchronize()
    assert sink.item() == 7.0
    with pytest.raises(_lib.HCError):
        ops.stream_read(buf[:3], sink=sink)
    with pytest.raises(_lib.HCError):
        ops.stream_read(buf, workgroups_per_cu=0, sink=sink)


def test_gather_sets_row_lengths_in_the_launch(dev):
    """hc_gather_store(set_len=row_len): the copied rows' device lengths
    become their counts in the same launch (gated rows keep theirs, rows
    outside the plan keep theirs), and the stores equal a gather followed
    by set_lengths."""
    from heterocache_amd import ops
    B, H, L = 1, 6, 300
    k = rand((B, H, L, 128), torch.bfloat16, dev, 11)
    v = rand((B, H, L, 128), torch.bfloat16, dev, 12)
    a = KVStore([L + 8] * H, torch.bfloat16, dev)
    b = KVStore([L + 8] * H, torch.bfloat16, dev)
    a.set_lengths([5] * H)
    b.set_lengths([5] * H)
    rows, counts = [0, 2, 3, 5], [300, 17, 0, 64]
    g = torch.Generator(device="cpu").manual_seed(13)
    idx = torch.sort(torch.randint(0, L, (len(rows), 300), generator=g), dim=1).values.to(torch.int32).to(dev)
    plan = a.plan_rows(k, [(0, r) for r in rows], rows, counts, idx=idx)
    a.launch_rows(plan, k, v, idx=idx, set_len=False, write_len=True)
    b.write_rows(k, v, [(0, r) for r in rows], rows, counts, idx=idx)
    torch.cuda.synchronize()
    assert a.row_len.tolist() == [300, 5, 17, 0, 5, 64]
    assert a.row_len.tolist() == b.row_len.tolist()
    for r, n in zip(rows, counts):
        if n:
            xa, ya = a.read_rows([r], n)
            xb, yb = b.read_rows([r], n)
            assert torch.equal(xa, xb) and torch.equal(ya, yb)
    # Gated off: lengths stay.
    trig = torch.zeros(1, dtype=torch.int32, device=dev)
    ops.gather_store(k, v, plan["src_off"], plan["tok_stride"], plan["src_len"], idx, plan["idx_off"], plan["counts"],
                     plan["rows"], a.k, a.v, a.row_tile_off, plan["max_count"], trigger=trig, trig_of=None,
                     set_len=a.row_len)
    torch.cuda.synchronize()
    assert a.row_len.tolist() == [300, 5, 17, 0, 5, 64]
