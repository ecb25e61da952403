"""hc_decode_attn_noalloc (device scratch, no workspace argument) against
hc_decode_attn with a caller workspace, through the C ABI: two calls in a
row, the second over a smaller input, each bit-identical to the
workspace entry point on a twin store (outputs, lengths after the fused
append, store contents); launches whose workspace would exceed the scratch
are refused before anything runs."""
import math

import numpy as np
import pytest
import torch

from heterocache_amd import _lib, ops
from heterocache_amd.store import KVStore
from tests.gpu_util import fill_store

pytestmark = pytest.mark.gpu


def _twin_stores(lens, dtype, dev, seed):
    rng = np.random.default_rng(seed)
    ks = [torch.as_tensor(rng.standard_normal((n, 128)), dtype=torch.float32).to(dev) for n in lens]
    vs = [torch.as_tensor(rng.standard_normal((n, 128)), dtype=torch.float32).to(dev) for n in lens]
    caps = [n + 40 for n in lens]
    a, b = KVStore(caps, dtype, dev), KVStore(caps, dtype, dev)
    for st in (a, b):
        fill_store(st, ks, vs, dev)
    return a, b


def _call(lib, st, q, kn, vn, out, parts, chunk, ws=None):
    common = (ops.dtype_code(q.dtype), q.data_ptr(), st.k.data_ptr(), st.v.data_ptr(), st.row_tile_off.data_ptr(),
              st.row_len.data_ptr(), st.row_cap.data_ptr(), st.row_order.data_ptr(), q.shape[0], q.shape[1],
              1 / math.sqrt(128), kn.data_ptr(), vn.data_ptr(), out.data_ptr())
    stream = torch.cuda.current_stream().cuda_stream
    if ws is None:
        return lib.hc_decode_attn_noalloc(*common, parts, chunk, st.status.data_ptr(), stream)
    return lib.hc_decode_attn(*common, ws.data_ptr(), ws.numel(), parts, chunk, st.status.data_ptr(), stream)


def _check_case(dev, lens, G, dtype, seed):
    lib = _lib.load()
    a, b = _twin_stores(lens, dtype, dev, seed)
    g = torch.Generator(device=dev).manual_seed(seed)
    rows = len(lens)
    q = torch.randn((rows, G, 128), device=dev, generator=g).to(dtype)
    kn = torch.randn((rows, 128), device=dev, generator=g).to(dtype)
    vn = torch.randn((rows, 128), device=dev, generator=g).to(dtype)
    chunk = ops.decode_chunk_tiles(a.host_len + 1, G, dtype)
    parts = ops.decode_num_parts(a.host_len + 1, chunk)
    ws = torch.empty(lib.hc_decode_workspace_size(rows, G, parts), dtype=torch.uint8, device=dev)
    out_ws = torch.empty_like(q)
    out_na = torch.full_like(q, float("nan"))
    assert _call(lib, a, q, kn, vn, out_ws, parts, chunk, ws) == 0
    rc = _call(lib, b, q, kn, vn, out_na, parts, chunk)
    assert rc == 0, lib.hc_last_error()
    torch.cuda.synchronize()
    assert torch.isfinite(out_ws.float()).all()
    assert torch.equal(out_ws, out_na)
    assert a.row_len.tolist() == b.row_len.tolist() == [n + 1 for n in lens]
    assert a.status.item() == b.status.item() == 0
    for r in range(rows):
        n = lens[r] + 1
        ka, va = a.read_rows([r], n)
        kb, vb = b.read_rows([r], n)
        assert torch.equal(ka, kb) and torch.equal(va, vb)


def test_noalloc_matches_workspace_entry_point_twice(dev):
    # Call 1: two sequences x 8 KV heads, ragged lengths (an empty row, a
    # one-token row, up to 40K tokens), GQA 4, bf16.
    rng = np.random.default_rng(21)
    big = [0, 1] + rng.integers(2, 40000, 14).tolist()
    _check_case(dev, big, 4, torch.bfloat16, 31)
    # Call 2, after it on the same device: a smaller input (5 rows, GQA 7,
    # float16) into the scratch the first call left behind.
    _check_case(dev, [700, 33, 2048, 5, 1200], 7, torch.float16, 32)


def _largest_fitting_parts(lib, rows, G, limit=16 << 20):
    """Largest part count whose workspace (hc_decode_workspace_size) fits the scratch."""
    lo, hi = 1, 1
    while lib.hc_decode_workspace_size(rows, G, hi) <= limit:
        lo, hi = hi, hi * 2
    while hi - lo > 1:
        mid = (lo + hi) // 2
        if lib.hc_decode_workspace_size(rows, G, mid) <= limit:
            lo = mid
        else:
            hi = mid
    return lo


def test_noalloc_accepts_the_largest_fitting_workspace_and_refuses_one_part_more(dev):
    """The scratch limit is exact: the largest grid whose workspace fits 16 MiB
    runs and matches the workspace entry point bit for bit (surplus
    workgroups find no chunk); one part more is refused before anything runs."""
    lib = _lib.load()
    lens, G, dtype = [64, 1, 0, 300, 31, 64, 2, 129], 16, torch.bfloat16
    rows = len(lens)
    parts = _largest_fitting_parts(lib, rows, G)
    assert lib.hc_decode_workspace_size(rows, G, parts) <= (16 << 20) < lib.hc_decode_workspace_size(rows, G, parts + 1)
    a, b = _twin_stores(lens, dtype, dev, 41)
    g = torch.Generator(device=dev).manual_seed(41)
    q = torch.randn((rows, G, 128), device=dev, generator=g).to(dtype)
    kn = torch.randn((rows, 128), device=dev, generator=g).to(dtype)
    vn = torch.randn((rows, 128), device=dev, generator=g).to(dtype)
    ws = torch.empty(lib.hc_decode_workspace_size(rows, G, parts), dtype=torch.uint8, device=dev)
    out_ws = torch.empty_like(q)
    out_na = torch.full_like(q, float("nan"))
    assert _call(lib, a, q, kn, vn, out_ws, parts, 4, ws) == 0
    rc = _call(lib, b, q, kn, vn, out_na, parts, 4)
    assert rc == 0, lib.hc_last_error()
    torch.cuda.synchronize()
    assert torch.isfinite(out_ws.float()).all() and torch.equal(out_ws, out_na)
    assert a.row_len.tolist() == b.row_len.tolist() == [n + 1 for n in lens]
    # One part more: refused, nothing launched (lengths and output unchanged).
    out = torch.zeros_like(q)
    rc = _call(lib, b, q, kn, vn, out, parts + 1, 4)
    assert rc == _lib.HC_ERR_INVALID
    assert b"16777216" in lib.hc_last_error()
    torch.cuda.synchronize()
    assert b.row_len.tolist() == [n + 1 for n in lens] and torch.equal(out, torch.zeros_like(out))
