"""Prefill attention (hc_prefill_attn) vs the float64 closed form of the oracle.

Parity bar: max-abs <= 2e-2 (bf16), 1e-2 (fp16), 1e-4 (fp32), the decode
bar: both kernels round the softmax probabilities to the input type for the
P.V product and accumulate in fp32.
"""
import math

import numpy as np
import pytest
import torch

from heterocache_amd import ops
from oracle import hc_oracle as O
from tests.gpu_util import ATTN_TOL, TORCH_DT, as_np

pytestmark = pytest.mark.gpu


def _inputs(dev, dt, B, Hq, Hkv, Lq, Lk, seed, layout="bhld", pad=0):
    """Seeded q [B, Hq, Lq, 128], k/v [B, Hkv, Lk, 128] on the device.

    layout "blhd" builds them as transposed views of [B, L, H, 128] tensors,
    the projections' layout.  `pad` extra NaN tokens follow each K/V row in
    memory, so a read past Lk would poison the output.
    """
    g = torch.Generator().manual_seed(seed)
    tdt = TORCH_DT[dt]
    q = torch.randn(B, Hq, Lq, 128, generator=g)
    k = torch.randn(B, Hkv, Lk, 128, generator=g)
    v = torch.randn(B, Hkv, Lk, 128, generator=g)
    k[..., :4] *= 6  # outlier channels, as post-RoPE keys carry
    if layout == "blhd":
        qd = q.transpose(1, 2).contiguous().to(tdt).to(dev).transpose(1, 2)
        kfull = torch.full((B, Lk + pad, Hkv, 128), float("nan"), dtype=tdt, device=dev)
        vfull = torch.full_like(kfull, float("nan"))
        kfull[:, :Lk] = k.transpose(1, 2).to(tdt).to(dev)
        vfull[:, :Lk] = v.transpose(1, 2).to(tdt).to(dev)
        kd, vd = kfull[:, :Lk].transpose(1, 2), vfull[:, :Lk].transpose(1, 2)
    else:
        qd = q.to(tdt).to(dev)
        kfull = torch.full((B, Hkv, Lk + pad, 128), float("nan"), dtype=tdt, device=dev)
        vfull = torch.full_like(kfull, float("nan"))
        kfull[:, :, :Lk] = k.to(tdt).to(dev)
        vfull[:, :, :Lk] = v.to(tdt).to(dev)
        kd, vd = kfull[:, :, :Lk], vfull[:, :, :Lk]
    return qd, kd, vd


CASES = [
    # B, Hq, Hkv, Lq, Lk
    (1, 8, 2, 300, 300),     # whole prompt, GQA 4, ragged last block
    (2, 4, 4, 64, 200),      # chunk over staged keys, no GQA, batch 2
    (1, 7, 1, 1, 129),       # one query (GQA 7), keys past a tile edge
    (1, 4, 1, 130, 1000),    # chunk spanning two query blocks
    (1, 2, 1, 1, 1),         # single key
    (1, 4, 2, 33, 33),       # just past one 32-token tile
    (1, 28, 4, 256, 256),    # Qwen2.5-7B head geometry
]


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("case", CASES)
def test_prefill_matches_oracle(dev, dt, case):
    B, Hq, Hkv, Lq, Lk = case
    seed = 2000 + sum(case)
    print(f"prefill_attn dt={dt} B={B} Hq={Hq} Hkv={Hkv} Lq={Lq} Lk={Lk} seed={seed}", flush=True)
    q, k, v = _inputs(dev, dt, B, Hq, Hkv, Lq, Lk, seed, pad=40)
    scale = 1.0 / math.sqrt(128)
    out = ops.prefill_attn(q, k, v, scale)
    torch.cuda.synchronize()
    ref = O.prefill_attention(as_np(q), as_np(k), as_np(v), scale)
    got = as_np(out)
    assert np.isfinite(got).all()
    err = np.abs(got - ref).max()
    assert err <= ATTN_TOL[dt], f"max-abs {err}"


@pytest.mark.parametrize("dt", ["bf16", "f32"])
def test_prefill_projection_layout_and_out_view(dev, dt):
    """Inputs as transposed [B, L, H, 128] views; output written into a view
    of a wider buffer; other elements untouched."""
    B, Hq, Hkv, Lq, Lk = 2, 8, 2, 150, 150
    print(f"prefill_attn layout dt={dt}", flush=True)
    q, k, v = _inputs(dev, dt, B, Hq, Hkv, Lq, Lk, 77, layout="blhd", pad=8)
    buf = torch.full((B, Lq, Hq, 256), 7.0, dtype=q.dtype, device=dev)
    out = buf[..., 64:192]
    ops.prefill_attn(q, k, v, 0.1, out=out)
    torch.cuda.synchronize()
    ref = O.prefill_attention(as_np(q), as_np(k), as_np(v), 0.1)
    assert np.abs(as_np(out) - ref).max() <= ATTN_TOL[dt]
    assert (buf[..., :64] == 7).all() and (buf[..., 192:] == 7).all()


def test_prefill_chunks_equal_whole_prompt(dev):
    """Chunked prefill: attention of each chunk over the keys staged so far
    matches the rows of the whole-prompt call (same kernel, same keys)."""
    B, Hq, Hkv, L, C = 1, 8, 2, 700, 256
    print("prefill_attn chunks", flush=True)
    q, k, v = _inputs(dev, "bf16", B, Hq, Hkv, L, L, 99)
    whole = ops.prefill_attn(q, k, v, 1 / math.sqrt(128))
    parts = []
    for s in range(0, L, C):
        e = min(L, s + C)
        parts.append(ops.prefill_attn(q[:, :, s:e], k[:, :, :e], v[:, :, :e], 1 / math.sqrt(128)))
    torch.cuda.synchronize()
    chunked = torch.cat(parts, dim=1)
    ref = O.prefill_attention(as_np(q), as_np(k), as_np(v))
    assert np.abs(as_np(chunked) - ref).max() <= ATTN_TOL["bf16"]
    assert np.abs(as_np(chunked) - as_np(whole)).max() <= ATTN_TOL["bf16"]


def test_prefill_rejects_bad_shapes(dev):
    q = torch.zeros(1, 4, 10, 128, dtype=torch.bfloat16, device=dev)
    k = torch.zeros(1, 2, 5, 128, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError):
        ops.prefill_attn(q, k, k, 0.1)          # more queries than keys
    k3 = torch.zeros(1, 3, 20, 128, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError):
        ops.prefill_attn(q, k3, k3, 0.1)        # 4 query heads over 3 KV heads


@pytest.mark.parametrize("dt", ["bf16", "f32"])
@pytest.mark.parametrize("case", [(1, 8, 2, 300, 300, 32), (2, 4, 4, 64, 200, 64), (1, 7, 1, 1, 129, 1),
                                  (1, 28, 4, 256, 256, 32), (1, 4, 1, 130, 1000, 7)])
def test_prefill_stats(dev, dt, case):
    """hc_prefill_attn_stats: the output is bit-identical to hc_prefill_attn's,
    and each of the last W queries' (M, L) gives the oracle's base-2
    log-normaliser over its visible keys, M + log2 L, within 1e-3 (log2
    units), with M inside [max s - 8, max s]."""
    B, Hq, Hkv, Lq, Lk, W = case
    seed = 3000 + sum(case)
    print(f"prefill_attn_stats dt={dt} B={B} Hq={Hq} Hkv={Hkv} Lq={Lq} Lk={Lk} W={W} seed={seed}", flush=True)
    q, k, v = _inputs(dev, dt, B, Hq, Hkv, Lq, Lk, seed, pad=40)
    scale = 1.0 / math.sqrt(128)
    plain = ops.prefill_attn(q, k, v, scale)
    st = torch.full((B, Hq, W, 2), float("nan"), dtype=torch.float32, device=dev)
    out = ops.prefill_attn(q, k, v, scale, stat_out=st)
    torch.cuda.synchronize()
    assert torch.equal(out, plain)
    G = Hq // Hkv
    qn, kn = as_np(q), as_np(k)
    rows, ks = [], []
    for b in range(B):
        for h in range(Hkv):
            for w in range(W):
                i = Lq - W + w
                rows.append(qn[b, h * G:(h + 1) * G, i])
                ks.append(kn[b, h, :Lk - Lq + i + 1])
    ref = O.softmax_lse2(np.stack(rows), ks, Lk, scale).reshape(B, Hkv, W, G).transpose(0, 1, 3, 2)
    ref = ref.reshape(B, Hq, W)
    got = as_np(st)
    M, Ls = got[..., 0], got[..., 1]
    assert np.isfinite(M).all() and (Ls >= 1.0).all()
    assert np.abs(M + np.log2(Ls) - ref).max() <= 1e-3
    # The bound: the row maxima of the scaled base-2 scores.
    smax = np.array([(scale * math.log2(math.e) * (r.astype(np.float64) @ kk.astype(np.float64).T)).max(axis=-1)
                     for r, kk in zip(rows, ks)]).reshape(B, Hkv, W, G).transpose(0, 1, 3, 2).reshape(B, Hq, W)
    assert (M <= smax + 1e-3).all() and (M >= smax - 8 - 1e-3).all()


def test_prefill_stats_rejects_bad_rows(dev):
    q, k, v = _inputs(dev, "bf16", 1, 4, 1, 16, 16, 5)
    for shape in ((1, 4, 17, 2), (1, 4, 0, 2), (1, 2, 8, 2)):
        st = torch.zeros(shape, dtype=torch.float32, device=dev)
        with pytest.raises((RuntimeError, ValueError)):
            ops.prefill_attn(q, k, v, 0.1, stat_out=st)


SPLIT_CASES = [
    # B, Hq, Hkv, Lq, Lk: one query block per (row, query head) over many keys
    (1, 32, 8, 1, 20000),     # a decode-like step (baseline caches)
    (1, 28, 4, 7, 9000),      # GQA 7, a few queries
    (2, 8, 2, 100, 30000),    # a short last chunk, batch 2
    (1, 4, 1, 128, 5000),     # a full query block
]


def _nbytes(dt, B, Hq, Hkv, Lq, Lk):
    from heterocache_amd import _lib
    lib = _lib.load()
    code = {"bf16": 2, "f16": 1, "f32": 0}[dt]
    return lib.hc_prefill_workspace_size(code, B, Hkv, Lk), lib.hc_prefill_workspace_bytes(code, B, Hq, Hkv, Lq, Lk)


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("case", SPLIT_CASES)
def test_prefill_key_split_matches_oracle(dev, dt, case):
    """Short calls over long key ranges split the keys across workgroups
    (the workspace of hc_prefill_workspace_bytes holds the partials): the
    output meets the oracle at the unsplit tolerance, and a call given only
    the unsplit workspace (one pass) agrees with it to the same bar."""
    from heterocache_amd import _lib
    B, Hq, Hkv, Lq, Lk = case
    seed = 4000 + sum(case)
    print(f"prefill_attn split dt={dt} B={B} Hq={Hq} Hkv={Hkv} Lq={Lq} Lk={Lk} seed={seed}", flush=True)
    vt, full = _nbytes(dt, B, Hq, Hkv, Lq, Lk)
    assert full > vt, "the shape should take the key split"
    q, k, v = _inputs(dev, dt, B, Hq, Hkv, Lq, Lk, seed, pad=40)
    scale = 1.0 / math.sqrt(128)
    out = ops.prefill_attn(q, k, v, scale)
    # The same call with only the V-tile workspace: one pass over the keys.
    lib = _lib.load()
    one = torch.empty((B, Lq, Hq, 128), dtype=q.dtype, device=dev)
    ws = torch.empty(vt, dtype=torch.uint8, device=dev)
    strides = np.array([[q.stride(0), q.stride(1), q.stride(2)], [k.stride(0), k.stride(1), k.stride(2)],
                        [v.stride(0), v.stride(1), v.stride(2)], [one.stride(0), one.stride(2), one.stride(1)]],
                       dtype=np.int64)
    base = strides.ctypes.data
    _lib.check(lib.hc_prefill_attn(ops.dtype_code(q.dtype), q.data_ptr(), base, k.data_ptr(), base + 24, v.data_ptr(),
                                   base + 48, one.data_ptr(), base + 72, B, Hq, Hkv, Lq, Lk, scale, ws.data_ptr(),
                                   ws.numel(), torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    ref = O.prefill_attention(as_np(q), as_np(k), as_np(v), scale)
    got = as_np(out)
    assert np.isfinite(got).all()
    assert np.abs(got - ref).max() <= ATTN_TOL[dt]
    assert np.abs(got - as_np(one)).max() <= ATTN_TOL[dt]


def test_prefill_key_split_statistics(dev):
    """Statistics from a split call: the merge folds the splits' (m, l) into
    the oracle's log-normaliser (1e-3, log2 units), M inside [max s - 8, max s]."""
    B, Hq, Hkv, Lq, Lk, W = 1, 8, 2, 32, 20000, 32
    vt, full = _nbytes("bf16", B, Hq, Hkv, Lq, Lk)
    assert full > vt
    q, k, v = _inputs(dev, "bf16", B, Hq, Hkv, Lq, Lk, 77)
    scale = 1.0 / math.sqrt(128)
    st = torch.full((B, Hq, W, 2), float("nan"), dtype=torch.float32, device=dev)
    out = ops.prefill_attn(q, k, v, scale, stat_out=st)
    plain = ops.prefill_attn(q, k, v, scale)
    torch.cuda.synchronize()
    assert torch.equal(out, plain)
    G = Hq // Hkv
    qn, kn = as_np(q), as_np(k)
    rows, ks = [], []
    for h in range(Hkv):
        for w in range(W):
            i = Lq - W + w
            rows.append(qn[0, h * G:(h + 1) * G, i])
            ks.append(kn[0, h, :Lk - Lq + i + 1])
    ref = O.softmax_lse2(np.stack(rows), ks, Lk, scale).reshape(1, Hkv, W, G).transpose(0, 1, 3, 2).reshape(1, Hq, W)
    got = as_np(st)
    assert np.abs(got[..., 0] + np.log2(got[..., 1]) - ref).max() <= 1e-3
    smax = np.array([(scale * math.log2(math.e) * (r.astype(np.float64) @ kk.astype(np.float64).T)).max(axis=-1)
                     for r, kk in zip(rows, ks)]).reshape(1, Hkv, W, G).transpose(0, 1, 3, 2).reshape(1, Hq, W)
    assert (got[..., 0] <= smax + 1e-3).all() and (got[..., 0] >= smax - 8 - 1e-3).all()


DECODE_SHAPED_CASES = [
    # B, Hq, Hkv, Lq, Lk: at most 16 (query head, query) columns per KV row
    (1, 32, 8, 1, 131072),    # a Llama-3-8B decode step at 128K
    (2, 28, 4, 2, 5000),      # GQA 7, two queries: 14 columns, batch 2
    (1, 8, 8, 16, 3001),      # no GQA, 16 queries, a ragged last tile
    (3, 4, 2, 8, 1100),       # GQA 2 x 8 queries, batch 3
]


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("case", DECODE_SHAPED_CASES)
def test_prefill_decode_shaped_matches_oracle(dev, dt, case):
    """Decode-shaped calls (a KV row's query heads x queries packed into one
    MFMA column block, K and V read in their natural layout, V transposed
    through LDS): the oracle at the unsplit tolerance, also with NaN-filled
    slots past the keys."""
    B, Hq, Hkv, Lq, Lk = case
    seed = 5000 + sum(case)
    print(f"prefill_attn decode-shaped dt={dt} B={B} Hq={Hq} Hkv={Hkv} Lq={Lq} Lk={Lk} seed={seed}", flush=True)
    vt, full = _nbytes(dt, B, Hq, Hkv, Lq, Lk)
    assert full > vt
    q, k, v = _inputs(dev, dt, B, Hq, Hkv, Lq, Lk, seed, pad=40)
    scale = 1.0 / math.sqrt(128)
    out = ops.prefill_attn(q, k, v, scale)
    torch.cuda.synchronize()
    ref = O.prefill_attention(as_np(q), as_np(k), as_np(v), scale)
    got = as_np(out)
    assert np.isfinite(got).all()
    assert np.abs(got - ref).max() <= ATTN_TOL[dt]


def test_prefill_decode_shaped_statistics(dev):
    """Statistics of a decode-shaped call: the oracle's log-normaliser within
    1e-3 (log2 units), the bound within 8 of the row maximum."""
    B, Hq, Hkv, Lq, Lk, W = 1, 8, 2, 4, 20000, 4
    q, k, v = _inputs(dev, "bf16", B, Hq, Hkv, Lq, Lk, 78)
    scale = 1.0 / math.sqrt(128)
    st = torch.full((B, Hq, W, 2), float("nan"), dtype=torch.float32, device=dev)
    out = ops.prefill_attn(q, k, v, scale, stat_out=st)
    plain = ops.prefill_attn(q, k, v, scale)
    torch.cuda.synchronize()
    assert torch.equal(out, plain)
    G = Hq // Hkv
    qn, kn = as_np(q), as_np(k)
    rows, ks = [], []
    for h in range(Hkv):
        for w in range(W):
            i = Lq - W + w
            rows.append(qn[0, h * G:(h + 1) * G, i])
            ks.append(kn[0, h, :Lk - Lq + i + 1])
    ref = O.softmax_lse2(np.stack(rows), ks, Lk, scale).reshape(1, Hkv, W, G).transpose(0, 1, 3, 2).reshape(1, Hq, W)
    got = as_np(st)
    assert np.abs(got[..., 0] + np.log2(got[..., 1]) - ref).max() <= 1e-3
    smax = np.array([(scale * math.log2(math.e) * (r.astype(np.float64) @ kk.astype(np.float64).T)).max(axis=-1)
                     for r, kk in zip(rows, ks)]).reshape(1, Hkv, W, G).transpose(0, 1, 3, 2).reshape(1, Hq, W)
    assert (got[..., 0] <= smax + 1e-3).all() and (got[..., 0] >= smax - 8 - 1e-3).all()
