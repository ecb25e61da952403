"""The reference's configurations run through the kernels at their own
shapes (or at reduced lengths where noted), checked against the oracle.

Config 0: one Llama-3-8B-shape layer in float32 at 4096 tokens -- SnapKV
window scoring (W = 32, max pool 7), per-head budgets 1024 / 3072 with the
window force-kept, the kept rows gathered into the store, then one decode
step (fused append + attention over the ragged cap_h + 1 rows).
"""
import math

import numpy as np
import pytest
import torch

from heterocache_amd import compress, workloads
from heterocache_amd.store import KVStore
from oracle import hc_oracle as O
from tests.gpu_util import as_np

pytestmark = pytest.mark.gpu


def test_config0_snapkv_layer_then_decode(dev):
    c = workloads.config0_inputs()
    L, W, Hkv, G = 4096, c["window"], 8, 4
    caps = [int(x) for x in c["caps"]]
    q = torch.as_tensor(c["q"]).to(dev)
    k = torch.as_tensor(c["k"]).to(dev)
    v = torch.as_tensor(c["v"]).to(dev)
    scores = compress.window_scores(q, k, range(Hkv), G, W, "maxpool", 7, window_keep=True)
    idx, counts = compress.select_kept(scores, caps, window=W)
    torch.cuda.synchronize()
    qw = np.stack([c["q"][0, h * G:(h + 1) * G, L - W:] for h in range(Hkv)])
    ref_s = O.window_scores(qw, c["k"][0], "maxpool", 7, window_keep=True)
    got_s = as_np(scores)
    assert np.max(np.abs(got_s - ref_s) / np.maximum(np.abs(ref_s), 1e-30)) < 2e-4
    idx_np, counts_np = idx.cpu().numpy(), counts.cpu().numpy()
    kept = []
    for h in range(Hkv):
        got = idx_np[h, :counts_np[h]].astype(np.int64)
        ref = O.select_with_window(ref_s[h], caps[h], L, W)
        assert len(got) == caps[h] and np.all(np.diff(got) > 0)
        assert got[-W:].tolist() == list(range(L - W, L))
        # Positions may only differ where the oracle score ties the budget
        # threshold within float32 noise.
        body = ref_s[h][:L - W]
        tau = np.sort(body)[::-1][caps[h] - W - 1]
        diff = set(got.tolist()).symmetric_difference(ref.tolist())
        assert all(abs(body[t] - tau) <= 1e-5 * abs(tau) for t in diff), f"head {h}"
        kept.append(got)
    # Gather the kept rows and run one decode step with the fused append.
    st = KVStore([cp + 1 for cp in caps], torch.float32, dev)
    st.write_rows(k, v, [(0, h) for h in range(Hkv)], list(range(Hkv)), caps, idx=idx)
    qd = torch.as_tensor(c["q_dec"]).to(dev).reshape(Hkv, G, 128)
    kd = torch.as_tensor(c["k_dec"]).to(dev).reshape(Hkv, 128)
    vd = torch.as_tensor(c["v_dec"]).to(dev).reshape(Hkv, 128)
    out = st.attend(qd, 1.0 / math.sqrt(128), k_new=kd, v_new=vd)
    torch.cuda.synchronize()
    ks = [np.concatenate([c["k"][0, h][kept[h]], c["k_dec"][0, h]]) for h in range(Hkv)]
    vs = [np.concatenate([c["v"][0, h][kept[h]], c["v_dec"][0, h]]) for h in range(Hkv)]
    ref = O.decode_attention(c["q_dec"][0].reshape(Hkv, G, 128), ks, vs)
    assert np.abs(as_np(out) - ref).max() <= 1e-4
    assert st.host_len.tolist() == [cp + 1 for cp in caps]


def test_config3_qwen_gqa7_ragged_batch_decode(dev):
    """Config 3 geometry (Qwen2.5-7B: 4 KV heads, GQA 7, ratio 0.25) with
    four sequences of ragged contexts 16/32/48/64K in one launch, one row
    per (sequence, KV head): each sequence's budgets follow its own context
    (the reference handles batch rows one sequence at a time).  One decode
    step with the fused append, bf16, against the float64 oracle."""
    NL, Hkv, G = 28, 4, 7
    contexts = [16384, 32768, 49152, 65536]
    # One full-KV head per layer pair (14 of 112 heads) and compressed heads
    # with allocation weights 0.5 / 1.0 / 1.5 (mean 1).
    lens = []
    for L in contexts:
        base = workloads.get_compress_len(0.25, 14, L, Hkv * NL)
        lens.extend([L] + [int(np.trunc(np.float32(base) * np.float32(w))) for w in (0.5, 1.0, 1.5)])
    rng = np.random.default_rng(1003)
    rows = len(lens)
    ks = [rng.standard_normal((n, 128)).astype(np.float32) for n in lens]
    vs = [rng.standard_normal((n, 128)).astype(np.float32) for n in lens]
    st = KVStore([n + 1 for n in lens], torch.bfloat16, dev)
    Lmax = max(lens)
    src_k = torch.zeros((1, rows, Lmax, 128), dtype=torch.bfloat16)
    src_v = torch.zeros_like(src_k)
    for r, n in enumerate(lens):
        src_k[0, r, :n] = torch.as_tensor(ks[r])
        src_v[0, r, :n] = torch.as_tensor(vs[r])
    st.write_rows(src_k.to(dev), src_v.to(dev), [(0, r) for r in range(rows)], list(range(rows)), lens)
    q = torch.as_tensor(rng.standard_normal((rows, G, 128)), dtype=torch.float32).to(torch.bfloat16).to(dev)
    kn = torch.as_tensor(rng.standard_normal((rows, 128)), dtype=torch.float32).to(torch.bfloat16).to(dev)
    vn = torch.as_tensor(rng.standard_normal((rows, 128)), dtype=torch.float32).to(torch.bfloat16).to(dev)
    out = st.attend(q, 1.0 / math.sqrt(128), k_new=kn, v_new=vn)
    torch.cuda.synchronize()
    kk = [np.concatenate([as_np(src_k[0, r, :n]), as_np(kn[r:r + 1])]) for r, n in enumerate(lens)]
    vv = [np.concatenate([as_np(src_v[0, r, :n]), as_np(vn[r:r + 1])]) for r, n in enumerate(lens)]
    ref = O.decode_attention(as_np(q), kk, vv)
    assert np.abs(as_np(out) - ref).max() <= 2e-2
    assert len(set(lens)) > 4  # ragged across sequences and heads
