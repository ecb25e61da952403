"""hc_drift_select and hc_score's key histogram against the oracle.

The drift selection is integer work on a given score array, so it is checked
bit-exact: per step row the overlap |top-K ∩ reference set| with the oracle's
ranking (descending score, ties -> lower position first;
oracle.hc_oracle.topk_indices), the trigger per leader as
oracle.hc_oracle.drift_check decides it (batch-mean overlap / K, median over
the steps, < threshold), and the rewritten reference sets (top-K of the last
step for sets whose leader triggered, untouched otherwise).  Score arrays with
heavy ties, constant rows, signed zeros and negative values exercise the
threshold bin, the tie cut and the key order.  Every case runs with the
histograms passed in (built here in numpy) and built by the selection itself.
"""
import numpy as np
import pytest
import torch

from heterocache_amd import ops
from oracle import hc_oracle as O
from tests.gpu_util import as_np

pytestmark = pytest.mark.gpu


def order_keys(x):
    """Order-preserving uint32 keys of float32 values (-0 ranks as +0)."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).copy()
    u[u == 0x80000000] = 0
    neg = (u & 0x80000000) != 0
    return np.where(neg, ~u, u | 0x80000000).astype(np.uint32)


def key_hist(scores):
    """[rows, 4096] counts of the top 12 key bits."""
    k = order_keys(scores) >> 20
    return np.stack([np.bincount(r, minlength=ops.HIST_BINS) for r in k]).astype(np.int32)


def make_scores(kind, rows, L, rng):
    if kind == "continuous":
        s = rng.random((rows, L), dtype=np.float32) * 1e-4
    elif kind == "ties":       # eight distinct values: the threshold lies inside a tie run
        s = (rng.integers(0, 8, (rows, L)) * 1e-5).astype(np.float32)
    elif kind == "constant":
        s = np.full((rows, L), 3e-5, dtype=np.float32)
    elif kind == "signed":     # negatives, both zeros, and a few large values
        s = rng.standard_normal((rows, L)).astype(np.float32)
        s[:, ::7] = 0.0
        s[:, 3::7] = -0.0
        s[:, 5::101] = 1e6
    else:
        raise ValueError(kind)
    return s


def bits_of(idx_sets, words):
    out = np.zeros((len(idx_sets), words), dtype=np.uint32)
    for j, ix in enumerate(idx_sets):
        t = np.asarray(ix, dtype=np.int64)
        np.bitwise_or.at(out[j], t >> 5, (np.uint32(1) << (t & 31).astype(np.uint32)))
    return out


def set_of(bits_row, L):
    b = np.asarray(bits_row, dtype=np.uint32)
    pos = np.nonzero((b[np.arange(L) >> 5] >> (np.arange(L) & 31).astype(np.uint32)) & 1)[0]
    return pos


@pytest.mark.parametrize("L,K,kind", [
    (4099, 1365, "continuous"),
    (4099, 1365, "ties"),
    (4099, 2000, "constant"),
    (3000, 1000, "signed"),
    (4099, 1, "ties"),
    (4099, 4098, "ties"),
    (1000, 1000, "continuous"),      # K = span: everything kept
    (131072, 49629, "continuous"),   # 128K context at ratio 0.5 of the reference's base budget
    (131072, 49629, "ties"),
])
@pytest.mark.parametrize("own_hist", [False, True])
def test_drift_select_matches_oracle(dev, L, K, kind, own_hist):
    rng = np.random.default_rng(L * 7 + K + len(kind))
    nlead, B, S, thr = 3, 2, 5, 0.5
    nsets, njobs = nlead * B, nlead * B * S
    words = (L + 31) // 32 + 3            # spare words past the span must end up zero
    scores = make_scores(kind, njobs, L, rng)
    Kc = min(K, L)
    # Reference sets: leader 0 = its last step's own top-K (overlap 1 on
    # that step), leader 1 = random (low overlap), leader 2 = half of its
    # first step's top-K and half random.
    ref_idx = []
    for i in range(nlead):
        for b in range(B):
            j = i * B + b
            if i == 0:
                ref_idx.append(O.topk_indices(scores[j * S + S - 1], Kc))
            elif i == 1:
                ref_idx.append(rng.choice(L, Kc, replace=False))
            else:
                top = O.topk_indices(scores[j * S], Kc)[: Kc // 2]
                rest = np.setdiff1d(np.arange(L), top)
                ref_idx.append(np.concatenate([top, rng.choice(rest, Kc - len(top), replace=False)]))
    ref_bits = bits_of(ref_idx, words)
    ref_bits[:, (L + 31) // 32:] = 0xFFFFFFFF       # junk past the span
    bits = torch.as_tensor(ref_bits.view(np.int32)).to(dev)
    caps = torch.full((njobs,), K, dtype=torch.int32, device=dev)
    trig_of = torch.arange(nlead, dtype=torch.int32, device=dev).repeat_interleave(B)
    trigger = torch.full((nlead,), 7, dtype=torch.int32, device=dev)
    hist = None if own_hist else torch.as_tensor(key_hist(scores)).to(dev)
    sc = torch.as_tensor(scores).to(dev)
    overlap = ops.drift_select(sc, caps, K, bits, L, trig_of, nlead, B, S, thr, trigger, hist)
    torch.cuda.synchronize()

    exp_overlap = np.zeros(njobs, dtype=np.int64)
    for j in range(nsets):
        ref = set(np.asarray(ref_idx[j]).tolist())
        for s in range(S):
            cur = O.topk_indices(scores[j * S + s], Kc)
            exp_overlap[j * S + s] = len(ref.intersection(cur.tolist()))
    np.testing.assert_array_equal(as_np(overlap).astype(np.int64), exp_overlap)

    exp_bits = ref_bits.copy()
    exp_trig = []
    for i in range(nlead):
        st = scores[i * B * S:(i + 1) * B * S].reshape(B, S, L)
        _, _, trig, cur_last = O.drift_check(st, [ref_idx[i * B + b] for b in range(B)], Kc, thr)
        exp_trig.append(int(trig))
        if trig:
            exp_bits[i * B:(i + 1) * B] = bits_of(cur_last, words)
    np.testing.assert_array_equal(as_np(trigger), np.asarray(exp_trig))
    got = bits.cpu().numpy().view(np.uint32)
    for j in range(nsets):
        if exp_trig[j // B]:
            np.testing.assert_array_equal(got[j], exp_bits[j], err_msg=f"set {j}")
            assert set_of(got[j], L).size == Kc
        else:
            np.testing.assert_array_equal(got[j], ref_bits[j], err_msg=f"untriggered set {j} changed")


def test_drift_select_repeat_and_smaller(dev):
    """Two calls in a row on the same buffers, the second over a shorter
    span: no state from the first call leaks into the second."""
    rng = np.random.default_rng(5)
    nlead, B, S = 2, 1, 5
    for L, K in ((8192, 3000), (2048, 700)):
        scores = make_scores("ties", nlead * B * S, L, rng)
        words = (L + 31) // 32
        ref_idx = [rng.choice(L, K, replace=False) for _ in range(nlead * B)]
        bits = torch.as_tensor(bits_of(ref_idx, words).view(np.int32)).to(dev)
        trigger = torch.zeros(nlead, dtype=torch.int32, device=dev)
        ov = ops.drift_select(torch.as_tensor(scores).to(dev), torch.full((nlead * B * S,), K, dtype=torch.int32,
                              device=dev), K, bits, L, torch.arange(nlead, dtype=torch.int32, device=dev), nlead,
                              B, S, 0.5, trigger, torch.as_tensor(key_hist(scores)).to(dev))
        exp = [len(set(ref_idx[j // S].tolist()).intersection(O.topk_indices(scores[j], K).tolist()))
               for j in range(nlead * B * S)]
        np.testing.assert_array_equal(as_np(ov), exp)


def test_score_hist_counts_the_scores(dev):
    """hc_score's histogram output equals the first-digit key histogram of
    the scores it wrote, for every (job, step) row."""
    g = torch.Generator().manual_seed(11)
    B, Hkv, G, W, L = 2, 2, 4, 5, 3000
    q = torch.randn((B, Hkv * G, W, 128), generator=g).to(torch.bfloat16).to(dev)
    k = torch.randn((B, Hkv, L, 128), generator=g).to(torch.bfloat16).to(dev)
    jobs = [(b, h) for b in range(B) for h in range(Hkv)]
    q_off = torch.tensor([b * q.stride(0) + h * G * q.stride(1) for b, h in jobs], dtype=torch.int64, device=dev)
    k_off = torch.tensor([b * k.stride(0) + h * k.stride(1) for b, h in jobs], dtype=torch.int64, device=dev)
    hist = torch.full((len(jobs) * W, ops.HIST_BINS), 99, dtype=torch.int32, device=dev)   # zeroed by the call
    for pooling in ("avgpool", "maxpool"):
        s = ops.score(q, q_off, q.stride(1), q.stride(2), k, k_off, k.stride(2), L, G, W, L, pooling, 5,
                      128 ** -0.5, hist=hist)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(as_np(hist), key_hist(as_np(s).reshape(len(jobs) * W, L)))


def test_score_hist_refused_for_large_query_sets(dev):
    B, Hkv, G, W, L = 1, 1, 7, 5, 512      # 35 query rows
    q = torch.randn((B, Hkv * G, W, 128), device=dev).to(torch.bfloat16)
    k = torch.randn((B, Hkv, L, 128), device=dev).to(torch.bfloat16)
    zero = torch.zeros(1, dtype=torch.int64, device=dev)
    hist = torch.zeros((W, ops.HIST_BINS), dtype=torch.int32, device=dev)
    with pytest.raises(Exception, match="histogram"):
        ops.score(q, zero, q.stride(1), q.stride(2), k, zero, k.stride(2), L, G, W, L, "avgpool", 5, 128 ** -0.5,
                  hist=hist)


@pytest.mark.parametrize("kind", ["ascending_dense", "ascending_sparse", "shuffled", "duplicates_and_out_of_range"])
def test_set_bits_matches_numpy(dev, kind):
    """hc_set_bits: bitmaps of position lists (the pivot reference sets) are
    the lists' sets exactly, for ascending lists dense and sparse in their
    words, shuffled ones, and lists with repeats and positions outside
    [0, nbits) (ignored); per-set counts and a fixed count; a set beyond the
    LDS path's 262144 positions; whole rows (row stride) cleared first."""
    rng = np.random.default_rng(len(kind))
    for nbits, nsets in ((131072, 3), (4099, 2), (300000, 2)):
        words = (nbits + 31) // 32
        lists, counts = [], []
        for j in range(nsets):
            n = {0: nbits // 2, 1: 1000, 2: 37}[j % 3]
            if kind == "ascending_sparse":
                n = min(n, nbits // 64)
            x = np.sort(rng.choice(nbits, size=min(n, nbits), replace=False))
            if kind == "shuffled":
                x = rng.permutation(x)
            if kind == "duplicates_and_out_of_range":
                x = np.concatenate([x, x[: len(x) // 3], [-5, nbits, nbits + 77, -1]])
                x = rng.permutation(x)
            lists.append(x.astype(np.int32))
            counts.append(len(x))
        width = max(counts) + 3
        idx = np.full((nsets, width), 7, dtype=np.int32)  # past each count: must be ignored
        for j, x in enumerate(lists):
            idx[j, :len(x)] = x
        bits = torch.full((nsets, words + 5), -1, dtype=torch.int32, device=dev)
        ops.set_bits(torch.tensor(idx, device=dev), torch.tensor(counts, dtype=torch.int32, device=dev), bits, nbits)
        got = bits.cpu().numpy()
        for j, x in enumerate(lists):
            ref = np.zeros(words * 32, dtype=bool)
            v = x[(x >= 0) & (x < nbits)]
            ref[v] = True
            row = np.unpackbits(got[j, :words].view(np.uint8), bitorder="little").astype(bool)
            assert np.array_equal(row, ref), (kind, nbits, j)
            assert np.all(got[j, words:] == 0), "the row's padding words are cleared too"
        # A fixed count: the first count positions of every row.
        k = min(counts)
        bits2 = torch.zeros((nsets, words), dtype=torch.int32, device=dev)
        ops.set_bits(torch.tensor(idx, device=dev), None, bits2, nbits, fixed_count=k)
        got2 = bits2.cpu().numpy()
        for j, x in enumerate(lists):
            ref = np.zeros(words * 32, dtype=bool)
            v = x[:k]
            ref[v[(v >= 0) & (v < nbits)]] = True
            assert np.array_equal(np.unpackbits(got2[j].view(np.uint8), bitorder="little").astype(bool), ref)


def test_set_bits_row_order_matches_reordered_lists(dev):
    """hc_set_bits(row_of): set j takes its list from row row_of[j] of a
    larger selection, the same bitmaps as the reordered lists copied first."""
    rng = np.random.default_rng(5)
    nbits, rows, width = 131072, 10, 50000
    idx = np.stack([np.sort(rng.choice(nbits, size=width, replace=False)) for _ in range(rows)]).astype(np.int32)
    order = np.asarray([7, 2, 9, 2], dtype=np.int64)
    words = nbits // 32
    got = torch.zeros((len(order), words), dtype=torch.int32, device=dev)
    ref = torch.zeros_like(got)
    ti = torch.tensor(idx, device=dev)
    ops.set_bits(ti, None, got, nbits, fixed_count=40000, row_of=torch.tensor(order, device=dev))
    ops.set_bits(ti[torch.tensor(order, device=dev)].contiguous(), None, ref, nbits, fixed_count=40000)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)
    g = got.cpu().numpy()
    for j, r in enumerate(order):
        want = np.zeros(words * 32, dtype=bool)
        want[idx[r, :40000]] = True
        assert np.array_equal(np.unpackbits(g[j].view(np.uint8), bitorder="little").astype(bool), want)
