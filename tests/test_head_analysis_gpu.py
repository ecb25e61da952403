"""Head-classification JSON producer (heterocache_amd.head_analysis) vs the
oracle's restatement of tools/get_cluster.py, on seeded synthetic attention
maps: the classification, star clusters, counts and allocation ratios must
match (sets are compared exactly; the maps are continuous random values, so
the pooled scores have no ties at the top-k threshold)."""
import numpy as np
import pytest
import torch

from heterocache_amd import head_analysis
from oracle import hc_oracle as O
from tests.gpu_util import as_np

pytestmark = pytest.mark.gpu


def synthetic_maps(rng, layers, B, Hq, Hkv, S, steps):
    """Per layer: KV heads 0 and 1 share a pattern (a star), KV head 2 is
    stable, the rest drift between steps."""
    G = Hq // Hkv
    maps = {}
    for layer in range(layers):
        base = rng.random((B, Hkv, 1, S)).astype(np.float32)
        base[:, 1] = base[:, 0] + 0.01 * rng.random((B, 1, S)).astype(np.float32)
        per = {}
        for step in range(steps):
            m = base + 0.01 * rng.random(base.shape).astype(np.float32)
            if step:
                m[:, 3:] = rng.random((B, Hkv - 3, 1, S))
            # query heads of a KV head: the KV pattern plus small per-head noise
            q = np.repeat(m, G, axis=1) + 0.001 * rng.random((B, Hq, 1, S)).astype(np.float32)
            per[step] = np.concatenate([rng.random((B, Hq, 2, S)).astype(np.float32), q], axis=2)  # 3 rows
        maps[layer] = per
    return maps


def test_head_analysis_json_matches_oracle(dev):
    rng = np.random.default_rng(21)
    L, B, Hq, Hkv, S = 3, 2, 24, 6, 700
    maps_np = synthetic_maps(rng, L, B, Hq, Hkv, S, 6)
    maps = {l: {s: torch.as_tensor(m).to(dev) for s, m in per.items()} for l, per in maps_np.items()}
    kw = dict(topk=64, max_length=650, stable_threshold=0.5, sim_threshold=0.5, decode_step=5)
    got = head_analysis.analyze(maps, L, Hq, Hkv, **kw)
    ref = O.head_analysis(maps_np, L, Hq, Hkv, **kw)
    assert got["classification_matrix"] == ref["classification_matrix"]
    assert got["leader_member_relations"] == ref["leader_member_relations"]
    assert got["meta"] == ref["meta"]
    np.testing.assert_allclose(np.asarray(got["allocation_matrix"]), np.asarray(ref["allocation_matrix"]),
                               rtol=1e-12, atol=1e-12)
    # The synthetic structure is found: a star over KV heads 0-1, head 2 an anchor.
    for layer in range(L):
        assert got["leader_member_relations"][layer] == {0: [1]}
        assert got["classification_matrix"][layer][:3] == [3, 4, 1]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_head_topk_sets_match_oracle(dev, dtype):
    rng = np.random.default_rng(22)
    a = rng.random((2, 8, 2, 300)).astype(np.float32)
    t = torch.as_tensor(a).to(dtype).to(dev)
    idx, k, H, span = head_analysis.head_topk_sets(t, 8, 2, 280, 30)
    sets, H2 = O.head_topk_sets(as_np(t), 8, 2, 280, 30, io_dtype=None if dtype == torch.float32 else "bfloat16")
    assert (H, k, span) == (H2, 30, 280)
    got = idx.cpu().numpy()
    for b in range(2):
        for h in range(H):
            assert set(got[b * H + h, :k].tolist()) == sets[h][b]
