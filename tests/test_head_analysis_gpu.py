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


def test_calibration_maps_match_eager_attention_and_feed_the_producer(dev, tmp_path):
    """collect_maps on a random-init Llama: the recorded last-row attention
    of the prefill and of every decode step equals the stock model's eager
    attention rows (float32); the files it writes load back with load_maps;
    the JSON built from the recorded maps equals the oracle's."""
    from transformers import LlamaConfig, LlamaForCausalLM
    from heterocache_amd import utils
    def config(impl):
        return LlamaConfig(vocab_size=512, hidden_size=8 * 128, intermediate_size=1024, num_hidden_layers=2,
                           num_attention_heads=8, num_key_value_heads=2, head_dim=128, max_position_embeddings=4096,
                           attn_implementation=impl)
    cfg = config("sdpa")
    with utils.install_attention_patch():
        torch.manual_seed(0)
        model = LlamaForCausalLM(cfg).to(torch.float32).to(dev).eval()
    ids = torch.randint(0, 512, (1, 300), generator=torch.Generator().manual_seed(9)).to(dev)
    maps, out = head_analysis.collect_maps(model, ids, 4, save_dir=str(tmp_path))
    assert sorted(maps) == [0, 1] and sorted(maps[0]) == [300, 301, 302, 303]
    torch.manual_seed(0)
    ref_model = LlamaForCausalLM(config("eager")).to(torch.float32).to(dev).eval()
    with torch.no_grad():
        att = ref_model(out[:, :303], output_attentions=True).attentions
    for layer in range(2):
        for n in range(300, 304):
            got = as_np(maps[layer][n])[0, :, 0]
            want = as_np(att[layer])[0, :, n - 1, :n]
            np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-6)
    back = head_analysis.load_maps(str(tmp_path), device=dev)
    assert sorted(back) == [0, 1] and all(torch.equal(back[l][n], maps[l][n]) for l in back for n in back[l])
    kw = dict(topk=32, max_length=300, stable_threshold=0.5, sim_threshold=0.3, decode_step=303)
    got = head_analysis.analyze(maps, 2, 8, 2, **kw)
    ref = O.head_analysis({l: {n: as_np(m) for n, m in per.items()} for l, per in maps.items()}, 2, 8, 2, **kw)
    assert got["classification_matrix"] == ref["classification_matrix"]
    assert got["leader_member_relations"] == ref["leader_member_relations"]
    np.testing.assert_allclose(np.asarray(got["allocation_matrix"]), np.asarray(ref["allocation_matrix"]),
                               rtol=1e-12, atol=1e-12)
