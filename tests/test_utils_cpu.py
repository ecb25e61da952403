"""Head reorder and head-data augmentation (CPU only)."""
import json
import os

import numpy as np
import pytest
import torch
from transformers import LlamaConfig, LlamaForCausalLM

from heterocache_amd import utils, workloads
from heterocache_amd.cache_utils import HeteroCacheConfig, get_compress_len
from oracle import hc_oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def test_augment_matches_oracle_plan_on_reference_json():
    raw = json.load(open(os.path.join(GOLDEN, "head_analysis_llama-3.1-8b-instruct.json")))
    perms = [utils.head_permutation(row) for row in raw["classification_matrix"]]
    data = utils.augment_head_data(raw, perms)
    for li, row in enumerate(raw["classification_matrix"]):
        plan = O.reorder_plan(row, raw["leader_member_relations"][li])
        assert perms[li] == plan["perm"]
        assert data["need_to_compress_counts"][li] == plan["compress"]
        assert data["need_to_select_counts"][li] == plan["select"]
        assert data["need_to_update_counts"][li] == plan["update"]
        assert data["need_to_keep_counts"][li] == plan["keep"]
        assert list(data["leader_member_relations"][li].items()) == list(plan["relations"].items())
        assert data["allocation_matrix"][li] == [raw["allocation_matrix"][li][h] for h in plan["perm"]]
    # the input record is not modified
    assert raw["leader_member_relations"][23] == {"6": [0, 1, 2, 3, 5], "4": [7]}


def tiny_llama(seed=0):
    torch.manual_seed(seed)
    cfg = LlamaConfig(vocab_size=97, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
                      num_attention_heads=8, num_key_value_heads=4, head_dim=16, max_position_embeddings=256,
                      attention_bias=True)
    cfg._attn_implementation = "eager"
    m = LlamaForCausalLM(cfg).eval()
    for layer in m.model.layers:  # non-zero biases so their permutation is exercised
        for p in (layer.self_attn.q_proj, layer.self_attn.k_proj, layer.self_attn.v_proj, layer.self_attn.o_proj):
            torch.nn.init.normal_(p.bias, std=0.1)
    return m


def test_reorder_preserves_the_model_function():
    m = tiny_llama()
    ids = torch.randint(0, 97, (1, 40), generator=torch.Generator().manual_seed(1))
    with torch.no_grad():
        before = m(ids).logits
    data = {"classification_matrix": [[3, 1, 4, 2], [2, 4, 4, 3]]}
    rec = utils.reorder_model_weights_by_classification(m, data)
    assert rec == [[1, 2, 3, 0], [1, 2, 0, 3]]
    with torch.no_grad():
        after = m(ids).logits
    assert torch.allclose(before, after, atol=1e-5)


def test_reorder_rejects_mismatched_json():
    m = tiny_llama()
    with pytest.raises(ValueError):
        utils.reorder_model_weights_by_classification(m, {"classification_matrix": [[1, 1, 1, 1]]})
    with pytest.raises(ValueError):
        utils.reorder_model_weights_by_classification(m, {})


def test_build_cache_config_ratio_assertion():
    m = tiny_llama()
    data = {"meta": {"counts": {"volatile": 3, "pivot": 2}}}
    cfg = utils.build_cache_config(m, data, compression_ratio=0.75)
    assert isinstance(cfg, HeteroCacheConfig) and cfg.num_kv_heads == 4 and cfg.num_layers == 2
    with pytest.raises(AssertionError):
        utils.build_cache_config(m, data, compression_ratio=0.5)  # int(0.5 * 8) = 4 <= 5 full heads


def test_synthetic_head_json_schema_and_budget_identity():
    d = workloads.synthetic_head_json(32, 8, 1002)
    assert set(d) == {"meta", "classification_matrix", "allocation_matrix", "leader_member_relations"}
    vals = [a for row in d["allocation_matrix"] for a in row if a > -0.5]
    assert abs(np.mean(vals) - 1.0) < 1e-9
    total = sum(workloads.row_budgets(d, l, 131072, 0.5, 32, 8)[0].sum() for l in range(32))
    assert abs(total / (0.5 * 256 * 131072) - 1.0) < 1e-3
    assert get_compress_len(0.5, 50, 131072, 256) == O.get_compress_len(0.5, 50, 131072, 256) == 49629


# -- load_model_and_tokenizer (heterocache/utils.py:178-384) ---------------------
def _saved_model_dir(tmp_path, classes, relations):
    """A random-init 2-layer Llama and a word-level tokenizer saved with
    save_pretrained, and its head-analysis JSON under the reference's name."""
    from tokenizers import Tokenizer, models, pre_tokenizers
    from transformers import PreTrainedTokenizerFast
    cfg = LlamaConfig(vocab_size=520, hidden_size=4 * 128, intermediate_size=512, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, head_dim=128, max_position_embeddings=1024)
    torch.manual_seed(0)
    model_dir = tmp_path / "Tiny-Llama-Test"
    LlamaForCausalLM(cfg).save_pretrained(model_dir)
    vocab = {f"w{i}": i for i in range(512)}
    vocab.update({"[UNK]": 512, "[PAD]": 513})
    tok = Tokenizer(models.WordLevel(vocab=vocab, unk_token="[UNK]"))
    tok.pre_tokenizer = pre_tokenizers.Whitespace()
    PreTrainedTokenizerFast(tokenizer_object=tok, unk_token="[UNK]", pad_token="[PAD]").save_pretrained(model_dir)
    names = {1: "anchor", 2: "volatile", 3: "pivot", 4: "satellite"}
    counts = {n: sum(t == k for row in classes for t in row) for k, n in names.items()}
    stab = [[0.5 if t in (1, 4) else -1.0 for t in row] for row in classes]
    raw = {"meta": {"type_map": dict(workloads.TYPE_MAP), "counts": counts}, "classification_matrix": classes,
           "allocation_matrix": workloads.inverse_stability_allocation(stab), "leader_member_relations": relations}
    load_dir = tmp_path / "clusters"
    load_dir.mkdir()
    path = utils.head_analysis_path(str(load_dir), str(model_dir), 1024, 0.5, 0.5, 5000)
    with open(path, "w") as f:
        json.dump(raw, f)
    return model_dir, load_dir, raw


def _args(model_dir, load_dir, method="heterocache", **kw):
    from types import SimpleNamespace
    a = SimpleNamespace(method=method, model_path=str(model_dir), load_dir=str(load_dir), topk=1024,
                        stable_threshold=0.5, sim_threshold=0.5, decode_step=5000, compression_ratio=0.75,
                        real_offload=True, max_gen_len=64, steps=5, quant=False, attn_implementation="sdpa",
                        torch_dtype=torch.float32, device_map="cpu")
    a.__dict__.update(kw)
    return a


def test_load_model_and_tokenizer_heterocache(tmp_path):
    from heterocache_amd.llama_model import LlamaAttention
    classes = [[3, 4], [1, 2]]
    model_dir, load_dir, raw = _saved_model_dir(tmp_path, classes, [{"0": [1]}, {}])
    model, tok = utils.load_model_and_tokenizer(_args(model_dir, load_dir))
    assert isinstance(model.model.layers[0].self_attn, LlamaAttention)
    assert tok.padding_side == "left" and tok("w3 w7")["input_ids"] == [3, 7]
    # Heads reordered by the JSON (layer 0: pivot, satellite -> satellite, pivot).
    plain = LlamaForCausalLM.from_pretrained(model_dir, torch_dtype=torch.float32)
    k0, k1 = model.model.layers[0].self_attn.k_proj.weight, plain.model.layers[0].self_attn.k_proj.weight
    assert torch.equal(k0[:128], k1[128:]) and torch.equal(k0[128:], k1[:128])
    assert torch.equal(model.model.layers[1].self_attn.k_proj.weight, plain.model.layers[1].self_attn.k_proj.weight)
    cc = model.config.cache_config
    assert isinstance(cc, HeteroCacheConfig) and cc.decode_step == 5 and cc.max_gen_len == 64
    assert cc.data["need_to_select_counts"] == [[1], []] and cc.data["need_to_update_counts"] == [[0], []]
    assert cc.data["leader_member_relations"] == [{"1": [0]}, {}]
    kwargs = {}
    model._prepare_cache_for_generation(None, kwargs)
    assert type(kwargs["past_key_values"]).__name__ == "HeteroCache"


def test_load_model_and_tokenizer_other_methods_and_errors(tmp_path):
    from heterocache_amd import cache_utils as C
    model_dir, load_dir, raw = _saved_model_dir(tmp_path, [[3, 4], [1, 2]], [{"0": [1]}, {}])
    for method, cls, window in (("snapkv", C.SnapKVCache, 1), ("cake", C.CAKECache, 32),
                                ("streamingllm", C.StreamingLLMKVCache, 1)):
        model, _ = utils.load_model_and_tokenizer(_args(model_dir, load_dir, method=method))
        assert model.config.cache_config.window_size == window
        kwargs = {}
        model._prepare_cache_for_generation(None, kwargs)
        assert isinstance(kwargs["past_key_values"], cls)
    model, _ = utils.load_model_and_tokenizer(_args(model_dir, load_dir, method="FullKV"))
    kwargs = {}
    model._prepare_cache_for_generation(None, kwargs)
    assert type(kwargs["past_key_values"]).__name__ == "DynamicCache"
    with pytest.raises(ValueError, match="unknown method"):
        utils.load_model_and_tokenizer(_args(model_dir, load_dir, method="rocketkv"))
    with pytest.raises(NotImplementedError):
        utils.load_model_and_tokenizer(_args(model_dir, load_dir, quant=True))
    with pytest.raises(FileNotFoundError):
        utils.load_model_and_tokenizer(_args(model_dir, load_dir, topk=512))
    # The reference's ratio assertion: 3 of 4 heads full at ratio 0.75.
    with open(utils.head_analysis_path(str(load_dir), str(model_dir), 1024, 0.5, 0.5, 5000), "w") as f:
        bad = dict(raw, classification_matrix=[[3, 2], [2, 1]],
                   meta={"type_map": raw["meta"]["type_map"],
                         "counts": {"anchor": 1, "volatile": 2, "pivot": 1, "satellite": 0}})
        json.dump(bad, f)
    with pytest.raises(AssertionError, match="Too many full KV cache heads"):
        utils.load_model_and_tokenizer(_args(model_dir, load_dir))
