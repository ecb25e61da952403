"""HeteroCache through transformers generate() on small random-init models.

* Budgets that keep every token (one anchor head at ratio 1.0, all other heads
  full): greedy tokens must equal the stock model's full-KV generation
  (float32 weights).
* Compressed bf16 Llama (ratio 0.5, pivots + satellites, decode_step 5) and
  Qwen2 (GQA 7, batch 2): generation runs through prefill selection, fused
  decode attention, drift checks and retrieval, with lengths advancing by
  one per generated token.
"""
import math

import numpy as np
import pytest
import torch
from transformers import LlamaConfig, LlamaForCausalLM, Qwen2Config, Qwen2ForCausalLM

from heterocache_amd import ops, utils, workloads
from heterocache_amd.cache_utils import HeteroCache
from oracle import hc_oracle as O
from tests.gpu_util import as_np

pytestmark = pytest.mark.gpu


def llama_cfg(layers=2, q_heads=4, kv_heads=2):
    return LlamaConfig(vocab_size=512, hidden_size=q_heads * 128, intermediate_size=1024, num_hidden_layers=layers,
                       num_attention_heads=q_heads, num_key_value_heads=kv_heads, head_dim=128,
                       max_position_embeddings=4096, attn_implementation="sdpa")


def head_json(classes, relations, stab_seed=0):
    rng = np.random.default_rng(stab_seed)
    names = {1: "anchor", 2: "volatile", 3: "pivot", 4: "satellite"}
    counts = {n: 0 for n in names.values()}
    for row in classes:
        for t in row:
            counts[names[t]] += 1
    stab = [[float(rng.uniform(0.3, 0.9)) if t in (1, 4) else -1.0 for t in row] for row in classes]
    return {"meta": {"type_map": dict(workloads.TYPE_MAP), "counts": counts},
            "classification_matrix": classes, "allocation_matrix": workloads.inverse_stability_allocation(stab),
            "leader_member_relations": relations}


def build(model_cls, cfg, raw, dtype, dev, **cache_kw):
    with utils.install_attention_patch():
        torch.manual_seed(0)
        model = model_cls(cfg).to(dtype).to(dev).eval()
    perms = utils.reorder_model_weights_by_classification(model, raw)
    data = utils.augment_head_data(raw, perms)
    cc = utils.build_cache_config(model, data, **cache_kw)
    utils.attach_cache(model, cc)
    return model, cc


def test_uncompressed_budgets_match_full_kv_generation(dev):
    cfg = llama_cfg()
    # 4 KV heads in total: 3 volatile + 1 anchor whose budget is the whole prompt.
    raw = head_json([[2, 1], [2, 2]], [{}, {}])
    raw["allocation_matrix"] = [[-1.0, 1.0], [-1.0, -1.0]]
    ids = torch.randint(0, 512, (1, 300), generator=torch.Generator().manual_seed(3)).to(dev)
    torch.manual_seed(0)
    ref_model = LlamaForCausalLM(cfg).to(torch.float32).to(dev).eval()
    with torch.no_grad():
        ref = ref_model.generate(ids, max_new_tokens=12, do_sample=False)
    model, cc = build(LlamaForCausalLM, cfg, raw, torch.float32, dev, compression_ratio=1.0, max_gen_len=16)
    with torch.no_grad():
        out = model.generate(ids, max_new_tokens=12, do_sample=False)
    assert torch.equal(out, ref)


def test_compressed_llama_generation_runs(dev):
    cfg = llama_cfg(layers=3, q_heads=8, kv_heads=4)
    classes = [[4, 3, 4, 1], [1, 1, 2, 4], [3, 4, 4, 1]]
    relations = [{"1": [0, 2]}, {}, {"0": [1, 2]}]
    raw = head_json(classes, relations)
    model, cc = build(LlamaForCausalLM, cfg, raw, torch.bfloat16, dev, compression_ratio=0.5, max_gen_len=24,
                      decode_step=5, retrieval_topk=64)
    ids = torch.randint(0, 512, (1, 1000), generator=torch.Generator().manual_seed(4)).to(dev)
    caches = []
    orig = HeteroCache.__init__

    def spy(self, c):
        orig(self, c)
        caches.append(self)
    HeteroCache.__init__ = spy
    try:
        with torch.no_grad():
            out = model.generate(ids, max_new_tokens=16, do_sample=False)
    finally:
        HeteroCache.__init__ = orig
    assert out.shape == (1, 1016)
    cache = caches[-1]
    torch.cuda.synchronize()
    lens = [t.tolist() for t in cache.heads_len]
    # 15 decode forwards after the prefill (the last token is never fed back).
    for layer, row in enumerate(lens):
        caps = cache.layer_head_capacities[layer]
        keep = set(cc.data["need_to_keep_counts"][layer])
        for h, n in enumerate(row):
            if h in keep:
                assert n == 1000 + 15
            else:
                assert n <= caps[h] + 15


def test_qwen2_gqa7_batch2_generation_runs(dev):
    cfg = Qwen2Config(vocab_size=512, hidden_size=7 * 2 * 128, intermediate_size=1024, num_hidden_layers=2,
                      num_attention_heads=14, num_key_value_heads=2, head_dim=128, max_position_embeddings=4096,
                      attn_implementation="sdpa")
    raw = head_json([[3, 4], [1, 2]], [{"0": [1]}, {}])
    model, cc = build(Qwen2ForCausalLM, cfg, raw, torch.bfloat16, dev, compression_ratio=0.75, max_gen_len=16,
                      decode_step=5)
    ids = torch.randint(0, 512, (2, 600), generator=torch.Generator().manual_seed(5)).to(dev)
    with torch.no_grad():
        out = model.generate(ids, attention_mask=torch.ones_like(ids), max_new_tokens=11, do_sample=False)
    assert out.shape == (2, 611)


def test_chunked_prefill_generation_matches_single_shot(dev):
    """generate(prefill_chunk_size=256) on a compressed Llama: the chunks'
    attention runs over the keys staged so far, selection runs once on the
    whole prompt, and the greedy tokens equal the single-shot run's."""
    cfg = llama_cfg(layers=3, q_heads=8, kv_heads=4)
    classes = [[4, 3, 4, 1], [1, 1, 2, 4], [3, 4, 4, 1]]
    relations = [{"1": [0, 2]}, {}, {"0": [1, 2]}]
    model, cc = build(LlamaForCausalLM, cfg, head_json(classes, relations), torch.bfloat16, dev,
                      compression_ratio=0.5, max_gen_len=24, decode_step=5, retrieval_topk=64)
    ids = torch.randint(0, 512, (1, 1000), generator=torch.Generator().manual_seed(6)).to(dev)
    with torch.no_grad():
        whole = model.generate(ids, max_new_tokens=16, do_sample=False)
        chunked = model.generate(ids, max_new_tokens=16, do_sample=False, prefill_chunk_size=256)
    assert torch.equal(whole, chunked)


@pytest.mark.parametrize("name", ["snapkv", "pyramidkv", "h2o", "streamingllm"])
def test_baseline_caches_generate(dev, name):
    """The baseline compressor caches through generate() on a random Llama:
    with a ratio that keeps every token the greedy tokens equal the stock
    model's; with ratio 0.3 each layer holds its compressor's kept rows plus
    the generated tokens."""
    from heterocache_amd import cache_utils as C
    classes = {"snapkv": C.SnapKVCache, "pyramidkv": C.PyramidKVCache, "h2o": C.H2OKVCache,
               "streamingllm": C.StreamingLLMKVCache}
    cfg = llama_cfg(layers=2, q_heads=8, kv_heads=2)
    with utils.install_attention_patch():
        torch.manual_seed(0)
        model = LlamaForCausalLM(cfg).to(torch.float32).to(dev).eval()
    torch.manual_seed(0)
    ref_model = LlamaForCausalLM(cfg).to(torch.float32).to(dev).eval()
    ids = torch.randint(0, 512, (1, 400), generator=torch.Generator().manual_seed(7)).to(dev)
    with torch.no_grad():
        ref = ref_model.generate(ids, max_new_tokens=8, do_sample=False)
        keep_all = C.CompressionCacheConfig(window_size=16, compression_ratio=50.0, num_attn_heads=8, num_kv_heads=2,
                                            num_layers=2)
        out = model.generate(ids, max_new_tokens=8, do_sample=False, past_key_values=classes[name](keep_all))
    assert torch.equal(out, ref)
    cache = classes[name](C.CompressionCacheConfig(window_size=16, compression_ratio=0.3, num_attn_heads=8,
                                                   num_kv_heads=2, num_layers=2))
    with torch.no_grad():
        out = model.generate(ids, max_new_tokens=8, do_sample=False, past_key_values=cache)
    assert out.shape == (1, 408)
    for layer in range(2):
        n = cache.key_cache[layer].shape[2]
        assert cache.key_cache[layer].shape[1] == 8           # repeated per query head
        assert n < 400 and n > 7                              # compressed, then 7 appended tokens


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_full_kv_decode_through_decode_shaped_attention(dev, dtype):
    """A long prompt (1500 tokens, above the 32 key tiles from which a decode
    step takes the decode-shaped attention) through a keep-every-token
    SnapKV cache: the decode steps attend over the whole cache through
    hc_prefill_attn's packed-column kernel.  fp32: the greedy tokens equal the
    stock model's; bf16: each decode step's attention output of the patched
    model stays within the bf16 bar of the float64 closed form."""
    from heterocache_amd import cache_utils as C
    from heterocache_amd import llama_model as LM
    cfg = llama_cfg(layers=2, q_heads=8, kv_heads=2)
    with utils.install_attention_patch():
        torch.manual_seed(0)
        model = LlamaForCausalLM(cfg).to(dtype).to(dev).eval()
    ids = torch.randint(0, 512, (1, 1500), generator=torch.Generator().manual_seed(8)).to(dev)
    keep_all = C.CompressionCacheConfig(window_size=16, compression_ratio=50.0, num_attn_heads=8, num_kv_heads=2,
                                        num_layers=2)
    if dtype == torch.float32:
        torch.manual_seed(0)
        ref_model = LlamaForCausalLM(cfg).to(dtype).to(dev).eval()
        with torch.no_grad():
            ref = ref_model.generate(ids, max_new_tokens=6, do_sample=False)
            out = model.generate(ids, max_new_tokens=6, do_sample=False, past_key_values=C.SnapKVCache(keep_all))
        assert torch.equal(out, ref)
        return
    seen = []

    def check(layer, q, k, mask, scale):
        if q.shape[2] == 1:
            seen.append((q.detach().clone(), k.detach().clone()))
    LM.ATTENTION_OBSERVERS.append(check)
    try:
        with torch.no_grad():
            model.generate(ids, max_new_tokens=3, do_sample=False, past_key_values=C.SnapKVCache(keep_all))
    finally:
        LM.ATTENTION_OBSERVERS.remove(check)
    assert seen and all(k.shape[2] >= 1500 for _, k in seen)
    # The observed decode calls re-run through ops.prefill_attn against the oracle.
    for q, k in seen[:2]:
        v = torch.randn(k.shape, generator=torch.Generator().manual_seed(9)).to(dtype).to(dev)
        got = ops.prefill_attn(q, k, v, 1 / math.sqrt(128))
        torch.cuda.synchronize()
        ref = O.prefill_attention(as_np(q), as_np(k), as_np(v), 1 / math.sqrt(128))
        assert np.abs(as_np(got) - ref).max() <= 2e-2


def test_cake_cache_generate(dev):
    """CAKECache through generate(): a ratio that keeps every token gives the
    stock model's greedy tokens; at ratio 0.3 the layer budgets add up to
    (int(0.3 L) - W) * layers and each layer holds its kept rows, the
    window and the generated tokens, one row per KV head."""
    from heterocache_amd import cache_utils as C
    cfg = llama_cfg(layers=2, q_heads=8, kv_heads=2)
    with utils.install_attention_patch():
        torch.manual_seed(0)
        model = LlamaForCausalLM(cfg).to(torch.float32).to(dev).eval()
    torch.manual_seed(0)
    ref_model = LlamaForCausalLM(cfg).to(torch.float32).to(dev).eval()
    ids = torch.randint(0, 512, (1, 400), generator=torch.Generator().manual_seed(8)).to(dev)

    def config(ratio):
        return C.CompressionCacheConfig(window_size=32, compression_ratio=ratio, num_attn_heads=8, num_kv_heads=2,
                                        num_layers=2)
    with torch.no_grad():
        ref = ref_model.generate(ids, max_new_tokens=8, do_sample=False)
        out = model.generate(ids, max_new_tokens=8, do_sample=False, past_key_values=C.CAKECache(config(50.0)))
    assert torch.equal(out, ref)
    cache = C.CAKECache(config(0.3))
    with torch.no_grad():
        out = model.generate(ids, max_new_tokens=8, do_sample=False, past_key_values=cache)
    assert out.shape == (1, 408)
    assert sum(cache.layer_budget) == (int(0.3 * 400) - 32) * 2
    for layer in range(2):
        assert cache.key_cache[layer].shape[1] == 2
        assert 32 + 7 < cache.key_cache[layer].shape[2] <= cache.layer_budget[layer] + 32 + 7


def test_temp_kv_cache_through_patched_attention(dev):
    """update_global_past_kv = False on the attention modules reaches the
    baseline cache (the reference passes it in cache_kwargs): a decode
    forward then keeps its token in the temporary cache, gives the same
    logits as a global append, and clear_temp_kv_cache drops it."""
    from heterocache_amd import cache_utils as C
    cfg = llama_cfg(layers=2, q_heads=8, kv_heads=2)
    with utils.install_attention_patch():
        torch.manual_seed(0)
        model = LlamaForCausalLM(cfg).to(torch.float32).to(dev).eval()
    ids = torch.randint(0, 512, (1, 300), generator=torch.Generator().manual_seed(8)).to(dev)
    mk = lambda: C.SnapKVCache(C.CompressionCacheConfig(window_size=16, compression_ratio=0.3, num_attn_heads=8,
                                                         num_kv_heads=2, num_layers=2))
    glob, temp = mk(), mk()
    nxt = torch.tensor([[5]], device=dev)
    pos = torch.tensor([[300]], device=dev)
    with torch.no_grad():
        model(ids, past_key_values=glob, use_cache=True)
        model(ids, past_key_values=temp, use_cache=True)
        kept = [temp.key_cache[l].shape[2] for l in range(2)]
        ref = model(nxt, past_key_values=glob, use_cache=True, position_ids=pos).logits
        attn = [layer.self_attn for layer in model.model.layers]
        for a in attn:
            a.update_global_past_kv = False
        try:
            got = model(nxt, past_key_values=temp, use_cache=True, position_ids=pos).logits
        finally:
            for a in attn:
                del a.update_global_past_kv
    assert [temp.key_cache[l].shape[2] for l in range(2)] == kept
    assert [tuple(t.shape[1:3]) for t in temp.temp_key_cache] == [(8, 1), (8, 1)]  # one token per query head
    assert torch.allclose(got, ref, atol=1e-5, rtol=0)
    seen = temp._seen_tokens
    temp.clear_temp_kv_cache()
    assert temp.temp_key_cache == [] and temp._seen_tokens == seen - 1


def test_load_model_and_tokenizer_generate(dev, tmp_path):
    """Models loaded by utils.load_model_and_tokenizer from a saved
    directory and a head JSON found by the reference's naming convention:
    HeteroCache generation in float16 (the reference's load dtype) runs
    through prefill selection, drift checks and retrieval; the full-KV
    method in float32 gives the stock model's greedy tokens."""
    from tests.test_utils_cpu import _args, _saved_model_dir
    model_dir, load_dir, _ = _saved_model_dir(tmp_path, [[3, 4], [1, 2]], [{"0": [1]}, {}])
    model, tok = utils.load_model_and_tokenizer(_args(model_dir, load_dir, torch_dtype=torch.float16,
                                                      device_map="cuda:0", max_gen_len=32))
    text = " ".join(f"w{(7 * i) % 512}" for i in range(600))
    ids = tok(text, return_tensors="pt")["input_ids"].to(dev)
    with torch.no_grad():
        out = model.generate(ids, max_new_tokens=12, do_sample=False)
    assert out.shape == (1, 612)
    full, _ = utils.load_model_and_tokenizer(_args(model_dir, load_dir, method="fullkv", torch_dtype=torch.float32,
                                                   device_map="cuda:0"))
    stock = LlamaForCausalLM.from_pretrained(model_dir, torch_dtype=torch.float32).to(dev).eval()
    with torch.no_grad():
        a = full.generate(ids[:, :300], max_new_tokens=10, do_sample=False)
        b = stock.generate(ids[:, :300], max_new_tokens=10, do_sample=False)
    assert torch.equal(a, b)
