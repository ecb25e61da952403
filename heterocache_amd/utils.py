"""Model set-up for HeteroCache: head reorder, head-data augmentation,
attention patching and cache injection.

Counterpart of heterocache/utils.py:
  reorder_model_weights_by_classification  (:71-175) permutes q/k/v/o head
      blocks so KV heads are ordered anchor, satellite, volatile, pivot
      (a stable sort, so heads of one type keep their order);
  augment_head_data                        (:300-343) derives the per-layer
      lists HeteroCache consumes and remaps leader_member_relations (leaders
      keep the JSON's order, members are sorted);
  install_attention_patch                  (:195-197) swaps the attention
      classes into transformers before a model is built;
  attach_cache                             (:372-383) makes generate() build a
      HeteroCache;
  load_model_and_tokenizer                 (:178-384) all of the above from a
      model directory, a method name and the head-analysis JSON found by its
      naming convention.
"""
import copy
import json
import os

import numpy as np
import torch

from .cache_utils import HeteroCache, HeteroCacheConfig

TYPE_ORDER = {1: 0, 4: 1, 2: 2, 3: 3}  # anchor, satellite, volatile, pivot


def head_permutation(layer_types):
    """KV-head order of one layer: stable sort by TYPE_ORDER (unknown types last)."""
    return sorted(range(len(layer_types)), key=lambda h: TYPE_ORDER.get(layer_types[h], 99))


def _permute_rows(weight, heads, head_dim, order):
    out_dim, d_in = weight.shape
    if out_dim != heads * head_dim:
        raise ValueError(f"weight has {out_dim} rows, expected {heads} x {head_dim}")
    return weight.reshape(heads, head_dim, d_in)[order].reshape(out_dim, d_in)


def _permute_cols(weight, heads, head_dim, order):
    d_out, in_dim = weight.shape
    if in_dim != heads * head_dim:
        raise ValueError(f"weight has {in_dim} columns, expected {heads} x {head_dim}")
    return weight.reshape(d_out, heads, head_dim)[:, order].reshape(d_out, in_dim)


@torch.no_grad()
def reorder_model_weights_by_classification(model, json_data):
    """Permute every layer's attention heads in place; returns the KV-head
    permutation (new position -> old head) of each layer."""
    cfg = model.config
    Hq, Hkv, L = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.num_hidden_layers
    head_dim = getattr(cfg, "head_dim", None) or cfg.hidden_size // Hq
    cls = json_data.get("classification_matrix")
    if cls is None:
        raise ValueError("JSON data must contain 'classification_matrix'.")
    if len(cls) != L:
        raise ValueError(f"Matrix layers ({len(cls)}) != Model layers ({L})")
    G = Hq // Hkv
    records = []
    for li, layer in enumerate(model.model.layers):
        types = cls[li][:Hkv]
        if len(types) != Hkv:
            raise ValueError(f"Layer {li}: JSON contains {len(types)} heads, but model has {Hkv} KV heads.")
        kv_order = head_permutation(types)
        q_order = [h * G + g for h in kv_order for g in range(G)]
        att = layer.self_attn
        att.q_proj.weight.copy_(_permute_rows(att.q_proj.weight, Hq, head_dim, q_order))
        att.k_proj.weight.copy_(_permute_rows(att.k_proj.weight, Hkv, head_dim, kv_order))
        att.v_proj.weight.copy_(_permute_rows(att.v_proj.weight, Hkv, head_dim, kv_order))
        for proj, heads, order in ((att.q_proj, Hq, q_order), (att.k_proj, Hkv, kv_order), (att.v_proj, Hkv, kv_order)):
            if proj.bias is not None:
                proj.bias.copy_(proj.bias.reshape(heads, head_dim)[order].reshape(-1))
        att.o_proj.weight.copy_(_permute_cols(att.o_proj.weight, Hq, head_dim, q_order))
        records.append(kv_order)
    return records


def augment_head_data(json_data, permutation_records):
    """Reordered allocation/classification plus the derived per-layer lists:
    need_to_compress_counts (anchor + satellite count: the first heads),
    need_to_select_counts (pivots), need_to_update_counts (satellites),
    need_to_keep_counts (volatile + pivot), and relations in new indices."""
    data = copy.deepcopy(json_data)
    for key in ("need_to_update_counts", "need_to_select_counts", "need_to_compress_counts", "need_to_keep_counts"):
        data.setdefault(key, [])
    for li, order in enumerate(permutation_records):
        order = list(order)
        cls = [data["classification_matrix"][li][h] for h in order]
        alloc = [data["allocation_matrix"][li][h] for h in order]
        data["classification_matrix"][li] = cls
        data["allocation_matrix"][li] = alloc
        data["need_to_compress_counts"].append(cls.count(1) + cls.count(4))
        data["need_to_select_counts"].append([i for i, t in enumerate(cls) if t == 3])
        data["need_to_update_counts"].append([i for i, t in enumerate(cls) if t == 4])
        data["need_to_keep_counts"].append([i for i, t in enumerate(cls) if t in (2, 3)])
        new_of = {old: new for new, old in enumerate(order)}
        rel = {}
        for leader, members in json_data["leader_member_relations"][li].items():
            if int(leader) in new_of:
                rel[str(new_of[int(leader)])] = sorted(new_of[m] for m in members if m in new_of)
        data["leader_member_relations"][li] = rel
    return data


def build_cache_config(model, data, compression_ratio=0.5, stable_threshold=0.5, real_offload=True,
                       max_gen_len=128, decode_step=5, pooling="avgpool", kernel_size=5, **extra):
    """HeteroCacheConfig for a model whose heads were reordered with `data`
    (heterocache/utils.py:289-362, including its ratio assertion)."""
    cfg = model.config
    total = cfg.num_key_value_heads * cfg.num_hidden_layers
    full = data["meta"]["counts"]["volatile"] + data["meta"]["counts"]["pivot"]
    if not int(compression_ratio * total) > full:
        raise AssertionError("Too many full KV cache heads retained (volatile+pivot) to satisfy the compression "
                             "ratio; lower the ratio or adjust clustering hyperparameters")
    return HeteroCacheConfig(data=data, compression_ratio=compression_ratio, stable_threshold=stable_threshold,
                             real_offload=real_offload, max_gen_len=max_gen_len, decode_step=decode_step,
                             pooling=pooling, kernel_size=kernel_size, num_attn_heads=cfg.num_attention_heads,
                             num_kv_heads=cfg.num_key_value_heads, num_layers=cfg.num_hidden_layers, **extra)


class install_attention_patch:
    """Swap this package's attention classes into transformers; do it before
    the model is constructed (the decoder layer instantiates the module
    global).  Usable as a plain call or as a context manager that restores
    the original classes on exit."""

    def __init__(self):
        import transformers.models.llama.modeling_llama as ml
        import transformers.models.qwen2.modeling_qwen2 as mq
        from .llama_model import LlamaAttention
        from .qwen_model import Qwen2Attention
        self._saved = [(ml, "LlamaAttention", ml.LlamaAttention), (mq, "Qwen2Attention", mq.Qwen2Attention)]
        ml.LlamaAttention = LlamaAttention
        mq.Qwen2Attention = Qwen2Attention

    def restore(self):
        for mod, name, cls in self._saved:
            setattr(mod, name, cls)

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.restore()
        return False


def attach_cache(model, cache_config):
    """Make generate() construct a HeteroCache(cache_config).

    With generation_config.prefill_chunk_size set (transformers' chunked
    prefill), the cache is told the prompt length, taken from the attention
    mask or else from max_length - max_new_tokens."""
    def _prepare_cache_for_generation(self, generation_config, model_kwargs, *args, **kwargs):
        cache = HeteroCache(cache_config)
        if getattr(generation_config, "prefill_chunk_size", None):
            mask = model_kwargs.get("attention_mask")
            if mask is not None:
                prompt = mask.shape[-1]
            elif generation_config.max_new_tokens is not None and generation_config.max_length is not None:
                prompt = generation_config.max_length - generation_config.max_new_tokens
            else:
                raise ValueError("chunked prefill needs the prompt length: pass attention_mask or max_new_tokens")
            cache.begin_prefill(prompt)
        model_kwargs["past_key_values"] = cache
    model._prepare_cache_for_generation = _prepare_cache_for_generation.__get__(model, model.__class__)
    return model


def head_analysis_path(load_dir, model_path, topk, stable_threshold, sim_threshold, decode_step):
    """The head-analysis JSON of a model, named as the reference names it
    (heterocache/utils.py:218-222)."""
    name = str(model_path).lower().rstrip("/").split("/")[-1]
    return os.path.join(load_dir, f"Head_Analysis_{name}_topk{topk}_th{stable_threshold}_sim{sim_threshold}"
                                  f"_step{decode_step}.json")


def attach_cache_factory(model, factory):
    """Make generate() construct its cache with factory()."""
    def _prepare_cache_for_generation(self, generation_config, model_kwargs, *args, **kwargs):
        model_kwargs["past_key_values"] = factory()
    model._prepare_cache_for_generation = _prepare_cache_for_generation.__get__(model, model.__class__)
    return model


def load_model_and_tokenizer(args):
    """Model and tokenizer with a KV-cache method attached
    (heterocache/utils.py:178-384).

    args (a namespace, as the reference's command line gives it): method
    (fullkv, snapkv, pyramidkv, streamingllm, h2o, cake, heterocache),
    model_path, compression_ratio, and for heterocache load_dir, topk,
    stable_threshold, sim_threshold, decode_step (the JSON's name),
    real_offload, max_gen_len, steps (the drift-check period).  Optional:
    attn_implementation (default "sdpa"), torch_dtype (default float16, as
    the reference), device_map (default "auto").  The attention classes are
    patched before the model is built (every method runs this package's
    kernels); heterocache reorders the heads by the JSON, augments it and
    checks the ratio as the reference does.  4-bit quantization (the
    reference's bitsandbytes path) is not provided.
    """
    from transformers import AutoModelForCausalLM, AutoTokenizer, DynamicCache
    from . import cache_utils as C
    method = args.method.lower()
    classes = {"fullkv": None, "snapkv": C.SnapKVCache, "pyramidkv": C.PyramidKVCache,
               "streamingllm": C.StreamingLLMKVCache, "h2o": C.H2OKVCache, "cake": C.CAKECache,
               "heterocache": HeteroCache}
    if method not in classes:
        raise ValueError(f"unknown method {args.method!r}; expected one of {sorted(classes)}")
    if getattr(args, "quant", False):
        raise NotImplementedError("4-bit quantization (bitsandbytes) is not provided by heterocache_amd")
    data = None
    if method == "heterocache":
        path = head_analysis_path(args.load_dir, args.model_path, args.topk, args.stable_threshold,
                                  args.sim_threshold, args.decode_step)
        with open(path, "r", encoding="utf-8") as f:
            data = json.load(f)
    dtype = getattr(args, "torch_dtype", torch.float16)
    with install_attention_patch():
        model = AutoModelForCausalLM.from_pretrained(
            args.model_path, torch_dtype=dtype, low_cpu_mem_usage=True,
            device_map=getattr(args, "device_map", "auto"),
            attn_implementation=getattr(args, "attn_implementation", "sdpa"))
    tokenizer = AutoTokenizer.from_pretrained(args.model_path, use_fast=True, padding_side="left")
    cfg = model.config
    common = {"pooling": "avgpool", "kernel_size": 5, "num_attn_heads": cfg.num_attention_heads,
              "num_kv_heads": cfg.num_key_value_heads, "num_layers": cfg.num_hidden_layers,
              "compression_ratio": args.compression_ratio}
    if method == "heterocache":
        perms = reorder_model_weights_by_classification(model, data)
        data = augment_head_data(data, perms)
        cache_config = build_cache_config(model, data, stable_threshold=args.stable_threshold,
                                          real_offload=args.real_offload, max_gen_len=args.max_gen_len,
                                          decode_step=args.steps, **{k: v for k, v in common.items()
                                                                     if k not in ("num_attn_heads", "num_kv_heads",
                                                                                  "num_layers")})
        attach_cache(model, cache_config)
    elif method == "fullkv":
        cache_config = {}
        attach_cache_factory(model, DynamicCache)
    else:
        cache_config = C.CompressionCacheConfig(window_size=32 if method == "cake" else 1, **common)
        cls = classes[method]
        attach_cache_factory(model, lambda: cls(cache_config))
    model.config.cache_config = cache_config
    return model, tokenizer
