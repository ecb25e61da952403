"""Llama attention with HeteroCache on libhc kernels.

Drop-in for heterocache/llama_model.py:279-405 (`LlamaAttention`): same
constructor, same forward contract, the same cache calls:
  prefill: update -> full causal attention over the uncompressed K/V
           (hc_prefill_attn, reporting the last queries' softmax
           statistics) -> init_coefficient -> prefill_select -> o_proj;
           the reference selects before it attends, but neither step reads
           what the other writes, so moving the attention first changes no
           result and lets the selection scorers reuse its normalisers.  In
           a chunked prefill every chunk runs this branch, and the two
           selection calls act once the declared prompt is complete
  decode:  update -> decode attention (hc_decode_attn, replacing
           flash_attn_with_kvcache) -> decode_select -> o_proj
The forward accepts the transformers 4.57 keyword set (attention_mask,
position_ids, output_attentions, use_cache, cache_position,
position_embeddings, past_key_values) and the 5.x one (extra **kwargs).
"""
import weakref
from typing import Optional, Tuple

import torch
import torch.nn as nn
from transformers.models.llama.modeling_llama import apply_rotary_pos_emb

from . import ops
from .cache_utils import HeteroCache

# Callables observer(layer_idx, query_states, key_states, attention_mask,
# scaling) run by the patched attention after a cache update that is not a
# HeteroCache's (keys are the layer's whole cache, one row per KV head): the
# attention recording of tools/get_weights.py:30-138 hooks in here
# (head_analysis.AttentionRecorder).
ATTENTION_OBSERVERS = []


# The last 4-D mask checked by _plain_causal (weakly held) and the result.
_MASK_CHECK = {"ref": None, "shape": None, "plain": False}


def _plain_causal(mask, Lq, Lk):
    """True when a 4-D attention mask encodes bottom-right causality and
    nothing else (no padding): allowed[i, t] == (t <= Lk - Lq + i) for every
    batch row.  Every layer of one forward receives the same mask object, so
    the device comparison (and its host sync) runs once per forward."""
    ref = _MASK_CHECK["ref"]
    if ref is not None and ref() is mask and _MASK_CHECK["shape"] == (Lq, Lk):
        return _MASK_CHECK["plain"]
    m = mask[..., :Lq, :Lk]
    allowed = m if m.dtype == torch.bool else (m == 0)
    want = torch.ones(Lq, Lk, dtype=torch.bool, device=m.device).tril(diagonal=Lk - Lq)
    plain = m.shape[-2:] == (Lq, Lk) and bool((allowed == want).all().item())
    _MASK_CHECK.update(ref=weakref.ref(mask), shape=(Lq, Lk), plain=plain)
    return plain


def _native_prefill(query_states, key_states, attention_mask):
    """Whether prefill_attention runs hc_prefill_attn for these inputs (a
    ROCm device, head_dim 128, no padding in the mask)."""
    L, D, Lk = query_states.shape[2], query_states.shape[3], key_states.shape[2]
    mask = attention_mask
    if mask is not None and mask.dim() == 4 and _plain_causal(mask, L, Lk):
        mask = None
    return query_states.is_cuda and mask is None and D == ops.HEAD_DIM


def prefill_attention(query_states, key_states, value_states, attention_mask, scaling, stat_out=None):
    """Causal attention of the L query positions over the Lk uncompressed
    keys; the queries are the last L positions (a whole prompt, or one chunk
    of a chunked prefill over the keys staged so far).  Returns [B, L, Hq*d].

    This is hc_prefill_attn (the reference calls flash-attn here,
    heterocache/llama_model.py:353-361).  There is no second code path: a
    mask that carries more than bottom-right causality (padding), inputs
    off the ROCm device or a head_dim other than 128 raise
    NotImplementedError.  The reference's HeteroCache scores and sizes its
    pool for one unpadded sequence (heterocache/cache_utils.py:704-722,
    :807-829), so its path never sees a padded prompt; ragged batches are
    served as one cache per sequence.
    stat_out ([B, Hq, W, 2] float32) receives the last W queries' softmax
    statistics (ops.prefill_attn)."""
    B, Hq, L, D = query_states.shape
    Lk = key_states.shape[2]
    mask = attention_mask
    if mask is not None and mask.dim() == 4 and _plain_causal(mask, L, Lk):
        mask = None
    if mask is not None:
        raise NotImplementedError("hc_prefill_attn takes causal prompts without padding; this attention mask "
                                  "carries padding (serve ragged prompts as one sequence per cache)")
    if not query_states.is_cuda or D != ops.HEAD_DIM:
        raise NotImplementedError(f"hc_prefill_attn needs ROCm device tensors of head_dim {ops.HEAD_DIM} "
                                  f"(got {query_states.device}, head_dim {D})")
    return ops.prefill_attn(query_states, key_states, value_states, scaling, stat_out=stat_out).view(B, L, Hq * D)


class LlamaAttention(nn.Module):
    """Multi-headed attention whose KV cache is a HeteroCache."""

    def __init__(self, config, layer_idx: Optional[int] = None):
        super().__init__()
        self.config = config
        self.layer_idx = layer_idx
        self.attention_dropout = config.attention_dropout
        self.hidden_size = config.hidden_size
        self.num_heads = config.num_attention_heads
        self.head_dim = getattr(config, "head_dim", None) or self.hidden_size // self.num_heads
        self.num_key_value_heads = config.num_key_value_heads
        self.num_key_value_groups = self.num_heads // self.num_key_value_heads
        self.max_position_embeddings = getattr(config, "max_position_embeddings", None)
        self.rope_theta = getattr(config, "rope_theta", None)
        self.is_causal = True
        self.scaling = self.head_dim ** -0.5
        bias = getattr(config, "attention_bias", False)
        self.q_proj = nn.Linear(self.hidden_size, self.num_heads * self.head_dim, bias=bias)
        self.k_proj = nn.Linear(self.hidden_size, self.num_key_value_heads * self.head_dim, bias=bias)
        self.v_proj = nn.Linear(self.hidden_size, self.num_key_value_heads * self.head_dim, bias=bias)
        self.o_proj = nn.Linear(self.num_heads * self.head_dim, self.hidden_size, bias=bias)

    # Qwen2 runs decode_select before the decode attention.
    select_before_attention = False

    def _project(self, hidden_states, position_embeddings):
        input_shape = hidden_states.shape[:-1]
        hidden_shape = (*input_shape, -1, self.head_dim)
        q = self.q_proj(hidden_states).view(hidden_shape).transpose(1, 2)
        k = self.k_proj(hidden_states).view(hidden_shape).transpose(1, 2)
        v = self.v_proj(hidden_states).view(hidden_shape).transpose(1, 2)
        cos, sin = position_embeddings
        q, k = apply_rotary_pos_emb(q, k, cos, sin)
        return q, k, v

    def forward(self, hidden_states: torch.Tensor, attention_mask: Optional[torch.Tensor] = None,
                position_ids: Optional[torch.LongTensor] = None, output_attentions: bool = False,
                use_cache: bool = False, cache_position: Optional[torch.LongTensor] = None,
                position_embeddings: Optional[Tuple[torch.Tensor, torch.Tensor]] = None, past_key_values=None,
                **kwargs) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
        if position_embeddings is None:
            raise ValueError("position_embeddings (cos, sin) are required")
        bsz, q_len, _ = hidden_states.size()
        query_states, key_states, value_states = self._project(hidden_states, position_embeddings)
        cache = past_key_values
        cos, sin = position_embeddings
        cache_kwargs = {"sin": sin, "cos": cos, "cache_position": cache_position, "attention_mask": attention_mask,
                        "num_key_value_groups": self.num_key_value_groups, "query_states": query_states,
                        "update_global_past_kv": getattr(self, "update_global_past_kv", True)}
        if cache is None or not isinstance(cache, HeteroCache):
            # No HeteroCache: causal attention over whatever the cache returns
            # (a plain DynamicCache, or a baseline compressor's cache, which
            # returns its compressed rows; heterocache/llama_model.py:45-94).
            if cache is not None:
                key_states, value_states = cache.update(key_states, value_states, self.layer_idx, cache_kwargs)
            for observer in ATTENTION_OBSERVERS:
                observer(self.layer_idx, query_states, key_states, attention_mask, self.scaling)
            out = prefill_attention(query_states, key_states, value_states, attention_mask, self.scaling)
            return self.o_proj(out), None
        # A chunked prefill stays in the prefill branch until the declared
        # prompt is complete, even for a one-token last chunk.
        prefill = query_states.shape[-2] != 1 or cache.prefill_pending(self.layer_idx)
        key_states, value_states = cache.update(key_states, value_states, self.layer_idx, cache_kwargs)
        if prefill:
            # The attention runs first so that it can hand the selection
            # scorers the softmax normalisers of the last queries; neither
            # reads what the other writes, so the results are those of the
            # reference's order (select, then attend).
            stats = None
            W = cache.prefill_stat_rows(query_states, self.layer_idx)
            if W and _native_prefill(query_states, key_states, attention_mask):
                stats = torch.empty((bsz, query_states.shape[1], W, 2), dtype=torch.float32,
                                    device=query_states.device)
            out = prefill_attention(query_states, key_states, value_states, attention_mask, self.scaling,
                                    stat_out=stats)
            cache.init_coefficient(query_states, key_states, self.layer_idx, stats=stats)
            cache.prefill_select(query_states, key_states, value_states, self.layer_idx, stats=stats)
        else:
            if self.select_before_attention:
                cache.decode_select(query_states, self.layer_idx)
            out = cache.decode_attention(query_states, self.layer_idx)
            if not self.select_before_attention:
                cache.decode_select(query_states, self.layer_idx)
        return self.o_proj(out), None
