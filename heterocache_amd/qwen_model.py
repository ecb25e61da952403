"""Qwen2 attention with HeteroCache on libhc kernels.

Drop-in for heterocache/qwen_model.py:93-212 (`Qwen2Attention`): the Llama
flow with biased q/k/v projections, an unbiased o_proj, and decode_select
called BEFORE the decode attention (heterocache/qwen_model.py:178 vs :194), so
a retrieval triggered at step t is visible to step t's attention.
"""
from typing import Optional

import torch.nn as nn

from .llama_model import LlamaAttention


class Qwen2Attention(LlamaAttention):
    select_before_attention = True

    def __init__(self, config, layer_idx: Optional[int] = None):
        super().__init__(config, layer_idx)
        self.q_proj = nn.Linear(config.hidden_size, self.num_heads * self.head_dim, bias=True)
        self.k_proj = nn.Linear(config.hidden_size, self.num_key_value_heads * self.head_dim, bias=True)
        self.v_proj = nn.Linear(config.hidden_size, self.num_key_value_heads * self.head_dim, bias=True)
        self.o_proj = nn.Linear(self.num_heads * self.head_dim, config.hidden_size, bias=False)
        layer_types = getattr(config, "layer_types", None)
        self.sliding_window = (config.sliding_window if layer_types is not None and layer_idx is not None
                               and layer_types[layer_idx] == "sliding_attention" else None)
