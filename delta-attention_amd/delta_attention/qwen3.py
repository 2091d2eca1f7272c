"""Qwen3 on the delta path (delta_attention/qwen3.py): Llama attention plus a
per-head RMSNorm of q and k between the projection and RoPE (qwen3.py:37-43),
and the dense Qwen3 causal LM built from it (qwen3.py:46-60: the Llama
decoder stack with that attention class). On the fused path the norm runs
inside the prologue kernel together with RoPE. Everything after RoPE,
including the three kernels, is shared with Llama; GQA ratios that are not
powers of two (40/8 = 5) are handled natively by the kernels' packed
(row, head) tiles.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

from .llama import LlamaAttention, LlamaRMSNorm
from .model import LlamaConfig, LlamaDecoderLayer, LlamaForCausalLM, LlamaModel


class Qwen3DeltaAttention(LlamaAttention):
    def __init__(self, config, layer_idx):
        super().__init__(config, layer_idx)
        eps = getattr(config, "rms_norm_eps", 1e-6)
        self.q_norm = LlamaRMSNorm(self.head_dim, eps=eps)
        self.k_norm = LlamaRMSNorm(self.head_dim, eps=eps)

    def _qkv(self, hidden_states, hidden_shape):
        q = self.q_norm(self.q_proj(hidden_states).view(hidden_shape)).transpose(1, 2)
        k = self.k_norm(self.k_proj(hidden_states).view(hidden_shape)).transpose(1, 2)
        v = self.v_proj(hidden_states).view(hidden_shape).transpose(1, 2)
        return q, k, v

    def _qk_norm(self):
        # the fused prologue kernel applies these norms before RoPE
        return self.q_norm.weight, self.k_norm.weight, self.q_norm.variance_epsilon


@dataclass
class Qwen3Config(LlamaConfig):
    """Qwen3-14B architecture (untied embeddings, default RoPE with theta 1e6,
    RMSNorm eps 1e-6) plus the delta-attention pipeline knobs."""
    vocab_size: int = 151936
    hidden_size: int = 5120
    intermediate_size: int = 17408
    num_hidden_layers: int = 40
    num_attention_heads: int = 40
    num_key_value_heads: int = 8
    head_dim: int = 128
    rope_theta: float = 1000000.0
    rope_scaling: Optional[dict] = None
    rms_norm_eps: float = 1e-6


class Qwen3DeltaDecoderLayer(LlamaDecoderLayer):
    attn_cls = Qwen3DeltaAttention


class Qwen3DeltaModel(LlamaModel):
    layer_cls = Qwen3DeltaDecoderLayer


class Qwen3ForCausalLM(LlamaForCausalLM):
    model_cls = Qwen3DeltaModel
