"""Qwen3 attention on the delta path (delta_attention/qwen3.py): Llama
attention plus a per-head RMSNorm of q and k between the projection and RoPE
(qwen3.py:37-43). On the fused path the norm runs inside the prologue
kernel together with RoPE. Everything after RoPE, including the three
kernels, is shared with Llama; GQA ratios that are not powers of two (40/8 = 5) are
handled natively by the kernels' packed (row, head) tiles.
"""

from __future__ import annotations

from .llama import LlamaAttention, LlamaRMSNorm


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
