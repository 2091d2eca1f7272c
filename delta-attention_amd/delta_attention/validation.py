"""Numeric self-check helpers of the delta path (delta_attention/validation.py:119-245):
seeded q/k/v, row cosine, the anchor/tail index set, and the anchor-exactness
gate (corrected output == dense at anchor and tail rows).

The dense reference here is plain torch arithmetic in float32 on the
selected rows (a checker, independent of the kernels it checks).
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch


class ValidationError(RuntimeError):
    pass


def make_random_qkv(s: int, seed: int, device, n_heads: int = 32, n_kv_heads: int = 8,
                    head_dim: int = 128, batch: int = 1):
    """CPU generator seeded with `seed`, float32 randn drawn in the order q, k, v,
    then bf16 on `device` (validation.py:133-145)."""
    gen = torch.Generator(device="cpu").manual_seed(seed)
    q = torch.randn(batch, n_heads, s, head_dim, generator=gen, dtype=torch.float32)
    k = torch.randn(batch, n_kv_heads, s, head_dim, generator=gen, dtype=torch.float32)
    v = torch.randn(batch, n_kv_heads, s, head_dim, generator=gen, dtype=torch.float32)
    return (q.to(device=device, dtype=torch.bfloat16), k.to(device=device, dtype=torch.bfloat16),
            v.to(device=device, dtype=torch.bfloat16))


def anchor_indices(s: int, gamma: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """(anchors, tail) exactly as delta_forward lays them out (validation.py:224-232)."""
    cut_n = s % gamma + max(128, gamma)
    s_p = s - cut_n
    return torch.arange(0, max(s_p, 0), step=gamma), torch.arange(max(s_p, 0), s)


def row_cos(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Per-row cosine over flattened (h, d) of [b, s, h, d] tensors (validation.py:215-221)."""
    a32 = a.reshape(a.size(0), a.size(1), -1).float()
    b32 = b.reshape(b.size(0), b.size(1), -1).float()
    return torch.nn.functional.cosine_similarity(a32, b32, dim=-1)


def dense_rows_reference(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, rows: torch.Tensor,
                         scaling: float, chunk: int = 64) -> torch.Tensor:
    """Causal attention at `rows` in float32 torch math: q [b,h,s,d], k/v
    [b,hkv,s,d] -> [b, len(rows), h, d]."""
    b, h, s, d = q.shape
    g = h // k.shape[1]
    kf = k.float().repeat_interleave(g, dim=1)
    vf = v.float().repeat_interleave(g, dim=1)
    rows = rows.to(q.device)
    outs = []
    for c0 in range(0, rows.numel(), chunk):
        r = rows[c0:c0 + chunk]
        kmax = int(r.max().item()) + 1
        sc = torch.matmul(q[:, :, r].float(), kf[:, :, :kmax].transpose(-1, -2).contiguous()) * scaling
        keys = torch.arange(kmax, device=q.device)
        sc = sc.masked_fill(keys[None, None, None, :] > r[None, None, :, None], float("-inf"))
        outs.append(torch.matmul(torch.softmax(sc, dim=-1), vf[:, :, :kmax]))
    return torch.cat(outs, dim=2).transpose(1, 2)


def anchor_exactness_check(module, *, gamma: int, window: int, s: int = 2048,
                           min_cos: float = 0.999, seed: int = 0) -> float:
    """Delta-corrected rows must equal dense rows at anchors and the tail
    (validation.py:235-245); raises ValidationError otherwise."""
    cfg = module.config
    device = next(module.parameters()).device
    q, k, v = make_random_qkv(s, seed, device, cfg.num_attention_heads, cfg.num_key_value_heads,
                              module.head_dim)
    saved = (cfg.mode, cfg.delta_lambda, cfg.sliding_window)
    cfg.mode, cfg.delta_lambda, cfg.sliding_window = "delta", gamma, window
    try:
        with torch.no_grad():
            out, _ = module.delta_forward(module, q, k, v, None, scaling=module.head_dim ** -0.5)
    finally:
        cfg.mode, cfg.delta_lambda, cfg.sliding_window = saved
    anchors, tail = anchor_indices(s, gamma)
    rows = torch.cat([anchors, tail])
    dense = dense_rows_reference(q, k, v, rows, module.head_dim ** -0.5)
    cos = row_cos(out[:, rows.to(device)], dense)[0]
    worst = cos.min().item()
    if worst < min_cos:
        raise ValidationError(f"anchor exactness: min anchor/tail row cos {worst:.6f} < {min_cos} "
                              f"(s={s}, gamma={gamma}, window={window})")
    return worst
