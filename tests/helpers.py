"""Shared helpers of the test suite (inputs, comparisons)."""

import numpy as np
import torch


def gen_qkv(B, H, Hkv, S, D, seed=0, dtype=torch.bfloat16, device="cuda", std=1.0, N=None,
            model_layout=False):
    """Seeded CPU randn (q, k, v order), rounded to `dtype`, moved to `device`.
    model_layout=True returns q/k/v as [B,H,S,D] views of [B,S,H,D] storage,
    the layout the attention module hands over after its projections."""
    N = S if N is None else N
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, S, D, generator=g) * std
    k = torch.randn(B, Hkv, N, D, generator=g) * std
    v = torch.randn(B, Hkv, N, D, generator=g) * std
    q, k, v = (x.to(dtype) for x in (q, k, v))
    if model_layout:
        q, k, v = (x.transpose(1, 2).contiguous().transpose(1, 2) for x in (q, k, v))
    return q.to(device), k.to(device), v.to(device)


def np64(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def assert_close(got, ref, cos_min=0.999, atol=2e-2, what=""):
    """Tolerance of the reference's T1 gate (tests/test_math_identities.py:85-89):
    per-row (last dim) cosine > cos_min and max |diff| < atol."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    num = (got * ref).sum(-1)
    den = np.sqrt((got * got).sum(-1) * (ref * ref).sum(-1))
    nz = den > 0
    cos = np.where(nz, num / np.where(nz, den, 1.0), 1.0)
    # rows that are zero in both are equal; a zero row against a non-zero one fails
    both_zero = (np.abs(got).sum(-1) == 0) & (np.abs(ref).sum(-1) == 0)
    cos = np.where(both_zero, 1.0, np.where(nz, cos, 0.0))
    diff = np.abs(got - ref).max() if got.size else 0.0
    print(f"{what}: cos min {cos.min():.6f} mean {cos.mean():.6f} max|diff| {diff:.5f}", flush=True)
    assert cos.min() > cos_min, f"{what}: per-row cos {cos.min():.6f} <= {cos_min}"
    assert diff < atol, f"{what}: max abs diff {diff:.4f} >= {atol}"


def workload_inputs(B, H, Hkv, S, D, theta, seed=0, qk_norm=False, q_scale=True):
    """Seeded N(0,1) q/k/v on the GPU drawn in q, k, v order; optional per-head
    RMSNorm of q/k (Qwen3), q * D^-0.5 (Llama workloads), RoPE with `theta`,
    cast to bf16. Generated in row chunks to bound the fp32 temporaries."""
    from delta_attention.llama import apply_rotary_pos_emb, rope_cos_sin
    g = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.empty(B, H, S, D, device="cuda", dtype=torch.bfloat16)
    k = torch.empty(B, Hkv, S, D, device="cuda", dtype=torch.bfloat16)
    v = torch.empty(B, Hkv, S, D, device="cuda", dtype=torch.bfloat16)
    cos, sin = rope_cos_sin(torch.arange(S, device="cuda")[None], D, theta, torch.float32)
    for c0 in range(0, S, 8192):
        c1 = min(S, c0 + 8192)
        qc = torch.randn(B, H, c1 - c0, D, device="cuda", generator=g)
        kc = torch.randn(B, Hkv, c1 - c0, D, device="cuda", generator=g)
        if qk_norm:
            qc = torch.nn.functional.rms_norm(qc, (D,), eps=1e-6)
            kc = torch.nn.functional.rms_norm(kc, (D,), eps=1e-6)
        if q_scale:
            qc = qc * D ** -0.5
        qc, kc = apply_rotary_pos_emb(qc, kc, cos[:, c0:c1], sin[:, c0:c1])
        q[:, :, c0:c1] = qc.to(torch.bfloat16)
        k[:, :, c0:c1] = kc.to(torch.bfloat16)
        v[:, :, c0:c1] = torch.randn(B, Hkv, c1 - c0, D, device="cuda", generator=g).to(torch.bfloat16)
    return q, k, v
