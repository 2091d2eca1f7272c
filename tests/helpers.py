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
