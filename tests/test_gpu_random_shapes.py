"""Seeded random-shape sweep of the GPU path against the oracle: delta-attention
layer prefill (llama.py:659-757) in all three modes, fused and three-kernel
orders, over GQA ratios, head dims, sequence lengths (including lengths below
one row block and at or under the dense tail, where every row is dense),
strides that do and do not divide 128, windows too short to reach any key and
sinks; delta_kernel.attention (delta_kernel.py:262-322) with unsorted and
out-of-range row limits; and decode rows (llama.py:537-549, 598-600). Each
case prints its parameters before it runs."""

import numpy as np
import pytest
import torch

from helpers import assert_close, gen_qkv, np64
from oracle import delta_oracle as O

pytestmark = pytest.mark.gpu

HEADS = [(8, 2), (4, 4), (6, 3), (10, 2), (8, 1), (12, 4), (16, 8), (2, 1)]
GAMMAS = [1, 2, 8, 16, 32, 48, 64, 96, 128, 256]


def _prefill_cases(n, seed):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        H, Hkv = HEADS[int(rng.integers(len(HEADS)))]
        if rng.random() < 0.25:
            S = int(rng.choice([1, 2, 63, 64, 65, 127, 129, 200, 257]))
        else:
            S = int(rng.integers(300, 1300))
        cases.append(dict(
            i=i, B=int(rng.choice([1, 2])), H=H, Hkv=Hkv, D=int(rng.choice([32, 64, 128])), S=S,
            gamma=int(rng.choice(GAMMAS)), window=int(rng.integers(1, 700)),
            sink=int(rng.choice([0, 1, 16, 64, 100])),
            mode=str(rng.choice(["delta", "delta", "delta", "recompute", "sparse-only"])),
            fused=bool(rng.random() < 0.7),
            dtype=torch.bfloat16 if rng.random() < 0.75 else torch.float16,
            model_layout=bool(rng.random() < 0.5)))
    return cases


def _ref_layer(qn, kn, vn, gamma, window, sink, scale, mode):
    """The layer from the oracle's pieces: key-sparse rows, dense rows at the
    selected indices, the delta of the anchor at or before each row (any
    gamma: owner = r // gamma), the dense tail; every row dense when the
    sequence is not longer than the tail."""
    sparse = O.sparse_attention(qn, kn, vn, window, sink, scale)
    if mode == "sparse-only":
        return sparse
    S = qn.shape[2]
    anchors, tail, s_p, _ = O.anchor_layout(S, gamma)
    if s_p <= 0:
        return O.causal_attention_rows(qn, kn, vn, np.arange(S), scale)
    idx = np.concatenate([anchors, tail])
    dense = O.causal_attention_rows(qn, kn, vn, idx, scale)
    if mode == "recompute":
        out = sparse.copy()
        out[:, idx] = dense
        return out
    body = O.apply_delta_variable(sparse, dense[:, :len(anchors)], anchors, s_p)
    return np.concatenate([body, dense[:, len(anchors):]], axis=1)


@pytest.mark.parametrize("c", _prefill_cases(40, 2026), ids=lambda c: f"case{c['i']}")
def test_prefill_random_shape(gpu, c):
    from delta_attention import ops
    print(f"prefill case {c}", flush=True)
    q, k, v = gen_qkv(c["B"], c["H"], c["Hkv"], c["S"], c["D"], seed=1000 + c["i"],
                      dtype=c["dtype"], model_layout=c["model_layout"])
    scale = c["D"] ** -0.5
    out = ops.delta_prefill(q, k, v, gamma=c["gamma"], window=c["window"], sink=c["sink"],
                            sm_scale=scale, mode=c["mode"], fused=c["fused"])
    torch.cuda.synchronize()
    assert out.shape == (c["B"], c["S"], c["H"], c["D"]) and out.dtype == c["dtype"]
    ref = _ref_layer(np64(q), np64(k), np64(v), c["gamma"], c["window"], c["sink"], scale, c["mode"])
    assert_close(np64(out), ref, what=str(c))


@pytest.mark.parametrize("seed", range(10))
def test_attention_random_limits(gpu, seed):
    """delta_kernel.attention with random, unsorted row limits, some past the
    last key (clamped) and some negative (no visible key: a zero row), with
    native GQA and with expanded K/V."""
    from delta_attention.delta_kernel import attention
    from delta_attention.llama import repeat_kv
    rng = np.random.default_rng(500 + seed)
    H, Hkv = HEADS[int(rng.integers(len(HEADS)))]
    B, D = int(rng.choice([1, 2])), int(rng.choice([32, 64, 128]))
    n, N = int(rng.integers(1, 300)), int(rng.integers(1, 2000))
    lim = rng.integers(-2, N + 5, size=n)
    print(f"attention case seed {seed}: B{B} H{H}/{Hkv} D{D} n{n} N{N}", flush=True)
    q, k, v = gen_qkv(B, H, Hkv, n, D, seed=600 + seed, N=N)
    mask = torch.from_numpy(lim).long()[None].cuda()
    scale = D ** -0.5
    ref = O.qsparse_attention(np64(q), np64(k), np64(v), lim, scale)
    got = attention(q, k, v, mask, scale)
    torch.cuda.synchronize()
    assert_close(np64(got), ref, what=f"attention seed {seed}")
    if Hkv != H:
        exp = attention(q, repeat_kv(k, H // Hkv), repeat_kv(v, H // Hkv), mask, scale)
        torch.cuda.synchronize()
        assert torch.equal(exp, got)   # per-row softmax: the head packing does not change bits


@pytest.mark.parametrize("seed", range(8))
def test_decode_random(gpu, seed):
    from delta_attention import ops
    rng = np.random.default_rng(700 + seed)
    H, Hkv = HEADS[int(rng.integers(len(HEADS)))]
    B, D = int(rng.choice([1, 2])), int(rng.choice([32, 64, 128]))
    n = int(rng.integers(1, 5000))
    window = int(rng.choice([0, int(rng.integers(1, 3000))]))
    sink = int(rng.choice([0, 4, 64]))
    print(f"decode case seed {seed}: B{B} H{H}/{Hkv} D{D} n{n} w{window} s{sink}", flush=True)
    g = torch.Generator().manual_seed(800 + seed)
    q = torch.randn(B, H, 1, D, generator=g).to(torch.bfloat16).cuda()
    k = torch.randn(B, Hkv, n, D, generator=g).to(torch.bfloat16).cuda()
    v = torch.randn(B, Hkv, n, D, generator=g).to(torch.bfloat16).cuda()
    scale = D ** -0.5
    got = ops.decode_attention(q, k, v, window=window, sink=sink, sm_scale=scale)
    torch.cuda.synchronize()
    assert_close(np64(got), O.decode_row(np64(q), np64(k), np64(v), window, sink, scale),
                 what=f"decode seed {seed}")
