"""The training path on the GPU (delta_forward_train, flex_delta.py:95-196):
forward equal to the inference layer, the saved row statistics against the
oracle's log-sum-exp, and dq / dk / dv against the oracle's float64
gradients (delta_train_grads, pinned by tests/test_oracle_train.py) for GQA
1-5 and 8, head_dim 32/64/128, bf16 and fp16, the detach and gradient-scale arms,
sinks beyond the window and a window covering every key. Each case prints
its parameters before it runs."""

import numpy as np
import pytest
import torch

from helpers import np64
from oracle import delta_oracle as O

pytestmark = pytest.mark.gpu


def _inputs(B, H, Hkv, S, D, seed, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, S, D, generator=g).to(dtype).cuda()
    k = torch.randn(B, Hkv, S, D, generator=g).to(dtype).cuda()
    v = torch.randn(B, Hkv, S, D, generator=g).to(dtype).cuda()
    up = torch.randn(B, S, H, D, generator=g).to(dtype).cuda()
    return q, k, v, up


def _grad_close(got, ref, what, branches=()):
    g, r = np64(got).ravel(), np.asarray(ref, dtype=np.float64).ravel()
    cos = float(g @ r / (np.linalg.norm(g) * np.linalg.norm(r) + 1e-30))
    err = float(np.abs(g - r).max())
    # Each branch's gradient is rounded to bf16 before the two are added (as
    # autograd adds the sparse and dense branches' bf16 gradients), and at the
    # anchor rows the branches cancel (rnd(g - ddelta) against rnd(ddelta)):
    # the absolute bound scales with the largest rounded quantity, the final
    # or a branch gradient; P and dS also enter the MFMAs in bf16.
    mag = max([float(np.abs(r).max())] + [float(np.abs(x).max()) for x in branches])
    bound = 2e-2 * max(1.0, mag)
    assert cos >= 0.999 and err <= bound, f"{what}: cos {cos:.6f} max|err| {err:.4g} bound {bound:.3g}"


CASES = [
    # B, H, Hkv, S, D, gamma, window, sink, dtype, arm
    (1, 8, 2, 512, 64, 16, 128, 64, torch.bfloat16, "plain"),
    (2, 4, 4, 384, 128, 64, 256, 16, torch.bfloat16, "plain"),
    (1, 10, 2, 640, 128, 32, 192, 100, torch.bfloat16, "plain"),     # GQA 5
    (1, 4, 1, 448, 32, 16, 64, 200, torch.float16, "plain"),         # sinks past the window
    (1, 4, 2, 320, 64, 16, 1024, 0, torch.bfloat16, "plain"),        # window covers every key
    (1, 8, 2, 512, 64, 16, 128, 64, torch.bfloat16, "detach"),
    (1, 8, 2, 512, 64, 16, 128, 64, torch.bfloat16, "scaled"),
    (1, 4, 2, 128, 64, 64, 64, 8, torch.bfloat16, "plain"),          # s <= cut_n: all rows dense
    (1, 16, 2, 448, 128, 32, 128, 16, torch.bfloat16, "plain"),      # GQA 8: two four-head dK/dV steps
    (1, 8, 2, 384, 128, 64, 128, 16, torch.float16, "plain"),        # fp16 at head_dim 128
]


@pytest.mark.parametrize("c", CASES, ids=lambda c: "-".join(str(x).replace("torch.", "") for x in c))
def test_delta_forward_train_grads(gpu, c):
    from delta_attention import ops
    from delta_attention.train.flex_delta import delta_forward_train
    B, H, Hkv, S, D, gamma, window, sink, dtype, arm = c
    print(f"train case {c}", flush=True)
    q, k, v, up = _inputs(B, H, Hkv, S, D, seed=S + D + H, dtype=dtype)
    scale = D ** -0.5
    detach, gs = arm == "detach", (0.25 if arm == "scaled" else 1.0)
    qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
    out = delta_forward_train(qq, kk, vv, gamma, window, sink, scale, detach_delta=detach,
                              delta_grad_scale=gs)
    out.backward(up)
    torch.cuda.synchronize()
    # forward: the inference layer's bits
    assert out.shape == (B, S, H, D)
    ref_out = ops.delta_prefill(q, k, v, gamma=gamma, window=window, sink=sink, sm_scale=scale,
                                fused=False)
    assert torch.equal(out.detach(), ref_out)
    (dq, dk, dv), br1, br2 = O.delta_train_grads(np64(q), np64(k), np64(v), gamma, window, sink,
                                                 scale, np64(up), grad_scale=gs, detach=detach,
                                                 parts=True)
    _grad_close(qq.grad, dq, "dq", (br1[0], br2[0]))
    _grad_close(kk.grad, dk, "dk", (br1[1], br2[1]))
    _grad_close(vv.grad, dv, "dv", (br1[2], br2[2]))


@pytest.mark.parametrize("c", [CASES[0], CASES[2], CASES[4]],
                         ids=lambda c: "-".join(str(x).replace("torch.", "") for x in c))
def test_delta_forward_train_grads_in_row_chunks(gpu, c):
    """The same gradients with every key block's rows cut into 64-row dK/dV
    items (the default cap of 8192 rows gives one item per block at these
    sizes): the sink blocks' row chunks, several chunks per window block and
    per selected-row list, and the reduce over their fp32 partials."""
    from delta_attention import ops
    from delta_attention.train.flex_delta import delta_forward_train
    B, H, Hkv, S, D, gamma, window, sink, dtype, arm = c
    print(f"train case {c}, 64-row chunks", flush=True)
    q, k, v, up = _inputs(B, H, Hkv, S, D, seed=S + D + H + 1, dtype=dtype)
    scale = D ** -0.5
    qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
    ops.set_bwd_rows_per_chunk(64)
    try:
        out = delta_forward_train(qq, kk, vv, gamma, window, sink, scale)
        out.backward(up)
        torch.cuda.synchronize()
    finally:
        ops.set_bwd_rows_per_chunk(0)
    (dq, dk, dv), br1, br2 = O.delta_train_grads(np64(q), np64(k), np64(v), gamma, window, sink,
                                                 scale, np64(up), parts=True)
    _grad_close(qq.grad, dq, "dq", (br1[0], br2[0]))
    _grad_close(kk.grad, dk, "dk", (br1[1], br2[1]))
    _grad_close(vv.grad, dv, "dv", (br1[2], br2[2]))


def test_forward_row_statistics(gpu):
    """lse of both forward kernels against the oracle's log2-sum-exp2 of the
    scaled scores (every visible key; +inf for rows without one)."""
    from delta_attention import ops
    B, H, Hkv, S, D = 1, 8, 2, 700, 64
    q, k, v, _ = _inputs(B, H, Hkv, S, D, seed=3)
    scale = D ** -0.5
    window, sink = 100, 16
    _, lse = ops.sparse_attention_lse(q, k, v, window=window, sink=sink, sm_scale=scale)
    rows = torch.tensor([0, 5, 64, 300, 699], dtype=torch.int64)
    _, lse_r = ops.rows_attention_lse(q, k, v, rows.cuda(), scale)
    torch.cuda.synchronize()
    qn, kn = np64(q), np.repeat(np64(k), H // Hkv, axis=1)
    sc = np.matmul(qn, kn.swapaxes(-1, -2)) * scale * np.log2(np.e)
    r = np.arange(S)
    vis = O.sparse_visible(r[:, None], r[None, :], window, sink)
    ref = np.log2(np.where(vis[None, None], np.exp2(sc - sc.max(-1, keepdims=True)), 0).sum(-1)) + sc.max(-1)
    assert np.abs(np64(lse) - ref).max() < 2e-3
    causal = r[None, :] <= rows.numpy()[:, None]
    scr = sc[:, :, rows.numpy()]
    mr = np.where(causal[None, None], scr, -np.inf).max(-1, keepdims=True)
    ref_r = np.log2(np.where(causal[None, None], np.exp2(scr - mr), 0).sum(-1)) + mr[..., 0]
    assert np.abs(np64(lse_r) - ref_r).max() < 2e-3


def test_backward_is_deterministic(gpu):
    from delta_attention.train.flex_delta import delta_forward_train
    q, k, v, up = _inputs(1, 8, 2, 1024, 128, seed=9)
    grads = []
    for _ in range(2):
        qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
        delta_forward_train(qq, kk, vv, 64, 256, 128).backward(up)
        grads.append((qq.grad, kk.grad, vv.grad))
    torch.cuda.synchronize()
    for a, b in zip(*grads):
        assert torch.equal(a, b)


def test_full_size_properties(gpu):
    """Llama-3.1-8B layer at 32K tokens (32/8 heads, head_dim 128, window 2048
    + 128 sinks, gamma 64): the training forward equals the inference layer
    bit for bit, and the backward is linear in the upstream gradient exactly
    for a power-of-two scale (every fp32 product and bf16 rounding scales by
    2 without error), over every row."""
    from delta_attention import ops
    from delta_attention.train.flex_delta import delta_forward_train
    B, H, Hkv, S, D = 1, 32, 8, 32768, 128
    print("full-size training properties: Llama 32K", flush=True)
    q, k, v, up = _inputs(B, H, Hkv, S, D, seed=77)
    q, k = q * D ** -0.25, k * D ** -0.25         # moderate logits, as after RoPE'd projections
    scale = D ** -0.5
    grads = []
    for mult in (1.0, 2.0):
        qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
        out = delta_forward_train(qq, kk, vv, 64, 2048, 128, scale)
        out.backward(up * mult)
        grads.append((out.detach(), qq.grad, kk.grad, vv.grad))
    torch.cuda.synchronize()
    ref = ops.delta_prefill(q, k, v, gamma=64, window=2048, sink=128, sm_scale=scale, fused=False)
    assert torch.equal(grads[0][0], ref)
    for a, b in zip(grads[0][1:], grads[1][1:]):
        assert torch.isfinite(a).all()
        assert torch.equal(a * 2, b)


def test_rows_bwd_q_rows_past_32bit_offsets(gpu):
    """Selected-rows backward with q rows spread over more than 4 GB (a view
    with a 4M-element row stride): the dK/dV kernel cannot address a head's
    gathered q rows with 32-bit offsets from its row 0, stages them through
    registers instead of by DMA, and gives the bits of a contiguous copy."""
    from delta_attention import ops
    B, H, Hkv, Sq, D = 1, 4, 2, 600, 128
    print("rows backward: q rows past 32-bit offsets", flush=True)
    g = torch.Generator().manual_seed(5)
    qc = torch.randn(B, H, Sq, D, generator=g).to(torch.bfloat16).cuda()
    k = torch.randn(B, Hkv, Sq, D, generator=g).to(torch.bfloat16).cuda()
    v = torch.randn(B, Hkv, Sq, D, generator=g).to(torch.bfloat16).cuda()
    rows = torch.arange(3, Sq, 7, dtype=torch.int64).cuda()
    scale = D ** -0.5
    out, lse = ops.rows_attention_lse(qc, k, v, rows, scale)
    dout = torch.randn(out.shape, generator=g).to(torch.bfloat16).cuda()
    stride = 4_000_000                      # elements per q row: Sq * stride * 2 B = 4.8 GB
    buf = torch.empty(Sq * stride, dtype=torch.bfloat16, device="cuda")
    qv = buf.as_strided((B, H, Sq, D), (Sq * stride, D, stride, 1))
    qv.copy_(qc)
    res = []
    for qq in (qc, qv):
        dq = torch.zeros(B, H, Sq, D, dtype=torch.bfloat16, device="cuda")
        res.append(ops.rows_attention_bwd(qq, k, v, rows, out, dout, lse, sm_scale=scale, dq=dq))
    torch.cuda.synchronize()
    del buf, qv
    for a, b in zip(*res):
        assert torch.isfinite(a).all()
        assert torch.equal(a, b)
