"""Pins the oracle's training-path gradients (delta_train_grads and its parts)
on the CPU: against torch float64 autograd of an independent restatement of
delta_forward_train's composition (flex_delta.py:95-196: masked softmax
attention for the sparse branch, masked SDPA for the anchor/tail rows,
reshape broadcast, the _ScaleGrad and detach arms), against central finite
differences of the oracle's own forward, and by a planted mistake that must
fail."""

import numpy as np
import pytest
import torch

import conftest  # noqa: F401
from oracle import delta_oracle as O


def _inputs(B, H, Hkv, S, d, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, S, d, generator=g, dtype=torch.float64)
    k = torch.randn(B, Hkv, S, d, generator=g, dtype=torch.float64)
    v = torch.randn(B, Hkv, S, d, generator=g, dtype=torch.float64)
    up = torch.randn(B, S, H, d, generator=g, dtype=torch.float64)
    return q, k, v, up


class _Scale(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, s):
        ctx.s = s
        return x.clone()

    @staticmethod
    def backward(ctx, g):
        return g * ctx.s, None


def _torch_delta(q, k, v, gamma, window, sink, scale, detach=False, grad_scale=1.0, qb=64):
    """delta_forward_train's math in torch float64 (GQA by repeat_interleave)."""
    B, H, S, d = q.shape
    G = H // k.shape[1]
    kr, vr = k.repeat_interleave(G, dim=1), v.repeat_interleave(G, dim=1)
    r = torch.arange(S)
    block_last = (r // qb) * qb + qb - 1
    allowed = (r[None, :] <= r[:, None]) & ((r[None, :] < sink) | (r[None, :] + window > block_last[:, None]))
    sc = (q @ kr.transpose(-1, -2)) * scale
    sparse = torch.softmax(sc.masked_fill(~allowed, float("-inf")), -1) @ vr     # [B,H,S,d]
    sparse = sparse.transpose(1, 2)
    cut_n = S % gamma + max(128, gamma)
    s_p = S - cut_n
    idx, tail = torch.arange(0, s_p, gamma), torch.arange(s_p, S)
    sel = torch.cat((idx, tail))
    row_mask = (r[None, :] <= sel[:, None]).view(1, 1, sel.numel(), S)
    dense = torch.nn.functional.scaled_dot_product_attention(q[:, :, sel], kr, vr, attn_mask=row_mask,
                                                             scale=scale).transpose(1, 2)
    delta = dense[:, :idx.numel()] - sparse[:, idx]
    if detach:
        delta = delta.detach()
    elif grad_scale != 1.0:
        delta = _Scale.apply(delta, grad_scale)
    n = idx.numel()
    corrected = (sparse[:, :s_p].reshape(B, n, gamma, H, d) + delta.reshape(B, n, 1, H, d)).reshape(B, s_p, H, d)
    return torch.cat((corrected, dense[:, n:]), dim=1)


def _close(a, b, rtol=1e-9):
    a, b = np.asarray(a), np.asarray(b)
    assert np.abs(a - b).max() <= rtol * max(1.0, np.abs(b).max()), np.abs(a - b).max()


@pytest.mark.parametrize("B,H,Hkv,S,d,gamma,window,sink", [
    (1, 4, 2, 320, 16, 16, 64, 8),      # GQA 2, several anchor groups
    (2, 2, 2, 384, 8, 64, 128, 0),      # no sinks
    (1, 6, 3, 256, 8, 32, 256, 200),    # window >= s: the sparse branch is causal
    (1, 2, 1, 192, 8, 16, 16, 64),      # short window, sinks beyond the window
])
@pytest.mark.parametrize("arm", ["plain", "detach", "scaled"])
def test_delta_train_grads_match_torch_autograd(B, H, Hkv, S, d, gamma, window, sink, arm):
    q, k, v, up = _inputs(B, H, Hkv, S, d, seed=S + d)
    scale = d ** -0.5
    detach, gs = arm == "detach", (0.25 if arm == "scaled" else 1.0)
    qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
    out = _torch_delta(qq, kk, vv, gamma, window, sink, scale, detach, gs)
    # the forward agrees with the oracle's composition
    _close(out.detach().numpy(), O.delta_forward(q.numpy(), k.numpy(), v.numpy(), gamma, window, sink, scale))
    out.backward(up)
    dq, dk, dv = O.delta_train_grads(q.numpy(), k.numpy(), v.numpy(), gamma, window, sink, scale,
                                     up.numpy(), grad_scale=gs, detach=detach)
    _close(dq, qq.grad.numpy())
    _close(dk, kk.grad.numpy())
    _close(dv, vv.grad.numpy())


def test_masked_attention_grads_match_autograd_and_empty_rows():
    q, k, v, up = _inputs(2, 4, 2, 40, 8, seed=3)
    rng = np.random.default_rng(0)
    allowed = rng.random((40, 40)) < 0.4
    allowed[np.arange(40), rng.integers(0, 40, 40)] = True    # every row sees a key
    allowed[7] = False                                       # ... but row 7: none
    scale = 0.3
    dout = up.transpose(1, 2).contiguous()
    dq, dk, dv = O.masked_attention_grads(q.numpy(), k.numpy(), v.numpy(), allowed, scale, dout.numpy())
    assert np.all(dq[:, :, 7] == 0)
    keep = np.ones(40, bool)
    keep[7] = False
    qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
    kr, vr = kk.repeat_interleave(2, 1), vv.repeat_interleave(2, 1)
    sc = (qq[:, :, keep] @ kr.transpose(-1, -2)) * scale
    o = torch.softmax(sc.masked_fill(~torch.from_numpy(allowed[keep]), float("-inf")), -1) @ vr
    o.backward(dout[:, :, keep])
    _close(dq[:, :, keep], qq.grad[:, :, keep].numpy())
    _close(dk, kk.grad.numpy())
    _close(dv, vv.grad.numpy())


def test_delta_train_grads_finite_differences():
    """Central differences of <g, delta_forward(q, k, v)> at a few coordinates
    of each input (float64, step 1e-6)."""
    q, k, v, up = (t.numpy() for t in _inputs(1, 2, 1, 256, 4, seed=11))
    gamma, window, sink, scale = 16, 32, 8, 0.5
    dq, dk, dv = O.delta_train_grads(q, k, v, gamma, window, sink, scale, up)
    f = lambda qq, kk, vv: float((O.delta_forward(qq, kk, vv, gamma, window, sink, scale) * up).sum())
    rng = np.random.default_rng(5)
    h = 1e-6
    for which, grad in ((0, dq), (1, dk), (2, dv)):
        for _ in range(4):
            idx = tuple(int(rng.integers(0, n)) for n in grad.shape)
            args = [q.copy(), k.copy(), v.copy()]
            args[which][idx] += h
            fp = f(*args)
            args[which][idx] -= 2 * h
            fm = f(*args)
            fd = (fp - fm) / (2 * h)
            assert abs(fd - grad[idx]) <= 1e-5 * max(1.0, abs(fd)), (which, idx, fd, grad[idx])


def test_planted_compose_mistake_fails():
    """The composition's backward without the -ddelta at the anchor rows
    disagrees with autograd (the checks above would catch it)."""
    q, k, v, up = _inputs(1, 2, 2, 256, 8, seed=7)
    qq = q.clone().requires_grad_(True)
    _torch_delta(qq, k, v, 16, 64, 8, 0.4).backward(up)
    good = O.delta_train_grads(q.numpy(), k.numpy(), v.numpy(), 16, 64, 8, 0.4, up.numpy())[0]
    orig = O.compose_grads

    def bad(g, gamma, s_p, grad_scale=1.0, detach=False):
        ds, dd = orig(g, gamma, s_p, grad_scale, detach)
        ds[:, :s_p] = g[:, :s_p]            # the anchor correction dropped
        return ds, dd
    O.compose_grads = bad
    try:
        wrong = O.delta_train_grads(q.numpy(), k.numpy(), v.numpy(), 16, 64, 8, 0.4, up.numpy())[0]
    finally:
        O.compose_grads = orig
    _close(good, qq.grad.numpy())
    assert np.abs(wrong - qq.grad.numpy()).max() > 1e-3
