"""Differentiable delta attention (delta_attention/train/flex_delta.py:48-208).

`delta_forward_train(q, k, v, gamma, window, sink=1024, scaling=None,
detach_delta=False, delta_grad_scale=1.0)` has the reference's signature,
result layout ([b, s, h, d]) and composition (:95-196): key-sparse attention
over every row (the block-anchored window + sinks of :59-61), causal
attention at the anchor and tail rows of `anchor_layout`, and
out = sparse + (dense_anchor - sparse_anchor) broadcast over each gamma-row
group, with the dense tail rows appended. The reference runs FlexAttention
and masked SDPA under autograd; here both directions are HIP kernels:

  forward   da_sparse_attn_fwd_lse, da_qsparse_attn_fwd_lse (saving each
            row's log-sum-exp), da_delta_add for the composition;
  backward  da_delta_compose_bwd (the composition, with the detach and
            gradient-scale arms of :187-190), then da_sparse_attn_bwd and
            da_qsparse_attn_bwd (flash-style recomputation from the saved
            statistics; their dq/dk/dv contributions are added in bf16, as
            autograd adds the two branches' gradients).

GQA is native (no repeat_interleave copies); gradients of k/v are summed over
each KV head's query heads, which is what the expansion's backward does.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from .. import ops

Q_BLOCK = 64  # hip's block_sparse_block_size_q (flex_delta.py:48)


def anchor_layout(s: int, gamma: int) -> Tuple[torch.Tensor, torch.Tensor, int]:
    """Anchor rows 0, gamma, .. < s_p and dense tail rows s_p .. s-1 with
    cut_n = s % gamma + max(128, gamma), s_p = s - cut_n (flex_delta.py:72-76)."""
    cut_n = s % gamma + max(128, gamma)
    s_p = s - cut_n
    return torch.arange(0, s_p, gamma), torch.arange(s_p, s), s_p


class _DeltaAttention(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, gamma, window, sink, scaling, detach_delta, delta_grad_scale):
        b, h, s, d = q.shape
        idx, tail, s_p = anchor_layout(s, gamma)
        if s_p <= 0:
            # no anchors: every row is a dense tail row
            idx, tail, s_p = idx[:0], torch.arange(0, s), 0
        sel = torch.cat((idx, tail)).to(q.device)
        sparse, lse_s = ops.sparse_attention_lse(q, k, v, window=window, sink=sink,
                                                 sm_scale=scaling, q_block=Q_BLOCK)
        dense_sel, lse_d = ops.rows_attention_lse(q, k, v, sel, scaling)
        n = idx.numel()
        out = torch.empty((b, s, h, d), device=q.device, dtype=q.dtype)
        if s_p > 0:
            # delta = rnd(dense_anchor - sparse[idx]); out = rnd(sparse + delta)
            ops.delta_add(sparse, s_p=s_p, out=out[:, :s_p], dense_sel=dense_sel[:, :n],
                          anchors=idx.to(q.device), gamma=gamma)
        out[:, s_p:] = dense_sel[:, n:]
        ctx.save_for_backward(q, k, v, sel, sparse, lse_s, dense_sel, lse_d)
        ctx.cfg = (gamma, window, sink, scaling, detach_delta, delta_grad_scale, s_p)
        return out

    @staticmethod
    def backward(ctx, grad):
        q, k, v, sel, sparse, lse_s, dense_sel, lse_d = ctx.saved_tensors
        gamma, window, sink, scaling, detach_delta, delta_grad_scale, s_p = ctx.cfg
        grad = grad.to(q.dtype)
        if s_p > 0:
            dsparse, ddense = ops.delta_compose_bwd(grad, gamma=gamma, s_p=s_p,
                                                    delta_grad_scale=delta_grad_scale,
                                                    detach_delta=detach_delta)
        else:
            dsparse, ddense = torch.zeros_like(sparse), grad.contiguous()
        dq, dk, dv = ops.sparse_attention_bwd(q, k, v, sparse, dsparse, lse_s, window=window,
                                              sink=sink, sm_scale=scaling, q_block=Q_BLOCK)
        ops.rows_attention_bwd(q, k, v, sel, dense_sel, ddense, lse_d, sm_scale=scaling,
                               dq=dq, dk=dk, dv=dv, accumulate=True)
        return dq, dk, dv, None, None, None, None, None, None


def delta_forward_train(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    gamma: int,
    window: int,
    sink: int = 1024,
    scaling: Optional[float] = None,
    detach_delta: bool = False,
    delta_grad_scale: float = 1.0,
) -> torch.Tensor:
    """Differentiable delta-corrected attention (flex_delta.py:95-196).

    q: [b, h, s, d]; k/v: [b, h_kv, s, d] (GQA native). Returns [b, s, h, d].
    detach_delta: no gradient through the correction term; delta_grad_scale:
    its gradient multiplied by this factor (the forward is unchanged).
    """
    b, h, s, d = q.shape
    assert s % Q_BLOCK == 0, (
        f"s={s} must be a multiple of {Q_BLOCK} (hip block-anchored window "
        "semantics are only reconciled for full query blocks)")
    assert k.shape[1] and h % k.shape[1] == 0, (q.shape, k.shape)
    if scaling is None:
        scaling = d ** -0.5
    if q.dtype == torch.float32:
        # the kernels compute in bf16 with fp32 accumulation
        q, k, v = q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16)
    return _DeltaAttention.apply(q, k, v, int(gamma), int(window), int(sink), float(scaling),
                                 bool(detach_delta), float(delta_grad_scale))


def anchor_grad_ratio(q_grad: torch.Tensor, gamma: int) -> float:
    """Mean per-row gradient norm at anchor and tail rows over the other rows
    (batch 0, mean over heads; flex_delta.py:199-208)."""
    s = q_grad.size(2)
    idx, tail, _ = anchor_layout(s, gamma)
    device = q_grad.device
    norms = q_grad.float().norm(dim=-1).mean(dim=1)[0]
    is_dense = torch.zeros(s, dtype=torch.bool, device=device)
    is_dense[idx.to(device)] = True
    is_dense[tail.to(device)] = True
    return (norms[is_dense].mean() / norms[~is_dense].mean().clamp_min(1e-12)).item()
