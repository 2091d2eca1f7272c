"""Query-sparse / key-dense attention: the `attention(q, k, v, mask, sm_scale)`
entry point of delta_attention/delta_kernel.py:259-329, on the MI355X kernel.

Row i of q attends keys 0..mask[i] (inclusive) of k/v; the rows need not be
sorted (delta_kernel.py:400 uses a permutation). k/v may carry all H query
heads (the reference callers expand them with repeat_kv) or the Hkv key/value
heads of a GQA model (no expansion needed here). float32 inputs run in bf16 on
the MFMA kernel and the result is cast back to float32, as the reference's
window branch treats float32 (llama.py:383-388, 493-494); bf16 and fp16 run
as they are.
"""

from __future__ import annotations

import torch

from . import ops

SUPPORTED_HEAD_DIMS = (32, 64, 128, 256)


class _attention(torch.autograd.Function):

    @staticmethod
    def forward(ctx, q, k, v, mask, sm_scale):
        HEAD_DIM_Q, HEAD_DIM_K, HEAD_DIM_V = q.shape[-1], k.shape[-1], v.shape[-1]
        assert HEAD_DIM_Q == HEAD_DIM_K and HEAD_DIM_K == HEAD_DIM_V
        assert HEAD_DIM_K in {16, 32, 64, 128, 256}
        assert HEAD_DIM_K in SUPPORTED_HEAD_DIMS, \
            f"head_dim {HEAD_DIM_K} has no MI355X kernel (supported: {SUPPORTED_HEAD_DIMS})"
        assert len(mask.size()) == 2, "expecting mask to be 2D"
        assert mask.shape[0] in (1, q.shape[0]), (mask.shape, q.shape)
        assert mask.shape[1] == q.shape[2], (mask.shape, q.shape)
        if q.dtype == torch.float32:
            q, k, v = q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16)
            return ops.qsparse_attention(q, k, v, mask, float(sm_scale)).to(torch.float32)
        return ops.qsparse_attention(q, k, v, mask, float(sm_scale))

    @staticmethod
    def backward(ctx, do):
        raise NotImplementedError("bwd not implemented for recompute kernel")


attention = _attention.apply
