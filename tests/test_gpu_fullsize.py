"""Parity at the benchmark configurations' full sizes (Llama-3.1-8B shape at 32K
and 128K tokens, Qwen3-14B shape at 64K with batch 2 and GQA 5), where the
oracle cannot run whole layers:

* exact, size-independent composition over EVERY row: the delta output equals
  rnd(sparse + rnd(dense[anchor] - sparse[anchor])) recomputed with torch bf16
  ops from the sparse-only and recompute outputs (llama.py:733-755), and the
  tail rows equal the dense rows;
* sampled rows of the sparse pass and of the dense pass against the oracle
  (float32) on the same bf16 inputs: per-row cosine > 0.999, max |diff| < 2e-2.
"""

import numpy as np
import pytest
import torch

from helpers import assert_close, workload_inputs
from oracle import delta_oracle as O

pytestmark = pytest.mark.gpu

CONFIGS = {
    "llama-32k": dict(B=1, H=32, Hkv=8, S=32768, D=128, window=2048, sink=128, gamma=64,
                      theta=500000.0, qk_norm=False, q_scale=True),
    "llama-128k": dict(B=1, H=32, Hkv=8, S=131072, D=128, window=2048, sink=128, gamma=64,
                       theta=500000.0, qk_norm=False, q_scale=True),
    "qwen3-64k-b2": dict(B=2, H=40, Hkv=8, S=65536, D=128, window=4096, sink=64, gamma=64,
                         theta=1000000.0, qk_norm=True, q_scale=False),
}


def _f32(t):
    return t.detach().float().cpu().numpy()


@pytest.mark.parametrize("name", list(CONFIGS))
def test_fullsize_layer(gpu, name):
    from delta_attention import ops
    c = CONFIGS[name]
    B, H, Hkv, S, D = c["B"], c["H"], c["Hkv"], c["S"], c["D"]
    window, sink, gamma = c["window"], c["sink"], c["gamma"]
    G = H // Hkv
    q, k, v = workload_inputs(B, H, Hkv, S, D, c["theta"], seed=0, qk_norm=c["qk_norm"],
                              q_scale=c["q_scale"])
    scale = D ** -0.5
    kw = dict(gamma=gamma, window=window, sink=sink, sm_scale=scale)
    sp = ops.delta_prefill(q, k, v, mode="sparse-only", **kw)
    rc = ops.delta_prefill(q, k, v, mode="recompute", **kw)
    out = ops.delta_prefill(q, k, v, mode="delta", **kw)
    torch.cuda.synchronize()

    # index set, exact
    cut_n, s_p, n_anchor = ops.anchor_layout(S, gamma)
    anchors, tail, s_p_o, _ = O.anchor_layout(S, gamma)
    assert s_p == s_p_o and n_anchor == len(anchors)
    np.testing.assert_array_equal(ops.selected_rows(S, gamma, "cuda").cpu().numpy(),
                                  np.concatenate([anchors, tail]))

    # exact composition over all rows
    a = torch.from_numpy(anchors).cuda()
    delta = rc[:, a] - sp[:, a]                                   # bf16 op, one rounding
    expect = sp[:, :s_p] + delta.repeat_interleave(gamma, dim=1)[:, :s_p]
    assert torch.equal(out[:, :s_p], expect), "delta composition differs from the bf16 reference ops"
    assert torch.equal(out[:, s_p:], rc[:, s_p:]), "tail rows are not the dense rows"
    sel = torch.zeros(S, dtype=torch.bool, device="cuda")
    sel[ops.selected_rows(S, gamma, "cuda")] = True
    assert torch.equal(rc[:, ~sel], sp[:, ~sel]), "recompute touched unselected rows"
    del expect, delta

    # sampled rows against the oracle, on the first and the last kv-head group
    rng = np.random.default_rng(1)
    srows = np.unique(np.concatenate([
        [0, 1, 63, 64, 127, sink - 1, sink, window - 1, window, window + 63, window + 64,
         S // 2, S // 2 + 63, S - 129, S - 64, S - 1],
        rng.integers(0, S, 8)]))
    drows = np.unique(np.concatenate([anchors[[0, 1, len(anchors) // 2, -1]], tail[[0, -1]],
                                      rng.choice(anchors, 4)]))
    for b in range(B):
        for hk in (0, Hkv - 1):
            hs = slice(hk * G, (hk + 1) * G)
            kk = _f32(k[b:b + 1, hk:hk + 1])
            vv = _f32(v[b:b + 1, hk:hk + 1])
            qs = _f32(q[b:b + 1, hs][:, :, torch.from_numpy(srows).cuda()])
            ref = O.sparse_attention(qs, kk, vv, window, sink, scale, rows=srows, q_is_rows=True)
            got = _f32(sp[b:b + 1, torch.from_numpy(srows).cuda(), hs])
            assert_close(got, ref, what=f"{name} sparse rows b{b} kv{hk}")
            qd = _f32(q[b:b + 1, hs][:, :, torch.from_numpy(drows).cuda()])
            refd = O.qsparse_attention(qd, kk, vv, drows, scale).transpose(0, 2, 1, 3)
            gotd = _f32(rc[b:b + 1, torch.from_numpy(drows).cuda(), hs])
            assert_close(gotd, refd, what=f"{name} dense rows b{b} kv{hk}")
