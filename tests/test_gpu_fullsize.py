"""Parity at the benchmark configurations' full sizes (Llama-3.1-8B shape at 32K
and 128K tokens, the 128K stride sweep gamma 16 / 32 / 64 / 128, Qwen3-14B shape
at 64K with batch 2 and GQA 5, and the 32-layer random-init Llama-3.1-8B model
prefilling 131072 tokens, and the reference's long-context geometry at 1M tokens),
where the oracle cannot run whole layers:

* exact, size-independent composition over EVERY row: the delta output equals
  rnd(sparse + rnd(dense[anchor] - sparse[anchor])) recomputed with torch bf16
  ops from the sparse-only and recompute outputs (llama.py:733-755), and the
  tail rows equal the dense rows;
* sampled rows of the sparse pass and of the dense pass, in every kv-head
  group, against the oracle (float32) on the same bf16 inputs: per-row cosine
  > 0.999, max |diff| < 2e-2.
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
    # the stride sweep at 128K (the other gammas of the long-context workload)
    "llama-128k-g16": dict(B=1, H=32, Hkv=8, S=131072, D=128, window=2048, sink=128, gamma=16,
                           theta=500000.0, qk_norm=False, q_scale=True),
    "llama-128k-g32": dict(B=1, H=32, Hkv=8, S=131072, D=128, window=2048, sink=128, gamma=32,
                           theta=500000.0, qk_norm=False, q_scale=True),
    "llama-128k-g128": dict(B=1, H=32, Hkv=8, S=131072, D=128, window=2048, sink=128, gamma=128,
                            theta=500000.0, qk_norm=False, q_scale=True),
    "qwen3-64k-b2": dict(B=2, H=40, Hkv=8, S=65536, D=128, window=4096, sink=64, gamma=64,
                         theta=1000000.0, qk_norm=True, q_scale=False),
    # the reference's published long-context geometry (1024 sinks) at 1M tokens:
    # kernel (2)'s items at their 512-tile cap, 32 splits per row tile
    "llama-1m-sink1024": dict(B=1, H=32, Hkv=8, S=1048576, D=128, window=2048, sink=1024,
                              gamma=64, theta=500000.0, qk_norm=False, q_scale=True,
                              dense_sample=4),
}


def _f32(t):
    return t.detach().float().cpu().numpy()


def check_layer(q, k, v, out, window, sink, gamma, name, dense_sample=8, kv_groups=None):
    """The size-independent checks of one delta layer output `out` [B,S,H,D]
    computed from q [B,H,S,D], k/v [B,Hkv,S,D]: exact index set, exact bf16
    composition over every row against the sparse-only and recompute outputs,
    and sampled sparse / dense rows of every kv-head group of every batch
    (or of `kv_groups`) against the oracle (float32 on the same bf16 inputs)."""
    from delta_attention import ops
    B, H, S, D = q.shape
    Hkv = k.shape[1]
    G = H // Hkv
    scale = D ** -0.5
    kw = dict(gamma=gamma, window=window, sink=sink, sm_scale=scale)
    sp = ops.delta_prefill(q, k, v, mode="sparse-only", **kw)
    rc = ops.delta_prefill(q, k, v, mode="recompute", **kw)
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
    assert torch.equal(out[:, :s_p], expect), f"{name}: delta composition differs from the bf16 reference ops"
    assert torch.equal(out[:, s_p:], rc[:, s_p:]), f"{name}: tail rows are not the dense rows"
    sel = torch.zeros(S, dtype=torch.bool, device="cuda")
    sel[ops.selected_rows(S, gamma, "cuda")] = True
    assert torch.equal(rc[:, ~sel], sp[:, ~sel]), f"{name}: recompute touched unselected rows"
    del expect, delta

    # sampled rows against the oracle, on every kv-head group
    rng = np.random.default_rng(1)
    srows = np.unique(np.concatenate([
        [0, 1, 63, 64, 127, sink - 1, sink, window - 1, window, window + 63, window + 64,
         S // 2, S // 2 + 63, S - 129, S - 64, S - 1],
        rng.integers(0, S, 8)]))
    drows = np.unique(np.concatenate([anchors[[0, 1, len(anchors) // 2, -1]], tail[[0, -1]],
                                      rng.choice(anchors, dense_sample)]))
    for b in range(B):
        for hk in (range(Hkv) if kv_groups is None else kv_groups):
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


@pytest.mark.parametrize("name", list(CONFIGS))
def test_fullsize_layer(gpu, name):
    from delta_attention import ops
    c = CONFIGS[name]
    B, H, Hkv, S, D = c["B"], c["H"], c["Hkv"], c["S"], c["D"]
    print(f"full-size layer {name}", flush=True)
    q, k, v = workload_inputs(B, H, Hkv, S, D, c["theta"], seed=0, qk_norm=c["qk_norm"],
                              q_scale=c["q_scale"])
    out = ops.delta_prefill(q, k, v, mode="delta", gamma=c["gamma"], window=c["window"],
                            sink=c["sink"], sm_scale=D ** -0.5)
    check_layer(q, k, v, out, c["window"], c["sink"], c["gamma"], name,
                dense_sample=c.get("dense_sample", 8), kv_groups=c.get("kv_groups"))


def test_fullsize_model_prefill_llama8b_128k(gpu):
    """The 32-layer random-init Llama-3.1-8B-architecture model (hidden 4096,
    32/8 heads, SwiGLU 14336, vocab 128256, bf16 weights ~ N(0, 0.02)) prefills
    131072 random token ids with delta attention in every layer (window 2048 +
    128 sinks, gamma 64). The attention inputs and output of layers 0 and 31 are
    captured in the forward and checked like a stand-alone layer (exact
    composition over every row, sampled rows against the oracle); the greedy
    next token's logits are finite and two prefills give the same token."""
    from delta_attention.model import LlamaConfig, random_llama
    cfg = LlamaConfig(delta_lambda=64, sliding_window=2048, sink_tokens=128)
    assert (cfg.num_hidden_layers, cfg.hidden_size, cfg.num_attention_heads,
            cfg.num_key_value_heads, cfg.head_dim, cfg.intermediate_size,
            cfg.vocab_size) == (32, 4096, 32, 8, 128, 14336, 128256)
    print("full model: building the random-init Llama-3.1-8B architecture", flush=True)
    model = random_llama(cfg, "cuda", torch.bfloat16, seed=0)
    S = 131072
    ids = torch.randint(0, cfg.vocab_size, (1, S), device="cuda",
                        generator=torch.Generator(device="cuda").manual_seed(1))
    captured = {}

    def hook(layer_idx, fn):
        def wrapped(module, q, k, v, *args, **kw):
            out = fn(module, q, k, v, *args, **kw)
            captured[layer_idx] = (q.clone(), k.clone(), v.clone(), out[0].clone())
            return out
        return wrapped

    for i in (0, cfg.num_hidden_layers - 1):
        at = model.model.layers[i].self_attn
        at.delta_forward = hook(i, at.delta_forward)
    with torch.inference_mode():
        h = model.model(ids)
        logits = model.lm_head(h[:, -1]).float()
        tok = logits.argmax(-1)
        del h
        for i in list(captured):
            at = model.model.layers[i].self_attn
            del at.delta_forward                  # the class method again
        tok2 = model.prefill_next_token(ids)
    torch.cuda.synchronize()
    assert torch.isfinite(logits).all()
    assert int(tok[0]) == int(tok2[0]), (int(tok[0]), int(tok2[0]))
    assert sorted(captured) == [0, cfg.num_hidden_layers - 1]
    del model
    torch.cuda.empty_cache()
    for i, (q, k, v, out) in captured.items():
        print(f"full model: layer {i}", flush=True)
        assert q.shape == (1, 32, S, 128) and out.shape == (1, S, 32, 128)
        check_layer(q, k, v, out, 2048, 128, 64, f"llama8b-128k layer {i}", dense_sample=4)
