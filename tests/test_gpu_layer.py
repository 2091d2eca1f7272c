"""GPU parity of the composed layer prefill (kernels 1 -> 2 -> 3) and of the
attention modules, against the oracle's delta_forward (llama.py:659-757) on
identical seeded inputs, plus the reference's identities T2-T4 on the GPU path.
"""

import types

import numpy as np
import pytest
import torch

from helpers import assert_close, gen_qkv, np64
from oracle import delta_oracle as O

pytestmark = pytest.mark.gpu


def _layer(B, H, Hkv, S, D, gamma, window, sink, mode="delta", seed=0, dtype=torch.bfloat16):
    from delta_attention import ops
    q, k, v = gen_qkv(B, H, Hkv, S, D, seed=seed, dtype=dtype)
    scale = D ** -0.5
    out = ops.delta_prefill(q, k, v, gamma=gamma, window=window, sink=sink, sm_scale=scale, mode=mode)
    torch.cuda.synchronize()
    qn, kn, vn = np64(q), np64(k), np64(v)
    ref = O.delta_forward(qn, kn, vn, gamma, window, sink, scale, mode=mode)
    return np64(out), ref, (qn, kn, vn)


@pytest.mark.parametrize("B,H,Hkv,S,D,gamma,window,sink", [
    (1, 8, 2, 4096, 64, 16, 512, 64),     # the CPU configuration's shape (bf16 on the GPU path)
    (1, 8, 2, 2048, 128, 64, 512, 128),   # Llama geometry, shortened
    (2, 10, 2, 1024, 128, 64, 256, 64),   # Qwen3 geometry (GQA 5, batch 2), shortened
    (1, 4, 4, 1200, 128, 32, 128, 8),     # s % gamma != 0
    (1, 4, 1, 768, 64, 128, 192, 0),      # gamma 128
    (1, 8, 2, 1300, 32, 64, 256, 16),     # head_dim 32 (fused order)
    (1, 4, 4, 900, 32, 128, 128, 8),      # head_dim 32, gamma 128 with MHA (fused, 128-row tiles)
    (1, 8, 2, 1500, 256, 64, 384, 16),    # head_dim 256 (one workgroup per CU), fused order
    (1, 4, 4, 700, 256, 32, 128, 4),      # head_dim 256, MHA: one head per 128-row tile
    (1, 16, 2, 1536, 128, 64, 384, 32),   # GQA 8 (Llama-3-70B ratio): four head splits per row block
    (1, 8, 1, 1000, 64, 32, 256, 8),      # GQA 8, one kv head, head_dim 64, s % gamma != 0
])
def test_delta_prefill_parity(gpu, B, H, Hkv, S, D, gamma, window, sink):
    got, ref, _ = _layer(B, H, Hkv, S, D, gamma, window, sink)
    assert_close(got, ref, what=f"delta B{B} H{H}/{Hkv} S{S} D{D} g{gamma} w{window} sink{sink}")


@pytest.mark.parametrize("mode", ["sparse-only", "recompute"])
def test_delta_prefill_modes(gpu, mode):
    got, ref, _ = _layer(1, 8, 2, 1024, 128, 32, 256, 16, mode=mode)
    assert_close(got, ref, what=mode)


def test_short_sequence_is_all_dense(gpu):
    # s <= cut_n: the reference crashes (negative s_p); here every row is dense
    from delta_attention import ops
    q, k, v = gen_qkv(1, 4, 2, 100, 128, seed=0)
    out = ops.delta_prefill(q, k, v, gamma=64, window=32, sink=4, sm_scale=128 ** -0.5)
    torch.cuda.synchronize()
    dense = O.causal_attention_rows(np64(q), np64(k), np64(v), np.arange(100), 128 ** -0.5)
    assert_close(np64(out), dense, what="short")


def test_t2_anchor_exactness_and_index_set(gpu):
    s, gamma = 2048, 64
    got, ref, (q, k, v) = _layer(1, 8, 2, s, 128, gamma, 256, 16, seed=1)
    anchors, tail, s_p, _ = O.anchor_layout(s, gamma)
    rows = np.concatenate([anchors, tail])
    dense = O.causal_attention_rows(q, k, v, rows, 128 ** -0.5)
    assert_close(got[:, rows], dense, what="T2 anchors+tail")
    # the rows the GPU path computed densely are exactly the oracle's index set
    from delta_attention import ops
    np.testing.assert_array_equal(ops.selected_rows(s, gamma, "cuda").cpu().numpy(), rows)


def test_t3_gamma1_is_dense(gpu):
    s = 1024
    got, _, (q, k, v) = _layer(1, 4, 2, s, 128, 1, 128, 4, seed=2)
    dense = O.causal_attention_rows(q, k, v, np.arange(s), 128 ** -0.5)
    assert_close(got, dense, what="T3")


def test_t4_full_window_is_dense(gpu):
    s = 1024
    got, _, (q, k, v) = _layer(1, 4, 2, s, 128, 64, s, 0, seed=3)
    dense = O.causal_attention_rows(q, k, v, np.arange(s), 128 ** -0.5)
    assert_close(got, dense, what="T4")


def _cfg(H, Hkv, D, **kw):
    base = dict(hidden_size=H * D, num_attention_heads=H, num_key_value_heads=Hkv, head_dim=D,
                attention_bias=False, attention_dropout=0.0, rms_norm_eps=1e-6,
                _attn_implementation="window", mode="delta", delta_lambda=64,
                sliding_window=256, sink_tokens=16, stride_policy="fixed", log_drift=False,
                adapt_chunk=512, adapt_threshold=0.95, gamma_min=16, gamma_max=256,
                stride_trigger="absolute", adapt_k=2.0)
    base.update(kw)
    return types.SimpleNamespace(**base)


def test_module_delta_forward_matches_ops(gpu):
    from delta_attention import ops
    from delta_attention.llama import LlamaAttention
    from delta_attention.validation import anchor_exactness_check
    cfg = _cfg(8, 2, 128, log_drift=True)
    m = LlamaAttention(cfg, layer_idx=0).cuda().to(torch.bfloat16)
    q, k, v = gen_qkv(1, 8, 2, 1536, 128, seed=4, model_layout=True)
    out, w = m.delta_forward(m, q, k, v, None, scaling=m.scaling)
    assert w is None
    ref = ops.delta_prefill(q, k, v, gamma=64, window=256, sink=16, sm_scale=m.scaling)
    assert torch.equal(out, ref)
    assert m._drift_stats["n"] == (ops.anchor_layout(1536, 64)[2] - 1) * 8
    _, delta = ops.delta_prefill(q, k, v, gamma=64, window=256, sink=16, sm_scale=m.scaling,
                                 return_delta=True)
    assert m._drift_stats["mean"] == pytest.approx(O.interanchor_cos(np64(delta)).mean(), abs=1e-5)
    # fp32 inputs run in bf16 and come back as fp32 (llama.py:382-388, 493-494)
    out32, _ = m.delta_forward(m, q.float(), k.float(), v.float(), None, scaling=m.scaling)
    assert out32.dtype == torch.float32 and torch.equal(out32.to(torch.bfloat16), out)
    assert anchor_exactness_check(m, gamma=64, window=256, s=2048) > 0.999


def test_module_drift_stats_read_from_another_stream(gpu):
    """The layer leaves its drift summary as a deferred read on the stream it
    ran on: a layer run on a side stream and read from the default stream
    gives the summary of the same deltas computed in one go."""
    from delta_attention import ops
    from delta_attention.drift import drift_summary
    from delta_attention.llama import LlamaAttention
    cfg = _cfg(8, 2, 128, log_drift=True)
    m = LlamaAttention(cfg, layer_idx=3).cuda().to(torch.bfloat16)
    q, k, v = gen_qkv(1, 8, 2, 4096, 128, seed=9, model_layout=True)
    _, delta = ops.delta_prefill(q, k, v, gamma=64, window=256, sink=16, sm_scale=m.scaling,
                                 return_delta=True)
    want = drift_summary(delta, 3, 64, 4096)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        m.delta_forward(m, q, k, v, None, scaling=m.scaling)
    got = m._drift_stats
    assert got == want
    assert m._drift_stats is got     # read back once, then kept
    torch.cuda.current_stream().wait_stream(side)


def test_module_forward_and_qwen3(gpu):
    from delta_attention.llama import LlamaAttention, rope_cos_sin
    from delta_attention.qwen3 import Qwen3DeltaAttention
    torch.manual_seed(0)
    for cls, H, Hkv in ((LlamaAttention, 8, 2), (Qwen3DeltaAttention, 10, 2)):
        cfg = _cfg(H, Hkv, 128)
        m = cls(cfg, layer_idx=1).cuda().to(torch.bfloat16)
        for p in m.parameters():
            torch.nn.init.normal_(p, std=0.02)
        x = torch.randn(1, 1024, H * 128, device="cuda", dtype=torch.bfloat16)
        pos = torch.arange(1024, device="cuda")[None]
        cos, sin = rope_cos_sin(pos, 128, 500000.0, torch.bfloat16)
        seen = []   # the attention output, as o_proj receives it
        hook = m.o_proj.register_forward_pre_hook(lambda mod, args: seen.append(args[0].clone()))
        try:
            y, _ = m(x, (cos, sin))
        finally:
            hook.remove()
        torch.cuda.synchronize()
        # oracle: the same prologue in numpy, then delta_forward
        hs = (1, 1024, -1, 128)
        qp = np64(m.q_proj(x).view(hs).transpose(1, 2))
        kp = np64(m.k_proj(x).view(hs).transpose(1, 2))
        vp = np64(m.v_proj(x).view(hs).transpose(1, 2))
        if cls is Qwen3DeltaAttention:   # per-head q/k RMSNorm with the (random) norm weights
            qp = O.rms_norm(qp, 1e-6, np64(m.q_norm.weight)).astype(np.float64)
            kp = O.rms_norm(kp, 1e-6, np64(m.k_norm.weight)).astype(np.float64)
        c, s_ = O.rope_cos_sin(1024, 128, 500000.0)
        qr, kr = O.apply_rope(qp, c, s_), O.apply_rope(kp, c, s_)
        # the module rounds the post-RoPE q/k to bf16 before the kernels
        qr, kr = O.round_bf16(qr).astype(np.float64), O.round_bf16(kr).astype(np.float64)
        vr = O.round_bf16(vp).astype(np.float64)
        att = O.delta_forward(qr, kr, vr, 64, 256, 16, 128 ** -0.5)
        # the layer's delta attention itself, at cosine 0.999 / max |diff| 2e-2
        assert len(seen) == 1 and seen[0].shape == (1, 1024, H * 128)
        assert_close(np64(seen[0]).reshape(1, 1024, H, 128), att, what=f"{cls.__name__} attention")
        # and through o_proj (a bf16 GEMM of 1024 x H*128 by the random weights)
        y_ref = att.reshape(1, 1024, -1) @ np64(m.o_proj.weight).T
        assert_close(np64(y)[0], y_ref[0], cos_min=0.99, atol=5e-2, what=f"{cls.__name__} forward")


@pytest.mark.parametrize("mode", ["delta", "recompute"])
def test_adaptive_stride_path(gpu, mode):
    """The adaptive policy in the reference's branch order (llama.py:695-711):
    it replaces the uniform stride for "delta" and for "recompute" alike."""
    from delta_attention.llama import LlamaAttention
    cfg = _cfg(4, 2, 128, stride_policy="adaptive", adapt_chunk=512, delta_lambda=64,
               adapt_threshold=0.5, gamma_min=16, gamma_max=128, mode=mode)
    m = LlamaAttention(cfg, layer_idx=0).cuda().to(torch.bfloat16)
    s = 2048
    q, k, v = gen_qkv(1, 4, 2, s, 128, seed=8)
    out, _ = m.delta_forward(m, q, k, v, None, scaling=m.scaling)
    torch.cuda.synchronize()
    st = m._stride_stats
    idx = []
    for c in st["chunks"]:
        end = min(c["start"] + 512, s - 128 - s % 64)
        idx += list(range(c["start"], end, c["gamma"]))
    idx = np.array(idx)
    assert len(idx) == st["n_anchors"]
    qn, kn, vn = np64(q), np64(k), np64(v)
    scale = 128 ** -0.5
    sparse = O.sparse_attention(qn, kn, vn, 256, 16, scale)
    s_p = s - (s % 64 + 128)
    dense_sel = O.causal_attention_rows(qn, kn, vn, idx, scale)
    tail = O.causal_attention_rows(qn, kn, vn, np.arange(s_p, s), scale)
    ref = np.concatenate([O.apply_delta_variable(sparse, dense_sel, idx, s_p), tail], 1)
    assert_close(np64(out), ref, what=f"adaptive ({mode})")


@pytest.mark.parametrize("trigger,threshold,k,B", [("absolute", None, 2.0, 1), ("relative", 0.95, 0.3, 1),
                                                    ("absolute", None, 2.0, 2)])
def test_adaptive_device_decisions_follow_the_host_rules(gpu, trigger, threshold, k, B):
    """The adaptive chunk loop decides each next stride on the device
    (da_adapt_chunk_step). Checked against the host rules of stride.py:
    every logged stride follows from the previous chunk's logged mean by
    next_gamma / next_gamma_relative, and each logged mean and min equal the
    chunk deltas' cosines recomputed here from the layer's own sparse pass
    and dense anchor rows (anchor_delta_cos, fp64 mean). The absolute
    threshold is set between the chunk means of a first run, so that the
    stride does move."""
    from delta_attention import ops
    from delta_attention.llama import LlamaAttention
    from delta_attention.stride import next_gamma, next_gamma_relative
    s, chunk, window, sink = 4096, 256, 256, 16
    q, k_, v = gen_qkv(B, 8, 2, s, 128, seed=12)

    def run(thr):
        cfg = _cfg(8, 2, 128, stride_policy="adaptive", adapt_chunk=chunk, delta_lambda=32,
                   adapt_threshold=thr, gamma_min=8, gamma_max=128, stride_trigger=trigger,
                   adapt_k=k, sliding_window=window, sink_tokens=sink)
        m = LlamaAttention(cfg, layer_idx=0).cuda().to(torch.bfloat16)
        m.delta_forward(m, q, k_, v, None, scaling=m.scaling)
        torch.cuda.synchronize()
        return m._stride_stats["chunks"]

    if threshold is None:
        means = sorted(c["cos_mean"] for c in run(0.5))
        threshold = means[len(means) // 2]
    chunks = run(threshold)
    gammas = [c["gamma"] for c in chunks]
    assert len(set(gammas)) > 1, gammas
    for c in range(len(chunks) - 1):
        g, cm = chunks[c]["gamma"], chunks[c]["cos_mean"]
        if trigger == "absolute":
            want = next_gamma(cm, g, threshold=threshold, gamma_min=8, gamma_max=128)
        else:
            want = next_gamma_relative(cm, [x["cos_mean"] for x in chunks[:c]], g, k=k,
                                       gamma_min=8, gamma_max=128)
        assert chunks[c + 1]["gamma"] == want, (c, chunks[c], chunks[c + 1])
    sparse = ops.sparse_attention(q, k_, v, window=window, sink=sink, sm_scale=128 ** -0.5)
    for c in chunks:
        rows = torch.arange(c["start"], c["start"] + chunk, c["gamma"], device="cuda")
        rows = rows[rows < s - (s % 32 + 128)]
        assert rows.numel() == c["n_anchors"]
        dense = ops.qsparse_attention(q, k_, v, rows, 128 ** -0.5, q_rows=rows).transpose(1, 2)
        if rows.numel() < 2:
            assert c["cos_mean"] == 1.0 and c["cos_min"] == 1.0
            continue
        cos = ops.anchor_delta_cos(dense, sparse=sparse, rows=rows).cpu().double().numpy()
        assert abs(cos.mean() - c["cos_mean"]) <= 1e-12, (cos.mean(), c)
        assert float(cos.min()) == c["cos_min"]


def _with_heads(cases, H=8, Hkv=2, D=128):
    """Pad (B, s, chunk, gamma0, gmin, dtype[, H, Hkv[, D]]) cases to full length."""
    return [c + (H, Hkv, D)[len(c) - 6:] for c in cases]


@pytest.mark.parametrize("B,s,chunk,gamma0,gmin,dtype,H,Hkv,D", _with_heads([
    (1, 4096, 512, 32, 8, torch.bfloat16), (1, 3000, 1024, 64, 16, torch.bfloat16),
    (1, 2500, 1000, 64, 16, torch.bfloat16),      # adapt_chunk not a multiple of gamma0
    # no rows ahead, and chunks of 63 and 125 anchors (more row tiles than the first chunk's 16)
    (1, 4500, 1000, 64, 8, torch.bfloat16),
    (2, 3072, 512, 32, 8, torch.bfloat16),        # batch 2: the cosines average over it
    (1, 1000, 2048, 64, 16, torch.bfloat16),      # one chunk, shorter than adapt_chunk
    (1, 2600, 256, 128, 16, torch.bfloat16),      # starting stride 128: chunks of 2 anchors
    (1, 1500, 96, 16, 4, torch.bfloat16),         # many short chunks, strides down to 4
    (1, 2048, 512, 32, 16, torch.float16), (2, 1800, 600, 64, 16, torch.float16),
    # head layouts other than 8 / 2 at head_dim 128: five query heads per KV
    # head (a row tile holds 25.6 query rows), one, and head_dim 64
    (1, 3000, 512, 32, 8, torch.bfloat16, 10, 2), (1, 2200, 1024, 64, 16, torch.bfloat16, 4, 4),
    (1, 2600, 512, 32, 8, torch.bfloat16, 8, 2, 64)]))
def test_adaptive_layer_composition_is_exact(gpu, B, s, chunk, gamma0, gmin, dtype, H, Hkv, D):
    """The one-call adaptive layer (da_adapt_layer_fwd) against the same
    steps issued one by one: the key-sparse pass over all rows; each chunk's
    dense anchor rows from the same kernel (2) launch as inside, i.e. when
    gamma0 divides adapt_chunk and the chunk's stride is a multiple of gamma0
    the rows-ahead launch (every multiple of gamma0 below s_p, keys < s_p),
    else the chunk's own launch (its -1-padded row list, keys < the chunk's
    end, the same live-row plan); the deltas rnd(dense - sparse[anchor]) and
    rows rnd(sparse + delta) in torch bf16 ops (stride.py:26-40); and the dense
    tail. Bit-identical: the row selection, the per-chunk in-place broadcast,
    the row ranges of the sparse pass and the tail scatter change no bits."""
    from delta_attention import ops
    from delta_attention.llama import LlamaAttention
    window, sink = 256, 16
    scale = D ** -0.5
    q, k, v = gen_qkv(B, H, Hkv, s, D, seed=21 + B, dtype=dtype)
    cfg = _cfg(H, Hkv, D, stride_policy="adaptive", adapt_chunk=chunk, delta_lambda=gamma0,
               adapt_threshold=0.97, gamma_min=gmin, gamma_max=128, sliding_window=window,
               sink_tokens=sink)
    m = LlamaAttention(cfg, layer_idx=0).cuda().to(dtype)
    out, _ = m.delta_forward(m, q, k, v, None, scaling=scale)
    st = m._stride_stats
    cut_n = s % gamma0 + max(128, gamma0)
    s_p = s - cut_n
    max_n = -(-min(chunk, s_p) // min(gamma0, gmin))
    n_live = min(max_n, max(1, -(-chunk // gamma0)))
    sparse = ops.sparse_attention(q, k, v, window=window, sink=sink, sm_scale=scale)
    ref = sparse.clone()
    assert len(st["chunks"]) == -(-s_p // chunk)
    ahead = None
    if chunk % gamma0 == 0:
        ahead_rows = torch.arange(0, s_p, gamma0, device="cuda")
        ahead = ops.qsparse_attention(q, k[:, :, :s_p], v[:, :, :s_p], ahead_rows, scale,
                                      q_rows=ahead_rows)
    recomputed = 0
    for c in st["chunks"]:
        start, g, n_c = c["start"], c["gamma"], c["n_anchors"]
        end = min(start + chunk, s_p)
        rows = torch.arange(start, end, g, device="cuda")
        assert rows.numel() == n_c
        if ahead is not None and g % gamma0 == 0:
            dense = ahead[:, :, start // gamma0::g // gamma0][:, :, :n_c]
        else:
            recomputed += 1
            padded = torch.full((max_n,), -1, dtype=torch.int64, device="cuda")
            padded[:n_c] = rows
            dense = ops.qsparse_attention(
                q, k[:, :, :end], v[:, :, :end], padded, scale, q_rows=padded, n_live=n_live,
                n_dev=torch.tensor([n_c], dtype=torch.int32, device="cuda"))[:, :, :n_c]
        assert dense.dtype == dtype
        delta = dense.transpose(1, 2) - sparse[:, rows]
        owner = torch.div(torch.arange(start, end, device="cuda") - start, g, rounding_mode="floor")
        ref[:, start:end] = sparse[:, start:end] + delta[:, owner]
    tail = torch.arange(s_p, s, device="cuda")
    ref[:, s_p:] = ops.qsparse_attention(q, k, v, tail, scale, q_rows=tail).transpose(1, 2)
    torch.cuda.synchronize()
    assert torch.equal(out, ref), (out.float() - ref.float()).abs().max().item()
    gammas = {c["gamma"] for c in st["chunks"]}
    print(f"chunks {len(st['chunks'])} strides {sorted(gammas)} recomputed {recomputed} "
          f"anchors {[c['n_anchors'] for c in st['chunks']]}", flush=True)
    if (s, chunk) == (4500, 1000):
        assert max(c["n_anchors"] for c in st["chunks"]) > 64, st["chunks"]


def test_adaptive_layer_strided_inputs(gpu):
    """The module hands over q/k/v as [B,H,S,D] views of [B,S,H,D] projections:
    the one-call adaptive layer reads them through their strides, with the
    bits of the same call on contiguous copies."""
    from delta_attention.llama import LlamaAttention
    q, k, v = gen_qkv(2, 8, 2, 2304, 128, seed=33, model_layout=True)
    assert not q.is_contiguous()
    cfg = _cfg(8, 2, 128, stride_policy="adaptive", adapt_chunk=512, delta_lambda=32,
               adapt_threshold=0.97, gamma_min=8, gamma_max=128)
    m = LlamaAttention(cfg, layer_idx=0).cuda().to(torch.bfloat16)
    out_v, _ = m.delta_forward(m, q, k, v, None, scaling=128 ** -0.5)
    st_v = m._stride_stats
    out_c, _ = m.delta_forward(m, q.contiguous(), k.contiguous(), v.contiguous(), None,
                               scaling=128 ** -0.5)
    torch.cuda.synchronize()
    assert m._stride_stats["chunks"] == st_v["chunks"]
    assert torch.equal(out_v, out_c)


def test_adaptive_policy_sparse_only_returns_the_sparse_pass(gpu):
    """mode "sparse-only" returns before the adaptive branch (llama.py:695-696)."""
    from delta_attention.llama import LlamaAttention
    cfg = _cfg(4, 2, 128, stride_policy="adaptive", adapt_chunk=512, delta_lambda=64,
               adapt_threshold=0.5, gamma_min=16, gamma_max=128, mode="sparse-only")
    m = LlamaAttention(cfg, layer_idx=0).cuda().to(torch.bfloat16)
    q, k, v = gen_qkv(1, 4, 2, 1024, 128, seed=9)
    out, _ = m.delta_forward(m, q, k, v, None, scaling=m.scaling)
    torch.cuda.synchronize()
    assert getattr(m, "_stride_stats", None) is None   # no adaptive pass ran
    ref = O.sparse_attention(np64(q), np64(k), np64(v), 256, 16, 128 ** -0.5)
    assert_close(np64(out), ref, what="adaptive policy, sparse-only")


@pytest.mark.parametrize("B,H,Hkv,S,D,gamma,window,sink", [
    (1, 8, 2, 4096, 128, 64, 512, 128),   # GQA 4: 64-row tiles, two heads each
    (2, 8, 2, 1200, 128, 16, 256, 8),     # s % gamma != 0, batch 2
    (1, 4, 4, 1000, 64, 128, 192, 4),     # MHA: 128-row tiles, gamma 128
    (1, 6, 3, 777, 128, 32, 100, 0),      # GQA 2
    (1, 8, 2, 600, 128, 1, 128, 16),      # gamma 1: every row before the tail is an anchor
    (2, 10, 2, 1100, 128, 64, 256, 16),   # GQA 5 (Qwen3): one head per 128-row tile
    (1, 8, 2, 1500, 128, 128, 256, 16),   # GQA 4, gamma 128: one head per 128-row tile,
                                          # against kernel (1)'s two-head packing
    (1, 8, 2, 1000, 256, 64, 256, 16),    # head_dim 256
])
def test_fused_delta_bit_identical(gpu, rows_per_wave, B, H, Hkv, S, D, gamma, window, sink):
    """Kernel (3) fused into kernel (1)'s epilogue (kernel (2) first) gives the
    same bits as the three-kernel sequence, deltas included, and matches the
    oracle's delta_forward."""
    from delta_attention import ops
    rows = ops.fused_delta_rows(H, Hkv)
    assert rows and rows % gamma == 0          # the fused path is the one taken
    q, k, v = gen_qkv(B, H, Hkv, S, D, seed=gamma + S, model_layout=True)
    scale = D ** -0.5
    a, da = ops.delta_prefill(q, k, v, gamma=gamma, window=window, sink=sink, sm_scale=scale,
                              return_delta=True)
    b, db = ops.delta_prefill(q, k, v, gamma=gamma, window=window, sink=sink, sm_scale=scale,
                              return_delta=True, fused=False)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    assert torch.equal(da, db)
    ref = O.delta_forward(np64(q), np64(k), np64(v), gamma, window, sink, scale)
    assert_close(np64(a), ref, what=f"fused B{B} H{H}/{Hkv} S{S} g{gamma}")


@pytest.mark.parametrize("H,Hkv,D,gamma", [(8, 2, 128, 64), (4, 4, 64, 32), (10, 2, 128, 16),
                                            (8, 2, 64, 128)])
def test_fused_delta_bit_identical_fp16(gpu, rows_per_wave, H, Hkv, D, gamma):
    """The fused order in fp16 (the delta and the add round to fp16): same bits
    as the three-kernel sequence, within the T1 gate of the oracle."""
    from delta_attention import ops
    S, window, sink = 1500, 256, 16
    assert ops.fused_delta_rows(H, Hkv) % gamma == 0
    q, k, v = gen_qkv(1, H, Hkv, S, D, seed=H + D, dtype=torch.float16, model_layout=True)
    scale = D ** -0.5
    a, da = ops.delta_prefill(q, k, v, gamma=gamma, window=window, sink=sink, sm_scale=scale,
                              return_delta=True)
    b, db = ops.delta_prefill(q, k, v, gamma=gamma, window=window, sink=sink, sm_scale=scale,
                              return_delta=True, fused=False)
    torch.cuda.synchronize()
    assert a.dtype == torch.float16 and da.dtype == torch.float16
    assert torch.equal(a, b)
    assert torch.equal(da, db)
    ref = O.delta_forward(np64(q), np64(k), np64(v), gamma, window, sink, scale)
    assert_close(np64(a), ref, what=f"fused fp16 H{H}/{Hkv} D{D} g{gamma}")


def test_unfused_when_gamma_exceeds_the_tile(gpu):
    # gamma 256 does not divide the largest fused tile: the three-kernel path runs
    from delta_attention import ops
    assert ops.fused_delta_rows(8, 2) % 256 != 0
    got, ref, _ = _layer(1, 8, 2, 1024, 128, 256, 256, 16, seed=3)
    assert_close(got, ref, what="gamma 256, gqa 4")
