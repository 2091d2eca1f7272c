"""GPU parity of the decode side (delta_attention/llama.py:498-657): the decode
row kernel against the oracle (sink + last-window keys, dense row), the
rectangle rows, the delta decode policies (the reference's T6/T8 and refresh
schedule checks, tests/test_delta_decode.py) and greedy generation with a
small random-init model (T7: gamma_dec 1 == dense decode; T9: repeated
generate calls agree)."""

import types

import numpy as np
import pytest
import torch

from helpers import assert_close, np64
from oracle import delta_oracle as O

pytestmark = pytest.mark.gpu


def _rand(B, H, Hkv, n, D, seed, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, 1, D, generator=g).to(dtype).cuda()
    k = torch.randn(B, Hkv, n, D, generator=g).to(dtype).cuda()
    v = torch.randn(B, Hkv, n, D, generator=g).to(dtype).cuda()
    return q, k, v


@pytest.mark.parametrize("B,H,Hkv,n,D,window,sink", [
    (1, 32, 8, 8192, 128, 2048, 128),    # sink + last window of a long cache
    (1, 32, 8, 8192, 128, 0, 0),         # the dense anchor row
    (2, 8, 2, 3000, 64, 256, 16),        # head_dim 64, batch 2
    (1, 8, 2, 3000, 32, 256, 16),        # head_dim 32
    (1, 8, 8, 1000, 128, 900, 200),      # n <= sink + window: every key
    (1, 4, 1, 1, 128, 16, 4),            # a one-key cache
    (1, 40, 8, 5000, 128, 4096, 64),     # GQA 5
    (1, 32, 8, 131072, 128, 2048, 128),  # 128K cache, sparse
    (1, 32, 8, 131072, 128, 0, 0),       # 128K cache, dense
    (1, 8, 2, 6000, 256, 1024, 64),      # head_dim 256
])
def test_decode_row_parity(gpu, B, H, Hkv, n, D, window, sink):
    from delta_attention import ops
    q, k, v = _rand(B, H, Hkv, n, D, seed=n + window)
    scale = D ** -0.5
    got = ops.decode_attention(q, k, v, window=window, sink=sink, sm_scale=scale)
    torch.cuda.synchronize()
    ref = O.decode_row(np64(q), np64(k), np64(v), window, sink, scale)
    assert_close(np64(got), ref, what=f"decode n{n} w{window} s{sink} {H}/{Hkv} D{D}")


@pytest.mark.parametrize("window,sink", [(0, 0), (512, 16)])
def test_decode_row_device_key_count(gpu, window, sink):
    """da_decode_attn_fwd_dev: k/v buffers of the cache's capacity, the key
    count read on the device when the kernels run. Each count against the
    oracle's row and the host-count call (to rounding: the split partition
    follows the capacity); then one recorded call replayed while the count
    changes gives the eager call's bits for every count."""
    from delta_attention import ops
    cap, D = 4096, 128
    q, k, v = _rand(1, 16, 4, cap, D, seed=31 + window)
    scale = D ** -0.5
    nk = torch.zeros(1, dtype=torch.int32, device="cuda")
    eager = {}
    for n in (1, 700, 2500, cap):
        nk.fill_(n)
        got = ops.decode_attention(q, k, v, window=window, sink=sink, sm_scale=scale, n_keys=nk)
        host = ops.decode_attention(q, k[:, :, :n], v[:, :, :n], window=window, sink=sink, sm_scale=scale)
        torch.cuda.synchronize()
        kn, vn = np64(k)[:, :, :n], np64(v)[:, :, :n]
        assert_close(np64(got), O.decode_row(np64(q), kn, vn, window, sink, scale),
                     what=f"device count n{n} w{window}")
        assert (got.float() - host.float()).abs().max().item() <= 4e-3
        eager[n] = got
        # the cached-delta add in the same launch: the bf16 tensor add's bits
        d = torch.randn(q.shape, generator=torch.Generator().manual_seed(n)).to(q.dtype).cuda()
        fused = ops.decode_attention(q, k, v, window=window, sink=sink, sm_scale=scale, n_keys=nk,
                                     add=d)
        torch.cuda.synchronize()
        assert torch.equal(fused, got + d)
    out = torch.empty_like(q)
    nk.fill_(1)
    ops.decode_attention(q, k, v, window=window, sink=sink, sm_scale=scale, n_keys=nk, out=out)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ops.decode_attention(q, k, v, window=window, sink=sink, sm_scale=scale, n_keys=nk, out=out)
    for n in (700, cap, 2500, 1, 700):
        nk.fill_(n)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager[n]), n


def test_rectangle_rows(gpu):
    from delta_attention.llama import LlamaAttention
    m = LlamaAttention(_cfg(), 0).cuda().to(torch.bfloat16)
    g = torch.Generator().manual_seed(4)
    n, s = 700, 5
    q = torch.randn(1, 8, s, 128, generator=g).to(torch.bfloat16).cuda()
    k = torch.randn(1, 2, n, 128, generator=g).to(torch.bfloat16).cuda()
    v = torch.randn(1, 2, n, 128, generator=g).to(torch.bfloat16).cuda()
    out, _ = m.sdpa_rectangle_forward(m, q, k, v, scaling=128 ** -0.5)
    qq = np.concatenate([np.zeros((1, 8, n - s, 128)), np64(q)], axis=2)
    ref = O.causal_attention_rows(qq, np64(k), np64(v), np.arange(n - s, n), 128 ** -0.5)
    assert_close(np64(out), ref, what="rectangle")


def _cfg(**kw):
    base = dict(hidden_size=1024, num_attention_heads=8, num_key_value_heads=2, head_dim=128,
                attention_bias=False, attention_dropout=0.0, rms_norm_eps=1e-6,
                _attn_implementation="sdpa_rectangle", mode="delta", delta_lambda=64,
                sliding_window=512, sink_tokens=64, stride_policy="fixed", log_drift=False,
                decode_mode="delta", gamma_dec=8, refresh_policy="fixed", drift_threshold=0.95,
                drift_k=2.0, gamma_dec_max=128)
    base.update(kw)
    return types.SimpleNamespace(**base)


def _step(m, q, k, v):
    with torch.no_grad():
        out, _ = m.sdpa_rectangle_forward(m, q, k, v, scaling=m.head_dim ** -0.5)
    return out


def _module(**kw):
    from delta_attention.llama import LlamaAttention
    return LlamaAttention(_cfg(**kw), 0).cuda().to(torch.bfloat16)


def test_t6_anchor_step_is_dense(gpu):
    q, k, v = _rand(1, 8, 2, 4096, 128, seed=0)      # > sink + window: sparse != dense
    m = _module(decode_mode="delta", gamma_dec=8)
    out_anchor = _step(m, q, k, v)                   # fresh state: anchor
    d = _module(decode_mode="dense")
    out_dense = _step(d, q, k, v)
    assert torch.equal(out_anchor, out_dense)
    s = _module(decode_mode="sparse")
    assert not torch.equal(_step(s, q, k, v), out_dense)


def test_t8_zero_delta_is_sparse(gpu):
    q, k, v = _rand(1, 8, 2, 4096, 128, seed=1)
    m = _module(decode_mode="delta", gamma_dec=10_000, gamma_dec_max=100_000)
    _step(m, q, k, v)
    m._dec_state["last_delta"] = torch.zeros_like(m._dec_state["last_delta"])
    q2, _, _ = _rand(1, 8, 2, 1, 128, seed=2)
    out_zero = _step(m, q2, k, v)
    s = _module(decode_mode="sparse")
    assert torch.equal(out_zero, _step(s, q2, k, v))


def test_refresh_schedule_is_per_layer(gpu):
    m0 = _module(gamma_dec=2, gamma_dec_max=100, log_drift=True)
    m1 = _module(gamma_dec=2, gamma_dec_max=100, log_drift=True)
    flags, steps = [], []
    for seed in (10, 11, 12):
        q, k, v = _rand(1, 8, 2, 4096, 128, seed=seed)
        _step(m0, q, k, v)
        flags.append(m0._dec_drift_points[-1]["anchor"])
        steps.append(m0._dec_state["steps"])
    assert flags == [True, False, True] and steps == [0, 1, 0]
    assert getattr(m1, "_dec_state", None) is None
    q, k, v = _rand(1, 8, 2, 4096, 128, seed=13)
    _step(m1, q, k, v)
    assert m1._dec_drift_points[-1]["anchor"] is True and m1._dec_state is not m0._dec_state


def test_fixed_policy_matches_oracle(gpu):
    _, k, v = _rand(1, 8, 2, 3000, 128, seed=20)
    qs = [_rand(1, 8, 2, 1, 128, seed=30 + i)[0] for i in range(6)]
    m = _module(gamma_dec=3)
    got = [np64(_step(m, q, k, v)).transpose(0, 2, 1, 3) for q in qs]
    ref = O.delta_decode_steps([np64(q) for q in qs], np64(k), np64(v), 512, 64,
                               128 ** -0.5, gamma_dec=3)
    for i, (g_, r) in enumerate(zip(got, ref)):
        assert_close(g_, r, what=f"step {i}")


def test_drift_policies(gpu):
    _, k, v = _rand(1, 8, 2, 3000, 128, seed=40)
    qs = [_rand(1, 8, 2, 1, 128, seed=50 + i)[0] for i in range(4)]
    always = _module(refresh_policy="drift", drift_threshold=2.0, log_drift=True)   # cos < 2
    never = _module(refresh_policy="drift", drift_threshold=-2.0, gamma_dec_max=3, log_drift=True)
    rel = _module(refresh_policy="drift_rel", log_drift=True)
    for q in qs:
        _step(always, q, k, v)
        _step(never, q, k, v)
        _step(rel, q, k, v)
    assert [p["anchor"] for p in always._dec_drift_points] == [True] * 4
    assert [p["anchor"] for p in never._dec_drift_points] == [True, False, False, True]  # the cap
    assert [p["anchor"] for p in rel._dec_drift_points] == [True, False, False, False]   # < 8 history
    assert len(rel._dec_state["cos_hist"]) == 3


def _walk_qs(n, seed, sig):
    """Query rows that random-walk with step sizes sig[t], kept at unit RMS:
    small steps keep consecutive sparse rows close (cosine near 1), large ones
    break them."""
    g = torch.Generator().manual_seed(seed)
    cur = torch.randn(1, 8, 1, 128, generator=g)
    qs = []
    for t in range(n):
        cur = cur + sig[t % len(sig)] * torch.randn(1, 8, 1, 128, generator=g)
        cur = cur / cur.pow(2).mean().sqrt()
        qs.append(cur.to(torch.bfloat16).cuda())
    return qs


def _margins(cos, policy, threshold, k):
    """Distance of each tested cosine from its decision bound (the oracle's
    rule without the count triggers): a comparison of GPU and oracle flags is
    only well posed when every margin is clear of the rows' rounding."""
    out, rec = [], []
    for c in cos[1:]:
        if policy == "drift":
            out.append(abs(c - threshold))
        else:
            if len(rec) >= 8:
                m = float(np.mean(rec))
                out.append(abs(c - (m - k * float(np.std(rec)))))
            rec = (rec + [c])[-16:]
    return out


@pytest.mark.parametrize("policy", ["fixed", "drift", "drift_rel"])
@pytest.mark.parametrize("log_drift", [False, True])
def test_policies_match_oracle(gpu, policy, log_drift):
    """Each refresh policy over 26 decode steps: outputs and anchor steps
    against the oracle's delta_decode_steps (llama.py:551-634), with the drift
    thresholds placed between the realised cosines of consecutive sparse rows."""
    _, k, v = _rand(1, 8, 2, 3000, 128, seed=60)
    qs = _walk_qs(26, seed=61, sig=[0.02, 0.03, 0.02, 1.5, 0.02, 0.04, 0.02, 0.03, 0.02,
                                    0.03, 0.02, 0.05, 3.0])
    scale = 128 ** -0.5
    qn = [np64(q) for q in qs]
    sp = [O.decode_row(q, np64(k), np64(v), 512, 64, scale) for q in qn]
    cos = [None] + [O.flat_cos(sp[t], sp[t - 1]) for t in range(1, len(sp))]
    params = dict(gamma_dec=5, gamma_dec_max=11, drift_threshold=0.9, drift_k=2.0)
    if policy == "drift":
        srt = sorted(c for c in cos[1:])
        gap = max(range(len(srt) - 1), key=lambda i: srt[i + 1] - srt[i])
        params["drift_threshold"] = 0.5 * (srt[gap] + srt[gap + 1])
    if policy != "fixed":
        marg = _margins(cos, policy, params["drift_threshold"], params["drift_k"])
        assert marg and min(marg) > 1e-3, f"test inputs too close to the bound: {min(marg)}"
    ref, flags = O.delta_decode_steps(qn, np64(k), np64(v), 512, 64, scale, policy=policy,
                                      return_flags=True, **params)
    assert any(flags[1:]) and not all(flags[1:]), flags
    m = _module(refresh_policy=policy, log_drift=log_drift, **params)
    got_flags = []
    for t, q in enumerate(qs):
        out = _step(m, q, k, v)
        got_flags.append(m._dec_state["steps"] == 0)
        assert_close(np64(out).transpose(0, 2, 1, 3), ref[t], what=f"{policy} step {t}")
    assert got_flags == flags
    if log_drift:
        pts = m._dec_drift_points
        assert [p["anchor"] for p in pts] == flags
        assert all(abs(p["drift_cos"] - 1.0) < 1e-5 for p, f in zip(pts, flags) if f)
        assert all(abs(p["applied_vs_true_cos"] - 1.0) < 1e-5 for p, f in zip(pts, flags) if f)


def _small_model(**kw):
    from delta_attention.model import LlamaConfig, random_llama
    cfg = LlamaConfig(vocab_size=512, hidden_size=2048, intermediate_size=4096, num_hidden_layers=2,
                      num_attention_heads=16, num_key_value_heads=4, head_dim=128,
                      delta_lambda=64, sliding_window=256, sink_tokens=16, **kw)
    return random_llama(cfg, "cuda", torch.bfloat16, seed=7)


def test_t7_gamma1_generation_equals_dense(gpu):
    m = _small_model()
    ids = torch.randint(0, 512, (1, 900), device="cuda", generator=torch.Generator(device="cuda").manual_seed(8))
    m.config.decode_mode = "dense"
    dense = m.generate_greedy(ids, 12)
    m.config.decode_mode, m.config.gamma_dec = "delta", 1
    delta = m.generate_greedy(ids, 12)
    assert torch.equal(dense, delta)


def test_t9_repeated_generate_is_identical(gpu):
    m = _small_model(decode_mode="delta", gamma_dec=4)
    ids = torch.randint(0, 512, (1, 900), device="cuda", generator=torch.Generator(device="cuda").manual_seed(9))
    a = m.generate_greedy(ids, 10)
    b = m.generate_greedy(ids, 10)
    assert torch.equal(a, b) and a.shape == (1, 10)
    m.config.decode_mode = "sparse"
    assert m.generate_greedy(ids, 10).shape == (1, 10)


@pytest.mark.parametrize("mode,gamma_dec", [("dense", 1), ("sparse", 1), ("delta", 3)])
def test_graph_decode_replays(gpu, mode, gamma_dec):
    """Greedy decode with each step recorded once per step kind and replayed
    (delta: anchor steps every gamma_dec steps and plain steps; the token's
    row and the key count advance on the device). Same logits, bit for bit,
    as the same static steps run eagerly, over several replays of each kind;
    and to rounding the logits of the host-length decode steps."""
    m = _small_model(decode_mode=mode, gamma_dec=gamma_dec)
    assert m.graph_decodable()
    ids = torch.randint(0, 512, (1, 700), device="cuda",
                        generator=torch.Generator(device="cuda").manual_seed(11))
    lg_graph, lg_static, lg_eager = [], [], []
    a = m.generate_greedy(ids, 10, graph=True, logits_out=lg_graph)
    b = m.generate_greedy(ids, 10, graph=True, record=False, logits_out=lg_static)
    c = m.generate_greedy(ids, 10, logits_out=lg_eager)
    torch.cuda.synchronize()
    assert a.shape == (1, 10) and torch.equal(a, b)
    assert len(lg_graph) == len(lg_static) == 10
    for x, y in zip(lg_graph, lg_static):
        assert torch.equal(x, y)
    # against the host-length steps while both decoded the same tokens
    n_same = int((a == c).long().cumprod(1).sum())
    assert n_same >= 2
    for i in range(n_same):
        d = (lg_graph[i] - lg_eager[i]).abs().max().item()
        assert d <= 2e-2 * max(1.0, lg_eager[i].abs().max().item()), (i, d)


def test_graph_decode_falls_back_for_drift_policies(gpu):
    m = _small_model(decode_mode="delta", gamma_dec=4, refresh_policy="drift", drift_threshold=0.9)
    assert not m.graph_decodable()
    ids = torch.randint(0, 512, (1, 300), device="cuda",
                        generator=torch.Generator(device="cuda").manual_seed(12))
    assert torch.equal(m.generate_greedy(ids, 5, graph=True), m.generate_greedy(ids, 5))
