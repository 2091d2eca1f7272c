"""Pins the CPU oracle (oracle/delta_oracle.py) before it is trusted as the
parity reference: brute force on tiny inputs, library routines (torch SDPA in
float64) on the special cases that reduce to them, closed forms and the
reference's own known-answer identities (T1-T4 of
tests/test_math_identities.py, the delta_kernel.py in-file tests).

The reference ships no numeric fixtures; the integer constants below are the
sizes of the reference's benchmark configurations derived by hand from the
formulas in validation.py:224-232 and flex_delta.py:59-61.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import delta_oracle as O


def _sdpa64(q, k, v, scale, mask=None, causal=False):
    """Library reference: torch SDPA in float64 on [B,H,n,d] numpy inputs."""
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).double()
    H = q.shape[1]
    kk = np.repeat(k, H // k.shape[1], axis=1)
    vv = np.repeat(v, H // v.shape[1], axis=1)
    m = None if mask is None else torch.from_numpy(mask)
    return F.scaled_dot_product_attention(t(q), t(kk), t(vv), attn_mask=m, is_causal=causal,
                                          scale=scale).numpy()


def _qkv(B, H, Hkv, S, d, seed=0, N=None):
    rng = np.random.default_rng(seed)
    N = S if N is None else N
    return (rng.standard_normal((B, H, S, d)), rng.standard_normal((B, Hkv, N, d)),
            rng.standard_normal((B, Hkv, N, d)))


# ---------------------------------------------------------------------------
# index layout

@pytest.mark.parametrize("s,gamma,n_anchor,n_sel", [
    (4096, 16, 248, 376),        # CPU config: s 4096, gamma 16
    (32768, 64, 510, 638),       # Llama 32K, gamma 64
    (131072, 16, 8184, 8312),    # Llama 128K gamma sweep
    (131072, 32, 4092, 4220),
    (131072, 64, 2046, 2174),
    (131072, 128, 1023, 1151),
    (65536, 64, 1022, 1150),     # Qwen3 64K
    (8192, 64, 126, 254),        # T2 / T13 size
    (8192, 1, 8064, 8192),       # T3: gamma 1 selects every row
    (4100, 64, 62, 194),         # s % gamma != 0: cut_n = 4 + 128
    (4160, 256, 15, 15 + 320),   # gamma > 128: cut_n = 64 + 256
])
def test_anchor_layout_sizes(s, gamma, n_anchor, n_sel):
    anchors, tail, s_p, cut_n = O.anchor_layout(s, gamma)
    assert len(anchors) == n_anchor and len(anchors) + len(tail) == n_sel
    assert cut_n == s % gamma + max(128, gamma) and s_p == s - cut_n
    assert anchors[0] == 0 and np.all(np.diff(anchors) == gamma) and anchors[-1] < s_p
    assert np.array_equal(tail, np.arange(s_p, s))


def test_anchor_layout_reshape_condition():
    # the reference's reshape (llama.py:748-749) needs gamma | s_p: true for gamma | 128
    for gamma in (1, 2, 4, 8, 16, 32, 64, 128, 256, 512):
        for s in (4096, 5000, 131072, 131071):
            anchors, _, s_p, _ = O.anchor_layout(s, gamma)
            if s_p > 0:
                assert s_p % gamma == 0 and len(anchors) * gamma == s_p


# ---------------------------------------------------------------------------
# key-sparse visibility

@pytest.mark.parametrize("s,window,sink,qb", [
    (200, 64, 10, 64), (300, 100, 0, 64), (257, 31, 5, 64), (130, 500, 3, 64),
    (190, 48, 200, 64), (128, 16, 4, 1), (96, 0, 7, 32), (333, 70, 64, 16),
])
def test_visible_pairs_brute_force(s, window, sink, qb):
    r = np.arange(s)[:, None]
    k = np.arange(s)[None, :]
    # the predicate as flex_delta.py:59-61 writes it
    block_last = (r // qb) * qb + (qb - 1)
    brute = (r >= k) & ((k < sink) | (k + window > block_last))
    assert np.array_equal(brute.sum(1), O.sparse_row_counts(s, window, sink, qb))
    assert np.array_equal(brute, O.sparse_visible(r, k, window, sink, qb))


@pytest.mark.parametrize("s,window,sink,pairs", [
    (4096, 512, 64, 2082816),
    (32768, 2048, 128, 67973120),
    (131072, 2048, 128, 278786048),
    (65536, 4096, 64, 262045696),
])
def test_visible_pairs_config_totals(s, window, sink, pairs):
    assert O.visible_pairs(s, window, sink) == pairs


def test_visible_pairs_closed_forms():
    # window >= s: full causal, s(s+1)/2
    assert O.visible_pairs(1000, 5000, 0) == 1000 * 1001 // 2
    # q_block 1, no sink: a plain band of `window` keys per row
    s, w = 777, 40
    assert O.visible_pairs(s, w, 0, q_block=1) == sum(min(i + 1, w) for i in range(s))


def test_qsparse_pairs_closed_form():
    # sum over anchors 0, g, ..., (n-1)g of (i+1) plus the tail
    for s, g in [(131072, 64), (32768, 64), (4096, 16)]:
        a, t, s_p, _ = O.anchor_layout(s, g)
        n = len(a)
        closed = g * n * (n - 1) // 2 + n + (s * (s + 1) - s_p * (s_p + 1)) // 2
        assert O.qsparse_pairs(np.concatenate([a, t])) == closed


# ---------------------------------------------------------------------------
# attention

def _brute_sparse(q, k, v, window, sink, scale, qb):
    """Per-element loops with math.exp on tiny inputs."""
    B, H, S, d = q.shape
    G = H // k.shape[1]
    out = np.zeros((B, S, H, d))
    for b in range(B):
        for h in range(H):
            for r in range(S):
                last = (r // qb) * qb + qb - 1
                keys = [j for j in range(S) if j <= r and (j < sink or j + window > last)]
                if not keys:
                    continue
                sc = [scale * float(np.dot(q[b, h, r], k[b, h // G, j])) for j in keys]
                m = max(sc)
                w = [math.exp(x - m) for x in sc]
                tot = sum(w)
                for wi, j in zip(w, keys):
                    out[b, r, h] += wi / tot * v[b, h // G, j]
    return out


@pytest.mark.parametrize("S,window,sink,qb", [(130, 40, 3, 64), (70, 20, 0, 16), (96, 64, 70, 32)])
def test_sparse_attention_brute_force(S, window, sink, qb):
    q, k, v = _qkv(1, 2, 1, S, 8, seed=S)
    got = O.sparse_attention(q, k, v, window, sink, 0.3, q_block=qb)
    ref = _brute_sparse(q, k, v, window, sink, 0.3, qb)
    np.testing.assert_allclose(got, ref, rtol=1e-10, atol=1e-12)


def test_sparse_full_window_is_causal_sdpa():
    q, k, v = _qkv(2, 4, 2, 200, 16, seed=1)
    got = O.sparse_attention(q, k, v, window=400, sink=0, scale=0.25)
    ref = _sdpa64(q, k, v, 0.25, causal=True).transpose(0, 2, 1, 3)
    np.testing.assert_allclose(got, ref, rtol=1e-10, atol=1e-12)


def test_sparse_all_sinks_is_causal_sdpa():
    q, k, v = _qkv(1, 2, 2, 150, 16, seed=2)
    got = O.sparse_attention(q, k, v, window=8, sink=150, scale=0.2)
    ref = _sdpa64(q, k, v, 0.2, causal=True).transpose(0, 2, 1, 3)
    np.testing.assert_allclose(got, ref, rtol=1e-10, atol=1e-12)


def test_sparse_qblock1_is_sliding_window_sdpa():
    S, w = 160, 24
    q, k, v = _qkv(1, 2, 1, S, 8, seed=3)
    band = np.tril(np.ones((S, S), bool)) & np.triu(np.ones((S, S), bool), -(w - 1))
    got = O.sparse_attention(q, k, v, window=w, sink=0, scale=0.5, q_block=1)
    ref = _sdpa64(q, k, v, 0.5, mask=band).transpose(0, 2, 1, 3)
    np.testing.assert_allclose(got, ref, rtol=1e-10, atol=1e-12)


def test_sparse_gqa_equals_expanded():
    q, k, v = _qkv(1, 6, 2, 140, 8, seed=4)
    a = O.sparse_attention(q, k, v, 32, 4, 0.3)
    b = O.sparse_attention(q, np.repeat(k, 3, 1), np.repeat(v, 3, 1), 32, 4, 0.3)
    np.testing.assert_array_equal(a, b)


def test_sparse_rows_subset_matches_full():
    q, k, v = _qkv(1, 2, 1, 300, 8, seed=5)
    full = O.sparse_attention(q, k, v, 100, 8, 0.3)
    rows = np.array([0, 5, 63, 64, 200, 299])
    np.testing.assert_allclose(O.sparse_attention(q, k, v, 100, 8, 0.3, rows=rows), full[:, rows],
                               rtol=1e-12, atol=1e-14)


def test_qsparse_causal_rows_is_sdpa():
    # delta_kernel.py:426-469 (mask = arange) and T1 (sorted subset of rows)
    S = 300
    q, k, v = _qkv(1, 4, 4, S, 16, seed=6)
    got = O.qsparse_attention(q, k, v, np.arange(S), 0.25)
    np.testing.assert_allclose(got, _sdpa64(q, k, v, 0.25, causal=True), rtol=1e-10, atol=1e-12)
    idx = np.array([0, 3, 77, 128, 129, 250, 299])
    m = np.arange(S)[None, :] <= idx[:, None]
    ref = _sdpa64(q[:, :, idx], k, v, 0.25, mask=m)
    np.testing.assert_allclose(O.qsparse_attention(q[:, :, idx], k, v, idx, 0.25), ref,
                               rtol=1e-10, atol=1e-12)


def test_qsparse_rectangular_and_unsorted():
    # delta_kernel.py:332-377 (N_KV = 2N, random limits) and :380-423 (randperm)
    n, N = 96, 192
    q, k, v = _qkv(1, 2, 2, n, 16, seed=7, N=N)
    rng = np.random.default_rng(8)
    for mask in (rng.integers(0, N, n), rng.permutation(n)):
        m = np.arange(N)[None, :] <= mask[:, None]
        np.testing.assert_allclose(O.qsparse_attention(q, k, v, mask, 0.3),
                                   _sdpa64(q, k, v, 0.3, mask=m), rtol=1e-10, atol=1e-12)


# ---------------------------------------------------------------------------
# composition: T2 / T3 / T4 and the modes

def _dense(q, k, v, scale):
    return _sdpa64(q, k, v, scale, causal=True).transpose(0, 2, 1, 3)


def test_t2_anchor_and_tail_rows_are_dense():
    s, g = 512, 32
    q, k, v = _qkv(1, 4, 2, s, 16, seed=9)
    out = O.delta_forward(q, k, v, g, window=64, sink=4, scale=0.25)
    dense = _dense(q, k, v, 0.25)
    anchors, tail, s_p, _ = O.anchor_layout(s, g)
    np.testing.assert_allclose(out[:, anchors], dense[:, anchors], rtol=1e-9, atol=1e-12)
    np.testing.assert_allclose(out[:, tail], dense[:, tail], rtol=1e-9, atol=1e-12)
    # and the other rows really are corrected sparse rows, not dense
    assert np.abs(out[:, 1:s_p] - dense[:, 1:s_p]).max() > 1e-3


def test_t3_gamma1_is_dense_everywhere():
    s = 320
    q, k, v = _qkv(1, 2, 1, s, 16, seed=10)
    out = O.delta_forward(q, k, v, 1, window=32, sink=0, scale=0.25)
    np.testing.assert_allclose(out, _dense(q, k, v, 0.25), rtol=1e-9, atol=1e-12)


def test_t4_full_window_zero_delta():
    s = 384
    q, k, v = _qkv(1, 2, 2, s, 16, seed=11)
    sparse = O.sparse_attention(q, k, v, window=s, sink=0, scale=0.3)
    np.testing.assert_allclose(O.delta_forward(q, k, v, 64, s, 0, 0.3, sparse=sparse),
                               _dense(q, k, v, 0.3), rtol=1e-9, atol=1e-12)


def test_modes_sparse_only_and_recompute():
    s, g = 400, 16
    q, k, v = _qkv(1, 2, 1, s, 8, seed=12)
    sparse = O.sparse_attention(q, k, v, 48, 4, 0.3)
    np.testing.assert_array_equal(O.delta_forward(q, k, v, g, 48, 4, 0.3, mode="sparse-only"), sparse)
    rec = O.delta_forward(q, k, v, g, 48, 4, 0.3, mode="recompute")
    dense = _dense(q, k, v, 0.3)
    idx = O.selected_rows(s, g)
    other = np.setdiff1d(np.arange(s), idx)
    np.testing.assert_allclose(rec[:, idx], dense[:, idx], rtol=1e-9, atol=1e-12)
    np.testing.assert_array_equal(rec[:, other], sparse[:, other])


def test_apply_delta_variable_uniform_is_reshape_bitwise():
    # stride.py:33-34: uniform anchors give the reshape path bit-for-bit (bf16 ops)
    s, g = 1024, 64
    rng = np.random.default_rng(13)
    sparse = O.round_bf16(rng.standard_normal((2, s, 3, 16)).astype(np.float32))
    a, t, s_p, _ = O.anchor_layout(s, g)
    dense = O.round_bf16(rng.standard_normal((2, len(a) + len(t), 3, 16)).astype(np.float32))
    via_reshape = O.compose_uniform(sparse, dense, s, g, bf16=True)[:, :s_p]
    via_owner = O.apply_delta_variable(sparse, dense[:, :len(a)], a, s_p, bf16=True)
    np.testing.assert_array_equal(via_reshape, via_owner)
    # the zero-delta identity: dense == sparse at anchors -> output == sparse
    zero = O.apply_delta_variable(sparse, sparse[:, a], a, s_p, bf16=True)
    np.testing.assert_array_equal(zero, sparse[:, :s_p])


def test_apply_delta_variable_owner():
    idx = np.array([3, 10, 11, 40])
    sp = np.zeros((1, 50, 1, 1))
    dense = np.array([1.0, 2.0, 3.0, 4.0]).reshape(1, 4, 1, 1)
    out = O.apply_delta_variable(sp, dense, idx, 50)[0, :, 0, 0]
    # rows 0-2 precede the first anchor: searchsorted-1 == -1 -> the last anchor
    expect = [4] * 3 + [1] * 7 + [2] + [3] * 29 + [4] * 10
    np.testing.assert_array_equal(out, expect)


# ---------------------------------------------------------------------------
# bf16 arithmetic and the input prologue

def test_round_bf16_matches_torch():
    rng = np.random.default_rng(14)
    x = np.concatenate([rng.standard_normal(100000).astype(np.float32) * 10.0 ** rng.integers(-8, 8, 100000),
                        np.array([0.0, -0.0, 1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8, 65504.0], np.float32)])
    x = x.astype(np.float32)
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(O.round_bf16(x), ref)
    a, b = O.round_bf16(x[:5000]), O.round_bf16(x[5000:10000])
    ta, tb = torch.from_numpy(a).to(torch.bfloat16), torch.from_numpy(b).to(torch.bfloat16)
    np.testing.assert_array_equal(O.sub_bf16(a, b), (ta - tb).float().numpy())
    np.testing.assert_array_equal(O.add_bf16(a, b), (ta + tb).float().numpy())


def test_rope_invariants():
    s, d = 64, 16
    cos, sin = O.rope_cos_sin(s, d, 10000.0)
    rng = np.random.default_rng(15)
    x = rng.standard_normal((1, 1, s, d)).astype(np.float32)
    y = O.apply_rope(x, cos, sin)
    np.testing.assert_allclose(y[:, :, 0], x[:, :, 0], rtol=1e-6)        # position 0: identity
    np.testing.assert_allclose(np.linalg.norm(y, axis=-1), np.linalg.norm(x, axis=-1), rtol=1e-5)
    # relative position: <R_m q, R_n k> depends on m - n only
    q1 = rng.standard_normal(d).astype(np.float32)
    k1 = rng.standard_normal(d).astype(np.float32)
    Q = O.apply_rope(np.broadcast_to(q1, (1, 1, s, d)).copy(), cos, sin)[0, 0]
    K = O.apply_rope(np.broadcast_to(k1, (1, 1, s, d)).copy(), cos, sin)[0, 0]
    np.testing.assert_allclose(Q[10] @ K[4], Q[30] @ K[24], rtol=1e-4, atol=1e-4)
    # pair (i, i + d/2) rotates by angle pos * theta^(-2i/d)
    ang = 5 * 10000.0 ** (-2 * 3 / d)
    e = np.zeros(d, np.float32)
    e[3] = 1.0
    r = O.apply_rope(np.broadcast_to(e, (1, 1, s, d)).copy(), cos, sin)[0, 0, 5]
    np.testing.assert_allclose([r[3], r[3 + d // 2]], [math.cos(ang), math.sin(ang)], rtol=1e-5, atol=1e-6)


def test_rms_norm_matches_torch():
    x = np.random.default_rng(16).standard_normal((3, 5, 128)).astype(np.float32)
    ref = F.rms_norm(torch.from_numpy(x), (128,), eps=1e-6).numpy()
    np.testing.assert_allclose(O.rms_norm(x, 1e-6), ref, rtol=1e-5, atol=1e-6)


def test_bf16_prologue_ops_match_torch():
    # the bf16 RoPE / RMSNorm restatements against torch's own bf16 tensor ops
    rng = np.random.default_rng(17)
    S, D = 40, 128
    x = O.round_bf16(rng.standard_normal((2, 3, S, D)).astype(np.float32))
    c32, s32 = O.rope_cos_sin(S, D, 500000.0)
    c, s = O.round_bf16(c32), O.round_bf16(s32)
    tx = torch.from_numpy(x).to(torch.bfloat16)
    tc, ts = torch.from_numpy(c).to(torch.bfloat16), torch.from_numpy(s).to(torch.bfloat16)
    h = D // 2
    ref = (tx * tc) + (torch.cat((-tx[..., h:], tx[..., :h]), dim=-1) * ts)
    np.testing.assert_array_equal(O.apply_rope_bf16(x, c, s), ref.float().numpy())
    w = O.round_bf16(rng.uniform(0.5, 1.5, D).astype(np.float32))
    tw = torch.from_numpy(w).to(torch.bfloat16)
    xf = tx.float()
    tref = tw * (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)).to(torch.bfloat16)
    got = O.rms_norm_bf16(x, w, 1e-6)
    diff = np.abs(got - tref.float().numpy())
    ulp = np.abs(tref.float().numpy()) * 2.0 ** -7
    assert (diff <= ulp + 1e-30).all() and (diff == 0).mean() > 0.99


# ---------------------------------------------------------------------------
# decode rows

@pytest.mark.parametrize("n,window,sink", [(40, 8, 4), (40, 36, 4), (40, 0, 4), (7, 3, 2), (1, 4, 2)])
def test_decode_row_brute_force(n, window, sink):
    # the reference's key set: concat(k[:sink], k[n-window:]) when n > sink + window
    if window and n > sink + window:
        keys = list(range(sink)) + list(range(n - window, n))
    else:
        keys = list(range(n))
    assert list(O.decode_keys(n, window, sink)) == keys
    q, k, v = _qkv(1, 4, 2, 1, 8, seed=n + window, N=n)
    got = O.decode_row(q, k, v, window, sink, 0.3)
    ref = np.zeros_like(got)
    for h in range(4):
        sc = [0.3 * float(np.dot(q[0, h, 0], k[0, h // 2, j])) for j in keys]
        m = max(sc)
        w = [math.exp(x - m) for x in sc]
        ref[0, h, 0] = sum(wi * v[0, h // 2, j] for wi, j in zip(w, keys)) / sum(w)
    np.testing.assert_allclose(got, ref, rtol=1e-10, atol=1e-12)


def test_decode_dense_row_is_last_causal_row():
    q, k, v = _qkv(2, 6, 3, 1, 16, seed=3, N=90)
    qq = np.concatenate([np.zeros((2, 6, 89, 16)), q], axis=2)
    ref = O.causal_attention_rows(qq, k, v, np.array([89]), 0.25).transpose(0, 2, 1, 3)
    np.testing.assert_allclose(O.decode_row(q, k, v, 0, 0, 0.25), ref, rtol=1e-12, atol=1e-14)
    # window covering everything past the sinks is the dense row too
    np.testing.assert_allclose(O.decode_row(q, k, v, 86, 4, 0.25), ref, rtol=1e-12, atol=1e-14)


def test_delta_decode_steps_schedule():
    q0 = _qkv(1, 2, 1, 1, 8, seed=1, N=50)
    k, v = q0[1], q0[2]
    qs = [_qkv(1, 2, 1, 1, 8, seed=10 + i, N=50)[0] for i in range(5)]
    outs = O.delta_decode_steps(qs, k, v, 8, 2, 0.5, gamma_dec=2)
    dense = [O.decode_row(q, k, v, 0, 0, 0.5) for q in qs]
    sparse = [O.decode_row(q, k, v, 8, 2, 0.5) for q in qs]
    for i in (0, 2, 4):        # anchors: the dense rows
        np.testing.assert_array_equal(outs[i], dense[i])
    for i in (1, 3):           # sparse + the delta of the previous anchor
        np.testing.assert_allclose(outs[i], sparse[i] + dense[i - 1] - sparse[i - 1], rtol=1e-12)
    # gamma_dec 1: every step is an anchor, i.e. dense decode
    for o, d in zip(O.delta_decode_steps(qs, k, v, 8, 2, 0.5, gamma_dec=1), dense):
        np.testing.assert_array_equal(o, d)


def test_interanchor_cos_closed_forms_and_library():
    d = np.zeros((1, 5, 2, 4))
    d[0, 0, :, 0] = 1.0
    d[0, 1, :, 0] = 3.0                     # parallel: 1
    d[0, 2, 0, 0] = -2.0                    # antiparallel: -1 (head 0)
    d[0, 2, 1, 1] = 5.0                     # orthogonal: 0 (head 1)
    d[0, 3] = 0.0                           # zero delta: clamped norm gives 0
    d[0, 4, :, 2] = 1.0
    c = O.interanchor_cos(d)
    np.testing.assert_allclose(c[0, :, 0], [1.0, -1.0, 0.0, 0.0], atol=1e-15)
    np.testing.assert_allclose(c[0, :, 1], [1.0, 0.0, 0.0, 0.0], atol=1e-15)
    # torch's cosine_similarity (the reference's call) on random deltas
    rng = np.random.default_rng(5)
    x = rng.standard_normal((2, 9, 3, 16))
    t = torch.from_numpy(x)
    ref = F.cosine_similarity(t[:, :-1], t[:, 1:], dim=-1).numpy()
    np.testing.assert_allclose(O.interanchor_cos(x), ref, rtol=1e-12, atol=1e-14)


def test_histc_edges_and_library():
    x = np.array([-1.0, -0.5, 0.0, 0.99, 1.0, 1.5, -1.01, np.nan], dtype=np.float32)
    np.testing.assert_array_equal(O.histc(x, 4, -1.0, 1.0), [1, 1, 1, 2])
    rng = np.random.default_rng(6)
    y = rng.uniform(-1.2, 1.2, 3000).astype(np.float32)
    ref = torch.histc(torch.from_numpy(y), bins=40, min=-1.0, max=1.0).numpy().astype(np.int64)
    np.testing.assert_array_equal(O.histc(y, 40, -1.0, 1.0), ref)


def test_head_row_cos_against_library_and_closed_forms():
    """The smoke check's cosine (over the head dim, T1's gate at
    tests/test_math_identities.py:85) against torch's cosine_similarity in
    float64 and the closed forms: parallel rows give 1, opposite rows -1,
    orthogonal rows 0, and scaling a row leaves it unchanged. A planted
    mistake (the norms without the square root) fails the library check."""
    rng = np.random.default_rng(7)
    a = rng.standard_normal((2, 5, 3, 64))
    b = rng.standard_normal((2, 5, 3, 64))
    got = O.head_row_cos(a, b)
    ref = torch.nn.functional.cosine_similarity(torch.from_numpy(a), torch.from_numpy(b),
                                                dim=-1).numpy()
    assert got.shape == (2, 5, 3)
    np.testing.assert_allclose(got, ref, rtol=0, atol=1e-13)
    np.testing.assert_allclose(O.head_row_cos(a, 3.5 * a), 1.0, atol=1e-14)
    np.testing.assert_allclose(O.head_row_cos(a, -a), -1.0, atol=1e-14)
    e0, e1 = np.zeros((1, 64)), np.zeros((1, 64))
    e0[0, 3], e1[0, 9] = 2.0, -5.0
    assert O.head_row_cos(e0, e1)[0] == 0.0
    np.testing.assert_allclose(O.head_row_cos(a, b), O.head_row_cos(0.01 * a, 40 * b), atol=1e-13)
    no_sqrt = (a * b).sum(-1) / ((a * a).sum(-1) * (b * b).sum(-1))
    assert np.abs(no_sqrt - ref).max() > 0.1


# ---------------------------------------------------------------------------
# delta decode refresh policies (llama.py:578-604), hand-built schedules

def test_decode_anchor_flags_fixed_and_cap():
    T, F = True, False
    # fixed: step 0 has no delta; then every gamma_dec-th step since the last anchor
    assert O.decode_anchor_flags([None] + [0.5] * 9, "fixed", gamma_dec=3) == \
        [T, F, F, T, F, F, T, F, F, T]
    # gamma_dec_max guards every policy: a drift threshold that never fires
    assert O.decode_anchor_flags([None] + [0.5] * 9, "drift", drift_threshold=-2.0,
                                 gamma_dec_max=4) == [T, F, F, F, T, F, F, F, T, F]
    # fixed with gamma_dec above the cap: the cap decides
    assert O.decode_anchor_flags([None] + [0.5] * 5, "fixed", gamma_dec=50,
                                 gamma_dec_max=2) == [T, F, T, F, T, F]


def test_decode_anchor_flags_drift():
    T, F = True, False
    # anchor exactly where cos(sparse_t, sparse_{t-1}) < threshold, including
    # the step right after an anchor
    cos = [None, 0.99, 0.5, 0.2, 0.99, 0.9, 0.89]
    assert O.decode_anchor_flags(cos, "drift", drift_threshold=0.9) == [T, F, T, T, F, F, T]
    # the drift policy ignores gamma_dec
    assert O.decode_anchor_flags([None] + [0.99] * 6, "drift", gamma_dec=2,
                                 drift_threshold=0.9) == [T] + [F] * 6


def test_decode_anchor_flags_drift_rel():
    T, F = True, False
    # no test until 8 cosines are recorded; then cos < mean - k * pstd
    base = [None] + [0.8, 1.0] * 4              # history 0.8 x4, 1.0 x4: mean 0.9, pstd 0.1
    assert O.decode_anchor_flags(base + [0.71], "drift_rel", drift_k=2.0) == [T] + [F] * 9
    assert O.decode_anchor_flags(base + [0.69], "drift_rel", drift_k=2.0) == [T] + [F] * 8 + [T]
    assert O.decode_anchor_flags(base + [0.69], "drift_rel", drift_k=3.0) == [T] + [F] * 9
    # a constant history (pstd 0): anything below the mean anchors
    assert O.decode_anchor_flags([None] + [0.9] * 8 + [0.89999, 0.9], "drift_rel") == \
        [T] + [F] * 8 + [T, F]
    # the 8th recorded cosine is the first one tested against: 7 recorded -> no test
    assert O.decode_anchor_flags([None] + [0.9] * 7 + [0.1], "drift_rel") == [T] + [F] * 8
    # a rolling window of 16: an early outlier (0.0) widens the spread while it
    # is in the window (0.85 passes), and once 16 later cosines have pushed it
    # out the spread is 0 and 0.85 anchors
    hist = [None, 0.0] + [0.9] * 15
    assert O.decode_anchor_flags(hist + [0.85], "drift_rel")[-1] is False
    assert O.decode_anchor_flags(hist + [0.9, 0.85], "drift_rel")[-1] is True
    # steps anchored by the count record nothing: with gamma_dec_max 3 every
    # third step anchors by the count, and its cosine (0.1 at step 3) never
    # enters the history; had it, the spread would keep 0.85 at step 13 (the
    # first test, 8 cosines of 0.9 recorded) from anchoring
    cos = [None, 0.9, 0.9, 0.1] + [0.9] * 9 + [0.85]
    assert O.decode_anchor_flags(cos, "drift_rel", gamma_dec_max=3) == \
        [T, F, F] * 4 + [T, T]
    cos2 = [None] + [0.9] * 8 + [0.1, 0.2]
    assert O.decode_anchor_flags(cos2, "drift_rel") == [T] + [F] * 8 + [T, T]


def test_delta_decode_steps_composition():
    """Outputs follow the flags: anchors are the dense row, the other steps
    sparse + the last anchor's delta (checked against decode_row directly)."""
    rng = np.random.default_rng(5)
    k = rng.standard_normal((1, 2, 300, 16))
    v = rng.standard_normal((1, 2, 300, 16))
    q0 = rng.standard_normal((1, 4, 1, 16))
    qs = [q0 + 0.05 * t * rng.standard_normal(q0.shape) for t in range(7)]
    outs, flags = O.delta_decode_steps(qs, k, v, 64, 8, 0.25, gamma_dec=3, policy="fixed",
                                       return_flags=True)
    assert flags == [True, False, False, True, False, False, True]
    delta = None
    for q, o, f in zip(qs, outs, flags):
        sp = O.decode_row(q, k, v, 64, 8, 0.25)
        dn = O.decode_row(q, k, v, 0, 0, 0.25)
        if f:
            delta = dn - sp
            np.testing.assert_allclose(o, dn, rtol=0, atol=1e-12)
        else:
            np.testing.assert_allclose(o, sp + delta, rtol=0, atol=1e-12)
    # drift: the flags come from the cosines of consecutive sparse rows
    sp = [O.decode_row(q, k, v, 64, 8, 0.25) for q in qs]
    cos = [None] + [O.flat_cos(sp[t], sp[t - 1]) for t in range(1, 7)]
    thr = float(np.median([c for c in cos[1:]]))
    _, fl = O.delta_decode_steps(qs, k, v, 64, 8, 0.25, gamma_dec=3, policy="drift",
                                 drift_threshold=thr, return_flags=True)
    assert fl == [True] + [c < thr for c in cos[1:]]
