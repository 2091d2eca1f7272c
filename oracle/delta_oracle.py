"""CPU oracle of the delta-attention prefill path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this module, and only as the checker or the CPU baseline; the product path
(delta-attention_amd/delta_attention) never imports it.

It restates, in numpy, what the reference computes for one attention layer
prefill (file:line cite the reference, singhh5050/delta-attention):

  anchor_layout          validation.py:224-232, flex_delta.py:72-76, llama.py:692-714
  sparse_visible         flex_delta.py:51-61 (block-anchored window, Q_BLOCK=64 at :48)
  sparse_attention       hip-attn block_sparse_attention as used at llama.py:407-449,
                         with the visibility above
  qsparse_attention      delta_kernel.py:36-97, 199-251 (row i attends keys 0..mask[i])
  delta_forward          llama.py:659-757 (modes delta / recompute / sparse-only)
  apply_delta_variable   stride.py:26-40
  decode_row             llama.py:537-549 (_decode_sparse_row: sink + last window
                         keys of the cache) and the dense decode row of :598-600
  decode_anchor_flags    llama.py:578-604: when a delta decode step recomputes its
                         dense row (fixed / drift / drift_rel policies and the
                         gamma_dec_max guard), from the per-step cosines of
                         consecutive sparse rows
  delta_decode_steps     llama.py:551-634 (delta decode composition under those
                         policies)
  round_bf16, *_bf16     the bf16 elementwise arithmetic of llama.py:740-751 and
                         stride.py:38-40 (fp32 op, one round-to-nearest-even)
  rope / rms_norm        llama.py:129-192 (rotate_half RoPE), llama.py:60-74 (RMSNorm),
                         qwen3.py:37-43 (per-head q/k norm before RoPE); *_bf16
                         variants round once per tensor op like the bf16 tensors
  visible_pairs          the algorithmic-work counts (pairs of the sparse pass,
                         sum(i+1) of the query-sparse pass)
  interanchor_cos        stride.py:43-52 / drift.py:30-32: cosine of consecutive
                         anchor deltas over the head dim (torch cosine_similarity,
                         each norm clamped to eps = 1e-8)
  histc                  drift.py:33: torch.histc's binning (bins over [lo, hi],
                         x == hi in the last bin, out-of-range and NaN dropped)
  head_row_cos           the per-row cosine over the head dim of the reference's
                         T1 gate (tests/test_math_identities.py:85)
  masked_attention_grads the attention backward that autograd forms for the
                         FlexAttention / masked SDPA branches of flex_delta.py:167-184
  compose_grads          the composition's backward (flex_delta.py:186-196, the
                         detach / gradient-scale arms at :187-190)
  delta_train_grads      gradients of delta_forward_train (flex_delta.py:95-196)

Pinning (tests/test_oracle.py): every function is checked against brute force
on tiny inputs, library routines (torch scaled_dot_product_attention in
float64) on special cases that reduce to them, closed forms, and the
reference's own known-answer identities (T1-T4). No function here is
"parity unpinned".
"""

from __future__ import annotations

import math
from typing import Iterable, Optional, Sequence, Tuple

import numpy as np

Q_BLOCK = 64


# ---------------------------------------------------------------------------
# index layout (integer, exact)

def anchor_layout(s: int, gamma: int) -> Tuple[np.ndarray, np.ndarray, int, int]:
    """(anchors, tail, s_p, cut_n) exactly as delta_forward builds them.

    cut_n = s % gamma + max(128, gamma); s_p = s - cut_n;
    anchors = 0, gamma, 2*gamma, ... < s_p; tail = s_p .. s-1.
    validation.py:224-232 / flex_delta.py:72-76 / llama.py:692-714.
    """
    cut_n = s % gamma + max(128, gamma)
    s_p = s - cut_n
    anchors = np.arange(0, max(s_p, 0), gamma, dtype=np.int64)
    tail = np.arange(max(s_p, 0), s, dtype=np.int64)
    return anchors, tail, s_p, cut_n


def selected_rows(s: int, gamma: int) -> np.ndarray:
    anchors, tail, _, _ = anchor_layout(s, gamma)
    return np.concatenate([anchors, tail])


# ---------------------------------------------------------------------------
# key-sparse visibility (flex_delta.py:59-61)

def window_start(r, window: int, q_block: int = Q_BLOCK):
    """First window key of row r: keys k with k + window > L(r) where
    L(r) = floor(r / q_block) * q_block + q_block - 1."""
    r = np.asarray(r, dtype=np.int64)
    return (r // q_block) * q_block + q_block - window


def sparse_visible(r, k, window: int, sink: int, q_block: int = Q_BLOCK):
    r = np.asarray(r, dtype=np.int64)
    k = np.asarray(k, dtype=np.int64)
    block_last = (r // q_block) * q_block + (q_block - 1)
    return (k <= r) & ((k < sink) | (k + window > block_last))


def sparse_row_counts(s: int, window: int, sink: int, q_block: int = Q_BLOCK) -> np.ndarray:
    """Number of visible keys of every row, from the interval form of the mask."""
    r = np.arange(s, dtype=np.int64)
    ws = np.maximum(window_start(r, window, q_block), 0)
    win = np.maximum(r - ws + 1, 0)                     # keys ws .. r
    sink_only = np.clip(np.minimum(sink, ws), 0, r + 1)  # keys 0 .. min(sink, ws)-1, causal
    return win + sink_only


def visible_pairs(s: int, window: int, sink: int, q_block: int = Q_BLOCK) -> int:
    return int(sparse_row_counts(s, window, sink, q_block).sum())


def qsparse_pairs(rows: Iterable[int]) -> int:
    return int(sum(int(r) + 1 for r in rows))


def flops_sparse(B: int, H: int, d: int, s: int, window: int, sink: int, q_block: int = Q_BLOCK) -> float:
    return 4.0 * d * H * B * visible_pairs(s, window, sink, q_block)


def flops_qsparse(B: int, H: int, d: int, rows: Iterable[int]) -> float:
    return 4.0 * d * H * B * qsparse_pairs(rows)


# ---------------------------------------------------------------------------
# bf16 arithmetic

def round_bf16(x) -> np.ndarray:
    """Round float32 values to the nearest bf16 (ties to even), kept as float32."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = x.view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    out = u.astype(np.uint32).view(np.float32)
    nan = np.isnan(x)
    if nan.any():
        out = out.copy()
        out[nan] = np.nan
    return out


def sub_bf16(a, b) -> np.ndarray:
    return round_bf16(np.asarray(a, np.float32) - np.asarray(b, np.float32))


def add_bf16(a, b) -> np.ndarray:
    return round_bf16(np.asarray(a, np.float32) + np.asarray(b, np.float32))


# ---------------------------------------------------------------------------
# attention

def _expand_kv(k: np.ndarray, H: int) -> np.ndarray:
    """GQA: query head h reads kv head h // (H // Hkv) (llama.py:218-229)."""
    Hkv = k.shape[1]
    assert H % Hkv == 0
    return np.repeat(k, H // Hkv, axis=1) if Hkv != H else k


def _softmax_rows(scores: np.ndarray) -> np.ndarray:
    m = scores.max(axis=-1, keepdims=True)
    m = np.where(np.isfinite(m), m, 0.0)
    p = np.exp(scores - m)
    l = p.sum(axis=-1, keepdims=True)
    return np.divide(p, l, out=np.zeros_like(p), where=l > 0)


def masked_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, allowed: np.ndarray,
                     scale: float) -> np.ndarray:
    """softmax(scale * q k^T + mask) v with a boolean mask [n, N] shared over
    batch and heads. q [B,H,n,d], k/v [B,Hkv,N,d] -> [B,H,n,d]. Rows with no
    visible key are zero."""
    H = q.shape[1]
    kk, vv = _expand_kv(k, H), _expand_kv(v, H)
    s = np.matmul(q, kk.swapaxes(-1, -2)) * scale
    s = np.where(allowed[None, None], s, -np.inf)
    return np.matmul(_softmax_rows(s), vv)


def sparse_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, window: int, sink: int,
                     scale: float, q_block: int = Q_BLOCK, rows: Optional[np.ndarray] = None,
                     q_is_rows: bool = False) -> np.ndarray:
    """Key-sparse attention. q [B,H,S,d], k/v [B,Hkv,S,d] -> [B,S,H,d]
    (the layout hip_attention_interface returns, llama.py:394-449).
    Computed per q_block row block on the union of its sink and window keys.
    rows: optional subset of rows (sorted); the result then has len(rows) rows.
    q_is_rows: q already holds only those rows ([B,H,len(rows),d])."""
    B, H, _, d = q.shape
    S = k.shape[2]
    kk, vv = _expand_kv(k, H), _expand_kv(v, H)
    all_rows = np.arange(S) if rows is None else np.asarray(rows, dtype=np.int64)
    out = np.zeros((B, len(all_rows), H, d), dtype=q.dtype)
    blocks = all_rows // q_block
    for blk in np.unique(blocks):
        sel = np.nonzero(blocks == blk)[0]
        r = all_rows[sel]
        ws = max(int(window_start(int(r[0]), window, q_block)), 0)
        keys = np.unique(np.concatenate([np.arange(min(sink, S)), np.arange(ws, int(r.max()) + 1)]))
        keys = keys[keys < S]
        allowed = sparse_visible(r[:, None], keys[None, :], window, sink, q_block)
        qr = q[:, :, sel] if q_is_rows else q[:, :, r]
        sc = np.matmul(qr, kk[:, :, keys].swapaxes(-1, -2)) * scale
        sc = np.where(allowed[None, None], sc, -np.inf)
        o = np.matmul(_softmax_rows(sc), vv[:, :, keys])
        out[:, sel] = o.transpose(0, 2, 1, 3)
    return out


def qsparse_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, mask: np.ndarray,
                      scale: float, chunk: int = 64) -> np.ndarray:
    """delta_kernel.attention semantics: row i of q attends keys 0..mask[i]
    inclusive (delta_kernel.py:57, 68). q [B,H,n,d], k/v [B,Hk,N,d] with Hk == H
    or a GQA divisor; mask [n] (shared over batch) -> [B,H,n,d]."""
    B, H, n, d = q.shape
    N = k.shape[2]
    kk, vv = _expand_kv(k, H), _expand_kv(v, H)
    mask = np.asarray(mask, dtype=np.int64).reshape(-1)
    out = np.zeros((B, H, n, d), dtype=q.dtype)
    for c0 in range(0, n, chunk):
        c1 = min(c0 + chunk, n)
        lim = mask[c0:c1]
        kmax = int(min(lim.max(), N - 1)) + 1 if c1 > c0 else 0
        if kmax <= 0:
            continue
        allowed = np.arange(kmax)[None, :] <= lim[:, None]
        sc = np.matmul(q[:, :, c0:c1], kk[:, :, :kmax].swapaxes(-1, -2)) * scale
        sc = np.where(allowed[None, None], sc, -np.inf)
        out[:, :, c0:c1] = np.matmul(_softmax_rows(sc), vv[:, :, :kmax])
    return out


def causal_attention_rows(q: np.ndarray, k: np.ndarray, v: np.ndarray, rows: np.ndarray,
                          scale: float) -> np.ndarray:
    """Full causal attention at the given rows of q [B,H,S,d] -> [B,len(rows),H,d]."""
    rows = np.asarray(rows, dtype=np.int64)
    return qsparse_attention(q[:, :, rows], k, v, rows, scale).transpose(0, 2, 1, 3)


def decode_keys(n: int, window: int, sink: int) -> np.ndarray:
    """Keys the decode row at position n-1 attends (llama.py:542-549): all of
    them when n <= sink + window (or window == 0), else the first `sink` and
    the last `window`."""
    if window <= 0 or n <= sink + window:
        return np.arange(n)
    return np.concatenate([np.arange(sink), np.arange(n - window, n)])


def decode_row(q: np.ndarray, k: np.ndarray, v: np.ndarray, window: int, sink: int,
               scale: float) -> np.ndarray:
    """The decode row: q [B,H,1,d] against k/v [B,Hkv,n,d] over decode_keys(...)
    -> [B,H,1,d]; window 0 is the dense row."""
    n = k.shape[2]
    keys = decode_keys(n, window, sink)
    allowed = np.zeros((1, n), dtype=bool)
    allowed[0, keys] = True
    return masked_attention(q, k, v, allowed, scale)


def decode_anchor_flags(cosines: Sequence[Optional[float]], policy: str = "fixed",
                        gamma_dec: int = 8, gamma_dec_max: int = 128,
                        drift_threshold: float = 0.95, drift_k: float = 2.0,
                        warmup: int = 8, history: int = 16) -> list:
    """Anchor decisions of a delta decode run (llama.py:578-604). cosines[t] is
    cos(sparse_t, sparse_{t-1}) over the whole row (None at t = 0, where there
    is no previous row). Step 0 anchors (no delta yet). Later steps count
    n = steps since the last anchor, and anchor when n reaches gamma_dec_max,
    or (fixed) gamma_dec; otherwise, for drift, when the cosine is below
    drift_threshold, and for drift_rel, when at least `warmup` cosines are
    recorded and the cosine is below their mean minus drift_k population
    standard deviations. drift_rel records each cosine it tests, after the
    test, keeping the last `history`; steps anchored by the count record
    nothing."""
    flags, since, rec = [], None, np.zeros(0)
    for t, c in enumerate(cosines):
        if since is None:
            flags.append(True)
            since = 0
            continue
        n = since + 1
        hit = n >= gamma_dec_max or (policy == "fixed" and n >= gamma_dec)
        if not hit and policy in ("drift", "drift_rel") and c is not None:
            if policy == "drift":
                hit = c < drift_threshold
            else:
                if rec.size >= warmup:
                    hit = c < rec.mean() - drift_k * np.sqrt(((rec - rec.mean()) ** 2).mean())
                rec = np.append(rec, c)[-history:]
        flags.append(bool(hit))
        since = 0 if hit else n
    return flags


def flat_cos(a: np.ndarray, b: np.ndarray) -> float:
    """Cosine of two arrays flattened (torch cosine_similarity over one dim,
    norms clamped to 1e-8)."""
    a, b = np.ravel(a).astype(np.float64), np.ravel(b).astype(np.float64)
    return float(a @ b / max(np.sqrt(a @ a) * np.sqrt(b @ b), 1e-8))


def delta_decode_steps(qs: Sequence[np.ndarray], k: np.ndarray, v: np.ndarray, window: int,
                       sink: int, scale: float, gamma_dec: int, policy: str = "fixed",
                       gamma_dec_max: int = 128, drift_threshold: float = 0.95,
                       drift_k: float = 2.0, return_flags: bool = False):
    """Delta decode over successive query rows against one cache
    (llama.py:551-634): anchor steps (decode_anchor_flags over the cosines of
    consecutive sparse rows) output the dense row and refresh delta = dense -
    sparse; the others output sparse + delta."""
    sparse = [decode_row(q, k, v, window, sink, scale) for q in qs]
    cos = [None] + [flat_cos(sparse[t], sparse[t - 1]) for t in range(1, len(sparse))]
    flags = decode_anchor_flags(cos, policy, gamma_dec, gamma_dec_max, drift_threshold, drift_k)
    outs, delta = [], None
    for q, sp, anchor in zip(qs, sparse, flags):
        if anchor:
            dn = decode_row(q, k, v, 0, 0, scale)
            delta = dn - sp
            outs.append(dn)
        else:
            outs.append(sp + delta)
    return (outs, flags) if return_flags else outs


# ---------------------------------------------------------------------------
# composition

def apply_delta_variable(sparse: np.ndarray, dense_sel: np.ndarray, idx: np.ndarray, s_p: int,
                         bf16: bool = False) -> np.ndarray:
    """stride.py:26-40: row i gets sparse[i] + (dense_sel - sparse[idx])[owner(i)],
    owner(i) = searchsorted(idx, i, right) - 1 (so -1, the LAST anchor, for rows
    before idx[0]). sparse [B,>=s_p,H,d], dense_sel [B,n,H,d] -> [B,s_p,H,d].
    bf16=True rounds each elementwise op like the reference's bf16 tensors."""
    idx = np.asarray(idx, dtype=np.int64)
    owner = np.searchsorted(idx, np.arange(s_p), side="right") - 1
    if bf16:
        deltas = sub_bf16(dense_sel, sparse[:, idx])
        return add_bf16(sparse[:, :s_p], deltas[:, owner])
    deltas = dense_sel - sparse[:, idx]
    return sparse[:, :s_p] + deltas[:, owner]


def compose_uniform(sparse: np.ndarray, dense_sel: np.ndarray, s: int, gamma: int,
                    bf16: bool = False) -> np.ndarray:
    """llama.py:733-755: reshape broadcast of the anchor deltas over gamma-row
    groups, then the dense tail. sparse [B,s,H,d] (rows >= s_p unused),
    dense_sel [B,n_anchor+cut_n,H,d] -> [B,s,H,d]."""
    B, _, H, d = sparse.shape
    anchors, tail, s_p, cut_n = anchor_layout(s, gamma)
    n = len(anchors)
    assert s_p == n * gamma, "the reference reshape needs gamma | s_p"
    dense_a, last = dense_sel[:, :n], dense_sel[:, n:]
    sp = sparse[:, :s_p]
    if bf16:
        diff = sub_bf16(dense_a, sp[:, anchors])
        corr = add_bf16(diff.reshape(B, n, 1, H, d), sp.reshape(B, n, gamma, H, d))
    else:
        diff = dense_a - sp[:, anchors]
        corr = diff.reshape(B, n, 1, H, d) + sp.reshape(B, n, gamma, H, d)
    return np.concatenate([corr.reshape(B, s_p, H, d), last], axis=1)


def delta_forward(q: np.ndarray, k: np.ndarray, v: np.ndarray, gamma: int, window: int,
                  sink: int, scale: float, mode: str = "delta",
                  sparse: Optional[np.ndarray] = None) -> np.ndarray:
    """LlamaAttention.delta_forward (llama.py:659-757). q [B,H,s,d], k/v
    [B,Hkv,s,d] -> [B,s,H,d]. `sparse` may be passed in to reuse a computed
    key-sparse output."""
    B, H, s, d = q.shape
    if sparse is None:
        sparse = sparse_attention(q, k, v, window, sink, scale)
    if mode == "sparse-only":
        return sparse
    anchors, tail, s_p, cut_n = anchor_layout(s, gamma)
    idx = np.concatenate([anchors, tail])
    dense = qsparse_attention(q[:, :, idx], k, v, idx, scale).transpose(0, 2, 1, 3)
    if mode == "recompute":
        out = np.zeros_like(sparse)
        out[:, :s_p] = sparse[:, :s_p]
        out[:, idx] = dense
        return out
    assert mode == "delta", mode
    return compose_uniform(sparse, dense, s, gamma)


# ---------------------------------------------------------------------------
# training path: gradients of the delta composition (flex_delta.py:95-196
# under autograd)

def masked_attention_grads(q: np.ndarray, k: np.ndarray, v: np.ndarray, allowed: np.ndarray,
                           scale: float, dout: np.ndarray):
    """Gradients of masked_attention for the upstream gradient dout [B,H,n,d]:
    P = softmax(scale q k^T + mask), O = P v;
      dV = P^T dO, dP = dO V^T, dS = P * (dP - rowsum(dO * O)),
      dQ = scale dS K, dK = scale dS^T Q,
    dK / dV summed over the query heads of each KV head (the backward of
    repeat_interleave). -> (dq [B,H,n,d], dk [B,Hkv,N,d], dv [B,Hkv,N,d])."""
    B, H, n, d = q.shape
    Hkv, N = k.shape[1], k.shape[2]
    kk, vv = _expand_kv(k, H), _expand_kv(v, H)
    sc = np.matmul(q, kk.swapaxes(-1, -2)) * scale
    sc = np.where(allowed[None, None], sc, -np.inf)
    p = _softmax_rows(sc)
    o = np.matmul(p, vv)
    dv_e = np.matmul(p.swapaxes(-1, -2), dout)
    dp = np.matmul(dout, vv.swapaxes(-1, -2))
    di = (dout * o).sum(-1, keepdims=True)
    ds = p * (dp - di)
    dq = scale * np.matmul(ds, kk)
    dk_e = scale * np.matmul(ds.swapaxes(-1, -2), q)
    G = H // Hkv
    return dq, dk_e.reshape(B, Hkv, G, N, d).sum(2), dv_e.reshape(B, Hkv, G, N, d).sum(2)


def compose_grads(g: np.ndarray, gamma: int, s_p: int, grad_scale: float = 1.0,
                  detach: bool = False):
    """Backward of compose_uniform (flex_delta.py:186-196 with the detach and
    _ScaleGrad arms of :187-190): g [B,s,H,d] -> (dsparse [B,s,H,d], ddense
    [B, n_anchor + s - s_p, H, d]). ddelta[i] = grad_scale * sum of g over
    group i (0 when detached); dsparse = g on rows < s_p minus ddelta at the
    anchors, 0 on the tail; ddense = (ddelta, g of the tail rows)."""
    B, s, H, d = g.shape
    s_p = max(s_p, 0)
    n = s_p // gamma
    ddelta = g[:, :s_p].reshape(B, n, gamma, H, d).sum(2) * grad_scale
    if detach:
        ddelta = np.zeros_like(ddelta)
    dsparse = np.zeros_like(g)
    dsparse[:, :s_p] = g[:, :s_p]
    dsparse[:, np.arange(0, s_p, gamma)] -= ddelta
    ddense = np.concatenate([ddelta, g[:, s_p:]], axis=1)
    return dsparse, ddense


def delta_train_grads(q: np.ndarray, k: np.ndarray, v: np.ndarray, gamma: int, window: int,
                      sink: int, scale: float, g: np.ndarray, grad_scale: float = 1.0,
                      detach: bool = False, q_block: int = Q_BLOCK, parts: bool = False):
    """Gradients of delta_forward_train for the upstream gradient g [B,s,H,d]:
    the composition's backward, then the key-sparse attention's (mask of
    sparse_visible) and the anchor/tail rows' causal attention's, their dq,
    dk, dv added. q [B,H,s,d], k/v [B,Hkv,s,d] -> (dq, dk, dv); with
    parts=True also each branch's (dq, dk, dv) (the sparse branch's, then the
    anchor/tail rows' with dq scattered to the full rows). Dense masks: small
    sizes only."""
    B, H, s, d = q.shape
    anchors, tail, s_p, _ = anchor_layout(s, gamma)
    sel = np.concatenate([anchors, tail])
    dsparse, ddense = compose_grads(g, gamma, s_p, grad_scale, detach)
    r = np.arange(s)
    allowed = sparse_visible(r[:, None], r[None, :], window, sink, q_block)
    dq, dk, dv = masked_attention_grads(q, k, v, allowed, scale, dsparse.transpose(0, 2, 1, 3))
    allowed_d = r[None, :] <= sel[:, None]
    dq2, dk2, dv2 = masked_attention_grads(q[:, :, sel], k, v, allowed_d, scale,
                                           ddense.transpose(0, 2, 1, 3))
    dq_full2 = np.zeros_like(dq)
    dq_full2[:, :, sel] = dq2
    total = (dq + dq_full2, dk + dk2, dv + dv2)
    if parts:
        return total, (dq, dk, dv), (dq_full2, dk2, dv2)
    return total


# ---------------------------------------------------------------------------
# input generation helpers (the benchmark workloads' prologue)

def rope_cos_sin(s: int, d: int, theta: float) -> Tuple[np.ndarray, np.ndarray]:
    """Default-rope cos/sin tables [s, d] (llama.py:129-158: inv_freq =
    theta^(-2i/d), emb = cat(freqs, freqs)), in float32."""
    inv_freq = 1.0 / (theta ** (np.arange(0, d, 2, dtype=np.int64).astype(np.float32) / d))
    pos = np.arange(s, dtype=np.float32)
    freqs = np.outer(pos, inv_freq.astype(np.float32)).astype(np.float32)
    emb = np.concatenate([freqs, freqs], axis=-1)
    return np.cos(emb).astype(np.float32), np.sin(emb).astype(np.float32)


def apply_rope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """x [B,H,s,d]: x*cos + rotate_half(x)*sin (llama.py:161-192)."""
    half = x.shape[-1] // 2
    rot = np.concatenate([-x[..., half:], x[..., :half]], axis=-1)
    return x * cos[None, None] + rot * sin[None, None]


def mul_bf16(a, b) -> np.ndarray:
    return round_bf16(np.asarray(a, np.float32) * np.asarray(b, np.float32))


def apply_rope_bf16(x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """apply_rope with the reference's bf16 tensors (llama.py:190-191): x, cos,
    sin hold bf16 values; q*cos, rotate_half(q)*sin and their sum each round once."""
    half = x.shape[-1] // 2
    rot = np.concatenate([-x[..., half:], x[..., :half]], axis=-1)
    return add_bf16(mul_bf16(x, cos), mul_bf16(rot, sin))


def rms_norm_bf16(x: np.ndarray, weight: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    """LlamaRMSNorm on bf16 input (llama.py:69-74): float32 normalisation, cast
    to bf16, then the bf16 product with the bf16 weight."""
    x32 = np.asarray(x, np.float32)
    y = round_bf16(x32 / np.sqrt((x32 * x32).mean(axis=-1, keepdims=True) + np.float32(eps)))
    return mul_bf16(weight, y)


def rms_norm(x: np.ndarray, eps: float = 1e-6, weight: Optional[np.ndarray] = None) -> np.ndarray:
    """llama.py:69-74 over the last dim (computed in float32)."""
    x32 = x.astype(np.float32)
    y = x32 / np.sqrt((x32 * x32).mean(axis=-1, keepdims=True) + eps)
    return y if weight is None else y * weight


# ---------------------------------------------------------------------------
# metrics (validation.py:215-221)

def head_row_cos(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Cosine over the last dim only (tests/test_math_identities.py:85)."""
    a = a.astype(np.float64)
    b = b.astype(np.float64)
    return (a * b).sum(-1) / np.maximum(np.sqrt((a * a).sum(-1) * (b * b).sum(-1)), 1e-300)


# ---------------------------------------------------------------------------
# drift signal (stride.py:43-52, drift.py:23-49)

def interanchor_cos(deltas: np.ndarray, eps: float = 1e-8) -> np.ndarray:
    """[B, n, H, D] deltas -> [B, n-1, H] cosine between consecutive anchors
    over D: <a, b> / (max(|a|, eps) * max(|b|, eps)), in float64."""
    d = deltas.astype(np.float64)
    a, b = d[:, :-1], d[:, 1:]
    na = np.maximum(np.sqrt((a * a).sum(-1)), eps)
    nb = np.maximum(np.sqrt((b * b).sum(-1)), eps)
    return (a * b).sum(-1) / (na * nb)


def histc(x: np.ndarray, bins: int, lo: float, hi: float) -> np.ndarray:
    """torch.histc counts (int64 [bins]): bin = floor((x - lo) * bins / (hi - lo))
    evaluated in float32 as the GPU code does, x == hi in the last bin, values
    outside [lo, hi] and NaN dropped. Pure-Python loop: small inputs only."""
    out = np.zeros(bins, dtype=np.int64)
    lo32, hi32, nb = np.float32(lo), np.float32(hi), np.float32(bins)
    for v in np.asarray(x, dtype=np.float32).ravel():
        if not (lo32 <= v <= hi32):
            continue
        k = int(np.float32(np.float32(v - lo32) * nb) / np.float32(hi32 - lo32))
        out[min(k, bins - 1)] += 1
    return out
