"""Torch-tensor entry points over the C ABI.

PyTorch is used here for device memory and the current HIP stream only; all
attention arithmetic runs in libdelta_attn.so. Every op launches
asynchronously on torch's current stream of the tensors' device and never
synchronises.
"""

from __future__ import annotations

import ctypes
import functools
from typing import Optional, Tuple

import torch

from . import _lib as L

_DTYPE = {torch.bfloat16: L.DA_BF16, torch.float16: L.DA_FP16}
Q_BLOCK = 64  # hip-attn's block_sparse_block_size_q (config.py:117, :136)


def _code(t: torch.Tensor) -> int:
    code = _DTYPE.get(t.dtype)
    assert code is not None, f"dtype {t.dtype} is not supported (bfloat16, float16)"
    return code


def _ready(t: torch.Tensor) -> torch.Tensor:
    """Rows contiguous and 16-byte aligned, as the kernels read them; other
    dimensions keep their strides (no copy for the usual transposed views)."""
    ok = (t.stride(-1) == 1 and t.data_ptr() % 16 == 0
          and all(s % 8 == 0 for s in t.stride()[:-1]))
    return t if ok else t.contiguous()


def _ptr(t: Optional[torch.Tensor]):
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def _stream(dev: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def _on_gpu(*ts: torch.Tensor) -> torch.device:
    dev = ts[0].device
    for t in ts:
        assert t.is_cuda, "delta-attention kernels need GPU tensors"
        assert t.device == dev, "all tensors must be on one device"
    return dev


# ---------------------------------------------------------------------------
# kernel (1)

def sparse_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, window: int,
                     sink: int, sm_scale: float, q_block: int = Q_BLOCK,
                     out: Optional[torch.Tensor] = None,
                     rows: Optional[Tuple[int, int]] = None) -> torch.Tensor:
    """Causal sink + block-anchored sliding-window attention.

    q [B,H,S,D], k/v [B,Hkv,S,D] (any strides, GQA native) -> out [B,S,H,D].
    A key k is visible to row r iff k <= r and (k < sink or
    k + window > floor(r/q_block)*q_block + q_block - 1)
    (delta_attention/train/flex_delta.py:59-61).
    rows = (row0, n): only rows row0 .. row0 + n - 1 are computed (the other
    rows of `out` are left as they are; da_sparse_attn_fwd_rows).
    """
    assert q.dim() == 4 and k.dim() == 4 and v.dim() == 4
    B, H, S, D = q.shape
    Hkv = k.shape[1]
    assert k.shape == (B, Hkv, S, D) and v.shape == (B, Hkv, S, D), (q.shape, k.shape, v.shape)
    assert H % Hkv == 0, (H, Hkv)
    assert q.dtype == k.dtype == v.dtype
    dev = _on_gpu(q, k, v)
    q, k, v = _ready(q), _ready(k), _ready(v)
    if out is None:
        out = torch.empty((B, S, H, D), device=dev, dtype=q.dtype)
    assert out.shape == (B, S, H, D) and out.dtype == q.dtype
    assert out.stride(-1) == 1 and out.data_ptr() % 16 == 0
    strides = (L.strides3(q.stride(0), q.stride(1), q.stride(2)),
               L.strides3(k.stride(0), k.stride(1), k.stride(2)),
               L.strides3(v.stride(0), v.stride(1), v.stride(2)),
               L.strides3(out.stride(0), out.stride(2), out.stride(1)))
    with torch.cuda.device(dev):
        if rows is not None:
            rc = L.lib().da_sparse_attn_fwd_rows(
                _ptr(q), _ptr(k), _ptr(v), _ptr(out), B, H, Hkv, S, D, *strides,
                int(window), int(sink), int(q_block), float(sm_scale), int(rows[0]), int(rows[1]),
                _code(q), _stream(dev))
        else:
            rc = L.lib().da_sparse_attn_fwd(
                _ptr(q), _ptr(k), _ptr(v), _ptr(out), B, H, Hkv, S, D, *strides,
                int(window), int(sink), int(q_block), float(sm_scale), _code(q), _stream(dev))
    L.check(rc, "da_sparse_attn_fwd")
    return out


def fused_delta_rows(H: int, Hkv: int) -> int:
    """Largest row-tile height of the fused delta launch (128): the fused
    order needs gamma to divide it (two heads per 64-row tile when the GQA
    ratio is even and gamma divides 64, else one head per 128-row tile)."""
    return int(L.lib().da_fused_delta_rows(int(H), int(Hkv)))


def set_sparse_rows_per_wave(rows: int) -> int:
    """Tile shape of the head_dim-128 key-sparse launches, process-wide: 32
    (default) or 64 query rows per wave. Returns the previous value; the
    outputs are bit-identical either way."""
    prev = int(L.lib().da_sparse_rows_per_wave())
    L.check(L.lib().da_set_sparse_rows_per_wave(int(rows)), "da_set_sparse_rows_per_wave")
    return prev


def set_bwd_rows_per_chunk(rows: int) -> None:
    """Rows per dK/dV work item at most in the training backward,
    process-wide (0: the default, 8192). Set it before the backward's
    workspace is sized; results agree to the rounding of the chunks'
    partial sums."""
    L.check(L.lib().da_set_bwd_rows_per_chunk(int(rows)), "da_set_bwd_rows_per_chunk")


def sparse_attention_delta(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, window: int,
                           sink: int, sm_scale: float, dense_sel: torch.Tensor, gamma: int,
                           s_p: int, out: torch.Tensor, delta_out: Optional[torch.Tensor] = None,
                           q_block: int = Q_BLOCK) -> torch.Tensor:
    """Kernel (1) with the delta broadcast-add in its epilogue: rows r < s_p of
    `out` [B,S,H,D] become rnd(rnd(sparse[r]) + delta[r // gamma]) with
    delta[g] = rnd(dense_sel[:, g] - rnd(sparse[g * gamma])) (llama.py:733-755);
    rows >= s_p are left as they are (the dense tail). dense_sel [B,n_anchor,H,D];
    delta_out (same shape) receives the deltas when given."""
    B, H, S, D = q.shape
    Hkv = k.shape[1]
    assert k.shape == (B, Hkv, S, D) and v.shape == (B, Hkv, S, D), (q.shape, k.shape, v.shape)
    assert q.dtype == k.dtype == v.dtype == out.dtype == dense_sel.dtype
    assert out.shape == (B, S, H, D) and out.stride(-1) == 1 and out.data_ptr() % 16 == 0
    n_anchor = -(-s_p // gamma) if s_p > 0 else 0
    assert dense_sel.shape == (B, n_anchor, H, D) and dense_sel.stride(-1) == 1, dense_sel.shape
    dev = _on_gpu(q, k, v, out, dense_sel)
    q, k, v = _ready(q), _ready(k), _ready(v)
    dl = L.strides3(0, 0, 0)
    if delta_out is not None:
        assert delta_out.shape == dense_sel.shape and delta_out.dtype == q.dtype
        assert delta_out.stride(-1) == 1
        dl = L.strides3(delta_out.stride(0), delta_out.stride(2), delta_out.stride(1))
    with torch.cuda.device(dev):
        rc = L.lib().da_sparse_attn_delta_fwd(
            _ptr(q), _ptr(k), _ptr(v), _ptr(out), B, H, Hkv, S, D,
            L.strides3(q.stride(0), q.stride(1), q.stride(2)),
            L.strides3(k.stride(0), k.stride(1), k.stride(2)),
            L.strides3(v.stride(0), v.stride(1), v.stride(2)),
            L.strides3(out.stride(0), out.stride(2), out.stride(1)),
            int(window), int(sink), int(q_block), float(sm_scale),
            _ptr(dense_sel), L.strides3(dense_sel.stride(0), dense_sel.stride(2), dense_sel.stride(1)),
            int(gamma), int(s_p), _ptr(delta_out), dl, _code(q), _stream(dev))
    L.check(rc, "da_sparse_attn_delta_fwd")
    return out


# ---------------------------------------------------------------------------
# kernel (2)

def qsparse_workspace(B: int, H: int, Hkv: int, n: int, Skv: int, D: int, device) -> torch.Tensor:
    nbytes = int(L.lib().da_qsparse_workspace_bytes(B, H, Hkv, n, Skv, D))
    return torch.empty(max(nbytes, 16), dtype=torch.uint8, device=device)


def _row_limits(row_last: torch.Tensor, B: int, n: int) -> Tuple[torch.Tensor, int]:
    rl = row_last
    if rl.dim() == 1:
        rl = rl.unsqueeze(0)
    assert rl.dim() == 2 and rl.shape[1] == n and rl.shape[0] in (1, B), (row_last.shape, B, n)
    if rl.dtype != torch.int64:
        rl = rl.to(torch.int64)
    rl = rl.contiguous()
    return rl, (0 if rl.shape[0] == 1 else rl.stride(0))


def qsparse_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                      row_last: torch.Tensor, sm_scale: float, *,
                      q_rows: Optional[torch.Tensor] = None,
                      epi: int = L.DA_EPI_OUTPUT, out: Optional[torch.Tensor] = None,
                      n_anchor: int = 0, delta: Optional[torch.Tensor] = None,
                      workspace: Optional[torch.Tensor] = None,
                      n_live: Optional[int] = None,
                      n_dev: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Query-sparse, key-dense attention: selected row i attends keys
    0..row_last[i] (inclusive), split over the key axis on the GPU.

    n_live (DA_EPI_OUTPUT only): about this many rows hold keys, the others
    being -1 rows; the split plan is sized for them (da_qsparse_attn_fwd_live).
    n_dev: with n_live, a device int32 holding the live row count; rows in
    row tiles wholly past it are neither computed nor written.

    q [B,H,Sq,D]; k/v [B,Hkv,Skv,D] (GQA native, any strides);
    q_rows: optional [n] int64 rows of q to use (default: rows 0..n-1, n = len(row_last)).
    epi == DA_EPI_OUTPUT: returns o [B,H,n,D] (new, or `out`).
    epi == DA_EPI_DELTA / DA_EPI_SCATTER / DA_EPI_DENSE: `out` is the [B,S,H,D]
    layer output; see include/delta_attn.h.
    """
    B, H, Sq, D = q.shape
    Hkv, Skv = k.shape[1], k.shape[2]
    assert k.shape == (B, Hkv, Skv, D) and v.shape == k.shape, (q.shape, k.shape, v.shape)
    assert H % Hkv == 0 and q.dtype == k.dtype == v.dtype
    n = row_last.shape[-1]
    dev = _on_gpu(q, k, v, row_last)
    q, k, v = _ready(q), _ready(k), _ready(v)
    rl, rl_b = _row_limits(row_last, B, n)
    if q_rows is not None:
        assert q_rows.numel() == n
        q_rows = q_rows.reshape(-1).to(device=dev, dtype=torch.int64).contiguous()
    else:
        assert n <= Sq, (n, Sq)
    if epi == L.DA_EPI_OUTPUT:
        if out is None:
            out = torch.empty((B, H, n, D), device=dev, dtype=q.dtype)
        assert out.shape == (B, H, n, D)
        o_str = L.strides3(out.stride(0), out.stride(1), out.stride(2))
    else:
        assert out is not None and out.dim() == 4 and out.shape[0] == B and out.shape[2] == H
        o_str = L.strides3(out.stride(0), out.stride(2), out.stride(1))
    assert out.dtype == q.dtype and out.stride(-1) == 1
    d_str = None
    if epi in (L.DA_EPI_DELTA, L.DA_EPI_DENSE) and n_anchor > 0:
        assert delta is not None and delta.shape == (B, n_anchor, H, D) and delta.dtype == q.dtype
        d_str = L.strides3(delta.stride(0), delta.stride(2), delta.stride(1))
    if n_live is not None and n > 0:
        assert epi == L.DA_EPI_OUTPUT and n_live >= 1
        if n_dev is not None:
            assert n_dev.dtype == torch.int32 and n_dev.device == dev
        if workspace is None:
            nb = L.lib().da_qsparse_workspace_bytes_live(B, H, Hkv, n, int(n_live), Skv, D)
            assert nb > 0, "selected-rows launch too large"
            workspace = torch.empty(nb, dtype=torch.uint8, device=dev)
        with torch.cuda.device(dev):
            rc = L.lib().da_qsparse_attn_fwd_live(
                _ptr(q), _ptr(k), _ptr(v), _ptr(q_rows), _ptr(rl), int(rl_b),
                n, int(n_live), _ptr(n_dev), B, H, Hkv, Sq, Skv, D,
                L.strides3(q.stride(0), q.stride(1), q.stride(2)),
                L.strides3(k.stride(0), k.stride(1), k.stride(2)),
                L.strides3(v.stride(0), v.stride(1), v.stride(2)),
                _ptr(out), o_str, float(sm_scale), _ptr(workspace), workspace.numel(), _code(q),
                _stream(dev))
        L.check(rc, "da_qsparse_attn_fwd_live")
        return out
    if workspace is None:
        workspace = qsparse_workspace(B, H, Hkv, n, Skv, D, dev)
    with torch.cuda.device(dev):
        rc = L.lib().da_qsparse_attn_fwd(
            _ptr(q), _ptr(k), _ptr(v), _ptr(q_rows), _ptr(rl), int(rl_b),
            n, B, H, Hkv, Sq, Skv, D,
            L.strides3(q.stride(0), q.stride(1), q.stride(2)),
            L.strides3(k.stride(0), k.stride(1), k.stride(2)),
            L.strides3(v.stride(0), v.stride(1), v.stride(2)),
            _ptr(out), o_str, int(epi), int(n_anchor), _ptr(delta), d_str,
            float(sm_scale), _ptr(workspace), workspace.numel(), _code(q), _stream(dev))
    L.check(rc, "da_qsparse_attn_fwd")
    return out


# ---------------------------------------------------------------------------
# kernel (3)

def delta_add(sparse: torch.Tensor, *, s_p: int, out: Optional[torch.Tensor] = None,
              delta: Optional[torch.Tensor] = None, dense_sel: Optional[torch.Tensor] = None,
              anchors: Optional[torch.Tensor] = None, gamma: int = 0) -> torch.Tensor:
    """out[:, r] = sparse[:, r] + delta[:, owner(r)] for r < s_p ([B,S,H,D] tensors).

    owner(r) = r // gamma (anchors None) or the last anchor <= r. The delta is
    `delta` [B,n,H,D], or rnd(dense_sel - sparse[:, anchors]) when `delta` is None.
    `out` defaults to a new [B,s_p,H,D] tensor; out=sparse runs in place
    (allowed with a precomputed delta only).
    """
    B, _, H, D = sparse.shape
    dev = _on_gpu(sparse)
    if out is None:
        out = torch.empty((B, s_p, H, D), device=dev, dtype=sparse.dtype)
    assert out.dtype == sparse.dtype and out.shape[0] == B and out.shape[2:] == (H, D)
    if delta is not None:
        n = delta.shape[1]
        d_str = L.strides3(delta.stride(0), delta.stride(2), delta.stride(1))
        ds_str = None
    else:
        assert dense_sel is not None and anchors is not None
        n = dense_sel.shape[1]
        d_str = None
        ds_str = L.strides3(dense_sel.stride(0), dense_sel.stride(2), dense_sel.stride(1))
    if anchors is not None:
        anchors = anchors.reshape(-1).to(device=dev, dtype=torch.int64).contiguous()
        assert anchors.numel() == n
    with torch.cuda.device(dev):
        rc = L.lib().da_delta_add(
            _ptr(sparse), L.strides3(sparse.stride(0), sparse.stride(2), sparse.stride(1)),
            _ptr(out), L.strides3(out.stride(0), out.stride(2), out.stride(1)),
            _ptr(delta), d_str, _ptr(dense_sel), ds_str, _ptr(anchors),
            int(n), int(gamma), int(s_p), B, H, D, _code(sparse), _stream(dev))
    L.check(rc, "da_delta_add")
    return out


# ---------------------------------------------------------------------------
# training path: forward with saved row log-sum-exp, and the backward

def _s3(t: torch.Tensor, a: int, b: int, c: int):
    return L.strides3(t.stride(a), t.stride(b), t.stride(c))


def sparse_attention_lse(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, window: int,
                         sink: int, sm_scale: float, q_block: int = Q_BLOCK
                         ) -> Tuple[torch.Tensor, torch.Tensor]:
    """sparse_attention plus each row's log2-domain log-sum-exp:
    -> (out [B,S,H,D], lse float32 [B,H,S])."""
    B, H, S, D = q.shape
    Hkv = k.shape[1]
    assert k.shape == (B, Hkv, S, D) and v.shape == k.shape and H % Hkv == 0
    dev = _on_gpu(q, k, v)
    q, k, v = _ready(q), _ready(k), _ready(v)
    out = torch.empty((B, S, H, D), device=dev, dtype=q.dtype)
    lse = torch.empty((B, H, S), device=dev, dtype=torch.float32)
    with torch.cuda.device(dev):
        rc = L.lib().da_sparse_attn_fwd_lse(
            _ptr(q), _ptr(k), _ptr(v), _ptr(out), B, H, Hkv, S, D,
            _s3(q, 0, 1, 2), _s3(k, 0, 1, 2), _s3(v, 0, 1, 2), _s3(out, 0, 2, 1),
            int(window), int(sink), int(q_block), float(sm_scale), _ptr(lse), _code(q),
            _stream(dev))
    L.check(rc, "da_sparse_attn_fwd_lse")
    return out, lse


def rows_attention_lse(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, rows: torch.Tensor,
                       sm_scale: float) -> Tuple[torch.Tensor, torch.Tensor]:
    """Rows `rows` (int64 [n]) of q attending keys 0 .. rows[i] (causal):
    -> (out [B,n,H,D], lse float32 [B,H,n])."""
    B, H, Sq, D = q.shape
    Hkv, Skv = k.shape[1], k.shape[2]
    assert k.shape == (B, Hkv, Skv, D) and v.shape == k.shape and H % Hkv == 0
    dev = _on_gpu(q, k, v, rows)
    q, k, v = _ready(q), _ready(k), _ready(v)
    rows = rows.reshape(-1).to(device=dev, dtype=torch.int64).contiguous()
    n = rows.numel()
    out = torch.empty((B, n, H, D), device=dev, dtype=q.dtype)
    lse = torch.empty((B, H, n), device=dev, dtype=torch.float32)
    ws = qsparse_workspace(B, H, Hkv, n, Skv, D, dev)
    with torch.cuda.device(dev):
        rc = L.lib().da_qsparse_attn_fwd_lse(
            _ptr(q), _ptr(k), _ptr(v), _ptr(rows), _ptr(rows), 0, n, B, H, Hkv, Sq, Skv, D,
            _s3(q, 0, 1, 2), _s3(k, 0, 1, 2), _s3(v, 0, 1, 2), _ptr(out), _s3(out, 0, 2, 1),
            _ptr(lse), float(sm_scale), _ptr(ws), ws.numel(), _code(q), _stream(dev))
    L.check(rc, "da_qsparse_attn_fwd_lse")
    return out, lse


def _grads_like(q, k, dq, dk, dv):
    dq = torch.empty_like(q) if dq is None else dq
    dk = torch.empty_like(k) if dk is None else dk
    dv = torch.empty_like(k) if dv is None else dv
    for t in (dq, dk, dv):
        assert t.stride(-1) == 1 and t.data_ptr() % 16 == 0 and all(x % 8 == 0 for x in t.stride()[:-1])
    return dq, dk, dv


def sparse_attention_bwd(q, k, v, out, dout, lse, *, window: int, sink: int, sm_scale: float,
                         q_block: int = Q_BLOCK, dq=None, dk=None, dv=None,
                         accumulate: bool = False):
    """Gradients of sparse_attention: q [B,H,S,D], k/v [B,Hkv,S,D], out/dout
    [B,S,H,D], lse [B,H,S] -> (dq, dk, dv) shaped like q, k, v (new, or the
    given tensors; accumulate=True adds into them)."""
    B, H, S, D = q.shape
    Hkv = k.shape[1]
    dev = _on_gpu(q, k, v, out, dout, lse)
    q, k, v, out, dout = _ready(q), _ready(k), _ready(v), _ready(out), _ready(dout)
    lse = lse.contiguous()
    assert out.shape == dout.shape == (B, S, H, D) and lse.shape == (B, H, S)
    dq, dk, dv = _grads_like(q, k, dq, dk, dv)
    nbytes = int(L.lib().da_sparse_attn_bwd_workspace_bytes(B, H, Hkv, S, D, int(window),
                                                            int(sink), int(q_block)))
    ws = torch.empty(max(nbytes, 16), device=dev, dtype=torch.uint8)
    with torch.cuda.device(dev):
        rc = L.lib().da_sparse_attn_bwd(
            _ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(dout), _ptr(lse),
            _ptr(dq), _ptr(dk), _ptr(dv), B, H, Hkv, S, D,
            _s3(q, 0, 1, 2), _s3(k, 0, 1, 2), _s3(v, 0, 1, 2), _s3(out, 0, 2, 1),
            _s3(dout, 0, 2, 1), _s3(dq, 0, 1, 2), _s3(dk, 0, 1, 2), _s3(dv, 0, 1, 2),
            int(window), int(sink), int(q_block), float(sm_scale), int(bool(accumulate)),
            _ptr(ws), ws.numel(), _code(q), _stream(dev))
    L.check(rc, "da_sparse_attn_bwd")
    return dq, dk, dv


def rows_attention_bwd(q, k, v, rows, out, dout, lse, *, sm_scale: float, dq=None, dk=None,
                       dv=None, accumulate: bool = False):
    """Gradients of rows_attention_lse (rows ascending and distinct): out/dout
    [B,n,H,D], lse [B,H,n] -> (dq, dk, dv) shaped like q, k, v; dq rows outside
    `rows` are zero (or untouched with accumulate=True)."""
    B, H, Sq, D = q.shape
    Hkv, Skv = k.shape[1], k.shape[2]
    dev = _on_gpu(q, k, v, rows, out, dout, lse)
    q, k, v, out, dout = _ready(q), _ready(k), _ready(v), _ready(out), _ready(dout)
    rows = rows.reshape(-1).to(device=dev, dtype=torch.int64).contiguous()
    lse = lse.contiguous()
    n = rows.numel()
    assert out.shape == dout.shape == (B, n, H, D) and lse.shape == (B, H, n)
    if dq is None and not accumulate:
        dq = torch.zeros_like(q)
    dq, dk, dv = _grads_like(q, k, dq, dk, dv)
    nbytes = int(L.lib().da_qsparse_attn_bwd_workspace_bytes(B, H, Hkv, n, Skv, D))
    ws = torch.empty(max(nbytes, 16), device=dev, dtype=torch.uint8)
    with torch.cuda.device(dev):
        rc = L.lib().da_qsparse_attn_bwd(
            _ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(dout), _ptr(lse), _ptr(rows), _ptr(rows), n,
            _ptr(dq), _ptr(dk), _ptr(dv), B, H, Hkv, Sq, Skv, D,
            _s3(q, 0, 1, 2), _s3(k, 0, 1, 2), _s3(v, 0, 1, 2), _s3(out, 0, 2, 1),
            _s3(dout, 0, 2, 1), _s3(dq, 0, 1, 2), _s3(dk, 0, 1, 2), _s3(dv, 0, 1, 2),
            float(sm_scale), int(bool(accumulate)), _ptr(ws), ws.numel(), _code(q), _stream(dev))
    L.check(rc, "da_qsparse_attn_bwd")
    return dq, dk, dv


def delta_compose_bwd(grad: torch.Tensor, *, gamma: int, s_p: int, delta_grad_scale: float = 1.0,
                      detach_delta: bool = False) -> Tuple[torch.Tensor, torch.Tensor]:
    """Backward of the delta composition: grad [B,S,H,D] -> (dsparse [B,S,H,D],
    ddense [B, s_p/gamma + S - s_p, H, D]) (include/delta_attn.h)."""
    B, S, H, D = grad.shape
    dev = _on_gpu(grad)
    grad = _ready(grad)
    n_sel = s_p // gamma + S - s_p
    dsparse = torch.empty((B, S, H, D), device=dev, dtype=grad.dtype)
    ddense = torch.empty((B, n_sel, H, D), device=dev, dtype=grad.dtype)
    with torch.cuda.device(dev):
        rc = L.lib().da_delta_compose_bwd(
            _ptr(grad), _s3(grad, 0, 2, 1), _ptr(dsparse), _s3(dsparse, 0, 2, 1),
            _ptr(ddense), _s3(ddense, 0, 2, 1), B, H, S, D, int(gamma), int(s_p),
            float(delta_grad_scale), int(bool(detach_delta)), _code(grad), _stream(dev))
    L.check(rc, "da_delta_compose_bwd")
    return dsparse, ddense


# ---------------------------------------------------------------------------
# attention prologue: per-head RMSNorm (optional) + RoPE, in place

def rope_qk_append(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cos: torch.Tensor,
                   sin: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                   pos: torch.Tensor, *, q_norm_w: Optional[torch.Tensor] = None,
                   k_norm_w: Optional[torch.Tensor] = None, eps: float = 1e-6) -> None:
    """One-token decode step: rope_qk on q (in place) and k, with the rotated k
    and v written to the [B, max_len, Hkv, D] caches at row pos (int64 [1] on
    the device) instead of a separate cache update. q/k/v [B, 1, H, D]. A pos
    outside [0, max_len) when the kernel runs leaves both caches unchanged."""
    B, S, Hq, D = q.shape
    Hkv = k.shape[2]
    assert S == 1 and k.shape == (B, 1, Hkv, D) and v.shape == k.shape
    assert k_cache.shape[0] == B and k_cache.shape[2:] == (Hkv, D) and v_cache.shape == k_cache.shape
    assert k_cache.dtype == v_cache.dtype == q.dtype
    dev = _on_gpu(q, k, v, k_cache, v_cache, pos)
    assert pos.dtype == torch.int64 and pos.numel() == 1
    cos = cos.to(device=dev, dtype=q.dtype)
    sin = sin.to(device=dev, dtype=q.dtype)
    if cos.dim() == 2:
        cos, sin = cos.unsqueeze(0), sin.unsqueeze(0)
    assert cos.shape[1:] == (1, D) and cos.shape[0] in (1, B)
    cos, sin = cos.contiguous(), sin.contiguous()
    ws = [None if w is None else w.to(device=dev, dtype=q.dtype).contiguous() for w in (q_norm_w, k_norm_w)]
    cs = (ctypes.c_int64 * 2)(0 if cos.shape[0] == 1 else cos.stride(0), cos.stride(1))
    with torch.cuda.device(dev):
        rc = L.lib().da_rope_qk_append(
            _ptr(q), _s3(q, 0, 1, 2), Hq, _ptr(k), _s3(k, 0, 1, 2), Hkv, _ptr(v), _s3(v, 0, 1, 2),
            B, D, _ptr(cos), _ptr(sin), cs, _ptr(ws[0]), _ptr(ws[1]), float(eps),
            _ptr(k_cache), _s3(k_cache, 0, 1, 2), _ptr(v_cache), _s3(v_cache, 0, 1, 2),
            int(k_cache.shape[1]), _ptr(pos), _code(q), _stream(dev))
    L.check(rc, "da_rope_qk_append")


def rope_qk(q: Optional[torch.Tensor], k: Optional[torch.Tensor], cos: torch.Tensor,
            sin: torch.Tensor, *, q_norm_w: Optional[torch.Tensor] = None,
            k_norm_w: Optional[torch.Tensor] = None, eps: float = 1e-6):
    """In place on q [B,S,Hq,D] and k [B,S,Hkv,D] (projection-output layout, any
    batch/seq/head strides): optional per-head RMSNorm with the given weights,
    then rotary embedding with cos/sin [B or 1, S, D] (cast to q's dtype, as the
    reference does). Returns (q, k)."""
    x = q if q is not None else k
    assert x is not None and x.dim() == 4
    B, S, _, D = x.shape
    dev = _on_gpu(*[t for t in (q, k) if t is not None])
    if S == 0:
        return q, k
    cos = cos.to(device=dev, dtype=x.dtype)
    sin = sin.to(device=dev, dtype=x.dtype)
    if cos.dim() == 2:
        cos, sin = cos.unsqueeze(0), sin.unsqueeze(0)
    assert cos.shape[1:] == (S, D) and cos.shape[0] in (1, B) and sin.shape == cos.shape
    cos, sin = cos.contiguous(), sin.contiguous()
    for t in (q, k):
        if t is not None:
            assert t.shape[0] == B and t.shape[1] == S and t.shape[3] == D and t.dtype == x.dtype
            assert t.stride(-1) == 1 and t.data_ptr() % 16 == 0, "rope_qk works in place on row-contiguous tensors"
    ws = [None if w is None else w.to(device=dev, dtype=x.dtype).contiguous() for w in (q_norm_w, k_norm_w)]
    cs = (ctypes.c_int64 * 2)(0 if cos.shape[0] == 1 else cos.stride(0), cos.stride(1))
    with torch.cuda.device(dev):
        rc = L.lib().da_rope_qk(
            _ptr(q), None if q is None else L.strides3(q.stride(0), q.stride(1), q.stride(2)),
            0 if q is None else q.shape[2],
            _ptr(k), None if k is None else L.strides3(k.stride(0), k.stride(1), k.stride(2)),
            0 if k is None else k.shape[2],
            B, S, D, _ptr(cos), _ptr(sin), cs, _ptr(ws[0]), _ptr(ws[1]), float(eps),
            _code(x), _stream(dev))
    L.check(rc, "da_rope_qk")
    return q, k


# ---------------------------------------------------------------------------
# decode rows

def decode_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, window: int, sink: int,
                     sm_scale: float, out: Optional[torch.Tensor] = None,
                     n_keys: Optional[torch.Tensor] = None,
                     add: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The query row at the end of the cache: q [B,H,1,D] against k/v
    [B,Hkv,n,D] (GQA native) over keys [0, sink) and the last `window` keys
    (window 0: all keys; llama.py:537-549, 598-600) -> [B,H,1,D].

    n_keys: an int32 device tensor holding the key count (k/v then hold the
    cache's capacity, n rows, of which the first *n_keys are valid). The call
    reads it when the kernels run, so a recorded call (HIP graph) serves every
    length of a growing cache. add (with n_keys): a [B,H,1,D] tensor added to
    the row in the same launch, rnd(rnd(row) + add) as the bf16 tensor add."""
    assert q.dim() == 4 and q.shape[2] == 1, q.shape
    B, H, _, D = q.shape
    Hkv, n = k.shape[1], k.shape[2]
    assert k.shape == (B, Hkv, n, D) and v.shape == k.shape and H % Hkv == 0, (q.shape, k.shape)
    assert q.dtype == k.dtype == v.dtype
    dev = _on_gpu(q, k, v)
    q, k, v = _ready(q), _ready(k), _ready(v)
    if out is None:
        out = torch.empty((B, H, 1, D), device=dev, dtype=q.dtype)
    assert out.shape == (B, H, 1, D) and out.stride(-1) == 1 and out.data_ptr() % 16 == 0
    w, sk = max(int(window), 0), max(int(sink), 0)
    nbytes = int(L.lib().da_decode_workspace_bytes(B, H, Hkv, n, D, w, sk))
    ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=dev)
    strides = (L.strides3(q.stride(0), q.stride(1), q.stride(2)),
               L.strides3(k.stride(0), k.stride(1), k.stride(2)),
               L.strides3(v.stride(0), v.stride(1), v.stride(2)),
               L.strides3(out.stride(0), out.stride(1), out.stride(2)))
    with torch.cuda.device(dev):
        if n_keys is None:
            assert add is None, "add= goes with a device key count"
            rc = L.lib().da_decode_attn_fwd(
                _ptr(q), _ptr(k), _ptr(v), _ptr(out), B, H, Hkv, n, D, *strides,
                w, sk, float(sm_scale), _ptr(ws), nbytes, _code(q), _stream(dev))
        else:
            assert n_keys.dtype == torch.int32 and n_keys.device == dev and n_keys.numel() == 1
            if add is not None:
                assert add.shape == (B, H, 1, D) and add.dtype == q.dtype and add.device == dev
                add = _ready(add)
            rc = L.lib().da_decode_attn_fwd_dev(
                _ptr(q), _ptr(k), _ptr(v), _ptr(out), B, H, Hkv, _ptr(n_keys), n, D, *strides,
                w, sk, float(sm_scale), _ptr(add),
                None if add is None else L.strides3(add.stride(0), add.stride(1), add.stride(2)),
                _ptr(ws), nbytes, _code(q), _stream(dev))
    L.check(rc, "da_decode_attn_fwd" if n_keys is None else "da_decode_attn_fwd_dev")
    return out


# ---------------------------------------------------------------------------
# decoder-layer element-wise kernels (full-model prefill)

def _rows2d(t: torch.Tensor) -> Tuple[int, int]:
    """(rows, row stride) of a tensor whose last dim is contiguous and whose
    leading dims collapse to one row index."""
    assert t.stride(-1) == 1, "last dim must be contiguous"
    n = t.shape[-1]
    rows = t.numel() // n if n else 0
    if t.dim() == 1:
        return 1, n
    lead = t.reshape(-1, n) if rows else t
    assert lead.data_ptr() == t.data_ptr(), "leading dims must collapse without a copy"
    return rows, lead.stride(0)


def add_rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float, *,
                residual: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None,
                residual_out: Optional[torch.Tensor] = None):
    """LlamaRMSNorm (llama.py:69-74) of x, or of rnd(x + residual) when a
    residual is given (the decoder layer's add, llama.py:968-979).
    Returns y, or (y, h) with h = x + residual (written to residual_out,
    default a new tensor)."""
    n = x.shape[-1]
    dev = _on_gpu(x, weight)
    rows, xs = _rows2d(x)
    if out is None:
        out = torch.empty_like(x)
    assert out.shape == x.shape and out.dtype == x.dtype
    _, ys = _rows2d(out)
    w = weight.to(device=dev, dtype=x.dtype).contiguous()
    h = None
    rs = hs = 0
    if residual is not None:
        assert residual.shape == x.shape and residual.dtype == x.dtype
        _, rs = _rows2d(residual)
        h = torch.empty_like(x) if residual_out is None else residual_out
        _, hs = _rows2d(h)
    with torch.cuda.device(dev):
        rc = L.lib().da_add_rmsnorm(_ptr(x), xs, _ptr(residual), rs, _ptr(h), hs, _ptr(out), ys,
                                    _ptr(w), rows, n, float(eps), _code(x), _stream(dev))
    L.check(rc, "da_add_rmsnorm")
    return out if residual is None else (out, h)


def swiglu(gate: torch.Tensor, up: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """silu(gate) * up with the reference's bf16 rounding per op (llama.py:212-213)."""
    assert gate.shape == up.shape and gate.dtype == up.dtype
    dev = _on_gpu(gate, up)
    rows, gs = _rows2d(gate)
    _, us = _rows2d(up)
    if out is None:
        out = torch.empty_like(gate)
    _, os_ = _rows2d(out)
    with torch.cuda.device(dev):
        rc = L.lib().da_swiglu(_ptr(gate), gs, _ptr(up), us, _ptr(out), os_, rows, gate.shape[-1],
                               _code(gate), _stream(dev))
    L.check(rc, "da_swiglu")
    return out


# ---------------------------------------------------------------------------
# the composed layer prefill (kernels 1 -> 2 -> 3)

# ---------------------------------------------------------------------------
# consecutive-anchor delta cosine (drift signal)

def anchor_delta_cos(a: torch.Tensor, *, sparse: Optional[torch.Tensor] = None,
                     rows: Optional[torch.Tensor] = None, hist_bins: int = 0,
                     hist_range: Tuple[float, float] = (-1.0, 1.0)):
    """Cosine between consecutive anchor deltas, per (batch, head) over the
    head dim: returns fp32 [B, n-1, H] (and, with hist_bins > 0, an int32
    histogram of the cosines over hist_range with torch.histc's bins).

    a: the deltas [B, n, H, D]; or, with `sparse` [B, S, H, D] given, the dense
    anchor rows, whose deltas rnd(a - sparse[:, rows]) are formed inside the
    kernel and never stored (rows: int64 [n] anchor rows, default 0..n-1)."""
    assert a.dim() == 4, a.shape
    B, n, H, D = a.shape
    ts = [a] + ([sparse] if sparse is not None else [])
    dev = _on_gpu(*ts)
    code = _code(a)
    if a.stride(-1) != 1 or a.data_ptr() % 4 or any(st % 2 for st in a.stride()[:-1]):
        a = a.contiguous()
    cos = torch.empty(B, max(n - 1, 0), H, device=dev, dtype=torch.float32)
    hist = torch.zeros(hist_bins, device=dev, dtype=torch.int32) if hist_bins > 0 else None
    s_str = None
    n_rows = 0
    if sparse is not None:
        assert sparse.dim() == 4 and sparse.shape[0] == B and sparse.shape[2:] == (H, D), sparse.shape
        assert sparse.dtype == a.dtype, (sparse.dtype, a.dtype)
        if sparse.stride(-1) != 1 or sparse.data_ptr() % 4 or any(st % 2 for st in sparse.stride()[:-1]):
            sparse = sparse.contiguous()
        s_str = L.I64x3(*sparse.stride()[:3])
        n_rows = sparse.shape[1]
        if rows is not None:
            rows = rows.to(device=dev, dtype=torch.int64).contiguous()
            assert rows.numel() == n, (rows.numel(), n)
    with torch.cuda.device(dev):
        rc = L.lib().da_anchor_delta_cos(
            _ptr(a), L.I64x3(*a.stride()[:3]), _ptr(sparse), s_str, _ptr(rows), n_rows,
            B, n, H, D, _ptr(cos), _ptr(hist), int(hist_bins),
            float(hist_range[0]), float(hist_range[1]), code, _stream(dev))
    L.check(rc, "da_anchor_delta_cos")
    return (cos, hist) if hist_bins > 0 else cos


def adapt_chunk_step(dense: torch.Tensor, sparse: torch.Tensor, rows: torch.Tensor,
                     state: torch.Tensor, cos_work: torch.Tensor, *, chunk: int,
                     next_start: int, next_end: int, rows_next: Optional[torch.Tensor],
                     trigger: str, threshold: float, margin: float, k: float,
                     gamma_min: int, gamma_max: int, log_mean: torch.Tensor,
                     log_min: torch.Tensor, log_gamma: torch.Tensor, log_n: torch.Tensor) -> None:
    """One chunk's stride decision of the adaptive path on the device
    (da_adapt_chunk_step): the chunk's delta cosines rnd(dense - sparse[rows])
    over its first state[1] anchors, their mean / min into the logs, the next
    stride into state[0] and the next chunk's anchor rows into rows_next.

    dense [B, max_n, H, D] (any strides with rows contiguous), sparse
    [B, S, H, D]; rows / rows_next int64 [max_n] (-1 past the anchors);
    state int32 [2]; cos_work fp32 >= B * (max_n - 1) * H; logs [n_chunks]
    (fp64 mean, fp32 min, int32 stride, int32 anchors)."""
    B, max_n, H, D = dense.shape
    dev = _on_gpu(dense, sparse, rows, state, cos_work, log_mean, log_min, log_gamma, log_n)
    assert sparse.shape[0] == B and sparse.shape[2:] == (H, D) and sparse.dtype == dense.dtype
    assert rows.dtype == torch.int64 and rows.is_contiguous() and rows.numel() == max_n
    assert state.dtype == torch.int32 and state.numel() >= 2
    assert cos_work.dtype == torch.float32 and cos_work.numel() >= B * max(max_n - 1, 1) * H
    assert log_mean.dtype == torch.float64 and log_min.dtype == torch.float32
    assert log_gamma.dtype == torch.int32 and log_n.dtype == torch.int32
    assert trigger in ("absolute", "relative"), trigger
    if rows_next is not None:
        assert rows_next.dtype == torch.int64 and rows_next.is_contiguous() and rows_next.numel() == max_n
    with torch.cuda.device(dev):
        rc = L.lib().da_adapt_chunk_step(
            _ptr(dense), L.I64x3(*dense.stride()[:3]), _ptr(sparse), L.I64x3(*sparse.stride()[:3]),
            int(sparse.shape[1]), _ptr(rows), B, H, D, max_n, _ptr(state), _ptr(cos_work), int(chunk),
            int(next_start), int(next_end), _ptr(rows_next), 0 if trigger == "absolute" else 1,
            float(threshold), float(margin), float(k), int(gamma_min), int(gamma_max),
            _ptr(log_mean), _ptr(log_min), _ptr(log_gamma), _ptr(log_n), _code(dense), _stream(dev))
    L.check(rc, "da_adapt_chunk_step")


def adapt_layer(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, out: torch.Tensor, *,
                s_p: int, window: int, sink: int, sm_scale: float, adapt_chunk: int,
                gamma0: int, gamma_min: int, gamma_max: int, trigger: str, threshold: float,
                margin: float, k_sd: float = 2.0, side_stream: Optional[torch.cuda.Stream] = None,
                q_block: int = Q_BLOCK):
    """The adaptive-stride layer in one library call (da_adapt_layer_fwd):
    per adapt_chunk rows of [0, s_p), kernel (2) over the chunk's anchors at
    its stride, the chunk's delta cosines and next stride on the device, and
    the chunk's broadcast-add in place in `out`; then the dense tail rows
    [s_p, S). With side_stream, the key-sparse pass runs here on it, chunk by
    chunk (out's rows [0, s_p) are written); without, out must already hold
    it. q [B,H,S,D], k/v [B,Hkv,S,D], out [B,S,H,D].

    Returns the per-chunk logs (log_mean fp64, log_min fp32, log_gamma int32,
    log_n int32) on the device; nothing is read back here."""
    B, H, S, D = q.shape
    Hkv = k.shape[1]
    assert k.shape == (B, Hkv, S, D) and v.shape == k.shape, (q.shape, k.shape, v.shape)
    assert q.dtype == k.dtype == v.dtype == out.dtype and out.shape == (B, S, H, D)
    assert out.stride(-1) == 1
    assert trigger in ("absolute", "relative"), trigger
    dev = _on_gpu(q, k, v, out)
    q, k, v = _ready(q), _ready(k), _ready(v)
    nc = -(-s_p // adapt_chunk) if adapt_chunk > 0 else 0
    nb = L.lib().da_adapt_layer_workspace_bytes(B, H, Hkv, S, D, int(s_p), int(adapt_chunk),
                                                int(gamma0), int(gamma_min))
    assert nb > 0, "adaptive layer sizes do not form a launch"
    workspace = torch.empty(nb, dtype=torch.uint8, device=dev)
    n_log = max(nc, 1)
    log_mean = torch.empty(n_log, dtype=torch.float64, device=dev)
    log_min = torch.empty(n_log, dtype=torch.float32, device=dev)
    log_gamma = torch.empty(n_log, dtype=torch.int32, device=dev)
    log_n = torch.empty(n_log, dtype=torch.int32, device=dev)
    with torch.cuda.device(dev):
        rc = L.lib().da_adapt_layer_fwd(
            _ptr(q), _ptr(k), _ptr(v), _ptr(out), B, H, Hkv, S, D,
            L.strides3(q.stride(0), q.stride(1), q.stride(2)),
            L.strides3(k.stride(0), k.stride(1), k.stride(2)),
            L.strides3(v.stride(0), v.stride(1), v.stride(2)),
            L.strides3(out.stride(0), out.stride(2), out.stride(1)),
            int(window), int(sink), int(q_block), float(sm_scale), int(s_p), int(adapt_chunk),
            int(gamma0), int(gamma_min), int(gamma_max), 0 if trigger == "absolute" else 1,
            float(threshold), float(margin), float(k_sd), _ptr(log_mean), _ptr(log_min),
            _ptr(log_gamma), _ptr(log_n), n_log, _ptr(workspace), nb, _code(q), _stream(dev),
            side_stream.cuda_stream if side_stream is not None else None)
    L.check(rc, "da_adapt_layer_fwd")
    return log_mean, log_min, log_gamma, log_n


def anchor_layout(s: int, gamma: int) -> Tuple[int, int, int]:
    """(cut_n, s_p, n_anchor) of delta_forward's fixed-stride layout
    (llama.py:692-693, 711-714): cut_n = s % gamma + max(128, gamma)."""
    cut_n = s % gamma + max(128, gamma)
    s_p = s - cut_n
    n_anchor = -(-s_p // gamma) if s_p > 0 else 0
    return cut_n, s_p, n_anchor


@functools.lru_cache(maxsize=64)
def selected_rows(s: int, gamma: int, device: str) -> torch.Tensor:
    """Anchor rows 0, gamma, ... < s_p followed by the dense tail s_p .. s-1
    (int64, on `device`)."""
    _, s_p, _ = anchor_layout(s, gamma)
    s_p = max(s_p, 0)
    return torch.cat([torch.arange(0, s_p, gamma, dtype=torch.int64),
                      torch.arange(s_p, s, dtype=torch.int64)]).to(device)


def delta_prefill(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, gamma: int,
                  window: int, sink: int, sm_scale: float, mode: str = "delta",
                  out: Optional[torch.Tensor] = None,
                  return_delta: bool = False, fused: bool = True):
    """One delta-attention layer prefill: q [B,H,s,D], k/v [B,Hkv,s,D] (post-RoPE)
    -> [B,s,H,D] (llama.py:659-757).

    mode "sparse-only": the key-sparse output; "recompute": sparse rows with
    the selected rows replaced by dense ones; "delta": sparse + the delta of
    the anchor at or before each row, dense tail rows.
    When s <= cut_n there are no anchors and every row is computed densely.
    return_delta: also return the [B,n_anchor,H,D] anchor deltas (drift telemetry).
    fused (mode "delta"): when the head geometry and gamma allow it
    (gamma | fused_delta_rows(H, Hkv)), kernel (2) runs first and kernel (3) is
    fused into kernel (1)'s epilogue; the result is bit-identical to the
    three-kernel sequence (fused=False).
    """
    assert mode in ("delta", "recompute", "sparse-only"), mode
    assert gamma >= 1
    B, H, s, D = q.shape
    cut_n, s_p, n_anchor = anchor_layout(s, gamma)
    rows = fused_delta_rows(H, k.shape[1])
    if mode == "delta" and s_p > 0 and fused and rows and rows % gamma == 0:
        # kernel (2) first (dense tail into the output, dense anchor rows
        # aside), then kernel (1) with the broadcast-add in its epilogue
        if out is None:
            out = torch.empty((B, s, H, D), device=q.device, dtype=q.dtype)
        idx = selected_rows(s, gamma, str(q.device))
        ws = qsparse_workspace(B, H, k.shape[1], idx.numel(), s, D, q.device)
        dense_sel = torch.empty((B, n_anchor, H, D), device=q.device, dtype=q.dtype)
        qsparse_attention(q, k, v, idx, sm_scale, q_rows=idx, epi=L.DA_EPI_DENSE, out=out,
                          n_anchor=n_anchor, delta=dense_sel, workspace=ws)
        delta = torch.empty_like(dense_sel) if return_delta else None
        sparse_attention_delta(q, k, v, window=window, sink=sink, sm_scale=sm_scale,
                               dense_sel=dense_sel, gamma=gamma, s_p=s_p, out=out,
                               delta_out=delta)
        return (out, delta) if return_delta else out
    out = sparse_attention(q, k, v, window=window, sink=sink, sm_scale=sm_scale, out=out)
    if mode == "sparse-only":
        return (out, None) if return_delta else out
    idx = selected_rows(s, gamma, str(q.device))
    ws = qsparse_workspace(B, H, k.shape[1], idx.numel(), s, D, q.device)
    if mode == "recompute" or s_p <= 0:
        qsparse_attention(q, k, v, idx, sm_scale, q_rows=idx, epi=L.DA_EPI_SCATTER,
                          out=out, workspace=ws)
        return (out, None) if return_delta else out
    delta = torch.empty((B, n_anchor, H, D), device=q.device, dtype=q.dtype)
    qsparse_attention(q, k, v, idx, sm_scale, q_rows=idx, epi=L.DA_EPI_DELTA, out=out,
                      n_anchor=n_anchor, delta=delta, workspace=ws)
    delta_add(out, s_p=s_p, out=out, delta=delta, gamma=gamma)
    return (out, delta) if return_delta else out
