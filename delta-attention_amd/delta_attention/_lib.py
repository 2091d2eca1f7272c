"""ctypes binding of libdelta_attn.so (the C ABI declared in include/delta_attn.h).

The library is the only compute path: there is no fallback. If it is missing
or fails to load, every op raises ExtensionMissing.
"""

from __future__ import annotations

import ctypes
import os
import threading

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libdelta_attn.so")

DA_OK = 0
DA_ERR_INVALID_ARG = -1
DA_ERR_HEAD_DIM = -2
DA_ERR_DTYPE = -3
DA_ERR_ALIGNMENT = -4
DA_ERR_WORKSPACE = -5
DA_ERR_LAUNCH = -6
DA_ERR_SCRATCH = -7

DA_BF16 = 0
DA_FP16 = 1

DA_EPI_OUTPUT = 0
DA_EPI_DELTA = 1
DA_EPI_SCATTER = 2
DA_EPI_DENSE = 3

EXPORTS = (
    "da_sparse_attn_fwd",
    "da_sparse_attn_delta_fwd",
    "da_fused_delta_rows",
    "da_qsparse_workspace_bytes",
    "da_qsparse_attn_fwd",
    "da_delta_add",
    "da_decode_workspace_bytes",
    "da_decode_attn_fwd",
    "da_decode_attn_fwd_dev",
    "da_rope_qk",
    "da_add_rmsnorm",
    "da_swiglu",
    "da_anchor_delta_cos",
    "da_sparse_attn_fwd_lse",
    "da_qsparse_attn_fwd_lse",
    "da_sparse_attn_bwd_workspace_bytes",
    "da_qsparse_attn_bwd_workspace_bytes",
    "da_sparse_attn_bwd",
    "da_qsparse_attn_bwd",
    "da_delta_compose_bwd",
    "da_rope_qk_append",
    "da_build_target",
    "da_decode_scratch_bytes",
    "da_decode_attn_fwd_dev_noalloc",
    "da_adapt_chunk_step",
    "da_qsparse_workspace_bytes_live",
    "da_qsparse_attn_fwd_live",
    "da_sparse_attn_fwd_rows",
    "da_adapt_layer_workspace_bytes",
    "da_adapt_layer_fwd",
    "da_set_sparse_rows_per_wave",
    "da_sparse_rows_per_wave",
    "da_set_bwd_rows_per_chunk",
)

_ERR_TEXT = {
    DA_ERR_INVALID_ARG: "invalid argument (shape, stride, range or null pointer)",
    DA_ERR_HEAD_DIM: "unsupported head_dim",
    DA_ERR_DTYPE: "unsupported dtype (bfloat16 and float16 are supported)",
    DA_ERR_ALIGNMENT: "tensor rows must be 16-byte aligned (strides multiple of 8 elements)",
    DA_ERR_WORKSPACE: "workspace missing or too small",
    DA_ERR_LAUNCH: "kernel launch failed",
    DA_ERR_SCRATCH: "sizes need more than the library's static scratch holds",
}


class ExtensionMissing(RuntimeError):
    """libdelta_attn.so is not built or cannot be loaded."""


_lib = None
_lib_lock = threading.Lock()

I64x3 = ctypes.c_int64 * 3
_vp = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64
_f = ctypes.c_float
_sz = ctypes.c_size_t
_p3 = ctypes.POINTER(ctypes.c_int64)


def lib() -> ctypes.CDLL:
    """Load the library once (thread-safe); raise ExtensionMissing if it is
    not there or lacks an entry point of this binding (a stale build)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lib_lock:
        if _lib is None:
            _lib = _load()
    return _lib


def _load() -> ctypes.CDLL:
    if not os.path.exists(LIB_PATH):
        raise ExtensionMissing(
            f"{LIB_PATH} is not built: run `python delta-attention_amd/build_lib.py` "
            "(or __graft_entry__.build()) first")
    try:
        L = ctypes.CDLL(LIB_PATH)
    except OSError as e:  # pragma: no cover - depends on the machine
        raise ExtensionMissing(f"cannot load {LIB_PATH}: {e}") from e
    missing = [name for name in EXPORTS if not hasattr(L, name)]
    if missing:
        raise ExtensionMissing(f"{LIB_PATH} lacks {', '.join(missing)}: rebuild it "
                               "(`python delta-attention_amd/build_lib.py`)")
    L.da_sparse_attn_fwd.restype = _i
    L.da_sparse_attn_fwd.argtypes = [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i,
                                     _p3, _p3, _p3, _p3, _i, _i, _i, _f, _i, _vp]
    L.da_sparse_attn_delta_fwd.restype = _i
    L.da_sparse_attn_delta_fwd.argtypes = [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i,
                                           _p3, _p3, _p3, _p3, _i, _i, _i, _f,
                                           _vp, _p3, _i, _i, _vp, _p3, _i, _vp]
    L.da_fused_delta_rows.restype = _i
    L.da_fused_delta_rows.argtypes = [_i, _i]
    L.da_set_sparse_rows_per_wave.restype = _i
    L.da_set_sparse_rows_per_wave.argtypes = [_i]
    L.da_sparse_rows_per_wave.restype = _i
    L.da_sparse_rows_per_wave.argtypes = []
    L.da_set_bwd_rows_per_chunk.restype = _i
    L.da_set_bwd_rows_per_chunk.argtypes = [_i]
    L.da_qsparse_workspace_bytes.restype = _sz
    L.da_qsparse_workspace_bytes.argtypes = [_i, _i, _i, _i, _i, _i]
    L.da_qsparse_attn_fwd.restype = _i
    L.da_qsparse_attn_fwd.argtypes = [_vp, _vp, _vp, _vp, _vp, _i64,
                                      _i, _i, _i, _i, _i, _i, _i,
                                      _p3, _p3, _p3, _vp, _p3,
                                      _i, _i, _vp, _p3, _f, _vp, _sz, _i, _vp]
    L.da_decode_workspace_bytes.restype = _sz
    L.da_decode_workspace_bytes.argtypes = [_i, _i, _i, _i, _i, _i, _i]
    L.da_decode_attn_fwd.restype = _i
    L.da_decode_attn_fwd.argtypes = [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i,
                                     _p3, _p3, _p3, _p3, _i, _i, _f, _vp, _sz, _i, _vp]
    L.da_decode_attn_fwd_dev.restype = _i
    L.da_decode_attn_fwd_dev.argtypes = [_vp, _vp, _vp, _vp, _i, _i, _i, _vp, _i, _i,
                                         _p3, _p3, _p3, _p3, _i, _i, _f, _vp, _p3,
                                         _vp, _sz, _i, _vp]
    L.da_delta_add.restype = _i
    L.da_delta_add.argtypes = [_vp, _p3, _vp, _p3, _vp, _p3, _vp, _p3, _vp,
                               _i, _i, _i, _i, _i, _i, _i, _vp]
    L.da_rope_qk.restype = _i
    L.da_rope_qk.argtypes = [_vp, _p3, _i, _vp, _p3, _i, _i, _i, _i, _vp, _vp,
                             ctypes.POINTER(ctypes.c_int64), _vp, _vp, _f, _i, _vp]
    L.da_add_rmsnorm.restype = _i
    L.da_add_rmsnorm.argtypes = [_vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _i, _f,
                                 _i, _vp]
    L.da_swiglu.restype = _i
    L.da_swiglu.argtypes = [_vp, _i64, _vp, _i64, _vp, _i64, _i64, _i, _i, _vp]
    L.da_anchor_delta_cos.restype = _i
    L.da_anchor_delta_cos.argtypes = [_vp, _p3, _vp, _p3, _vp, _i64, _i, _i, _i, _i,
                                      _vp, _vp, _i, _f, _f, _i, _vp]
    L.da_sparse_attn_fwd_lse.restype = _i
    L.da_sparse_attn_fwd_lse.argtypes = [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i,
                                         _p3, _p3, _p3, _p3, _i, _i, _i, _f, _vp, _i, _vp]
    L.da_qsparse_attn_fwd_lse.restype = _i
    L.da_qsparse_attn_fwd_lse.argtypes = [_vp, _vp, _vp, _vp, _vp, _i64, _i, _i, _i, _i, _i, _i,
                                          _i, _p3, _p3, _p3, _vp, _p3, _vp, _f, _vp, _sz, _i, _vp]
    L.da_sparse_attn_bwd_workspace_bytes.restype = _sz
    L.da_sparse_attn_bwd_workspace_bytes.argtypes = [_i, _i, _i, _i, _i, _i, _i, _i]
    L.da_qsparse_attn_bwd_workspace_bytes.restype = _sz
    L.da_qsparse_attn_bwd_workspace_bytes.argtypes = [_i, _i, _i, _i, _i, _i]
    L.da_sparse_attn_bwd.restype = _i
    L.da_sparse_attn_bwd.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                     _i, _i, _i, _i, _i, _p3, _p3, _p3, _p3, _p3, _p3, _p3, _p3,
                                     _i, _i, _i, _f, _i, _vp, _sz, _i, _vp]
    L.da_qsparse_attn_bwd.restype = _i
    L.da_qsparse_attn_bwd.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i,
                                      _vp, _vp, _vp, _i, _i, _i, _i, _i, _i,
                                      _p3, _p3, _p3, _p3, _p3, _p3, _p3, _p3,
                                      _f, _i, _vp, _sz, _i, _vp]
    L.da_delta_compose_bwd.restype = _i
    L.da_delta_compose_bwd.argtypes = [_vp, _p3, _vp, _p3, _vp, _p3, _i, _i, _i, _i, _i, _i,
                                       _f, _i, _i, _vp]
    L.da_rope_qk_append.restype = _i
    L.da_rope_qk_append.argtypes = [_vp, _p3, _i, _vp, _p3, _i, _vp, _p3, _i, _i, _vp, _vp,
                                    _vp, _vp, _vp, _f, _vp, _p3, _vp, _p3, _i64, _vp, _i, _vp]
    L.da_decode_scratch_bytes.restype = _sz
    L.da_decode_scratch_bytes.argtypes = []
    L.da_decode_attn_fwd_dev_noalloc.restype = _i
    L.da_decode_attn_fwd_dev_noalloc.argtypes = [_vp, _vp, _vp, _vp, _i, _i, _i, _vp, _i, _i,
                                                 _p3, _p3, _p3, _p3, _i, _i, _f, _vp, _p3,
                                                 _i, _vp]
    L.da_qsparse_workspace_bytes_live.restype = _sz
    L.da_qsparse_workspace_bytes_live.argtypes = [_i, _i, _i, _i, _i, _i, _i]
    L.da_qsparse_attn_fwd_live.restype = _i
    L.da_qsparse_attn_fwd_live.argtypes = [_vp, _vp, _vp, _vp, _vp, _i64, _i, _i, _vp,
                                           _i, _i, _i, _i, _i, _i,
                                           _p3, _p3, _p3, _vp, _p3, _f, _vp, _sz, _i, _vp]
    L.da_sparse_attn_fwd_rows.restype = _i
    L.da_sparse_attn_fwd_rows.argtypes = [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i,
                                          _p3, _p3, _p3, _p3, _i, _i, _i, _f, _i, _i, _i, _vp]
    L.da_adapt_chunk_step.restype = _i
    L.da_adapt_chunk_step.argtypes = [_vp, _p3, _vp, _p3, _i64, _vp, _i, _i, _i, _i,
                                      _vp, _vp, _i, _i, _i, _vp,
                                      _i, ctypes.c_double, ctypes.c_double, ctypes.c_double, _i, _i,
                                      _vp, _vp, _vp, _vp, _i, _vp]
    _d = ctypes.c_double
    L.da_adapt_layer_workspace_bytes.restype = _sz
    L.da_adapt_layer_workspace_bytes.argtypes = [_i, _i, _i, _i, _i, _i, _i, _i, _i]
    L.da_adapt_layer_fwd.restype = _i
    L.da_adapt_layer_fwd.argtypes = [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i,
                                     _p3, _p3, _p3, _p3, _i, _i, _i, _f,
                                     _i, _i, _i, _i, _i, _i, _d, _d, _d,
                                     _vp, _vp, _vp, _vp, _i, _vp, _sz, _i, _vp, _vp]
    L.da_build_target.restype = ctypes.c_char_p
    L.da_build_target.argtypes = []
    return L


def check(rc: int, what: str) -> None:
    """Map a DA_ERR_* code to the exception the reference raises for it:
    argument problems are AssertionError (the reference asserts, e.g.
    delta_kernel.py:267-268, 287), launch failures RuntimeError."""
    if rc == DA_OK:
        return
    msg = f"{what}: {_ERR_TEXT.get(rc, 'error')} (code {rc})"
    if rc == DA_ERR_LAUNCH:
        raise RuntimeError(msg)
    raise AssertionError(msg)


def strides3(*s: int):
    return I64x3(*[int(x) for x in s])
