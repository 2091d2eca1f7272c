"""The C-ABI library: it builds, loads, exports every declared symbol, and
rejects bad arguments with the documented codes before touching the GPU."""

import ctypes
import os
import re

import pytest

import conftest  # noqa: F401  (paths)
from delta_attention import _lib as L

HEADER = os.path.join(conftest.REPO, "include", "delta_attn.h")


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(L.LIB_PATH):
        import build_lib
        build_lib.build()
    return L.lib()


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^[a-z][\w\s\*]*?\b(da_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_the_entry_points():
    assert declared_symbols() == sorted(L.EXPORTS)


def test_library_exports_every_declared_symbol(lib):
    for name in declared_symbols():
        assert hasattr(lib, name), name
    assert lib.da_build_target() == b"gfx950"
    blob = open(L.LIB_PATH, "rb").read()
    assert b"gfx950" in blob


def _s3(*v):
    return L.strides3(*v)


def _sparse(lib, **kw):
    a = dict(q=16, k=16, v=16, out=16, B=1, Hq=8, Hkv=2, S=128, D=128,
             qs=(8 * 128 * 128, 128 * 128, 128), ks=(2 * 128 * 128, 128 * 128, 128),
             os_=(128 * 8 * 128, 128, 8 * 128), window=64, sink=4, qb=64, dtype=L.DA_BF16)
    a.update(kw)
    return lib.da_sparse_attn_fwd(ctypes.c_void_p(a["q"]), ctypes.c_void_p(a["k"]),
                                  ctypes.c_void_p(a["v"]), ctypes.c_void_p(a["out"]),
                                  a["B"], a["Hq"], a["Hkv"], a["S"], a["D"],
                                  _s3(*a["qs"]), _s3(*a["ks"]), _s3(*a["ks"]), _s3(*a["os_"]),
                                  a["window"], a["sink"], a["qb"], 0.1, a["dtype"], None)


def test_sparse_rejects_bad_arguments(lib):
    assert _sparse(lib, dtype=7) == L.DA_ERR_DTYPE
    assert _sparse(lib, D=96) == L.DA_ERR_HEAD_DIM
    assert _sparse(lib, D=512) == L.DA_ERR_HEAD_DIM
    assert _sparse(lib, Hq=6, Hkv=4) == L.DA_ERR_INVALID_ARG
    assert _sparse(lib, q=0) == L.DA_ERR_INVALID_ARG
    assert _sparse(lib, q=24) == L.DA_ERR_ALIGNMENT
    assert _sparse(lib, qs=(8 * 128 * 128, 128 * 128, 132)) == L.DA_ERR_ALIGNMENT
    assert _sparse(lib, window=-1) == L.DA_ERR_INVALID_ARG
    assert _sparse(lib, qb=0) == L.DA_ERR_INVALID_ARG
    assert _sparse(lib, S=0) == L.DA_OK          # nothing to do, nothing launched


def test_sparse_rows_rejects_bad_ranges(lib):
    def call(row0, n, **kw):
        a = dict(q=16, D=128, dtype=L.DA_BF16)
        a.update(kw)
        return lib.da_sparse_attn_fwd_rows(
            ctypes.c_void_p(a["q"]), ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16),
            1, 8, 2, 128, a["D"], _s3(8 * 128 * 128, 128 * 128, 128), _s3(2 * 128 * 128, 128 * 128, 128),
            _s3(2 * 128 * 128, 128 * 128, 128), _s3(128 * 8 * 128, 128, 8 * 128),
            64, 4, 64, 0.1, row0, n, a["dtype"], None)
    assert call(-1, 10) == L.DA_ERR_INVALID_ARG
    assert call(0, -1) == L.DA_ERR_INVALID_ARG
    assert call(100, 29) == L.DA_ERR_INVALID_ARG      # past S = 128
    assert call(64, 0) == L.DA_OK                     # nothing to do, nothing launched
    assert call(0, 10, dtype=9) == L.DA_ERR_DTYPE
    assert call(0, 10, D=96) == L.DA_ERR_HEAD_DIM
    assert call(0, 10, q=0) == L.DA_ERR_INVALID_ARG


def test_qsparse_workspace_and_checks(lib):
    ws = lib.da_qsparse_workspace_bytes
    assert ws(1, 32, 8, 2174, 131072, 128) > 0
    assert ws(1, 32, 8, 2174, 131072, 128) >= ws(1, 32, 8, 100, 131072, 128)
    assert ws(1, 32, 8, 10, 100, 96) == 0
    assert ws(1, 6, 4, 10, 100, 128) == 0
    need = ws(1, 8, 2, 64, 1024, 128)
    s3 = _s3(8 * 1024 * 128, 1024 * 128, 128)

    def call(workspace=4096, nbytes=None, epi=L.DA_EPI_OUTPUT, D=128, row_last=16, n_anchor=0, delta=0):
        return lib.da_qsparse_attn_fwd(
            ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16), None,
            ctypes.c_void_p(row_last), 0, 64, 1, 8, 2, 1024, 1024, D, s3, s3, s3,
            ctypes.c_void_p(16), s3, epi, n_anchor, ctypes.c_void_p(delta), s3, 0.1,
            ctypes.c_void_p(workspace), need if nbytes is None else nbytes, L.DA_BF16, None)

    assert call(nbytes=need - 1) == L.DA_ERR_WORKSPACE
    assert call(workspace=0) == L.DA_ERR_WORKSPACE
    assert call(epi=9) == L.DA_ERR_INVALID_ARG
    assert call(D=80) == L.DA_ERR_HEAD_DIM
    assert call(row_last=0) == L.DA_ERR_INVALID_ARG
    assert call(epi=L.DA_EPI_DELTA, n_anchor=65, delta=16) == L.DA_ERR_INVALID_ARG
    assert call(epi=L.DA_EPI_DELTA, n_anchor=4, delta=0) == L.DA_ERR_INVALID_ARG


def test_delta_add_checks(lib):
    s3 = _s3(4096 * 32 * 128, 128, 32 * 128)

    def call(delta=16, dense=0, anchors=0, n=64, gamma=64, s_p=4096, sparse=16, out=32):
        return lib.da_delta_add(ctypes.c_void_p(sparse), s3, ctypes.c_void_p(out), s3,
                                ctypes.c_void_p(delta), s3, ctypes.c_void_p(dense), s3,
                                ctypes.c_void_p(anchors), n, gamma, s_p, 1, 32, 128, L.DA_BF16, None)

    assert call(n=63) == L.DA_ERR_INVALID_ARG                 # too few deltas for s_p / gamma
    assert call(gamma=0) == L.DA_ERR_INVALID_ARG
    assert call(delta=0, dense=16, anchors=0) == L.DA_ERR_INVALID_ARG    # dense form needs anchors
    assert call(delta=0, dense=16, anchors=16, out=16) == L.DA_ERR_INVALID_ARG  # no aliasing
    assert call(delta=8) == L.DA_ERR_ALIGNMENT
    assert call(s_p=0) == L.DA_OK


def test_rope_checks(lib):
    s3 = _s3(128 * 8 * 128, 8 * 128, 128)
    c2 = (ctypes.c_int64 * 2)

    def call(q=16, D=128, dtype=L.DA_BF16, cos=16, cs=(0, 128), S=128, qs=s3, w=0):
        return lib.da_rope_qk(ctypes.c_void_p(q), qs, 8, None, None, 0, 1, S, D,
                              ctypes.c_void_p(cos), ctypes.c_void_p(16), c2(*cs),
                              ctypes.c_void_p(w), None, 1e-6, dtype, None)

    assert call(dtype=5) == L.DA_ERR_DTYPE
    assert call(D=96) == L.DA_ERR_HEAD_DIM
    assert call(D=80) == L.DA_ERR_HEAD_DIM       # the prologue takes 32, 64, 128 and 256
    assert call(cos=0) == L.DA_ERR_INVALID_ARG
    assert call(cs=(0, 64)) == L.DA_ERR_INVALID_ARG          # table rows shorter than D
    assert call(cos=24) == L.DA_ERR_ALIGNMENT
    assert call(q=8) == L.DA_ERR_ALIGNMENT
    assert call(w=8) == L.DA_ERR_ALIGNMENT
    assert call(qs=_s3(128 * 8 * 128, 8 * 128, 100)) == L.DA_ERR_ALIGNMENT
    assert call(S=0) == L.DA_OK


def test_fused_delta_rows_and_checks(lib):
    # gamma must divide 128 whatever the head packing (two heads per 64-row
    # tile for gamma | 64 and an even GQA ratio, else one head per 128 rows)
    for hq, hkv in ((32, 8), (8, 8), (6, 3), (40, 8)):
        assert lib.da_fused_delta_rows(hq, hkv) == 128
    assert lib.da_fused_delta_rows(6, 4) == 0 and lib.da_fused_delta_rows(0, 1) == 0
    s3 = _s3(128 * 32 * 128, 128, 32 * 128)
    q3 = _s3(32 * 4096 * 128, 4096 * 128, 128)
    k3 = _s3(8 * 4096 * 128, 4096 * 128, 128)

    def call(gamma=64, s_p=3968, dense=16, S=4096, Hq=32, Hkv=8, dout=0):
        return lib.da_sparse_attn_delta_fwd(
            ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16),
            1, Hq, Hkv, S, 128, q3, k3, k3, s3, 512, 64, 64, 0.1,
            ctypes.c_void_p(dense), s3, gamma, s_p, ctypes.c_void_p(dout), s3, L.DA_BF16, None)

    assert call(gamma=256, s_p=3840) == L.DA_ERR_INVALID_ARG     # gamma must divide 128
    assert call(gamma=48, s_p=3840) == L.DA_ERR_INVALID_ARG
    assert call(s_p=3900) == L.DA_ERR_INVALID_ARG                # s_p % gamma != 0
    assert call(s_p=4160) == L.DA_ERR_INVALID_ARG                # s_p > S
    assert call(dense=0) == L.DA_ERR_INVALID_ARG
    assert call(Hq=40, gamma=256, s_p=3840) == L.DA_ERR_INVALID_ARG   # 256 does not divide 128
    assert call(dense=8) == L.DA_ERR_ALIGNMENT
    assert call(dout=8) == L.DA_ERR_ALIGNMENT
    assert call(s_p=0) == L.DA_OK
    assert call(S=0, s_p=0) == L.DA_OK


def test_sparse_rows_per_wave_setting(lib):
    # 32 (default) or 64 query rows per wave; anything else is refused and
    # leaves the setting as it was
    assert lib.da_sparse_rows_per_wave() == 32
    for bad in (0, 16, 48, 96, 128, -32):
        assert lib.da_set_sparse_rows_per_wave(bad) == L.DA_ERR_INVALID_ARG
        assert lib.da_sparse_rows_per_wave() == 32
    assert lib.da_set_sparse_rows_per_wave(64) == L.DA_OK
    assert lib.da_sparse_rows_per_wave() == 64
    assert lib.da_set_sparse_rows_per_wave(32) == L.DA_OK
    assert lib.da_sparse_rows_per_wave() == 32


def test_norm_and_swiglu_checks(lib):
    P = ctypes.c_void_p
    assert lib.da_add_rmsnorm(P(16), 4096, None, 0, None, 0, P(16), 4096, P(16), 8, 3000, 1e-5,
                              L.DA_BF16, None) == L.DA_ERR_INVALID_ARG      # unsupported row length
    assert lib.da_add_rmsnorm(P(16), 4096, P(16), 4096, None, 0, P(16), 4096, P(16), 8, 4096, 1e-5,
                              L.DA_BF16, None) == L.DA_ERR_INVALID_ARG      # residual without h
    assert lib.da_add_rmsnorm(P(24), 4096, None, 0, None, 0, P(16), 4096, P(16), 8, 4096, 1e-5,
                              L.DA_BF16, None) == L.DA_ERR_ALIGNMENT
    assert lib.da_add_rmsnorm(P(16), 4096, None, 0, None, 0, P(16), 4096, P(16), 0, 4096, 1e-5,
                              L.DA_BF16, None) == L.DA_OK                   # no rows
    assert lib.da_add_rmsnorm(P(16), 4096, None, 0, None, 0, P(16), 4096, P(16), 8, 4096, 1e-5,
                              9, None) == L.DA_ERR_DTYPE
    assert lib.da_swiglu(P(16), 64, P(16), 64, P(16), 64, 8, 60, L.DA_BF16, None) == L.DA_ERR_INVALID_ARG
    assert lib.da_swiglu(P(16), 64, P(8), 64, P(16), 64, 8, 64, L.DA_BF16, None) == L.DA_ERR_ALIGNMENT
    assert lib.da_swiglu(P(16), 64, P(16), 64, P(16), 64, 0, 64, L.DA_BF16, None) == L.DA_OK


def test_decode_checks(lib):
    P = ctypes.c_void_p
    s3 = _s3(32 * 128, 128, 128)
    k3 = _s3(8 * 8192 * 128, 8192 * 128, 128)
    ws = lib.da_decode_workspace_bytes
    assert ws(1, 32, 8, 8192, 128, 2048, 128) > 0
    assert ws(1, 32, 8, 8192, 128, 2048, 128) < ws(1, 32, 8, 8192, 128, 0, 0) * 4
    assert ws(1, 32, 8, 8192, 96, 0, 0) == 0 and ws(1, 32, 8, 0, 128, 0, 0) == 0
    need = ws(1, 32, 8, 8192, 128, 2048, 128)

    def call(n=8192, window=2048, sink=128, w=16, nbytes=None, D=128):
        return lib.da_decode_attn_fwd(P(16), P(16), P(16), P(16), 1, 32, 8, n, D, s3, k3, k3, s3,
                                      window, sink, 0.1, P(w), need if nbytes is None else nbytes,
                                      L.DA_BF16, None)
    assert call(nbytes=need - 1) == L.DA_ERR_WORKSPACE
    assert call(w=0) == L.DA_ERR_WORKSPACE
    assert call(n=0) == L.DA_ERR_INVALID_ARG
    assert call(window=-1) == L.DA_ERR_INVALID_ARG
    assert call(D=80) == L.DA_ERR_HEAD_DIM


def test_decode_dev_checks(lib):
    """The device-key-count decode entry: its plan and workspace follow
    max_keys, and every refusal happens before a launch."""
    P = ctypes.c_void_p
    s3 = _s3(32 * 128, 128, 128)
    k3 = _s3(8 * 8192 * 128, 8192 * 128, 128)
    need = lib.da_decode_workspace_bytes(1, 32, 8, 8192, 128, 0, 0)

    a3 = s3

    def call(nk=64, max_keys=8192, w=16, nbytes=None, D=128, window=0, add=0):
        return lib.da_decode_attn_fwd_dev(P(16), P(16), P(16), P(16), 1, 32, 8,
                                          P(nk) if nk else None, max_keys, D, s3, k3, k3, s3,
                                          window, 0, 0.1, P(add) if add else None, a3,
                                          P(w), need if nbytes is None else nbytes,
                                          L.DA_BF16, None)
    assert call(nk=0) == L.DA_ERR_INVALID_ARG          # no key-count pointer
    assert call(nk=66) == L.DA_ERR_ALIGNMENT           # int32 needs 4-byte alignment
    assert call(max_keys=0) == L.DA_ERR_INVALID_ARG
    assert call(nbytes=need - 1) == L.DA_ERR_WORKSPACE
    assert call(w=0) == L.DA_ERR_WORKSPACE
    assert call(window=-1) == L.DA_ERR_INVALID_ARG
    assert call(D=80) == L.DA_ERR_HEAD_DIM
    assert call(add=8) == L.DA_ERR_ALIGNMENT            # addend rows 16-byte aligned


def test_decode_noalloc_checks(lib):
    """The no-workspace decode entry refuses bad arguments, and sizes whose
    partials exceed its static scratch, before it looks up the scratch or
    launches anything."""
    P = ctypes.c_void_p
    assert lib.da_decode_scratch_bytes() == 16 << 20

    def call(H=32, Hkv=8, max_keys=8192, D=128, window=0, dtype=L.DA_BF16):
        s3 = _s3(H * D, D, D)
        k3 = _s3(Hkv * max_keys * D, max_keys * D, D)
        return lib.da_decode_attn_fwd_dev_noalloc(P(16), P(16), P(16), P(16), 1, H, Hkv, P(16),
                                                  max_keys, D, s3, k3, k3, s3, window, 0, 0.1,
                                                  None, None, dtype, None)
    assert call(dtype=5) == L.DA_ERR_DTYPE
    assert call(D=80) == L.DA_ERR_HEAD_DIM
    assert call(max_keys=0) == L.DA_ERR_INVALID_ARG
    assert call(window=-1) == L.DA_ERR_INVALID_ARG
    assert call(H=1024, max_keys=131072) == L.DA_ERR_SCRATCH
    need = lib.da_decode_workspace_bytes(1, 1024, 8, 131072, 128, 0, 0)
    assert need > lib.da_decode_scratch_bytes()


def test_anchor_delta_cos_checks(lib):
    P = ctypes.c_void_p
    a3 = _s3(64 * 8 * 128, 8 * 128, 128)

    def call(a=16, n=64, D=128, dtype=L.DA_BF16, cos=16, hist=None, bins=0, lo=-1.0, hi=1.0,
             sparse=None, n_rows=0, s3=None, a_str=a3):
        return lib.da_anchor_delta_cos(P(a), a_str, P(sparse) if sparse else None, s3, None, n_rows,
                                       1, n, 8, D, P(cos), P(hist) if hist else None, bins,
                                       lo, hi, dtype, None)
    assert call(dtype=5) == L.DA_ERR_DTYPE
    assert call(D=96) == L.DA_ERR_HEAD_DIM
    assert call(n=-1) == L.DA_ERR_INVALID_ARG
    assert call(n=1) == L.DA_OK and call(n=0) == L.DA_OK      # no consecutive pair: nothing to do
    assert call(a=0) == L.DA_ERR_INVALID_ARG
    assert call(cos=0) == L.DA_ERR_INVALID_ARG
    assert call(hist=16, bins=0) == L.DA_ERR_INVALID_ARG
    assert call(hist=16, bins=40, lo=1.0, hi=1.0) == L.DA_ERR_INVALID_ARG
    assert call(sparse=16, n_rows=0, s3=a3) == L.DA_ERR_INVALID_ARG
    assert call(sparse=16, n_rows=100, s3=None) == L.DA_ERR_INVALID_ARG
    assert call(a=18) == L.DA_ERR_ALIGNMENT
    assert call(a_str=_s3(64 * 8 * 128, 8 * 128, 127)) == L.DA_ERR_ALIGNMENT


def test_adapt_chunk_step_checks(lib):
    """Refusals of the adaptive stride's device-side chunk step (every check
    precedes the launches; nothing runs on a GPU here)."""
    P = ctypes.c_void_p
    d3 = _s3(64 * 8 * 128, 8 * 128, 128)

    def call(dense=16, sparse=16, rows=16, state=16, cos=16, logs=16, max_n=64, D=128,
             dtype=L.DA_BF16, trigger=0, gmin=16, gmax=128, chunk=0, nxt=(0, 0), rows_next=None,
             n_rows=4096, d_str=d3):
        return lib.da_adapt_chunk_step(
            P(dense) if dense else None, d_str, P(sparse) if sparse else None, d3, n_rows,
            P(rows) if rows else None, 1, 8, D, max_n, P(state) if state else None,
            P(cos) if cos else None, chunk, nxt[0], nxt[1], P(rows_next) if rows_next else None,
            trigger, 0.95, 0.02, 2.0, gmin, gmax,
            P(logs) if logs else None, P(logs) if logs else None, P(logs) if logs else None,
            P(logs) if logs else None, dtype, None)
    assert call(dtype=7) == L.DA_ERR_DTYPE
    assert call(D=80) == L.DA_ERR_HEAD_DIM
    for kw in ({"dense": 0}, {"sparse": 0}, {"rows": 0}, {"state": 0}, {"cos": 0}, {"logs": 0},
               {"max_n": 0}, {"trigger": 2}, {"gmin": 0}, {"gmin": 64, "gmax": 32}, {"chunk": -1},
               {"n_rows": 0}, {"nxt": (4096, 8192)}, {"nxt": (-1, 8), "rows_next": 16}):
        assert call(**kw) == L.DA_ERR_INVALID_ARG, kw
    assert call(dense=18) == L.DA_ERR_ALIGNMENT
    assert call(d_str=_s3(64 * 8 * 128, 8 * 128, 127)) == L.DA_ERR_ALIGNMENT


def test_adapt_layer_sizes_and_checks(lib):
    """The adaptive layer's workspace query (the largest chunk's split plan,
    one chunk of dense rows, the row lists) and its refusals, all of which
    precede any launch or event (nothing runs on a GPU here)."""
    P = ctypes.c_void_p
    B, H, Hkv, S, D = 1, 32, 8, 131072, 128
    s_p = S - 128
    nb = lib.da_adapt_layer_workspace_bytes(B, H, Hkv, S, D, s_p, 4096, 64, 16)
    # at least: 32 chunk row lists of 256 slots, two buffers of a chunk's 256
    # dense rows, the 2046 rows at multiples of 64 computed ahead and their
    # row list, the last chunk's split workspace, the rows-ahead launch's and
    # the tail's
    split = lib.da_qsparse_workspace_bytes_live(B, H, Hkv, 256, 64, s_p, D)
    ahead = lib.da_qsparse_workspace_bytes(B, H, Hkv, 2046, s_p, D)
    tail = lib.da_qsparse_workspace_bytes(B, H, Hkv, 128, S, D)
    least = (32 * 256 * 8 + 2 * B * H * 256 * D * 2 + 2046 * 8 + B * H * 2046 * D * 2
             + split + ahead + tail)
    assert least <= nb < least + 10 * 256 + B * H * 256 * 4
    # adapt_chunk not a multiple of the first stride: no rows ahead
    nb2 = lib.da_adapt_layer_workspace_bytes(B, H, Hkv, S, D, s_p, 4000, 64, 16)
    assert 0 < nb2 < nb - B * H * 2046 * D * 2 - ahead
    # no prefix rows: no chunk, only the tail
    assert lib.da_adapt_layer_workspace_bytes(B, H, Hkv, 128, D, 0, 4096, 64, 16) > 0
    for args in ((B, H, Hkv, S, 80, s_p, 4096, 64, 16), (B, H, 7, S, D, s_p, 4096, 64, 16),
                 (B, H, Hkv, S, D, S, 4096, 64, 16), (B, H, Hkv, S, D, -1, 4096, 64, 16),
                 (B, H, Hkv, S, D, s_p, 0, 64, 16), (B, H, Hkv, S, D, s_p, 4096, 0, 16),
                 (B, H, Hkv, S, D, s_p, 4096, 64, 0), (0, H, Hkv, S, D, s_p, 4096, 64, 16)):
        assert lib.da_adapt_layer_workspace_bytes(*args) == 0, args

    q3 = _s3(H * S * D, S * D, D)
    k3 = _s3(Hkv * S * D, S * D, D)
    o3 = _s3(S * H * D, D, H * D)

    def call(q=16, out=16, ws=256, ws_bytes=nb, logs=16, n_log=32, D=D, dtype=L.DA_BF16,
             trigger=0, gmin=16, gmax=256, o_str=o3, s_p=s_p):
        return lib.da_adapt_layer_fwd(
            P(q) if q else None, P(16), P(16), P(out) if out else None, B, H, Hkv, S, D,
            q3, k3, k3, o_str, 2048, 128, 64, 0.088, s_p, 4096, 64, gmin, gmax, trigger,
            0.95, 0.02, 2.0, P(logs) if logs else None, P(logs) if logs else None,
            P(logs) if logs else None, P(logs) if logs else None, n_log,
            P(ws) if ws else None, ws_bytes, dtype, None, None)
    assert call(dtype=7) == L.DA_ERR_DTYPE
    assert call(D=80) == L.DA_ERR_HEAD_DIM
    for kw in ({"q": 0}, {"out": 0}, {"ws": 0}, {"ws_bytes": nb - 1}, {"logs": 0},
               {"n_log": 31}, {"trigger": 2}, {"gmin": 64, "gmax": 32}, {"s_p": S}):
        assert call(**kw) == L.DA_ERR_INVALID_ARG, kw
    assert call(ws=512 + 16) == L.DA_ERR_ALIGNMENT
    assert call(out=24) == L.DA_ERR_ALIGNMENT
    assert call(o_str=_s3(S * H * D, D, H * D + 4)) == L.DA_ERR_ALIGNMENT


def test_qsparse_live_plan_sizes(lib):
    """The live-rows plan: the grid (and the workspace's item count) covers
    all n slots, the splits per row tile follow n_live rows; n_live >= n is the
    plain plan, n_live < 1 is refused."""
    plain = lib.da_qsparse_workspace_bytes(1, 32, 8, 256, 131072, 128)
    assert lib.da_qsparse_workspace_bytes_live(1, 32, 8, 256, 256, 131072, 128) == plain
    assert lib.da_qsparse_workspace_bytes_live(1, 32, 8, 256, 1000, 131072, 128) == plain
    assert lib.da_qsparse_workspace_bytes_live(1, 32, 8, 256, 0, 131072, 128) == 0
    # 64 live rows of 256: the short-list plan's splits over all 8 row tiles per kv head
    live = lib.da_qsparse_workspace_bytes_live(1, 32, 8, 256, 64, 131072, 128)
    small = lib.da_qsparse_workspace_bytes(1, 32, 8, 64, 131072, 128)
    assert live == 4 * small


def test_split_plans_refuse_grid_overflow(lib):
    # a selected-rows launch whose work items would not fit a 32-bit grid
    assert lib.da_qsparse_workspace_bytes(1, 32, 8, 2_000_000_000, 131072, 128) == 0
    assert lib.da_qsparse_workspace_bytes(1, 32, 8, 2174, 131072, 128) > 0


def test_bwd_rows_per_chunk_setting(lib):
    """The dK/dV rows-per-item cap: positive multiples of 32 up to 2^20, 0 for
    the default (8192); read when a plan is made, so a smaller cap cuts the
    key blocks into more items, whose partials the workspace holds."""
    B, H, Hkv, S, D = 1, 8, 2, 4096, 128
    base = lib.da_sparse_attn_bwd_workspace_bytes(B, H, Hkv, S, D, 2048, 16, 64)
    base_rows = lib.da_qsparse_attn_bwd_workspace_bytes(B, H, Hkv, 1000, S, D)
    for bad in (-32, 16, 33, 100, (1 << 20) + 32):
        assert lib.da_set_bwd_rows_per_chunk(bad) == L.DA_ERR_INVALID_ARG
    try:
        assert lib.da_set_bwd_rows_per_chunk(64) == L.DA_OK
        assert lib.da_sparse_attn_bwd_workspace_bytes(B, H, Hkv, S, D, 2048, 16, 64) > base
        assert lib.da_qsparse_attn_bwd_workspace_bytes(B, H, Hkv, 1000, S, D) > base_rows
    finally:
        assert lib.da_set_bwd_rows_per_chunk(0) == L.DA_OK
    assert lib.da_sparse_attn_bwd_workspace_bytes(B, H, Hkv, S, D, 2048, 16, 64) == base
    assert lib.da_qsparse_attn_bwd_workspace_bytes(B, H, Hkv, 1000, S, D) == base_rows


def test_training_entry_checks(lib):
    """The training-path entries: workspace sizes, and every refusal happens
    before a launch (null pointers, head_dim, dtype, row alignment, lse
    alignment, workspace, composition stride rules)."""
    P = ctypes.c_void_p
    B, H, Hkv, S, D = 1, 8, 2, 1024, 128
    q3 = _s3(H * S * D, S * D, D)
    k3 = _s3(Hkv * S * D, S * D, D)
    o3 = _s3(S * H * D, D, H * D)
    need = lib.da_sparse_attn_bwd_workspace_bytes(B, H, Hkv, S, D, 256, 16, 64)
    assert need > 0
    assert lib.da_sparse_attn_bwd_workspace_bytes(B, H, 3, S, D, 256, 16, 64) == 0   # H % Hkv
    assert lib.da_sparse_attn_bwd_workspace_bytes(B, H, Hkv, S, 80, 256, 16, 64) == 0
    # sink blocks are cut into row chunks: more sinks, more partial slots
    assert lib.da_sparse_attn_bwd_workspace_bytes(B, H, Hkv, S, D, 256, 512, 64) > need
    nr = lib.da_qsparse_attn_bwd_workspace_bytes(B, H, Hkv, 200, S, D)
    assert nr > 0 and lib.da_qsparse_attn_bwd_workspace_bytes(B, H, Hkv, 0, S, D) == 0

    def sparse(q=16, lse=16, D=D, dtype=L.DA_BF16, ws=16, nbytes=None, q_block=64, k_row=None):
        kk = k3 if k_row is None else _s3(Hkv * S * D, S * D, k_row)
        return lib.da_sparse_attn_bwd(P(q) if q else None, P(16), P(16), P(16), P(16),
                                      P(lse) if lse else None, P(16), P(16), P(16),
                                      B, H, Hkv, S, D, q3, kk, kk, o3, o3, q3, k3, k3,
                                      256, 16, q_block, 0.1, 0, P(ws) if ws else None,
                                      need if nbytes is None else nbytes, dtype, None)
    assert sparse(q=0) == L.DA_ERR_INVALID_ARG
    assert sparse(lse=0) == L.DA_ERR_INVALID_ARG
    assert sparse(lse=18) == L.DA_ERR_ALIGNMENT
    assert sparse(q=24) == L.DA_ERR_ALIGNMENT
    assert sparse(D=80) == L.DA_ERR_HEAD_DIM
    assert sparse(D=256) == L.DA_ERR_HEAD_DIM    # the backward takes 32, 64 and 128
    assert lib.da_sparse_attn_bwd_workspace_bytes(B, H, Hkv, S, 256, 256, 16, 64) == 0
    assert sparse(dtype=7) == L.DA_ERR_DTYPE
    assert sparse(q_block=0) == L.DA_ERR_INVALID_ARG
    assert sparse(k_row=1 << 23) == L.DA_ERR_INVALID_ARG     # row offsets beyond 32 bits
    assert sparse(ws=0) == L.DA_ERR_WORKSPACE
    assert sparse(nbytes=need - 1) == L.DA_ERR_WORKSPACE

    def rows(rl=16, n=200, nbytes=None):
        return lib.da_qsparse_attn_bwd(P(16), P(16), P(16), P(16), P(16), P(16),
                                       P(16), P(rl) if rl else None, n, P(16), P(16), P(16),
                                       B, H, Hkv, S, S, D, q3, k3, k3, o3, o3, q3, k3, k3,
                                       0.1, 1, P(16), nr if nbytes is None else nbytes,
                                       L.DA_BF16, None)
    assert rows(rl=0) == L.DA_ERR_INVALID_ARG
    assert rows(n=0) == L.DA_ERR_INVALID_ARG
    assert rows(nbytes=nr - 1) == L.DA_ERR_WORKSPACE

    def compose(gamma=64, s_p=896, D=D, g=16):
        return lib.da_delta_compose_bwd(P(g), o3, P(16), o3, P(16), o3, B, H, S, D, gamma, s_p,
                                        1.0, 0, L.DA_BF16, None)
    assert compose(s_p=900) == L.DA_ERR_INVALID_ARG        # s_p % gamma
    assert compose(s_p=S + 64) == L.DA_ERR_INVALID_ARG
    assert compose(gamma=0) == L.DA_ERR_INVALID_ARG
    assert compose(D=48) == L.DA_ERR_HEAD_DIM
    assert compose(g=8) == L.DA_ERR_ALIGNMENT

    # forward with row statistics: lse required and 4-byte aligned
    f = lib.da_sparse_attn_fwd_lse(P(16), P(16), P(16), P(16), B, H, Hkv, S, D, q3, k3, k3, o3,
                                   256, 16, 64, 0.1, None, L.DA_BF16, None)
    assert f == L.DA_ERR_INVALID_ARG
    f = lib.da_qsparse_attn_fwd_lse(P(16), P(16), P(16), P(16), P(16), 0, 10, B, H, Hkv, S, S, D,
                                    q3, k3, k3, P(16), q3, P(18), 0.1, P(16), 1 << 30,
                                    L.DA_BF16, None)
    assert f == L.DA_ERR_ALIGNMENT


def test_rope_append_checks(lib):
    """da_rope_qk_append refuses bad arguments before a launch."""
    P = ctypes.c_void_p
    x3 = _s3(12 * 128, 12 * 128, 128)
    c3 = _s3(40 * 2 * 128, 2 * 128, 128)
    cs = (ctypes.c_int64 * 2)(0, 128)

    def call(pos=16, D=128, dtype=L.DA_BF16, v=16, kc=16, cos=16, max_len=40):
        return lib.da_rope_qk_append(P(16), x3, 8, P(16), x3, 2, P(v) if v else None, x3, 1, D,
                                     P(cos) if cos else None, P(16), cs, None, None, 1e-6,
                                     P(kc) if kc else None, c3, P(16), c3, max_len,
                                     P(pos) if pos else None, dtype, None)
    assert call(max_len=0) == L.DA_ERR_INVALID_ARG     # the caches' row count
    assert call(max_len=-5) == L.DA_ERR_INVALID_ARG
    assert call(pos=0) == L.DA_ERR_INVALID_ARG
    assert call(pos=20) == L.DA_ERR_ALIGNMENT          # int64 position
    assert call(v=0) == L.DA_ERR_INVALID_ARG
    assert call(kc=0) == L.DA_ERR_INVALID_ARG
    assert call(kc=24) == L.DA_ERR_ALIGNMENT
    assert call(cos=0) == L.DA_ERR_INVALID_ARG
    assert call(D=96) == L.DA_ERR_HEAD_DIM
    assert call(dtype=3) == L.DA_ERR_DTYPE
