"""da_decode_attn_fwd_dev_noalloc: the decode row with its split-KV partials in
the library's static device scratch instead of a caller workspace. Called
through the C ABI and compared with da_decode_attn_fwd_dev (same plan, same
kernels: bit for bit) on consecutive calls, the second one smaller, so that
the second call runs over the first call's leftovers in the scratch."""

import ctypes

import pytest
import torch

from delta_attention import _lib as L

pytestmark = pytest.mark.gpu


def _s3(t, a, b, c):
    return L.strides3(t.stride(a), t.stride(b), t.stride(c))


def _inputs(B, H, Hkv, cap, D, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, 1, D, generator=g).to(torch.bfloat16).cuda()
    k = torch.randn(B, Hkv, cap, D, generator=g).to(torch.bfloat16).cuda()
    v = torch.randn(B, Hkv, cap, D, generator=g).to(torch.bfloat16).cuda()
    add = torch.randn(B, H, 1, D, generator=g).to(torch.bfloat16).cuda()
    return q, k, v, add


def _call(lib, q, k, v, nk, cap, window, sink, add, ws=None):
    B, H, _, D = q.shape
    Hkv = k.shape[1]
    out = torch.full_like(q, float("nan"))
    P = ctypes.c_void_p
    strides = (_s3(q, 0, 1, 2), _s3(k, 0, 1, 2), _s3(v, 0, 1, 2), _s3(out, 0, 1, 2))
    a_ptr = P(add.data_ptr()) if add is not None else None
    a_str = _s3(add, 0, 1, 2) if add is not None else None
    stream = P(torch.cuda.current_stream().cuda_stream)
    if ws is None:
        rc = lib.da_decode_attn_fwd_dev_noalloc(
            P(q.data_ptr()), P(k.data_ptr()), P(v.data_ptr()), P(out.data_ptr()), B, H, Hkv,
            P(nk.data_ptr()), cap, D, *strides, window, sink, D ** -0.5, a_ptr, a_str,
            L.DA_BF16, stream)
    else:
        rc = lib.da_decode_attn_fwd_dev(
            P(q.data_ptr()), P(k.data_ptr()), P(v.data_ptr()), P(out.data_ptr()), B, H, Hkv,
            P(nk.data_ptr()), cap, D, *strides, window, sink, D ** -0.5, a_ptr, a_str,
            P(ws.data_ptr()), ws.numel(), L.DA_BF16, stream)
    assert rc == L.DA_OK, rc
    return out


@pytest.mark.parametrize("first,second", [
    # (B, H, Hkv, capacity, keys, D, window, sink, with addend)
    ((1, 32, 8, 131072, 131072, 128, 0, 0, False), (1, 32, 8, 8192, 5000, 128, 2048, 128, True)),
    ((2, 40, 8, 65536, 40000, 128, 4096, 64, True), (1, 8, 2, 3000, 1, 64, 256, 16, False)),
])
def test_noalloc_decode_matches_workspace_entry(gpu, first, second):
    lib = L.lib()
    assert lib.da_decode_scratch_bytes() == 16 << 20
    for i, (B, H, Hkv, cap, n, D, window, sink, with_add) in enumerate((first, second)):
        q, k, v, add = _inputs(B, H, Hkv, cap, D, seed=100 + i)
        add = add if with_add else None
        nk = torch.full((1,), n, dtype=torch.int32, device="cuda")
        need = lib.da_decode_workspace_bytes(B, H, Hkv, cap, D, window, sink)
        assert 0 < need <= lib.da_decode_scratch_bytes()
        ws = torch.empty(need, dtype=torch.uint8, device="cuda")
        ref = _call(lib, q, k, v, nk, cap, window, sink, add, ws=ws)
        got = _call(lib, q, k, v, nk, cap, window, sink, add)
        torch.cuda.synchronize()
        assert torch.isfinite(got).all()
        assert torch.equal(got, ref), (i, (got.float() - ref.float()).abs().max().item())


def test_noalloc_decode_refuses_sizes_past_the_scratch(gpu):
    """GQA 128 x 8 KV heads at 131072 keys needs more partials than the 16 MiB
    scratch holds: refused on the host before any launch. The call gets real
    device buffers of the shapes it names (q, out [1, 1024, 1, 128], k/v
    [1, 8, 131072, 128], the key count), so that only the scratch size is out
    of range."""
    lib = L.lib()
    B, H, Hkv, cap, D = 1, 1024, 8, 131072, 128
    need = lib.da_decode_workspace_bytes(B, H, Hkv, cap, D, 0, 0)
    assert need > lib.da_decode_scratch_bytes()
    q = torch.zeros(B, H, 1, D, dtype=torch.bfloat16, device="cuda")
    out = torch.empty_like(q)
    k = torch.zeros(B, Hkv, cap, D, dtype=torch.bfloat16, device="cuda")
    v = torch.zeros_like(k)
    nk = torch.full((1,), cap, dtype=torch.int32, device="cuda")
    P = ctypes.c_void_p
    s3 = L.strides3(H * D, D, D)
    k3 = L.strides3(Hkv * cap * D, cap * D, D)
    rc = lib.da_decode_attn_fwd_dev_noalloc(P(q.data_ptr()), P(k.data_ptr()), P(v.data_ptr()),
                                            P(out.data_ptr()), B, H, Hkv, P(nk.data_ptr()), cap, D,
                                            s3, k3, k3, s3, 0, 0, 0.1, None, None, L.DA_BF16,
                                            None)
    torch.cuda.synchronize()
    assert rc == L.DA_ERR_SCRATCH
