"""The online softmax's lazy rescale under inputs that move the running max a
lot: key norms that grow along the sequence (the max rises tile after tile),
rare outlier keys whose scores jump far above everything before them, and
wide-range inputs. The running max of a row only moves when a tile's max
exceeds it by more than 40 (log2 domain; 15 for fp16, whose packed
probabilities must stay below 65504), per row, and the kernels' first pass
takes no per-tile row max at all: a workgroup with a row whose max would have
moved runs its tiles again with every max taken. These inputs send workgroups
through that second pass in every kernel: kernel (1), kernel (2) (split,
merged), the fused layer and the decode rows, each against the oracle's exact
softmax (delta_kernel.py:71-80 is the online-softmax reference), and rows keep
the same bits whichever rows share their workgroup."""

import numpy as np
import pytest
import torch

from helpers import assert_close, np64
from oracle import delta_oracle as O

pytestmark = pytest.mark.gpu


def _inputs(kind, B, H, Hkv, S, D, seed, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, S, D, generator=g)
    k = torch.randn(B, Hkv, S, D, generator=g)
    v = torch.randn(B, Hkv, S, D, generator=g)
    if kind == "growing":
        # key norms grow 12x along the sequence: later tiles' maxima keep
        # exceeding the running max
        k = k * torch.linspace(1.0, 12.0, S)[None, None, :, None]
    elif kind == "outliers":
        # ~1 % of keys aligned with every query direction at 40x scale: their
        # scores jump far above the running max wherever they appear
        idx = torch.randperm(S, generator=g)[: max(S // 100, 1)]
        k[:, :, idx] = k[:, :, idx] * 40.0
    elif kind == "wide":
        q, k = q * 4.0, k * 4.0
    return (x.to(dtype).cuda() for x in (q, k, v))


KINDS = ["growing", "outliers", "wide"]


@pytest.mark.parametrize("kind", KINDS)
def test_rescale_key_sparse(gpu, rows_per_wave, kind):
    from delta_attention import ops
    q, k, v = _inputs(kind, 1, 8, 2, 1500, 128, seed=41)
    scale = 128 ** -0.5
    got = ops.sparse_attention(q, k, v, window=512, sink=16, sm_scale=scale)
    torch.cuda.synchronize()
    ref = O.sparse_attention(np64(q), np64(k), np64(v), 512, 16, scale)
    assert_close(np64(got), ref, what=f"key-sparse {kind}")


@pytest.mark.parametrize("kind", KINDS)
def test_rescale_query_sparse(gpu, kind):
    from delta_attention.delta_kernel import attention
    q, k, v = _inputs(kind, 1, 8, 2, 3000, 64, seed=42)
    rows = np.arange(0, 3000, 37)
    scale = 64 ** -0.5
    got = attention(q[:, :, rows], k, v, torch.from_numpy(rows)[None].cuda(), scale)
    torch.cuda.synchronize()
    ref = O.qsparse_attention(np64(q)[:, :, rows], np64(k), np64(v), rows, scale)
    assert_close(np64(got), ref, what=f"query-sparse {kind}")


@pytest.mark.parametrize("kind", KINDS)
def test_rescale_fused_layer(gpu, rows_per_wave, kind):
    from delta_attention import ops
    q, k, v = _inputs(kind, 1, 8, 2, 1300, 128, seed=43)
    scale = 128 ** -0.5
    a = ops.delta_prefill(q, k, v, gamma=64, window=256, sink=16, sm_scale=scale)
    b = ops.delta_prefill(q, k, v, gamma=64, window=256, sink=16, sm_scale=scale, fused=False)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    ref = O.delta_forward(np64(q), np64(k), np64(v), 64, 256, 16, scale)
    # These peaky softmaxes give outputs near single V rows (|out| up to ~4),
    # where one bf16 ulp is 0.016-0.03 and the delta composition rounds three
    # times in bf16 (as the reference's tensor ops do): the absolute bound
    # scales with the output magnitude; the cosine gate is unchanged.
    atol = 2e-2 * max(1.0, float(np.abs(ref).max()) / 2)
    assert_close(np64(a), ref, atol=atol, what=f"fused layer {kind}")


@pytest.mark.parametrize("kind", KINDS)
def test_rescale_decode(gpu, kind):
    from delta_attention import ops
    q, k, v = _inputs(kind, 1, 8, 2, 6000, 128, seed=44)
    q = q[:, :, -1:].contiguous()
    scale = 128 ** -0.5
    for window, sink in ((0, 0), (1024, 64)):
        got = ops.decode_attention(q, k, v, window=window, sink=sink, sm_scale=scale)
        torch.cuda.synchronize()
        ref = O.decode_row(np64(q), np64(k), np64(v), window, sink, scale)
        assert_close(np64(got), ref, what=f"decode {kind} w{window}")


@pytest.mark.parametrize("kind", KINDS)
def test_rescale_bits_independent_of_packing(gpu, kind):
    """GQA 4 packs two heads per key-sparse tile and four per query-sparse
    tile; the same heads expanded to GQA 1 pack one. A row that needs its max
    moved sends its whole workgroup through the exact pass, so the other rows
    of that workgroup change pass with the packing: their bits must not."""
    from delta_attention import ops
    from delta_attention.delta_kernel import attention
    from delta_attention.llama import repeat_kv
    q, k, v = _inputs(kind, 1, 8, 2, 1500, 128, seed=45)
    ke, ve = repeat_kv(k, 4), repeat_kv(v, 4)
    scale = 128 ** -0.5
    a = ops.sparse_attention(q, k, v, window=512, sink=16, sm_scale=scale)
    b = ops.sparse_attention(q, ke, ve, window=512, sink=16, sm_scale=scale)
    assert torch.equal(a, b)
    rows = np.arange(0, 1500, 37)
    rt = torch.from_numpy(rows)[None].cuda()
    c = attention(q[:, :, rows], k, v, rt, scale)
    d = attention(q[:, :, rows], ke, ve, rt, scale)
    assert torch.equal(c, d)
    ref = O.qsparse_attention(np64(q)[:, :, rows], np64(k), np64(v), rows, scale)
    assert_close(np64(c), ref, what=f"query-sparse packing {kind}")


@pytest.mark.parametrize("kind", ["growing", "outliers"])
def test_rescale_fp16(gpu, rows_per_wave, kind):
    """fp16 inputs whose scores jump by far more than 2^16 in the exponential
    (outlier keys at 40x): with a lazy-rescale bound above 16 the packed fp16
    probabilities would overflow to inf. Kernel (1), kernel (2) and the decode
    rows against the oracle."""
    from delta_attention import ops
    from delta_attention.delta_kernel import attention
    q, k, v = _inputs(kind, 1, 8, 2, 1500, 128, seed=46, dtype=torch.float16)
    scale = 128 ** -0.5
    got = ops.sparse_attention(q, k, v, window=512, sink=16, sm_scale=scale)
    rows = np.arange(0, 1500, 37)
    gq = attention(q[:, :, rows], k, v, torch.from_numpy(rows)[None].cuda(), scale)
    qd = q[:, :, -1:].contiguous()
    gd = ops.decode_attention(qd, k, v, window=0, sink=0, sm_scale=scale)
    torch.cuda.synchronize()
    for t in (got, gq, gd):
        assert torch.isfinite(t).all()
    assert_close(np64(got), O.sparse_attention(np64(q), np64(k), np64(v), 512, 16, scale),
                 what=f"fp16 key-sparse {kind}")
    assert_close(np64(gq), O.qsparse_attention(np64(q)[:, :, rows], np64(k), np64(v), rows, scale),
                 what=f"fp16 query-sparse {kind}")
    assert_close(np64(gd), O.decode_row(np64(qd), np64(k), np64(v), 0, 0, scale),
                 what=f"fp16 decode {kind}")


def test_fp16_split_partials_keep_fp16_precision(gpu):
    """Kernel (2) and the decode row split each row's keys over several items
    and merge the partial O / l rows, stored in the input's element type. For
    fp16 inputs the result stays within a few fp16 ulps of the exact softmax
    (partials rounded to bf16 would be 8x coarser)."""
    from delta_attention import ops
    from delta_attention.delta_kernel import attention
    g = torch.Generator().manual_seed(47)
    S, D = 16384, 128
    q = torch.randn(1, 8, S, D, generator=g)
    k = torch.randn(1, 2, S, D, generator=g)
    v = torch.randn(1, 2, S, D, generator=g) * 8.0
    q, k, v = (x.to(torch.float16).cuda() for x in (q, k, v))
    scale = 4 * D ** -0.5
    rows = np.arange(S - 512, S, 7)
    got = attention(q[:, :, rows], k, v, torch.from_numpy(rows)[None].cuda(), scale)
    qd = q[:, :, -1:].contiguous()
    gd = ops.decode_attention(qd, k, v, window=0, sink=0, sm_scale=scale)
    torch.cuda.synchronize()
    for t, ref, what in ((got, O.qsparse_attention(np64(q)[:, :, rows], np64(k), np64(v), rows, scale), "rows"),
                         (gd, O.decode_row(np64(qd), np64(k), np64(v), 0, 0, scale), "decode")):
        # error per row in units of 2^-10 of the row's largest |value| (its
        # fp16 ulp scale): one bf16 rounding of a partial row would be 4 units
        unit = 2.0 ** -10 * np.abs(ref).max(-1, keepdims=True)
        err = (np.abs(np64(t) - ref) / unit).max()
        print(f"fp16 {what}: max error {err:.2f} units of 2^-10 of the row max", flush=True)
        assert err < 2.0, what
