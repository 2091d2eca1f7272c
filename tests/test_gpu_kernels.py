"""GPU parity of the three kernels against the oracle on identical seeded
inputs (the oracle runs in float64 on the bf16/fp16-rounded values).

Tolerance (the reference's T1 gate, tests/test_math_identities.py:85-89, and
the layer's parity bar): per-row cosine > 0.999 and max |diff| < 2e-2 for the
attention kernels; the delta-add kernel is bit-exact against the reference's
bf16 elementwise arithmetic.
"""

import numpy as np
import pytest
import torch

from helpers import assert_close, gen_qkv, np64
from oracle import delta_oracle as O

pytestmark = pytest.mark.gpu


def _sparse_case(B, H, Hkv, S, D, window, sink, qb=64, dtype=torch.bfloat16, seed=0,
                 model_layout=False, scale=None):
    from delta_attention import ops
    q, k, v = gen_qkv(B, H, Hkv, S, D, seed=seed, dtype=dtype, model_layout=model_layout)
    scale = D ** -0.5 if scale is None else scale
    out = ops.sparse_attention(q, k, v, window=window, sink=sink, sm_scale=scale, q_block=qb)
    torch.cuda.synchronize()
    ref = O.sparse_attention(np64(q), np64(k), np64(v), window, sink, scale, q_block=qb)
    assert_close(np64(out), ref, what=f"sparse B{B} H{H}/{Hkv} S{S} D{D} w{window} sink{sink} qb{qb}")


@pytest.mark.parametrize("B,H,Hkv,S,D,window,sink", [
    (1, 8, 2, 1024, 64, 256, 64),      # CPU-config geometry, shortened
    (1, 8, 2, 2048, 128, 512, 128),    # Llama geometry (GQA 4)
    (2, 4, 1, 700, 128, 128, 20),      # batch 2, S and sink not multiples of 64
    (1, 10, 2, 512, 128, 200, 7),      # Qwen3 GQA ratio 5
    (1, 2, 2, 300, 64, 96, 0),         # MHA, no sink
    (1, 4, 4, 256, 128, 40, 3),        # window < q_block: rows with few keys
    (1, 4, 2, 384, 128, 4096, 0),      # window covers everything: causal
    (1, 4, 2, 384, 64, 8, 1000),       # sinks cover everything: causal
    (1, 8, 2, 1100, 32, 300, 16),      # head_dim 32
    (2, 6, 3, 500, 32, 64, 0),         # head_dim 32, GQA 2, batch 2
])
def test_sparse_attention_parity(gpu, rows_per_wave, B, H, Hkv, S, D, window, sink):
    _sparse_case(B, H, Hkv, S, D, window, sink)


def test_sparse_attention_fp16_and_q_block(gpu, rows_per_wave):
    _sparse_case(1, 8, 2, 640, 128, 160, 16, qb=32, dtype=torch.float16)
    _sparse_case(1, 4, 1, 256, 64, 64, 8, qb=1)


@pytest.mark.parametrize("H,Hkv,D,window,sink,cuts", [
    (8, 2, 128, 256, 16, (0, 300, 301, 1024, 1500)),   # GQA 4: two heads per 64-row tile
    (5, 1, 64, 100, 0, (0, 64, 500, 1500)),            # GQA 5: one head per 128-row tile
])
def test_sparse_attention_row_ranges(gpu, rows_per_wave, H, Hkv, D, window, sink, cuts):
    """Row ranges of the key-sparse pass (da_sparse_attn_fwd_rows), launched
    one after another into one output, give the full launch's bits; rows
    outside a launched range are left untouched."""
    from delta_attention import ops
    q, k, v = gen_qkv(1, H, Hkv, 1500, D, seed=31)
    scale = D ** -0.5
    full = ops.sparse_attention(q, k, v, window=window, sink=sink, sm_scale=scale)
    out = torch.full_like(full, 7.0)
    for a, b in zip(cuts[:-1], cuts[1:]):
        ops.sparse_attention(q, k, v, window=window, sink=sink, sm_scale=scale, out=out, rows=(a, b - a))
    torch.cuda.synchronize()
    assert torch.equal(out, full)
    part = torch.full_like(full, 7.0)
    ops.sparse_attention(q, k, v, window=window, sink=sink, sm_scale=scale, out=part, rows=(301, 700))
    assert torch.equal(part[:, 301:1001], full[:, 301:1001])
    assert bool((part[:, :301] == 7.0).all()) and bool((part[:, 1001:] == 7.0).all())


@pytest.mark.parametrize("H,Hkv,S,window,sink,gamma", [
    (8, 2, 3000, 1024, 128, 64),    # GQA 4: two heads per 64-row tile (32 rows per wave) or four (64)
    (10, 2, 1700, 512, 16, 16),     # GQA 5: one head per 128- or 256-row tile
    (4, 4, 900, 128, 3, 32),        # MHA
])
def test_sparse_bits_independent_of_rows_per_wave(gpu, H, Hkv, S, window, sink, gamma):
    """Kernel (1) and the fused delta launch at 64 query rows per wave (one
    workgroup per CU, O in AGPRs) give the bits of the 32-rows-per-wave
    launch: same row maxima, same accumulation order, per-row rescale."""
    from delta_attention import ops
    q, k, v = gen_qkv(1, H, Hkv, S, 128, seed=S + H, model_layout=True)
    scale = 128 ** -0.5
    res = {}
    for rows in (32, 64):
        prev = ops.set_sparse_rows_per_wave(rows)
        try:
            res[rows] = (ops.sparse_attention(q, k, v, window=window, sink=sink, sm_scale=scale),
                         ops.delta_prefill(q, k, v, gamma=gamma, window=window, sink=sink, sm_scale=scale))
            torch.cuda.synchronize()
        finally:
            ops.set_sparse_rows_per_wave(prev)
    assert torch.equal(res[32][0], res[64][0])
    assert torch.equal(res[32][1], res[64][1])


def test_sparse_attention_model_layout(gpu):
    # q/k/v as transposed views of [B,S,H,D] storage (no copies on the way in)
    _sparse_case(1, 8, 2, 1024, 128, 256, 64, model_layout=True, seed=3)


def _qsa(q, k, v, mask, scale):
    from delta_attention.delta_kernel import attention
    out = attention(q, k, v, mask, scale)
    torch.cuda.synchronize()
    return out


def test_qsparse_t1(gpu):
    # tests/test_math_identities.py:61-89: 37 sorted rows incl. both ends
    b, h, s, d = 1, 32, 4096, 128
    q, k, v = gen_qkv(b, h, h, s, d, seed=0)
    mid = torch.randperm(s - 2, generator=torch.Generator().manual_seed(1))[:35] + 1
    idx = torch.cat([torch.tensor([0, s - 1]), mid]).unique().sort().values
    out = _qsa(q[:, :, idx.cuda()], k, v, idx.cuda().unsqueeze(0), d ** -0.5)
    ref = O.qsparse_attention(np64(q)[:, :, idx.numpy()], np64(k), np64(v), idx.numpy(), d ** -0.5)
    assert_close(np64(out), ref, what="T1")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_qsparse_one_merge_lane_per_task(gpu, dtype):
    """A selected-rows launch with 2^18 merge tasks (8 kv heads x 16 row tiles
    of 128 (row, head) pairs x 16 sixteen-byte columns) and 5 splits per row
    tile at 16K keys merges each task's splits in one lane; smaller launches
    share a task between lanes. Both dtypes against the oracle; fp16 at a
    bound near its own rounding (the split partials are stored in the
    element type)."""
    from delta_attention import ops
    B, H, Hkv, S, D = 1, 32, 8, 16384, 128
    q, k, v = gen_qkv(B, H, Hkv, S, D, seed=11, dtype=dtype)
    rows = torch.randperm(S, generator=torch.Generator().manual_seed(12))[:512].sort().values
    print(f"qsparse 512 rows x 32 heads, {dtype}", flush=True)
    out = ops.qsparse_attention(q, k, v, rows.cuda(), D ** -0.5, q_rows=rows.cuda())
    torch.cuda.synchronize()
    ref = O.qsparse_attention(np64(q)[:, :, rows.numpy()], np64(k), np64(v), rows.numpy(), D ** -0.5)
    assert_close(np64(out), ref, atol=2e-2 if dtype == torch.bfloat16 else 2e-3,
                 what=f"one merge lane per task ({dtype})")


@pytest.mark.parametrize("kind", ["rectangle", "irregular", "causal"])
def test_qsparse_reference_kernel_tests(gpu, kind):
    # delta_kernel.py:332-469: Z=1, H=2, N_CTX=1024, D=64, std 0.5, seed 20, atol 1e-2
    n = 1024
    N = {"rectangle": 2 * n, "irregular": 4 * n, "causal": n}[kind]
    q, k, v = gen_qkv(1, 2, 2, n, 64, seed=20, std=0.5, N=N)
    g = torch.Generator().manual_seed(20)
    mask = {"rectangle": torch.randint(0, N, (1, n), generator=g),
            "irregular": torch.randperm(n, generator=g).unsqueeze(0),
            "causal": torch.arange(n).unsqueeze(0)}[kind]
    out = _qsa(q, k, v, mask.cuda(), 64 ** -0.5)
    ref = O.qsparse_attention(np64(q), np64(k), np64(v), mask[0].numpy(), 64 ** -0.5)
    assert_close(np64(out), ref, atol=1e-2, what=f"qsa {kind}")


def test_qsparse_gqa_native_equals_expanded(gpu):
    from delta_attention.llama import repeat_kv
    q, k, v = gen_qkv(2, 8, 2, 1500, 128, seed=4)
    rows = torch.tensor([0, 1, 63, 64, 500, 1000, 1499], device="cuda")
    a = _qsa(q[:, :, rows], k, v, rows.unsqueeze(0), 0.1)
    b = _qsa(q[:, :, rows], repeat_kv(k, 4), repeat_kv(v, 4), rows.unsqueeze(0), 0.1)
    assert torch.equal(a, b)
    ref = O.qsparse_attention(np64(q)[:, :, rows.cpu().numpy()], np64(k), np64(v), rows.cpu().numpy(), 0.1)
    assert_close(np64(a), ref, what="qsa GQA")


def test_qsparse_edge_limits(gpu):
    from delta_attention import ops
    q, k, v = gen_qkv(2, 4, 2, 64, 128, seed=5, N=300)
    # per-batch limits, a negative limit (empty row -> zeros) and one beyond the keys (clamped)
    lim = torch.tensor([[5, -1, 299, 1000] * 16, [0, 63, 128, 7] * 16], device="cuda")
    out = ops.qsparse_attention(q, k, v, lim, 0.2)
    torch.cuda.synchronize()
    for b in range(2):
        l = np.minimum(lim[b].cpu().numpy(), 299)
        ref = O.qsparse_attention(np64(q)[b:b + 1], np64(k)[b:b + 1], np64(v)[b:b + 1], l, 0.2)
        assert_close(np64(out)[b:b + 1], ref, what=f"edge b{b}")
    assert torch.count_nonzero(out[0, :, 1::4]) == 0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_delta_add_bit_exact(gpu, dtype):
    from delta_attention import ops
    B, S, H, D, g = 2, 1280, 8, 128, 64
    gen = torch.Generator().manual_seed(6)
    sparse = torch.randn(B, S, H, D, generator=gen).to(dtype)
    _, _, s_p, _ = O.anchor_layout(S, g)
    n = s_p // g
    dense = torch.randn(B, n, H, D, generator=gen).to(dtype)
    anchors = torch.arange(0, s_p, g)
    # delta precomputed the way kernel (2) writes it, then the in-place uniform add
    delta = (dense - sparse[:, anchors])
    out = sparse.clone().cuda()
    ops.delta_add(out, s_p=s_p, out=out, delta=delta.cuda(), gamma=g)
    torch.cuda.synchronize()
    if dtype == torch.bfloat16:
        ref = O.compose_uniform(np64(sparse).astype(np.float32),
                                np.concatenate([np64(dense), np64(sparse)[:, s_p:]], 1).astype(np.float32),
                                S, g, bf16=True)
        np.testing.assert_array_equal(out.float().cpu().numpy(), ref)
    ref_t = sparse.clone()
    ref_t[:, :s_p] = (sparse[:, :s_p].reshape(B, n, g, H, D) + delta.reshape(B, n, 1, H, D)).reshape(B, s_p, H, D)
    assert torch.equal(out.cpu(), ref_t)


def test_apply_delta_variable_bit_exact(gpu):
    from delta_attention.stride import apply_delta_variable
    B, S, H, D = 1, 2000, 4, 64
    gen = torch.Generator().manual_seed(7)
    sparse = torch.randn(B, S, H, D, generator=gen).to(torch.bfloat16)
    idx = torch.tensor([5, 17, 18, 100, 640, 641, 1500])       # variable stride, first row != 0
    dense = torch.randn(B, len(idx), H, D, generator=gen).to(torch.bfloat16)
    s_p = 1900
    got = apply_delta_variable(sparse.cuda(), dense.cuda(), idx.cuda(), s_p)
    torch.cuda.synchronize()
    ref = O.apply_delta_variable(np64(sparse).astype(np.float32), np64(dense).astype(np.float32),
                                 idx.numpy(), s_p, bf16=True)
    np.testing.assert_array_equal(got.float().cpu().numpy(), ref)
    # the reference's own torch ops on the same bf16 tensors (stride.py:38-40)
    deltas = dense - sparse[:, idx]
    owner = torch.searchsorted(idx, torch.arange(s_p), right=True) - 1
    assert torch.equal(got.cpu(), sparse[:, :s_p] + deltas[:, owner])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_qsparse_head_dim_32(gpu, dtype):
    """delta_kernel.attention with head_dim 32 (the reference's wrapper accepts
    it, delta_kernel.py:268): sorted rows and an unsorted mask, native GQA."""
    q, k, v = gen_qkv(1, 8, 2, 1500, 32, seed=9, dtype=dtype)
    rows = torch.tensor([0, 7, 64, 640, 999, 1499], device="cuda")
    out = _qsa(q[:, :, rows], k, v, rows.unsqueeze(0), 32 ** -0.5)
    ref = O.qsparse_attention(np64(q)[:, :, rows.cpu().numpy()], np64(k), np64(v), rows.cpu().numpy(),
                              32 ** -0.5)
    assert_close(np64(out), ref, what="qsa d32")
    mask = torch.randperm(1500, generator=torch.Generator().manual_seed(3))[:200].unsqueeze(0)
    out = _qsa(q[:, :, :200], k, v, mask.cuda(), 32 ** -0.5)
    ref = O.qsparse_attention(np64(q)[:, :, :200], np64(k), np64(v), mask[0].numpy(), 32 ** -0.5)
    assert_close(np64(out), ref, what="qsa d32 unsorted")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_qsparse_head_dim_256(gpu, dtype):
    """delta_kernel.attention with head_dim 256 (accepted by the reference's
    wrapper, delta_kernel.py:268; one workgroup per CU): sorted rows over a
    long key range (several split items per row tile), an unsorted mask, and
    expanded K/V equal to native GQA bit for bit."""
    q, k, v = gen_qkv(1, 8, 2, 2500, 256, seed=11, dtype=dtype)
    rows = torch.tensor([0, 5, 63, 64, 700, 1999, 2400, 2499], device="cuda")
    out = _qsa(q[:, :, rows], k, v, rows.unsqueeze(0), 256 ** -0.5)
    ref = O.qsparse_attention(np64(q)[:, :, rows.cpu().numpy()], np64(k), np64(v),
                              rows.cpu().numpy(), 256 ** -0.5)
    assert_close(np64(out), ref, what=f"qsa d256 {dtype}")
    mask = torch.randperm(2500, generator=torch.Generator().manual_seed(4))[:300].unsqueeze(0)
    out = _qsa(q[:, :, :300], k, v, mask.cuda(), 256 ** -0.5)
    ref = O.qsparse_attention(np64(q)[:, :, :300], np64(k), np64(v), mask[0].numpy(), 256 ** -0.5)
    assert_close(np64(out), ref, what="qsa d256 unsorted")
    ke, ve = (t.repeat_interleave(4, dim=1) for t in (k, v))
    assert torch.equal(_qsa(q[:, :, :300], ke, ve, mask.cuda(), 256 ** -0.5), out)


def test_sparse_attention_head_dim_256(gpu):
    _sparse_case(1, 8, 2, 1100, 256, 300, 16)
    _sparse_case(2, 4, 4, 400, 256, 128, 0, dtype=torch.float16)


def test_attention_fp32_inputs(gpu):
    """float32 callers of delta_kernel.attention (the reference's Triton
    kernel takes them): the rows run in bf16 and come back as float32
    (llama.py:383-388, 493-494), within the bf16 gate of the float64 result."""
    g = torch.Generator().manual_seed(12)
    q, k, v = (torch.randn(1, h, 900, 128, generator=g).cuda() for h in (8, 2, 2))
    rows = torch.tensor([3, 64, 500, 899], device="cuda")
    out = _qsa(q[:, :, rows], k, v, rows.unsqueeze(0), 128 ** -0.5)
    assert out.dtype == torch.float32 and out.shape == (1, 8, 4, 128)
    ref = O.qsparse_attention(np64(q)[:, :, rows.cpu().numpy()], np64(k), np64(v),
                              rows.cpu().numpy(), 128 ** -0.5)
    assert_close(np64(out), ref, what="qsa fp32 inputs")
