"""GPU parity of the consecutive-anchor delta cosine kernel (da_anchor_delta_cos)
against the oracle's restatement of stride.py:43-52 / drift.py:23-49, and of the
two callers built on it: the adaptive stride's interanchor_cos and the prefill
drift summary."""

import numpy as np
import pytest
import torch

from helpers import np64
from oracle import delta_oracle as O

pytestmark = pytest.mark.gpu


def _randn(shape, seed, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).to(dtype).cuda()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [128, 64])
def test_delta_buffer_mode(gpu, dtype, D):
    from delta_attention import ops
    d = _randn((2, 33, 8, D), seed=D, dtype=dtype)
    # correlated neighbours, so the cosines spread over [-1, 1]
    d[:, 1:] += 0.7 * d[:, :-1].clone()
    cos, hist = ops.anchor_delta_cos(d, hist_bins=40)
    torch.cuda.synchronize()
    ref = O.interanchor_cos(np64(d))
    assert cos.shape == (2, 32, 8) and cos.dtype == torch.float32
    np.testing.assert_allclose(cos.cpu().numpy(), ref, atol=2e-6)
    # the histogram bins the kernel's own cosines with torch.histc's rule
    np.testing.assert_array_equal(hist.cpu().numpy(), O.histc(cos.cpu().numpy(), 40, -1.0, 1.0))
    assert int(hist.sum()) == cos.numel()


def test_dense_minus_sparse_mode(gpu):
    """Deltas formed in the kernel from dense anchor rows and the key-sparse
    output at the anchor rows: rnd(dense - sparse[:, rows]), the reference's
    bf16 tensor subtraction (llama.py:784-788)."""
    from delta_attention import ops
    B, S, H, D = 2, 700, 4, 128
    sparse = _randn((B, S, H, D), seed=1)
    rows = torch.arange(5, S, 48, device="cuda")
    dense = _randn((B, rows.numel(), H, D), seed=2) * 0.3 + sparse[:, rows]
    cos = ops.anchor_delta_cos(dense, sparse=sparse, rows=rows)
    torch.cuda.synchronize()
    deltas = dense - sparse[:, rows]                 # bf16 subtraction, as the reference
    np.testing.assert_allclose(cos.cpu().numpy(), O.interanchor_cos(np64(deltas)), atol=2e-6)
    # dense given as a [B, H, n, D] buffer's transposed view (the qsparse output layout)
    dense_t = dense.transpose(1, 2).contiguous().transpose(1, 2)
    cos_t = ops.anchor_delta_cos(dense_t, sparse=sparse, rows=rows)
    torch.cuda.synchronize()
    assert torch.equal(cos, cos_t)


def test_zero_and_degenerate_deltas(gpu):
    from delta_attention import ops
    d = torch.zeros(1, 4, 2, 128, device="cuda", dtype=torch.bfloat16)
    d[0, 0, :, 0] = 1.0
    d[0, 1, :, 0] = 4.0          # parallel
    d[0, 2] = 0.0                # zero delta: cosine 0 on both sides
    d[0, 3, 0, 0] = -1.0         # then antiparallel would be -1, but after a zero it is 0
    cos, hist = ops.anchor_delta_cos(d, hist_bins=4)
    torch.cuda.synchronize()
    np.testing.assert_allclose(cos.cpu().numpy(), O.interanchor_cos(np64(d)), atol=1e-7)
    np.testing.assert_array_equal(hist.cpu().numpy(), [0, 0, 4, 2])
    one = ops.anchor_delta_cos(d[:, :1])           # a single anchor: no pair
    assert one.shape == (1, 0, 2)


def test_interanchor_cos_and_drift_summary(gpu):
    from delta_attention import drift, stride
    d = _randn((1, 65, 32, 128), seed=7)
    d[:, 1:] += 1.5 * d[:, :-1].clone()
    ref = O.interanchor_cos(np64(d))
    mean, mn = stride.interanchor_cos(d)
    assert mean == pytest.approx(ref.mean(), abs=1e-5)
    assert mn == pytest.approx(ref.min(), abs=1e-5)
    s = drift.drift_summary(d, layer_idx=2, gamma=64, seq_len=65 * 64 + 128)
    assert s["n"] == 64 * 32 and s["layer"] == 2 and s["gamma"] == 64
    assert s["mean"] == pytest.approx(ref.mean(), abs=1e-5)
    q = np.quantile(ref.ravel(), [0.1, 0.5, 0.9])
    assert [s["p10"], s["p50"], s["p90"]] == pytest.approx(list(q), abs=1e-4)
    assert sum(s["hist"]) == s["n"] and len(s["hist"]) == drift.HIST_BINS
