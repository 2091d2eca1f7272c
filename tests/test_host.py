"""Host-side logic of the delta path on the CPU: the exact sampled-row index
set, knobs, the stride rules / cost model, drift aggregation, and that the
product ops refuse to run anywhere but on the GPU library."""

import dataclasses
import json

import numpy as np
import pytest
import torch

import conftest  # noqa: F401
from oracle import delta_oracle as O
from delta_attention import config as C
from delta_attention import drift, ops, stride
from delta_attention.delta_kernel import attention
from delta_attention.validation import anchor_indices


@pytest.mark.parametrize("s,gamma", [(4096, 16), (32768, 64), (131072, 16), (131072, 32),
                                     (131072, 64), (131072, 128), (65536, 64), (8192, 1),
                                     (4100, 64), (200, 64), (100, 64)])
def test_index_set_exact(s, gamma):
    ref = O.selected_rows(s, gamma)
    got = ops.selected_rows(s, gamma, "cpu").numpy()
    np.testing.assert_array_equal(got, ref)
    cut_n, s_p, n_anchor = ops.anchor_layout(s, gamma)
    a, t, s_p_o, cut_o = O.anchor_layout(s, gamma)
    assert (cut_n, s_p) == (cut_o, s_p_o) and n_anchor == len(a)
    va, vt = anchor_indices(s, gamma)
    np.testing.assert_array_equal(np.concatenate([va.numpy(), vt.numpy()]), ref)


def test_config_knobs():
    cfg = C.Config()
    assert cfg.delta_lambda == 64 and cfg.sliding_window == 2048 and cfg.sink_tokens == 1024
    names = {f.name for f in dataclasses.fields(C.Config)}
    assert set(C.PIPELINE_FIELDS) <= names and "sink_tokens" in C.PIPELINE_FIELDS
    cfg2 = C.Config.from_args(["--delta_lambda", "16", "--sink_tokens", "128", "--log_drift",
                               "--mode", "recompute"])
    assert (cfg2.delta_lambda, cfg2.sink_tokens, cfg2.log_drift, cfg2.mode) == (16, 128, True, "recompute")

    class M:
        pass
    m = M()
    C.copy_pipeline_fields(cfg2, m)
    assert all(getattr(m, f) == getattr(cfg2, f) for f in C.PIPELINE_FIELDS)


def test_sparse_pass_cost_closed_form():
    for s, w, sk in [(4096, 2048, 1024), (1000, 2048, 1024), (131072, 2048, 128), (10, 3, 2)]:
        brute = sum(min(i + 1, w + sk) for i in range(s))
        assert stride._sparse_pass_cost(s, w, sk) == brute


def test_effective_sparsity_uniform_matches_tensor_form():
    for s, g in [(32768, 64), (8192, 16), (131072, 128)]:
        idx = torch.from_numpy(O.selected_rows(s, g))
        assert stride.uniform_effective_sparsity(s, g, 2048, 1024) == pytest.approx(
            stride.effective_sparsity(idx, s, 2048, 1024), rel=1e-12)


def test_next_gamma_rules():
    kw = dict(threshold=0.9, gamma_min=16, gamma_max=256)
    assert stride.next_gamma(0.5, 64, **kw) == 32
    assert stride.next_gamma(0.5, 16, **kw) == 16
    assert stride.next_gamma(0.91, 64, **kw) == 64           # inside the hysteresis band
    assert stride.next_gamma(0.93, 64, **kw) == 128
    assert stride.next_gamma(0.99, 256, **kw) == 256
    kr = dict(k=1.0, gamma_min=16, gamma_max=256)
    assert stride.next_gamma_relative(0.1, [0.5], 64, **kr) == 64   # needs >= 2 entries
    hist = [0.5, 0.7]                                                # mean .6, std .1
    assert stride.next_gamma_relative(0.45, hist, 64, **kr) == 32
    assert stride.next_gamma_relative(0.75, hist, 64, **kr) == 128
    assert stride.next_gamma_relative(0.6, hist, 64, **kr) == 64
    assert stride.plan_chunks(10000, 4096) == [(0, 4096), (4096, 8192), (8192, 10000)]


def test_interanchor_cos_needs_gpu_deltas():
    d = torch.zeros(1, 3, 2, 64, dtype=torch.bfloat16)
    assert stride.interanchor_cos(d[:, :1]) == (1.0, 1.0)     # fewer than two anchors
    with pytest.raises(AssertionError):
        stride.interanchor_cos(d)                              # the product runs the kernel
    with pytest.raises(AssertionError):
        drift.drift_summary(d, layer_idx=0, gamma=64, seq_len=256)


def test_aggregate_drift():
    hist = [0] * drift.HIST_BINS
    hist[30] = 32
    s = {"layer": 3, "gamma": 64, "seq_len": 640, "n": 32, "mean": 0.5, "p10": 0.4, "p50": 0.5,
         "p90": 0.6, "hist_bins": drift.HIST_BINS, "hist_range": list(drift.HIST_RANGE), "hist": hist}
    json.dumps(s)
    agg = drift.aggregate_drift([s, dict(s, mean=1.0)])
    assert agg[3]["n"] == 64 and agg[3]["requests"] == 2
    assert agg[3]["mean"] == pytest.approx((s["mean"] + 1.0) / 2)
    assert agg[3]["hist"][30] == 64 and sum(agg[3]["hist"]) == 64
    with pytest.raises(ValueError, match="mixed-version"):
        drift.aggregate_drift([dict(s, hist_bins=10)])
    with pytest.raises(ValueError, match="mixed-version"):
        drift.aggregate_drift([dict(s, hist_range=[0.0, 1.0])])
    # the reference pairs histograms with zip: a shorter one truncates the sum
    assert len(drift.aggregate_drift([s, dict(s, hist=hist[:-1])])[3]["hist"]) == drift.HIST_BINS - 1
    # several layers, unequal weights, an empty request
    h2 = [0] * drift.HIST_BINS
    h2[0], h2[39] = 5, 3
    agg = drift.aggregate_drift([s, dict(s, layer=7, n=8, mean=-0.25, hist=h2),
                                 dict(s, n=96, mean=0.1), dict(s, layer=7, n=0, mean=0.9,
                                                               hist=[0] * drift.HIST_BINS)])
    assert sorted(agg) == [3, 7]
    assert agg[3]["mean"] == pytest.approx((32 * 0.5 + 96 * 0.1) / 128) and agg[3]["n"] == 128
    assert agg[7]["mean"] == pytest.approx(-0.25) and agg[7]["requests"] == 2
    assert agg[7]["hist"] == h2 and agg[7]["gamma"] == 64
    assert drift.aggregate_drift([dict(s, n=0)])[3]["mean"] == 0.0
    assert set(agg[3]) == {"layer", "n", "mean", "requests", "hist", "hist_bins", "hist_range",
                           "gamma"}
    # means fold one summary at a time, (m * n + m_i * n_i) / (n + n_i), the
    # order whose roundings the reference's sidecar aggregates carry: these
    # three summaries give a different last bit than sum(m_i n_i) / sum(n_i)
    parts = [(47, 0.604), (38, 0.891), (21, -0.939)]
    m, n = 0.0, 0
    for n_i, m_i in parts:
        m, n = (m * n + m_i * n_i) / (n + n_i), n + n_i
    assert m != sum(a * b for a, b in parts) / n
    agg = drift.aggregate_drift([dict(s, n=n_i, mean=m_i) for n_i, m_i in parts])
    assert agg[3]["mean"] == m
    # the edges are torch.histc's: a value just inside each edge lands in that bin
    edges = drift.hist_bin_edges()
    assert edges == [-1.0 + i * (2.0 / drift.HIST_BINS) for i in range(drift.HIST_BINS + 1)]
    np.testing.assert_allclose(edges, np.linspace(*drift.HIST_RANGE, drift.HIST_BINS + 1),
                               rtol=0, atol=1e-15)
    probe = torch.tensor(edges[:-1], dtype=torch.float64) + 1e-9
    counts = torch.histc(probe, bins=drift.HIST_BINS, min=drift.HIST_RANGE[0],
                         max=drift.HIST_RANGE[1])
    assert counts.tolist() == [1.0] * drift.HIST_BINS


def test_product_ops_refuse_cpu_tensors():
    q = torch.zeros(1, 2, 64, 64, dtype=torch.bfloat16)
    with pytest.raises(AssertionError):
        ops.sparse_attention(q, q, q, window=32, sink=0, sm_scale=0.1)
    with pytest.raises(AssertionError):
        attention(q, q, q, torch.arange(64)[None], 0.1)
    with pytest.raises(AssertionError):           # head_dim 96 has no kernel
        attention(torch.zeros(1, 2, 8, 96), torch.zeros(1, 2, 8, 96), torch.zeros(1, 2, 8, 96),
                  torch.arange(8)[None], 0.1)
    with pytest.raises(AssertionError):           # mask must be 2-D
        attention(q, q, q, torch.arange(64), 0.1)


def test_stale_library_is_extension_missing(tmp_path, monkeypatch):
    """A library without this binding's entry points (an old build) is refused
    with ExtensionMissing at load, not with an AttributeError mid-call."""
    import subprocess
    from delta_attention import _lib as L
    src = tmp_path / "old.c"
    src.write_text("int da_sparse_attn_fwd(void) { return 0; }\n")
    so = tmp_path / "libold.so"
    subprocess.run(["gcc", "-shared", "-fPIC", str(src), "-o", str(so)], check=True)
    monkeypatch.setattr(L, "LIB_PATH", str(so))
    monkeypatch.setattr(L, "_lib", None)
    with pytest.raises(L.ExtensionMissing, match="lacks da_sparse_attn_delta_fwd"):
        L.lib()


def test_fused_projections_are_views():
    """fuse_projections keeps names, values and state-dict keys; the fused
    product equals the separate ones; a replaced parameter (or a long input)
    falls back to separate products."""
    from delta_attention.llama import FUSED_MAX_ROWS, LlamaAttention
    from delta_attention.model import LlamaConfig, LlamaMLP
    cfg = LlamaConfig(vocab_size=64, hidden_size=256, intermediate_size=512, num_hidden_layers=1,
                      num_attention_heads=4, num_key_value_heads=2, head_dim=64)
    torch.manual_seed(0)
    at, mlp = LlamaAttention(cfg, 0), LlamaMLP(cfg)
    x = torch.randn(3, 256)
    ref = torch.cat([at.q_proj(x), at.k_proj(x), at.v_proj(x)], -1)
    keys, vals = list(at.state_dict()), {k: v.clone() for k, v in at.state_dict().items()}
    at.fuse_projections()
    mlp.fuse_projections()
    assert list(at.state_dict()) == keys
    assert all(torch.equal(at.state_dict()[k], vals[k]) for k in keys)
    with torch.no_grad():
        torch.testing.assert_close(at._qkv_product(x), ref)
        assert at._qkv_product(torch.randn(FUSED_MAX_ROWS + 1, 256)) is None
        g = mlp.forward(x)
        mlp._gate_up_fused = None
        torch.testing.assert_close(g, mlp.forward(x))
    assert at._qkv_product(x) is None           # gradients wanted: separate products
    at.k_proj.weight = torch.nn.Parameter(at.k_proj.weight.detach().clone())
    with torch.no_grad():
        assert at._qkv_product(x) is None


def test_fused_projection_params_keep_gradients():
    """fuse_linears re-points the modules' weights at slices of one buffer
    that is not an autograd leaf: with gradients enabled (and parameters that
    require them) fused_params declines, so the separate products run and
    every parameter gets its gradient; under no_grad the fused product is used."""
    import torch
    from torch import nn
    from delta_attention.llama import fuse_linears, fused_params
    torch.manual_seed(0)
    mods = [nn.Linear(16, n, bias=False) for n in (8, 4, 4)]
    fused = fuse_linears(*mods)
    assert fused_params(fused, mods, rows=1) == (None, None)
    with torch.no_grad():
        w, b = fused_params(fused, mods, rows=1)
        assert w is fused[0] and b is None
        assert fused_params(fused, mods, rows=65) == (None, None)   # long inputs: separate GEMMs
    for m in mods:
        m.weight.requires_grad_(False)
    w, _ = fused_params(fused, mods, rows=1)
    assert w is fused[0]
    for m in mods:
        m.weight.requires_grad_(True)
    x = torch.randn(2, 16)
    sum(m(x).sum() for m in mods).backward()
    assert all(m.weight.grad is not None for m in mods)
