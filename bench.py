"""Delta-attention layer prefill benchmark on one MI355X.

Workload: one Llama-3.1-8B-shaped attention layer prefill at 128K tokens --
batch 1, 32 query heads / 8 key-value heads, head_dim 128, seq 131072,
Q/K/V ~ N(0,1) (Q scaled by 1/sqrt(128)), RoPE theta 500000 on Q/K, bf16,
causal, window 2048 + 128 sink tokens, gamma 64. A step is one full layer
prefill: kernel (1) key-sparse attention, kernel (2) query-sparse dense rows
with the fused delta epilogue, kernel (3) delta broadcast-add, with the inputs
resident in HBM.

Prints ONE JSON line: value = TFLOP/s of the layer (algorithmic FLOPs of
kernels 1+2 / layer time), ms_per_step = layer time, plus the roofline of the
dominant kernel (HIP events on the launch stream), per-kernel figures and the
CPU oracle timed on a bounded sample of the same workload.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "delta-attention_amd"))
sys.path.insert(0, REPO)

METRIC = "delta-attn layer prefill ms + TFLOP/s (%MFMA peak) at 128K, Llama-3.1-8B shape"
PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
PEAK_SCLK_MHZ = 2400.0      # engine clock the MFMA peak is quoted at


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--seq", type=int, default=131072)
    p.add_argument("--gamma", type=int, default=64)
    p.add_argument("--window", type=int, default=2048)
    p.add_argument("--sink", type=int, default=128)
    p.add_argument("--heads", type=int, default=32)
    p.add_argument("--kv-heads", type=int, default=8)
    p.add_argument("--batch", type=int, default=1)
    p.add_argument("--head-dim", type=int, default=128)
    p.add_argument("--rope-theta", type=float, default=500000.0)
    p.add_argument("--cpu-budget", type=float, default=15.0,
                   help="approximate seconds of CPU oracle work for cpu_baseline (0: skip)")
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--gamma-sweep", type=str, default="",
                   help="comma-separated gammas: print one JSON line per gamma (layer time, "
                        "TFLOP/s, row cosine to full causal attention on sampled rows) "
                        "instead of the headline line")
    p.add_argument("--prologue", action="store_true",
                   help="time only the fused RoPE (+ optional per-head q/k RMSNorm with "
                        "--qk-norm) prologue kernel on the workload's [B,S,H,D] q/k projection "
                        "outputs and print one JSON line with its HBM roofline")
    p.add_argument("--qk-norm", action="store_true",
                   help="per-head RMSNorm (weight 1, eps 1e-6) on q and k before RoPE (the Qwen3 "
                        "recipe); with --prologue, time the kernel with the norm")
    p.add_argument("--no-q-scale", action="store_true",
                   help="q ~ N(0,1) without the d^-0.5 factor (the Qwen3 recipe)")
    p.add_argument("--workload", type=str, default="",
                   help="name recorded in config.workload (default: derived from the shape)")
    p.add_argument("--model", action="store_true",
                   help="full random-init Llama-3.1-8B-architecture prefill of --seq random token "
                        "ids with delta attention in every layer: time to first token and the "
                        "attention kernels' share (one JSON line; --steps/--warmup count prefills)")
    p.add_argument("--layers", type=int, default=32, help="decoder layers of --model")
    p.add_argument("--decode", action="store_true",
                   help="decode step of one layer against a --seq key cache: the sparse decode row "
                        "(sinks + last window keys), the dense anchor row and the delta step at "
                        "--gamma-dec, with their HBM rooflines (one JSON line)")
    p.add_argument("--gamma-dec", type=int, default=32)
    p.add_argument("--decode-tokens", type=int, default=0,
                   help="with --model: also generate this many tokens after the prefill, with "
                        "dense and with delta decode, and report ms per decode token")
    p.add_argument("--train", action="store_true",
                   help="time delta_forward_train's forward and backward (the training "
                        "path) at --seq/--gamma/--window/--sink instead of the prefill")
    p.add_argument("--adaptive", action="store_true",
                   help="time the adaptive-stride layer (stride_policy \"adaptive\", one "
                        "library call: per --adapt-chunk rows the inter-anchor delta cosine and "
                        "the next stride decided on the device) beside the fixed-stride layer; "
                        "with --model, every layer of the model uses it")
    p.add_argument("--adapt-chunk", type=int, default=4096)
    p.add_argument("--adapt-threshold", type=float, default=0.95)
    p.add_argument("--energy", action="store_true",
                   help="power-limit evidence: the fused kernel (1)+(3) at 32 and 64 query rows "
                        "per wave, kernel (2), and a hipBLASLt bf16 GEMM (8192^3), each run back "
                        "to back for about 1.5 s on the workload's N(0,1) inputs and on zeros, "
                        "with engine clock and package power sampled; one JSON line")
    p.add_argument("--copy-calibration", action="store_true",
                   help="only run a plain 1 GiB device-to-device copy 3 times (the known-size "
                        "kernel that calibrates rocprofv3 FETCH_SIZE / WRITE_SIZE) and exit")
    return p.parse_args()


def copy_calibration():
    import torch
    x = torch.ones(1 << 28, dtype=torch.float32, device="cuda")   # 1 GiB
    y = torch.empty_like(x)
    for _ in range(3):
        y.copy_(x)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": x.numel() * 4, "launches": 3}), flush=True)


def make_inputs(a, device):
    """Seeded N(0,1) q/k/v drawn in q, k, v order, q * d^-0.5 (unless
    --no-q-scale), per-head RMSNorm on q and k (with --qk-norm), RoPE on q and k
    (rotate_half, inv_freq = theta^(-2i/d), fp32 tables), cast to bf16."""
    import torch
    from delta_attention.llama import apply_rotary_pos_emb, rope_cos_sin

    g = torch.Generator(device=device).manual_seed(a.seed)
    B, H, Hkv, S, D = a.batch, a.heads, a.kv_heads, a.seq, a.head_dim
    q = torch.empty(B, H, S, D, device=device, dtype=torch.bfloat16)
    k = torch.empty(B, Hkv, S, D, device=device, dtype=torch.bfloat16)
    v = torch.empty(B, Hkv, S, D, device=device, dtype=torch.bfloat16)
    pos = torch.arange(S, device=device)[None]
    cos, sin = rope_cos_sin(pos, D, a.rope_theta, torch.float32)
    CH = 8192
    for c0 in range(0, S, CH):
        c1 = min(S, c0 + CH)
        qc = torch.randn(B, H, c1 - c0, D, device=device, generator=g)
        if not a.no_q_scale:
            qc = qc * D ** -0.5
        kc = torch.randn(B, Hkv, c1 - c0, D, device=device, generator=g)
        if a.qk_norm:
            qc = qc * torch.rsqrt(qc.pow(2).mean(-1, keepdim=True) + 1e-6)
            kc = kc * torch.rsqrt(kc.pow(2).mean(-1, keepdim=True) + 1e-6)
        qc, kc = apply_rotary_pos_emb(qc, kc, cos[:, c0:c1], sin[:, c0:c1])
        q[:, :, c0:c1] = qc.to(torch.bfloat16)
        k[:, :, c0:c1] = kc.to(torch.bfloat16)
        v[:, :, c0:c1] = torch.randn(B, Hkv, c1 - c0, D, device=device, generator=g).to(torch.bfloat16)
    return q, k, v


def cpu_threads():
    """Host threads for the CPU oracle: the cores this process may run on
    (sched_getaffinity), capped by OMP_NUM_THREADS when it is set (the CPU
    share of a shared machine). -> (threads, affinity count)."""
    aff = len(os.sched_getaffinity(0))
    cap = os.environ.get("OMP_NUM_THREADS", "")
    n = min(aff, int(cap)) if cap.isdigit() and int(cap) > 0 else aff
    return n, aff


def cpu_c1(O, np, runs=3):
    """The CPU configuration in full (batch 1, 8/2 heads, head_dim 64, seq
    4096, fp32, window 512 + 64 sinks, gamma 16), q/k/v ~ N(0,1) from a CPU
    generator seeded 0 in q, k, v order (validation.py:133-145): the oracle's
    delta_forward, one warm-up then the median of `runs` timed runs."""
    import torch
    g = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn(1, h, 4096, 64, generator=g).numpy() for h in (8, 2, 2))
    scale = 64 ** -0.5
    O.delta_forward(q, k, v, 16, 512, 64, scale)
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        O.delta_forward(q, k, v, 16, 512, 64, scale)
        ts.append(time.perf_counter() - t0)
    flops = (O.flops_sparse(1, 8, 64, 4096, 512, 64)
             + O.flops_qsparse(1, 8, 64, O.selected_rows(4096, 16)))
    t = statistics.median(ts)
    return {"workload": "cpu configuration in full: B1, 8/2 heads, d64, s4096, fp32, "
                        "window 512 + 64 sinks, gamma 16",
            "ms": round(t * 1e3, 2), "tflops": round(flops / t / 1e12, 6), "flop": flops,
            "runs": runs, "warmup": 1, "stat": "median"}


def cpu_baseline(a, q, k, v, flops_layer):
    """The CPU oracle (numpy, BLAS threads) on a bounded sample of the same
    workload: the key-sparse pass for a block of rows and the dense pass for
    the longest anchor rows, both on the heads of one kv group, plus the CPU
    configuration run in full. BLAS and torch threads are set to cpu_threads()."""
    import numpy as np
    import torch
    from oracle import delta_oracle as O
    cores, aff = cpu_threads()
    torch.set_num_threads(cores)
    try:
        from threadpoolctl import threadpool_limits
        limits = threadpool_limits(limits=cores)
    except Exception:  # pragma: no cover
        limits = None
    G = a.heads // a.kv_heads
    S, D = a.seq, a.head_dim
    scale = D ** -0.5
    qh = q[:, :G].float().cpu().numpy()
    kh = k[:, :1].float().cpu().numpy()
    vh = v[:, :1].float().cpu().numpy()
    anchors, tail, s_p, _ = O.anchor_layout(S, a.gamma)
    flops = 0.0
    t0 = time.perf_counter()
    n_rows = 0
    # key-sparse rows from the middle of the sequence, 1024 at a time
    r0 = S // 2
    while time.perf_counter() - t0 < a.cpu_budget / 2 and r0 + 1024 <= S:
        rows = np.arange(r0, r0 + 1024)
        O.sparse_attention(qh, kh, vh, a.window, a.sink, scale, rows=rows)
        flops += 4.0 * D * G * O.sparse_row_counts(S, a.window, a.sink)[rows].sum()
        n_rows += 1024
        r0 += 1024
    t1 = time.perf_counter()
    # the longest dense anchor rows, 8 at a time
    n_dense = 0
    i = len(anchors)
    while time.perf_counter() - t1 < a.cpu_budget / 2 and i >= 8:
        rows = anchors[i - 8:i]
        O.qsparse_attention(qh[:, :, rows], kh, vh, rows, scale)
        flops += 4.0 * D * G * float((rows + 1).sum())
        n_dense += 8
        i -= 8
    dt = time.perf_counter() - t0
    tflops = flops / dt / 1e12
    c1 = cpu_c1(O, np)
    if limits is not None:
        limits.unregister()
    return {
        "value": round(tflops, 6), "unit": "TFLOP/s", "cores": int(cores), "kind": "port",
        "affinity_cores": int(aff),
        "sample": (f"oracle/delta_oracle.py (numpy fp32, BLAS on {cores} threads) on heads "
                   f"0-{G - 1} (kv group 0) of this workload: key-sparse pass over {n_rows} rows "
                   f"from row {S // 2} plus the dense pass over the last {n_dense} anchor rows; "
                   f"{flops / 1e9:.1f} GFLOP in {dt:.1f} s"),
        "full_layer_s_extrapolated": round(flops_layer / (tflops * 1e12), 1),
        "c1_full": c1,
    }


def gamma_sweep(a, q, k, v, gammas):
    """Per gamma: layer prefill time and the correction quality, i.e. the
    per-row cosine (over heads x dims) between the delta output and full causal
    attention at 512 sampled rows (dense rows from the query-sparse kernel)."""
    import torch
    from delta_attention import ops
    from oracle import delta_oracle as O
    B, H, Hkv, S, D = a.batch, a.heads, a.kv_heads, a.seq, a.head_dim
    scale = D ** -0.5
    g = torch.Generator().manual_seed(1)
    rows = torch.randperm(S, generator=g)[:512].sort().values.cuda()
    dense = ops.qsparse_attention(q, k, v, rows, scale, q_rows=rows).transpose(1, 2)
    sparse = ops.delta_prefill(q, k, v, gamma=64, window=a.window, sink=a.sink, sm_scale=scale,
                               mode="sparse-only")
    cs = torch.nn.functional.cosine_similarity(sparse[:, rows].reshape(B, 512, -1).float(),
                                               dense.reshape(B, 512, -1).float(), dim=-1)
    del sparse
    f_sparse = O.flops_sparse(B, H, D, S, a.window, a.sink)
    for gm in gammas:
        fn = lambda: ops.delta_prefill(q, k, v, gamma=gm, window=a.window, sink=a.sink, sm_scale=scale)
        for _ in range(a.warmup):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(a.steps):
            out = fn()
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) / a.steps * 1e3
        cos = torch.nn.functional.cosine_similarity(out[:, rows].reshape(B, 512, -1).float(),
                                                    dense.reshape(B, 512, -1).float(), dim=-1)
        f_q = O.flops_qsparse(B, H, D, O.selected_rows(S, gm))
        print(json.dumps({
            "gamma": gm, "ms_per_layer": round(ms, 4),
            "tflops": round((f_sparse + f_q) / (ms * 1e-3) / 1e12, 2),
            "flop_sparse": f_sparse, "flop_qsparse": f_q,
            "selected_rows": int(len(O.selected_rows(S, gm))),
            "cos_to_full_mean": round(cos.mean().item(), 6), "cos_to_full_min": round(cos.min().item(), 6),
            "sparse_only_cos_mean": round(cs.mean().item(), 6), "sparse_only_cos_min": round(cs.min().item(), 6),
            "seq_len": S, "window": a.window, "sink": a.sink}), flush=True)


def adaptive_layer(a, q, k, v):
    """The adaptive-stride layer: LlamaAttention.delta_forward with
    stride_policy "adaptive" (the reference's llama.py:695-711, 759-824), one
    library call that enqueues the key-sparse pass in row chunks on a second
    stream and, per adapt_chunk rows, a dense pass over the chunk's anchors at
    the current stride, the inter-anchor delta cosines with the next stride
    decided on the device and the chunk's broadcast-add, then the dense tail.
    Nothing is read back inside the layer (the per-chunk log is read after
    the timed steps, for the stride statistics). Wall clock per layer, with
    the fixed-stride layer at the starting and at the smallest stride beside
    it."""
    import types
    import torch
    from delta_attention import ops
    from delta_attention.llama import LlamaAttention
    B, H, Hkv, S, D = a.batch, a.heads, a.kv_heads, a.seq, a.head_dim
    scale = D ** -0.5
    cfg = types.SimpleNamespace(
        hidden_size=H * D, num_attention_heads=H, num_key_value_heads=Hkv, head_dim=D,
        attention_bias=False, attention_dropout=0.0, rms_norm_eps=1e-6,
        _attn_implementation="window", mode="delta", delta_lambda=a.gamma,
        sliding_window=a.window, sink_tokens=a.sink, stride_policy="adaptive", log_drift=False,
        adapt_chunk=a.adapt_chunk, adapt_threshold=a.adapt_threshold, gamma_min=16,
        gamma_max=256, stride_trigger="absolute", adapt_k=2.0)
    m = LlamaAttention(cfg, layer_idx=0).to(q.device).to(torch.bfloat16)

    def timed(fn):
        for _ in range(a.warmup):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(a.steps):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / a.steps * 1e3

    with torch.inference_mode():
        ms = timed(lambda: m.delta_forward(m, q, k, v, None, scaling=scale))
        st = m._stride_stats
        fixed = {g: round(timed(lambda: ops.delta_prefill(q, k, v, gamma=g, window=a.window,
                                                          sink=a.sink, sm_scale=scale)), 4)
                 for g in sorted({a.gamma, 16})}
        sparse_ms = timed(lambda: ops.sparse_attention(q, k, v, window=a.window, sink=a.sink,
                                                       sm_scale=scale))
    gammas = [c["gamma"] for c in st["chunks"]]
    n = len(gammas)
    print(json.dumps({
        "metric": "adaptive-stride layer prefill (wall clock)",
        "value": round(ms, 4), "unit": "ms", "higher_is_better": False,
        "steps": a.steps, "warmup": a.warmup, "chunks": n, "adapt_chunk": a.adapt_chunk,
        "adapt_threshold": a.adapt_threshold, "n_anchors": st["n_anchors"],
        "gamma_first_chunks": gammas[:6], "gamma_last": gammas[-1] if gammas else None,
        "effective_sparsity": round(st["effective_sparsity"], 6),
        "sparse_pass_ms": round(sparse_ms, 4),
        "beyond_sparse_pass_ms_per_chunk": round((ms - sparse_ms) / max(n, 1), 4),
        "fixed_stride_layer_ms": fixed,
        "config": {"batch": B, "seq_len": S, "heads": H, "kv_heads": Hkv, "head_dim": D,
                   "window": a.window, "sink": a.sink, "gamma_start": a.gamma}}), flush=True)


def prologue(a, dev):
    """The fused prologue kernel (da_rope_qk) in place on a packed projection
    buffer [B, S, (Hq + 2 Hkv) D]: algorithmic bytes = read + write of every q
    and k element, plus the bf16 cos/sin rows once per token."""
    import torch
    from delta_attention import ops
    from delta_attention.llama import rope_cos_sin
    B, H, Hkv, S, D = a.batch, a.heads, a.kv_heads, a.seq, a.head_dim
    buf = torch.randn(B, S, (H + 2 * Hkv) * D, device=dev, dtype=torch.bfloat16)
    q = buf[..., :H * D].view(B, S, H, D)
    k = buf[..., H * D:(H + Hkv) * D].view(B, S, Hkv, D)
    cos, sin = rope_cos_sin(torch.arange(S, device=dev)[None], D, a.rope_theta, torch.bfloat16)
    w = torch.ones(D, device=dev, dtype=torch.bfloat16) if a.qk_norm else None
    fn = lambda: ops.rope_qk(q, k, cos, sin, q_norm_w=w, k_norm_w=w)
    for _ in range(a.warmup):
        fn()
    stream = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(a.steps):
        fn()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / a.steps
    nbytes = 2 * B * S * (H + Hkv) * D * 2 + 2 * S * D * 2 + (4 * D if a.qk_norm else 0)
    gbs = nbytes / (ms * 1e-3) / 1e9
    print(json.dumps({
        "metric": "fused RoPE prologue (da_rope_qk, one launch over the q and k rows)", "value": round(gbs, 1),
        "unit": "GB/s", "ms_per_call": round(ms, 4), "steps": a.steps, "warmup": a.warmup,
        "qk_norm": bool(a.qk_norm), "bytes_per_call": nbytes,
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4)},
        "config": {"batch": B, "seq_len": S, "heads": H, "kv_heads": Hkv, "head_dim": D}}), flush=True)


def model_prefill(a, dev):
    """Time to first token of a random-init Llama-3.1-8B-architecture model
    (32 layers, hidden 4096, 32/8 heads, MLP 14336, vocab 128256, bf16 weights
    ~ N(0, 0.02)) on a.seq random token ids: embedding, every decoder layer
    (projections, fused RoPE, delta attention, o_proj, fused add+RMSNorm,
    SwiGLU MLP), final norm, lm_head on the last position and the greedy token."""
    import numpy as np
    import torch
    from delta_attention import ops
    from delta_attention.model import LlamaConfig, random_llama
    from delta_attention.timing import Timer
    from oracle import delta_oracle as O
    cfg = LlamaConfig(num_hidden_layers=a.layers, delta_lambda=a.gamma, sliding_window=a.window,
                      sink_tokens=a.sink)
    if a.adaptive:
        # --model --adaptive: every layer with stride_policy "adaptive"
        cfg.stride_policy, cfg.adapt_chunk = "adaptive", a.adapt_chunk
        cfg.adapt_threshold, cfg.gamma_min, cfg.gamma_max = a.adapt_threshold, 16, 256
    B, S = a.batch, a.seq
    t0 = time.perf_counter()
    model = random_llama(cfg, dev, torch.bfloat16, seed=a.seed)
    torch.cuda.synchronize()
    init_s = time.perf_counter() - t0
    g = torch.Generator(device=dev).manual_seed(a.seed + 1)
    ids = torch.randint(0, cfg.vocab_size, (B, S), device=dev, generator=g)
    for _ in range(a.warmup):
        model.prefill_next_token(ids)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(a.steps):
        tok = model.prefill_next_token(ids)
    torch.cuda.synchronize()
    ttft = (time.perf_counter() - t0) / a.steps * 1e3
    timer = Timer()
    model.prefill_next_token(ids, timer)
    parts = {k: round(v, 3) for k, v in timer.totals().items()}
    timed_total = sum(parts.values())
    H, Hkv, D, L = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim, cfg.num_hidden_layers
    cut_n, s_p, n_anchor = ops.anchor_layout(S, a.gamma)
    counts = O.sparse_row_counts(S, a.window, a.sink)
    rows = ops.fused_delta_rows(H, Hkv)
    f_sparse = 4.0 * D * H * B * float(counts[:s_p].sum() if rows and rows % a.gamma == 0 else counts.sum())
    strides = None
    if a.adaptive:
        # each layer's own anchors (from its stride statistics) plus the dense tail
        f_attn = 0.0
        strides = {"anchors_per_layer": [], "chunks_per_stride": {}}
        for layer in model.model.layers:
            st = layer.self_attn._stride_stats
            strides["anchors_per_layer"].append(st["n_anchors"])
            for c in st["chunks"]:
                key = str(c["gamma"])
                strides["chunks_per_stride"][key] = strides["chunks_per_stride"].get(key, 0) + 1
            sel = [r for c in st["chunks"]
                   for r in range(c["start"], c["start"] + c["n_anchors"] * c["gamma"], c["gamma"])]
            sel = np.array(sel + list(range(s_p, S)))
            # the key-sparse pass covers rows below s_p (the tail rows are dense)
            f_attn += 4.0 * D * H * B * float(counts[:s_p].sum()) + O.flops_qsparse(B, H, D, sel)
    else:
        f_attn = L * (f_sparse + O.flops_qsparse(B, H, D, O.selected_rows(S, a.gamma)))
    hid, inter = cfg.hidden_size, cfg.intermediate_size
    per_tok = 2 * (hid * (H + 2 * Hkv) * D + H * D * hid + 3 * hid * inter)
    f_gemm = L * per_tok * B * S + 2 * B * hid * cfg.vocab_size
    attn_ms = parts.get("attention_kernels", 0.0)
    gemm_ms = sum(parts.get(k, 0.0) for k in ("qkv_gemm", "o_gemm", "mlp_gemm", "lm_head"))
    line = {
        "metric": "llama-3.1-8b-architecture prefill time to first token at 128K",
        "value": round(ttft, 2), "unit": "ms", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "higher_is_better": False, "dtype": "bf16",
        "data": "synthetic (random token ids, weights ~ N(0, 0.02) per the reference's _init_weights)",
        "config": {"workload": "llama-3.1-8b-architecture causal LM prefill, delta attention in every layer",
                   "layers": L, "batch": B, "seq_len": S, "window": a.window, "sink": a.sink,
                   "gamma": a.gamma, "stride_policy": cfg.stride_policy,
                   "params": sum(p.numel() for p in model.parameters()),
                   "rope_scaling": cfg.rope_scaling, "parallelism": "none (1 GPU)"},
        "attention_share": round(attn_ms / timed_total, 4),
        "tokens_per_s": round(B * S / (ttft * 1e-3), 1),
        "breakdown_ms": parts, "breakdown_total_ms": round(timed_total, 2),
        "flop": {"attention": f_attn, "gemm": f_gemm},
        "tflops": {"attention_kernels": round(f_attn / attn_ms / 1e9, 1) if attn_ms else None,
                   "gemm": round(f_gemm / gemm_ms / 1e9, 1) if gemm_ms else None,
                   "model": round((f_attn + f_gemm) / (ttft * 1e-3) / 1e12, 1)},
        "first_token": int(tok[0]), "init_s": round(init_s, 2),
    }
    if strides is not None:
        line["adaptive_strides"] = strides
    if a.decode_tokens > 1:
        # generation after the prefill: ms per decode token, dense vs delta
        # decode, each step launched eagerly or replayed from HIP graphs
        dec = {}
        for mode in ("dense", "delta"):
            for graph in (False, True):
                cfg.decode_mode, cfg.gamma_dec = mode, a.gamma_dec
                steps_ms = []
                toks = model.generate_greedy(ids, a.decode_tokens, step_ms=steps_ms, graph=graph)
                later = steps_ms[2:] or steps_ms     # graphs: the first step of each kind records
                dec[mode + ("_graph" if graph else "")] = {
                    "ms_per_token": round(float(np.median(steps_ms)), 3),
                    "mean_ms_after_step2": round(float(np.mean(later)), 3),
                    "tokens": int(toks.shape[1])}
        line["decode"] = dict(dec, gamma_dec=a.gamma_dec, context=S,
                              note="median wall time of one decode step (all layers + lm_head); "
                                   "_graph: each step kind recorded once and replayed")
    print(json.dumps(line), flush=True)


def decode_layer(a, dev):
    """One layer's decode step against a KV cache of a.seq keys (batch 1):
    the sparse decode row, the dense anchor row, and the delta step averaged
    over gamma_dec steps (one dense + gamma_dec - 1 sparse rows + the add)."""
    import torch
    from delta_attention import ops
    H, Hkv, D, n = a.heads, a.kv_heads, a.head_dim, a.seq
    g = torch.Generator(device=dev).manual_seed(a.seed)
    q = torch.randn(1, H, 1, D, device=dev, generator=g).to(torch.bfloat16)
    k = torch.randn(1, Hkv, n, D, device=dev, generator=g).to(torch.bfloat16)
    v = torch.randn(1, Hkv, n, D, device=dev, generator=g).to(torch.bfloat16)
    scale = D ** -0.5
    delta = torch.zeros(1, H, 1, D, device=dev, dtype=torch.bfloat16)

    def timed(fn, iters):
        for _ in range(max(a.warmup, 3)):
            fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(iters):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / iters * 1e3   # us
    iters = max(a.steps, 50)
    us_sparse = timed(lambda: ops.decode_attention(q, k, v, window=a.window, sink=a.sink,
                                                   sm_scale=scale), iters)
    us_dense = timed(lambda: ops.decode_attention(q, k, v, window=0, sink=0, sm_scale=scale), iters)
    us_add = timed(lambda: ops.decode_attention(q, k, v, window=a.window, sink=a.sink,
                                                sm_scale=scale).add_(delta), iters) - us_sparse
    n_sparse = min(n, a.sink + a.window)
    row_b = Hkv * D * 2 * 2                     # one key's K and V bytes
    b_sparse, b_dense = n_sparse * row_b, n * row_b
    gd = a.gamma_dec
    us_delta = (us_dense + (gd - 1) * (us_sparse + max(us_add, 0.0))) / gd

    def hbm(b, us):
        gbs = b / (us * 1e-6) / 1e9
        return {"bytes": b, "us": round(us, 2), "gbs": round(gbs, 1),
                "frac_hbm": round(gbs / PEAK_HBM_GBS, 4)}
    print(json.dumps({
        "metric": "delta-attention decode step latency (one layer)", "value": round(us_delta, 2),
        "unit": "us", "higher_is_better": False, "dtype": "bf16", "n_gpus": 1,
        "config": {"workload": "decode row against a KV cache", "keys": n, "q_heads": H,
                   "kv_heads": Hkv, "head_dim": D, "window": a.window, "sink": a.sink,
                   "gamma_dec": gd},
        "sparse_row": hbm(b_sparse, us_sparse), "dense_row": hbm(b_dense, us_dense),
        "delta_step_avg_us": round(us_delta, 2),
        "roofline": dict(hbm(b_dense, us_dense), bound="hbm", kernel="dense decode row",
                         peak=PEAK_HBM_GBS, unit="GB/s"),
    }), flush=True)


class GpuState:
    """Samples the amdgpu sysfs files of the (single) GPU in a background
    thread while the timed work runs: current engine clock (pp_dpm_sclk, the
    level marked '*'), package power (hwmon power1_input) and junction
    temperature (hwmon temp2_input). Fields whose files are absent are None."""

    def __init__(self, period_s=0.002):
        import glob
        self.period = period_s
        devs = sorted(glob.glob("/sys/class/drm/card*/device/pp_dpm_sclk"))
        self.dev = os.path.dirname(devs[0]) if devs else None
        hw = sorted(glob.glob(os.path.join(self.dev, "hwmon", "hwmon*"))) if self.dev else []
        self.hwmon = hw[0] if hw else None
        self.samples = {"sclk_mhz": [], "power_w": [], "temp_c": []}
        self._stop = None
        self._thread = None

    @staticmethod
    def _read(path):
        try:
            with open(path) as f:
                return f.read()
        except OSError:
            return None

    def _sample(self):
        import re
        if self.dev:
            t = self._read(os.path.join(self.dev, "pp_dpm_sclk"))
            for line in (t or "").splitlines():
                m = re.search(r"(\d+)\s*Mhz\s*\*", line)
                if m:
                    self.samples["sclk_mhz"].append(float(m.group(1)))
        if self.hwmon:
            p = self._read(os.path.join(self.hwmon, "power1_input"))
            if p and p.strip().isdigit():
                self.samples["power_w"].append(int(p) / 1e6)
            c = self._read(os.path.join(self.hwmon, "temp2_input"))
            if c and c.strip().lstrip("-").isdigit():
                self.samples["temp_c"].append(int(c) / 1e3)

    def __enter__(self):
        import threading
        self._stop = threading.Event()

        def loop():
            while not self._stop.is_set():
                self._sample()
                self._stop.wait(self.period)
        self._thread = threading.Thread(target=loop, daemon=True)
        self._thread.start()
        return self

    def __exit__(self, *exc):
        self._stop.set()
        self._thread.join()

    def summary(self):
        import statistics
        out = {}
        for k, v in self.samples.items():
            out[k] = ({"min": round(min(v), 1), "median": round(statistics.median(v), 1),
                       "max": round(max(v), 1), "n": len(v)} if v else None)
        cap = self._read(os.path.join(self.hwmon, "power1_cap")) if self.hwmon else None
        out["power_cap_w"] = int(cap) / 1e6 if cap and cap.strip().isdigit() else None
        return out


TRAFFIC_SOURCE = ("profiles/hbm_traffic_llama8b_128k.md: rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE "
                  "of this workload, scaled by a 1 GiB copy; committed, not measured in this run")


def load_traffic(name):
    """HBM bytes per launch of `name` from the committed rocprofv3 PMC summary."""
    path = os.path.join(REPO, "profiles", "hbm_traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f)
        return rec.get(name, {}).get("bytes_per_launch")
    except (OSError, ValueError):
        return None


def energy(a, q, k, v, dev, O):
    """The same instruction stream on N(0,1) data and on zeros, beside a
    hipBLASLt GEMM: under the package power cap the engine clock drops with
    the switching activity of the operands, so the time per launch follows
    the energy per launch (package power x time). Prints one JSON line."""
    import torch
    from delta_attention import ops
    from delta_attention import _lib as L
    B, H, Hkv, S, D = a.batch, a.heads, a.kv_heads, a.seq, a.head_dim
    scale = D ** -0.5
    cut_n, s_p, n_anchor = ops.anchor_layout(S, a.gamma)
    idx = ops.selected_rows(S, a.gamma, str(dev))
    out = torch.empty(B, S, H, D, device=dev, dtype=torch.bfloat16)
    dense_sel = torch.zeros(B, n_anchor, H, D, device=dev, dtype=torch.bfloat16)
    ws = ops.qsparse_workspace(B, H, Hkv, idx.numel(), S, D, dev)
    zeros = tuple(torch.zeros_like(x) for x in (q, k, v))
    # algorithmic work: the fused launch covers rows < s_p, kernel (2) the selected rows
    f_fused = 4.0 * D * H * B * float(O.sparse_row_counts(S, a.window, a.sink)[:s_p].sum())
    f_rows = O.flops_qsparse(B, H, D, O.selected_rows(S, a.gamma))

    def run(fn, flop, seconds=1.5):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(); fn(); e1.record(); torch.cuda.synchronize()
        n = max(10, int(seconds * 1e3 / max(e0.elapsed_time(e1), 1e-3)))
        st = GpuState()
        with st:
            e0.record()
            for _ in range(n):
                fn()
            e1.record(); torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / n
        g = st.summary()
        w = g["power_w"]["median"] if g["power_w"] else None
        tf = flop / (ms * 1e-3) / 1e12
        return {"ms": round(ms, 4), "tflops": round(tf, 1), "frac_mfma": round(tf / PEAK_BF16_TFLOPS, 4),
                "sclk_mhz": g["sclk_mhz"]["median"] if g["sclk_mhz"] else None, "power_w": w,
                "joule": round(w * ms * 1e-3, 4) if w else None,
                "pj_per_flop": round(w * ms * 1e-3 / flop * 1e12, 4) if w else None, "launches": n}

    recs = []
    prev = ops.set_sparse_rows_per_wave(32)
    try:
        for rows in (32, 64):
            ops.set_sparse_rows_per_wave(rows)
            for data, (qq, kk, vv) in (("normal", (q, k, v)), ("zeros", zeros)):
                r = run(lambda: ops.sparse_attention_delta(qq, kk, vv, window=a.window, sink=a.sink,
                                                           sm_scale=scale, dense_sel=dense_sel,
                                                           gamma=a.gamma, s_p=s_p, out=out), f_fused)
                recs.append({"kernel": "sparse_attn_delta", "rows_per_wave": rows, "data": data, **r})
    finally:
        ops.set_sparse_rows_per_wave(prev)
    for data, (qq, kk, vv) in (("normal", (q, k, v)), ("zeros", zeros)):
        r = run(lambda: ops.qsparse_attention(qq, kk, vv, idx, scale, q_rows=idx, epi=L.DA_EPI_DENSE,
                                              out=out, n_anchor=n_anchor, delta=dense_sel, workspace=ws),
                f_rows)
        recs.append({"kernel": "qsparse_attn+merge", "data": data, **r})
    M = 8192
    x = torch.randn(M, M, device=dev).to(torch.bfloat16)
    y = torch.randn(M, M, device=dev).to(torch.bfloat16)
    z = torch.empty(M, M, device=dev, dtype=torch.bfloat16)
    for data in ("normal", "zeros"):
        if data == "zeros":
            x.zero_(); y.zero_()
        r = run(lambda: torch.matmul(x, y, out=z), 2.0 * M ** 3)
        recs.append({"kernel": "hipblaslt_gemm_8192_bf16", "data": data, **r})
    cap = GpuState().summary().get("power_cap_w")
    print(json.dumps({"metric": "energy per launch under the package power cap", "power_cap_w": cap,
                      "config": {"workload": "llama-3.1-8b-shaped delta-attention layer prefill",
                                 "seq_len": S, "gamma": a.gamma, "window": a.window, "sink": a.sink},
                      "records": recs}), flush=True)


def train_step(a, q, k, v):
    """delta_forward_train forward and backward on the workload's q/k/v with
    a seeded N(0,1) upstream gradient: median ms of each over --steps after
    --warmup, from HIP events on the current stream. Work: the forward's
    algorithmic FLOPs (both attentions); the backward's counted as 2.5x
    (five products per attended pair against two; the kernels recompute S
    and dP, 3.5x in MFMA work)."""
    import torch
    from delta_attention.train.flex_delta import delta_forward_train
    from oracle import delta_oracle as O
    B, H, Hkv, S, D = a.batch, a.heads, a.kv_heads, a.seq, a.head_dim
    g = torch.Generator(device=q.device).manual_seed(a.seed + 1)
    up = torch.randn(B, S, H, D, device=q.device, generator=g).to(torch.bfloat16)
    qq, kk, vv = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    f_fwd = (O.flops_sparse(B, H, D, S, a.window, a.sink)
             + O.flops_qsparse(B, H, D, O.selected_rows(S, a.gamma)))
    fw, bw = [], []
    for i in range(a.warmup + a.steps):
        e = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
        qq.grad = kk.grad = vv.grad = None
        e[0].record()
        out = delta_forward_train(qq, kk, vv, a.gamma, a.window, a.sink, D ** -0.5)
        e[1].record()
        out.backward(up)
        e[2].record()
        torch.cuda.synchronize()
        if i >= a.warmup:
            fw.append(e[0].elapsed_time(e[1]))
            bw.append(e[1].elapsed_time(e[2]))
    fm, bm = statistics.median(fw), statistics.median(bw)
    print(json.dumps({
        "metric": "delta_forward_train forward + backward ms per layer",
        "forward_ms": round(fm, 3), "backward_ms": round(bm, 3), "step_ms": round(fm + bm, 3),
        "forward_tflops": round(f_fwd / (fm * 1e-3) / 1e12, 1),
        "backward_tflops": round(2.5 * f_fwd / (bm * 1e-3) / 1e12, 1),
        "flop_forward": f_fwd, "steps": a.steps, "warmup": a.warmup, "dtype": "bf16",
        "config": {"workload": a.workload or "delta_forward_train layer", "batch": B, "heads": H,
                   "kv_heads": Hkv, "seq_len": S, "head_dim": D, "gamma": a.gamma,
                   "window": a.window, "sink": a.sink}}), flush=True)


def main():
    a = parse()
    if a.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {a.gpus}); the delta-attention path "
              "is not sharded across GPUs in this build.", file=sys.stderr)
        sys.exit(2)
    import torch
    from delta_attention import ops
    from delta_attention import _lib as L
    from oracle import delta_oracle as O

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    if a.copy_calibration:
        copy_calibration()
        return
    L.lib()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if a.prologue:
        prologue(a, dev)
        return
    if a.model:
        model_prefill(a, dev)
        return
    if a.decode:
        decode_layer(a, dev)
        return
    B, H, Hkv, S, D = a.batch, a.heads, a.kv_heads, a.seq, a.head_dim
    scale = D ** -0.5
    q, k, v = make_inputs(a, dev)

    if a.gamma_sweep:
        gamma_sweep(a, q, k, v, [int(x) for x in a.gamma_sweep.split(",")])
        return
    if a.train:
        train_step(a, q, k, v)
        return
    if a.energy:
        energy(a, q, k, v, dev, O)
        return
    if a.adaptive:
        adaptive_layer(a, q, k, v)
        return

    cut_n, s_p, n_anchor = ops.anchor_layout(S, a.gamma)
    idx = ops.selected_rows(S, a.gamma, str(dev))
    n_sel = idx.numel()
    rows = ops.fused_delta_rows(H, Hkv)
    fused = bool(rows) and rows % a.gamma == 0
    assert s_p > 0, "the sequence must be longer than the dense tail"
    out = torch.empty(B, S, H, D, device=dev, dtype=torch.bfloat16)
    dense_sel = torch.empty(B, n_anchor, H, D, device=dev, dtype=torch.bfloat16)
    ws = ops.qsparse_workspace(B, H, Hkv, n_sel, S, D, dev)

    # one layer prefill. Fused order: kernel (2) writes the dense tail rows into
    # the output and the dense anchor rows aside, then kernel (1) runs with
    # kernel (3) (the delta broadcast-add) fused into its epilogue. Otherwise
    # (GQA ratio 5, gamma 128 with GQA): kernel (1), kernel (2) writing the
    # tail and the deltas, kernel (3) in place.
    def step(ev=None):
        if ev is not None:
            ev[0].record()
        if fused:
            ops.qsparse_attention(q, k, v, idx, scale, q_rows=idx, epi=L.DA_EPI_DENSE, out=out,
                                  n_anchor=n_anchor, delta=dense_sel, workspace=ws)
            if ev is not None:
                ev[1].record()
            ops.sparse_attention_delta(q, k, v, window=a.window, sink=a.sink, sm_scale=scale,
                                       dense_sel=dense_sel, gamma=a.gamma, s_p=s_p, out=out)
            if ev is not None:
                ev[2].record()
                ev[3].record()
        else:
            ops.sparse_attention(q, k, v, window=a.window, sink=a.sink, sm_scale=scale, out=out)
            if ev is not None:
                ev[1].record()
            ops.qsparse_attention(q, k, v, idx, scale, q_rows=idx, epi=L.DA_EPI_DELTA, out=out,
                                  n_anchor=n_anchor, delta=dense_sel, workspace=ws)
            if ev is not None:
                ev[2].record()
            ops.delta_add(out, s_p=s_p, out=out, delta=dense_sel, gamma=a.gamma)
            if ev is not None:
                ev[3].record()

    for _ in range(a.warmup):
        step()
    torch.cuda.synchronize()

    # timed region: exactly `steps` layer prefills (engine clock, power and
    # temperature sampled meanwhile and through the per-kernel event pass)
    gpu_state = GpuState()
    with gpu_state:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(a.steps):
            step()
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) / a.steps * 1e3

        # per-kernel durations from HIP events on the launch stream (separate pass)
        evs = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(a.steps)]
        for e in evs:
            step(e)
        torch.cuda.synchronize()
    k_ms = [sum(e[i].elapsed_time(e[i + 1]) for e in evs) / a.steps for i in range(3)]

    # outside the step: the stand-alone kernels (1) and (3) on the same data, the
    # forms the sparse-only / recompute modes and the variable-stride path use
    def timed(fn):
        for _ in range(2):
            fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(a.steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / a.steps
    sparse_buf = torch.empty_like(out)
    ms_sparse = timed(lambda: ops.sparse_attention(q, k, v, window=a.window, sink=a.sink,
                                                   sm_scale=scale, out=sparse_buf))
    delta = torch.zeros(B, n_anchor, H, D, device=dev, dtype=torch.bfloat16)
    ms_add = timed(lambda: ops.delta_add(sparse_buf, s_p=s_p, out=sparse_buf, delta=delta,
                                         gamma=a.gamma))
    del sparse_buf, delta

    counts = O.sparse_row_counts(S, a.window, a.sink)
    f_fused = 4.0 * D * H * B * float(counts[:s_p].sum())   # kernel (1) rows < s_p
    f_sparse = O.flops_sparse(B, H, D, S, a.window, a.sink)  # kernel (1) over every row
    f_q = O.flops_qsparse(B, H, D, idx.cpu().numpy())
    bytes_add = B * H * D * 2 * (2 * s_p + n_anchor)
    # the layer's work: the sparse rows it needs (all rows when kernel (1) runs alone)
    f_layer = (f_fused if fused else f_sparse) + f_q
    tflops = f_layer / (ms * 1e-3) / 1e12

    def mf(f, t):
        return {"ms": round(t, 4), "tflops": round(f / t / 1e9, 2),
                "frac_mfma": round(f / t / 1e9 / PEAK_BF16_TFLOPS, 4), "flop": f}
    add = {"ms": round(ms_add, 4), "gbs": round(bytes_add / ms_add / 1e6, 1),
           "frac_hbm": round(bytes_add / ms_add / 1e6 / PEAK_HBM_GBS, 4), "bytes": bytes_add}
    if fused:
        kernels = {
            "qsparse_attn": dict(mf(f_q, k_ms[0]), rows=n_sel, in_step=True),
            "sparse_attn_delta": dict(mf(f_fused, k_ms[1]), in_step=True),
            "sparse_attn": dict(mf(f_sparse, ms_sparse), in_step=False),
            "delta_add": dict(add, in_step=False),
        }
        dom = "sparse_attn_delta" if k_ms[1] >= k_ms[0] else "qsparse_attn"
    else:
        kernels = {
            "sparse_attn": dict(mf(f_sparse, k_ms[0]), in_step=True),
            "qsparse_attn": dict(mf(f_q, k_ms[1]), rows=n_sel, in_step=True),
            "delta_add": dict(add, ms=round(k_ms[2], 4),
                              gbs=round(bytes_add / k_ms[2] / 1e6, 1),
                              frac_hbm=round(bytes_add / k_ms[2] / 1e6 / PEAK_HBM_GBS, 4),
                              in_step=True),
        }
        dom = "sparse_attn" if k_ms[0] >= k_ms[1] else "qsparse_attn"
    standard = (B, H, Hkv, S, D, a.window, a.sink, a.gamma) == (1, 32, 8, 131072, 128, 2048, 128, 64)
    for name in kernels:
        # committed rocprofv3 traffic figures are for the default workload only
        kernels[name]["traffic"] = load_traffic(name) if standard else None
    achieved = kernels[dom]["tflops"]
    roofline = {"bound": "mfma", "kernel": dom, "achieved": achieved, "peak": PEAK_BF16_TFLOPS,
                "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                "traffic": kernels[dom]["traffic"],
                "traffic_source": (TRAFFIC_SOURCE if kernels[dom]["traffic"] is not None
                                   else None)}
    # the published peak is quoted at the 2400 MHz maximum engine clock; the
    # fraction of the peak at the clock the GPU actually held is given beside it
    st = gpu_state.summary()
    if st["sclk_mhz"]:
        sclk = st["sclk_mhz"]["median"]
        roofline["sclk_mhz"] = sclk
        roofline["frac_at_sclk"] = round(achieved / (PEAK_BF16_TFLOPS * sclk / PEAK_SCLK_MHZ), 4)

    cpu = None
    if a.cpu_budget > 0:
        cpu = cpu_baseline(a, q, k, v, f_layer)

    line = {
        "metric": METRIC, "value": round(tflops, 3), "unit": "TFLOP/s", "n_gpus": 1,
        "steps": a.steps, "warmup": a.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": ("synthetic (N(0,1) q/k/v from torch's device generator seeded "
                 f"{a.seed}, drawn q, k, v" + ("" if a.no_q_scale else ", q*d^-0.5")
                 + (", per-head q/k RMSNorm" if a.qk_norm else "")
                 + f", RoPE theta {a.rope_theta:g}, bf16)"),
        "config": {"workload": a.workload or (
                       "llama-3.1-8b-shaped delta-attention layer prefill" if (H, Hkv, D) == (32, 8, 128)
                       else f"delta-attention layer prefill, {H}/{Hkv} heads, head_dim {D}"),
                   "order": "fused (2) -> (1)+(3)" if fused else "(1) -> (2) -> (3)",
                   "batch": B, "seq_len": S, "q_heads": H, "kv_heads": Hkv, "head_dim": D,
                   "window": a.window, "sink": a.sink, "gamma": a.gamma,
                   "selected_rows": n_sel, "parallelism": "none (1 GPU)"},
        "roofline": roofline, "cpu_baseline": cpu, "kernels": kernels, "gpu_state": st,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
