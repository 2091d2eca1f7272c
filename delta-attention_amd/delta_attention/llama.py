"""Llama attention with the delta-attention prefill path
(delta_attention/llama.py:60-192, 218-229, 364-496, 659-914 of the reference).

`LlamaAttention.forward` projects q/k/v, applies the fused RoPE (+ Qwen3 q/k
norm) prologue kernel and routes `config._attn_implementation == "window"` to
`delta_forward`: query-sparse dense rows (kernel 2, dense tail into the output,
dense anchor rows aside), then key-sparse attention (kernel 1) with the delta
broadcast-add (kernel 3) fused into its epilogue, or kernels 1 -> 2 -> 3 when
the stride does not divide the row tile. "sdpa_rectangle" (decode after the
prefill) routes to `sdpa_rectangle_forward` and the sparse / delta decode.
The module's config object needs the Llama fields
(hidden_size, num_attention_heads, num_key_value_heads, optional head_dim,
attention_bias, attention_dropout, rms_norm_eps, _attn_implementation) and the
pipeline knobs of `config.PIPELINE_FIELDS`.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch
from torch import nn

from . import _lib as L
from . import ops
from .delta_kernel import attention as qsa_kernel
from .timing import region


# per-device side streams of the adaptive path (LlamaAttention._side_stream)
_SIDE_STREAMS: dict = {}

class LlamaRMSNorm(nn.Module):
    """x / sqrt(mean(x^2) + eps) in float32, times the weight, in the input
    dtype (llama.py:60-74)."""

    def __init__(self, hidden_size: int, eps: float = 1e-6):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(hidden_size))
        self.variance_epsilon = eps

    def forward(self, hidden_states: torch.Tensor) -> torch.Tensor:
        dt = hidden_states.dtype
        x = hidden_states.to(torch.float32)
        x = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + self.variance_epsilon)
        return self.weight.to(dt) * x.to(dt)


def llama3_inv_freq(inv_freq: torch.Tensor, factor: float = 8.0, low_freq_factor: float = 1.0,
                    high_freq_factor: float = 4.0,
                    original_max_position_embeddings: int = 8192) -> torch.Tensor:
    """Llama 3.1's RoPE frequency scaling (the "llama3" rope type the
    reference's LlamaRotaryEmbedding takes from the model config,
    llama.py:83-127): wavelengths longer than original/low_freq_factor are
    divided by `factor`, shorter than original/high_freq_factor kept, and the
    band between interpolated linearly in original/wavelength."""
    low_wl = original_max_position_embeddings / low_freq_factor
    high_wl = original_max_position_embeddings / high_freq_factor
    wavelen = 2 * torch.pi / inv_freq
    scaled = torch.where(wavelen > low_wl, inv_freq / factor, inv_freq)
    smooth = (original_max_position_embeddings / wavelen - low_freq_factor) / (high_freq_factor - low_freq_factor)
    smoothed = (1 - smooth) * scaled / factor + smooth * scaled
    medium = (wavelen >= high_wl) & (wavelen <= low_wl)
    return torch.where(medium, smoothed, scaled)


def rope_cos_sin(position_ids: torch.Tensor, head_dim: int, theta: float,
                 dtype: torch.dtype, rope_scaling: Optional[dict] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Default RoPE tables for position_ids [b, s] -> cos/sin [b, s, head_dim]:
    inv_freq = theta^(-2i/d), angles in float32, emb = cat(freqs, freqs)
    (llama.py:129-158). rope_scaling {"rope_type": "llama3", factor, ...}
    applies llama3_inv_freq."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64,
                                             device=position_ids.device).float() / head_dim))
    if rope_scaling:
        kw = dict(rope_scaling)
        kind = kw.pop("rope_type", kw.pop("type", "llama3"))
        kw.pop("type", None)
        if kind != "default":
            if kind != "llama3":
                raise NotImplementedError(f"rope_scaling type {kind!r} (built: default, llama3)")
            inv_freq = llama3_inv_freq(inv_freq, **kw)
    freqs = position_ids[..., None].float() * inv_freq[None, None, :]
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def fuse_linears(*mods: nn.Linear):
    """Concatenate the weights (and biases) of linears that read the same input
    into one buffer along the output dim and re-point each module's parameters
    at its slice. -> (weight, bias or None) of the fused product."""
    with torch.no_grad():
        w = torch.cat([m.weight.detach() for m in mods], 0)
        has_b = all(m.bias is not None for m in mods)
        b = torch.cat([m.bias.detach() for m in mods], 0) if has_b else None
        o = 0
        for m in mods:
            n = m.out_features
            m.weight = nn.Parameter(w[o:o + n], requires_grad=m.weight.requires_grad)
            if has_b:
                m.bias = nn.Parameter(b[o:o + n], requires_grad=m.bias.requires_grad)
            o += n
    return (w, b)


# Token counts up to which the fused products run (decode steps, short
# prompts: one GEMV instead of two or three). Long prefills keep the separate
# GEMMs: at 131072 tokens the fused gate/up product plus the down product on
# its strided half measured 1 % slower (30.2 vs 29.8 ms per layer).
FUSED_MAX_ROWS = 64


def fused_params(fused, mods, rows: int = 1):
    """(weight, bias) of a fuse_linears product while every module's parameters
    are still its slices and the input has at most FUSED_MAX_ROWS rows;
    (None, None) otherwise. The fused buffer is not an autograd leaf, so with
    gradients enabled for any of the modules' parameters the separate products
    (which give each parameter its gradient) are used."""
    if fused is None or rows > FUSED_MAX_ROWS:
        return None, None
    if torch.is_grad_enabled() and any(
            p.requires_grad for m in mods for p in (m.weight, m.bias) if p is not None):
        return None, None
    w, b = fused
    o = 0
    for m in mods:
        if (m.weight.data_ptr() != w.data_ptr() + o * w.stride(0) * w.element_size()
                or m.weight.shape[0] != m.out_features or m.weight.dtype != w.dtype):
            return None, None
        if b is not None and (m.bias is None or m.bias.data_ptr() != b.data_ptr() + o * b.element_size()):
            return None, None
        o += m.out_features
    return w, b


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def apply_rotary_pos_emb(q, k, cos, sin, position_ids=None, unsqueeze_dim: int = 1):
    """q*cos + rotate_half(q)*sin, same for k (llama.py:168-192)."""
    cos = cos.unsqueeze(unsqueeze_dim)
    sin = sin.unsqueeze(unsqueeze_dim)
    return (q * cos) + (rotate_half(q) * sin), (k * cos) + (rotate_half(k) * sin)


def repeat_kv(hidden_states: torch.Tensor, n_rep: int) -> torch.Tensor:
    """[b, hkv, s, d] -> [b, hkv * n_rep, s, d], head h reading kv head h // n_rep
    (llama.py:218-229). The delta path never needs it: its kernels read the
    Hkv heads directly."""
    b, hkv, s, d = hidden_states.shape
    if n_rep == 1:
        return hidden_states
    return hidden_states[:, :, None].expand(b, hkv, n_rep, s, d).reshape(b, hkv * n_rep, s, d)


def _adaptive_stride_stats(logs, layer, s, s_p, adapt_chunk, window, sink):
    """The stride statistics of one adaptive pass (llama.py:806-824) from its
    per-chunk device logs: per chunk its first row, stride, mean / min delta
    cosine and anchor count, the anchor total and the effective sparsity of
    the anchors plus the dense tail."""
    from .stride import effective_sparsity, plan_chunks

    log_mean, log_min, log_gamma, log_n = (t.tolist() for t in logs)
    chunk_log, idx_parts = [], []
    for c, (start, end) in enumerate(plan_chunks(s_p, adapt_chunk)):
        idx_parts.append(torch.arange(start, end, log_gamma[c], dtype=torch.int64)[:log_n[c]])
        chunk_log.append({"start": int(start), "gamma": int(log_gamma[c]),
                          "cos_mean": float(log_mean[c]), "cos_min": float(log_min[c]),
                          "n_anchors": int(log_n[c])})
    idx = torch.cat(idx_parts) if idx_parts else torch.empty(0, dtype=torch.int64)
    tail_idx = torch.arange(s_p, s, dtype=torch.int64)
    return {
        "kind": "stride", "layer": layer, "seq_len": s,
        "effective_sparsity": effective_sparsity(torch.cat((idx, tail_idx)), s, window, sink),
        "n_anchors": int(idx.numel()), "chunks": chunk_log,
    }


class _LazyStats:
    """An attribute that may be set to a zero-argument callable which builds
    its value: the first read calls it and keeps the result. The layer stores
    its telemetry this way, so that reading it back (a device sync) waits
    until someone asks."""

    def __set_name__(self, owner, name):
        self.key = "_lazy" + name

    def __get__(self, obj, objtype=None):
        if obj is None:
            return self
        value = obj.__dict__.get(self.key)
        if callable(value):
            value = obj.__dict__[self.key] = value()
        return value

    def __set__(self, obj, value):
        obj.__dict__[self.key] = value


def _deferred(fn, *args, device=None):
    """A zero-argument call of fn(*args) that runs on the stream current now
    (the one that produced the device values fn reads back), whatever stream
    is current when it is finally called."""
    stream = torch.cuda.current_stream(device) if device is not None and device.type == "cuda" else None

    def call():
        if stream is None:
            return fn(*args)
        with torch.cuda.stream(stream):
            return fn(*args)

    return call


class LlamaAttention(nn.Module):
    # telemetry of the last prefill, read back on first access: the drift
    # summary (log_drift) and the adaptive stride's statistics
    _drift_stats = _LazyStats()
    _stride_stats = _LazyStats()

    def __init__(self, config, layer_idx: int):
        super().__init__()
        self.config = config
        self.layer_idx = layer_idx
        self.head_dim = getattr(config, "head_dim", None) or config.hidden_size // config.num_attention_heads
        self.num_key_value_groups = config.num_attention_heads // config.num_key_value_heads
        self.scaling = self.head_dim ** -0.5
        self.attention_dropout = getattr(config, "attention_dropout", 0.0)
        self.is_causal = True
        bias = getattr(config, "attention_bias", False)
        self.q_proj = nn.Linear(config.hidden_size, config.num_attention_heads * self.head_dim, bias=bias)
        self.k_proj = nn.Linear(config.hidden_size, config.num_key_value_heads * self.head_dim, bias=bias)
        self.v_proj = nn.Linear(config.hidden_size, config.num_key_value_heads * self.head_dim, bias=bias)
        self.o_proj = nn.Linear(config.num_attention_heads * self.head_dim, config.hidden_size, bias=bias)
        self._drift_stats = None
        self._stride_stats = None
        self._qkv_fused = None

    def fuse_projections(self):
        """Move the q/k/v projection weights (and biases) into one
        [(Hq + 2 Hkv) * d, hidden] buffer and make the three modules'
        parameters views of it, so that one product computes all three (one
        GEMV per decode step instead of three; inputs of more than
        FUSED_MAX_ROWS tokens keep the three products). Module names,
        state-dict keys and values are unchanged; if the parameters are later
        replaced (e.g. by .to()), the forward falls back to three products."""
        self._qkv_fused = fuse_linears(self.q_proj, self.k_proj, self.v_proj)

    def _qkv_product(self, hidden_states):
        """The fused q/k/v product [..., (Hq + 2 Hkv) * d], or None when the
        projections are not (or no longer) fused."""
        w, b = fused_params(self._qkv_fused, (self.q_proj, self.k_proj, self.v_proj),
                            hidden_states.numel() // hidden_states.shape[-1])
        if w is None:
            return None
        return nn.functional.linear(hidden_states, w, b)

    # -- knobs -------------------------------------------------------------
    def _sink(self) -> int:
        return int(getattr(self.config, "sink_tokens", 1024))

    # -- kernel (1) ----------------------------------------------------------
    def hip_attention_interface(self, module, query, key, value, attention_mask,
                                dropout: float = 0.0, scaling: Optional[float] = None,
                                sliding_window: Optional[int] = None, softcap=None,
                                position_ids=None, output_attentions: bool = False,
                                use_cache: bool = False, rope_cos=None, rope_sin=None,
                                out: Optional[torch.Tensor] = None):
        """Key-sparse (sink + sliding window) attention; returns ([b, s, h, d], None)
        (llama.py:364-449, "window" branch). fp32 inputs run in bf16 and the
        result is cast back (llama.py:382-388, 493-494)."""
        assert self.config._attn_implementation == "window", (
            f"{self.config._attn_implementation!r}: only the 'window' sparse pass is built")
        assert softcap is None and not output_attentions
        original_dtype = query.dtype
        if query.dtype == torch.float32:
            query, key, value = query.to(torch.bfloat16), key.to(torch.bfloat16), value.to(torch.bfloat16)
        assert query.dtype in (torch.bfloat16, torch.float16), query.dtype
        scaling = self.scaling if scaling is None else scaling
        window = sliding_window if sliding_window is not None else 1024
        output = ops.sparse_attention(query, key, value, window=int(window), sink=self._sink(),
                                      sm_scale=float(scaling), out=out)
        if output.dtype != original_dtype:
            output = output.to(original_dtype)
        return output, None

    # -- the delta composition -------------------------------------------------
    def delta_forward(self, module, query_states, key_states, value_states,
                      attention_mask=None, dropout: float = 0.0, scaling: float = 1.0, **kwargs):
        """Delta attention prefill (llama.py:659-757). q [b, h, s, d] and k/v
        [b, hkv, s, d] post-RoPE -> ([b, s, h, d], None).

        mode "sparse-only": kernel (1) only. "recompute": kernel (1), then the
        selected rows (anchors every delta_lambda rows + the cut_n dense tail)
        are replaced by dense rows. "delta": sparse + the anchor delta over each
        stride group, dense tail rows (ops.delta_prefill: kernel (2) then kernel
        (1) with the broadcast-add in its epilogue, bit-identical to kernels
        (1) -> (2) -> (3)).
        """
        cfg = self.config
        lambd = int(cfg.delta_lambda)
        window = int(cfg.sliding_window)
        mode = cfg.mode
        b, h, s, d = query_states.size()
        assert h == cfg.num_attention_heads, (h, s)

        # the reference's branch order (llama.py:695-711): "sparse-only" returns
        # the sparse pass, then the adaptive policy replaces the uniform stride
        # for every other mode ("recompute" included)
        if getattr(cfg, "stride_policy", "fixed") == "adaptive" and mode != "sparse-only":
            # the key-sparse pass runs inside, in row chunks beside the chunk loop
            cut_n = s % lambd + max(128, lambd)
            s_p = s - cut_n
            return self.delta_adaptive_forward(query_states, key_states, value_states, None,
                                               s, s_p, cut_n, scaling), None

        original_dtype = query_states.dtype
        q, k, v = query_states, key_states, value_states
        if q.dtype == torch.float32:
            q, k, v = q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16)
        log_drift = bool(getattr(cfg, "log_drift", False)) and mode == "delta"
        out = ops.delta_prefill(q, k, v, gamma=lambd, window=window, sink=self._sink(),
                                sm_scale=float(scaling), mode=mode, return_delta=log_drift)
        delta = None
        if log_drift:
            out, delta = out
        if delta is not None and delta.shape[1] >= 2:
            from .drift import drift_cosines, drift_summary_of

            # the cosines are launched now; the summary is read back on first access
            self._drift_stats = _deferred(drift_summary_of, *drift_cosines(delta),
                                          int(self.layer_idx), lambd, s, device=delta.device)
        if out.dtype != original_dtype:
            out = out.to(original_dtype)
        return out, None

    def delta_adaptive_forward(self, query_states, key_states, value_states, sparse_attn_output,
                               s, s_p, cut_n, scaling):
        """Chunked adaptive anchor placement (llama.py:759-824): anchors at the
        current stride inside each adapt_chunk rows, stride re-planned from the
        chunk's mean consecutive-delta cosine, variable-stride broadcast
        (kernel 3 with an anchor list), dense cut_n tail.

        The whole layer is one library call (da_adapt_layer_fwd), which
        enqueues the chunk loop without reading anything back: each chunk's
        dense anchor rows (kernel (2) over a row list of max_n slots, -1 past
        the chunk's anchors), its delta cosines rnd(dense - sparse[idx]) with
        their mean / min logged and the next stride (stride.py:55-86) and row
        list decided on the device, then the chunk's broadcast-add in place.
        With sparse_attn_output None the key-sparse pass runs in the same call,
        one launch per chunk on a second stream, and each chunk's decision
        waits only for its own rows of it, so the latency-bound chunk loop runs
        beside the MFMA-heavy sparse launches (rows >= s_p, which the dense tail
        replaces, are not computed). The result equals the reference's
        cat(apply_delta_variable(...), tail_dense): every stride group lies
        inside one chunk, its delta is rnd(dense - sparse[anchor]) (the
        rounding of stride.py:38) and its rows get rnd(sparse + delta); the tail
        rows come from the query-sparse kernel's scatter epilogue. The stride
        statistics are read from the per-chunk logs when first asked for."""
        from .stride import ADAPT_MARGIN

        cfg = self.config
        device = query_states.device
        q, k, v = query_states, key_states, value_states
        if q.dtype == torch.float32:
            q, k, v = q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16)
        b, h, _, d = q.shape
        overlap = sparse_attn_output is None
        if overlap:
            out = torch.empty((b, s, h, d), dtype=q.dtype, device=device)
        else:
            out = sparse_attn_output
            if out.dtype != q.dtype:
                out = out.to(q.dtype)
            out = out.contiguous()
        adapt_chunk = int(cfg.adapt_chunk)
        logs = ops.adapt_layer(
            q, k, v, out, s_p=s_p, window=int(cfg.sliding_window), sink=self._sink(),
            sm_scale=float(scaling), adapt_chunk=adapt_chunk, gamma0=int(cfg.delta_lambda),
            gamma_min=int(cfg.gamma_min), gamma_max=int(cfg.gamma_max),
            trigger=getattr(cfg, "stride_trigger", "absolute"),
            threshold=float(cfg.adapt_threshold), margin=ADAPT_MARGIN,
            k_sd=float(getattr(cfg, "adapt_k", 2.0)),
            side_stream=self._side_stream(device) if overlap else None)
        self._stride_stats = _deferred(
            _adaptive_stride_stats, logs, int(self.layer_idx), int(s), int(s_p), adapt_chunk,
            int(cfg.sliding_window), self._sink(), device=device)
        return out.to(query_states.dtype)


    @staticmethod
    def _side_stream(device):
        """The second stream (default priority) of the adaptive path's
        row-chunked key-sparse pass: one per device, shared by every layer
        (the layers run one after another)."""
        idx = torch.device(device).index
        idx = torch.cuda.current_device() if idx is None else idx
        st = _SIDE_STREAMS.get(idx)
        if st is None:
            st = _SIDE_STREAMS[idx] = torch.cuda.Stream(device=idx)
        return st

    # -- decode (llama.py:498-657) ---------------------------------------------------
    def sdpa_rectangle_forward(self, module, query_states, key_states, value_states,
                               attention_mask=None, dropout: float = 0.0, scaling: float = 1.0,
                               **kwargs):
        """Queries at the end of the KV cache: row i of s attends keys
        0 .. n - s + i (llama.py:498-535) -> ([b, s, h, d], None). One-row
        steps with decode_mode "sparse" / "delta" go to delta_decode_forward."""
        b, h, s, d = query_states.size()
        n_keys = kwargs.get("n_keys")
        if s == 1 and getattr(self.config, "decode_mode", "dense") != "dense":
            return self.delta_decode_forward(module, query_states, key_states, value_states,
                                             scaling=scaling, **kwargs)
        q, k, v = self._half(query_states, key_states, value_states)
        n = k.size(2)
        if s == 1:
            out = ops.decode_attention(q, k, v, window=0, sink=0, sm_scale=float(scaling),
                                       n_keys=n_keys)
        else:
            assert n_keys is None, "a device key count serves one-row decode steps"
            mask = torch.arange(n - s, n, device=q.device, dtype=torch.int64)[None]
            out = qsa_kernel(q, k, v, mask, float(scaling))
        return out.transpose(1, 2).contiguous().to(query_states.dtype), None

    @staticmethod
    def _half(q, k, v):
        if q.dtype == torch.float32:
            return q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16)
        return q, k, v

    def _decode_sparse_row(self, q, k, v, scaling, n_keys=None):
        """One decode row over the sink tokens + the last sliding_window keys of
        the cache, softmax over exactly that set (llama.py:537-549; every key
        when the cache holds at most sink + window keys). GQA native."""
        return ops.decode_attention(q, k, v, window=int(self.config.sliding_window),
                                    sink=self._sink(), sm_scale=float(scaling), n_keys=n_keys)

    def _delta_decode_recorded(self, q, k, v, scaling, n_keys, anchor: bool, out_dtype):
        """delta_decode_forward's fixed-policy step in the form a recorded
        decode step needs: the key count is on the device, the anchor decision
        comes from the caller (the same schedule: the first step, then every
        min(gamma_dec, gamma_dec_max) steps), and the cached delta is one
        persistent buffer per layer, written in place on anchor steps."""
        if self.config.decode_mode == "delta" and not anchor:
            st = getattr(self, "_dec_static", None)
            assert st is not None, "a delta decode step needs an anchor step first"
            # the sparse row and the cached delta's add in one launch
            out = ops.decode_attention(q, k, v, window=int(self.config.sliding_window),
                                       sink=self._sink(), sm_scale=float(scaling),
                                       n_keys=n_keys, add=st["last_delta"])
            return out.transpose(1, 2).contiguous().to(out_dtype), None
        sparse_out = self._decode_sparse_row(q, k, v, scaling, n_keys)
        if self.config.decode_mode == "sparse":
            out = sparse_out
        elif anchor:
            dense_out = ops.decode_attention(q, k, v, window=0, sink=0, sm_scale=float(scaling),
                                             n_keys=n_keys)
            st = getattr(self, "_dec_static", None)
            if st is None:    # first anchor step (run eagerly before any recording)
                st = self._dec_static = {"last_delta": torch.empty_like(dense_out)}
            torch.sub(dense_out, sparse_out, out=st["last_delta"])
            out = dense_out
        return out.transpose(1, 2).contiguous().to(out_dtype), None

    def delta_decode_forward(self, module, query_states, key_states, value_states,
                             scaling: float = 1.0, **kwargs):
        """Decode step of the sparse / delta decode (semantics: llama.py:551-634).
        `decode_policy.RefreshRule` decides whether this step is an anchor;
        anchors output the dense row and keep dense - sparse in `_dec_state`,
        the other steps output sparse + that correction (recorded decode steps
        take `_delta_decode_recorded`, whose non-anchor steps add it in the
        sparse row's launch). log_drift appends a record per step to
        `_dec_drift_points`."""
        from . import decode_policy as dp
        assert query_states.size(0) == 1, "sparse/delta decode supports batch size 1 only"
        mode = self.config.decode_mode
        assert mode in ("sparse", "delta"), mode
        q, k, v = self._half(query_states, key_states, value_states)
        if kwargs.get("n_keys") is not None:
            return self._delta_decode_recorded(q, k, v, scaling, kwargs["n_keys"],
                                               bool(kwargs.get("decode_anchor")), query_states.dtype)

        def emit(x):
            return x.transpose(1, 2).contiguous().to(query_states.dtype), None

        if mode == "sparse":
            return emit(self._decode_sparse_row(q, k, v, scaling))
        state = getattr(self, "_dec_state", None) or dp.new_state()
        rule = dp.RefreshRule.of(self.config)
        logging = bool(getattr(self.config, "log_drift", False))
        sparse = self._decode_sparse_row(q, k, v, scaling)
        anchor, since = rule.decide(state, sparse)
        dense = (ops.decode_attention(q, k, v, window=0, sink=0, sm_scale=float(scaling))
                 if anchor or logging else None)
        out = dense if anchor else sparse + state["last_delta"]
        dp.commit(state, anchor, since, sparse, dense, out)
        if logging:
            pts = getattr(self, "_dec_drift_points", None) or []
            pts.append(dp.drift_point(state, since, anchor, sparse, dense, out))
            self._dec_drift_points = pts
        self._dec_state = state
        return emit(out)

    # -- projections and dispatch -----------------------------------------------
    def _qkv(self, hidden_states, hidden_shape):
        """The reference's model-family hook (llama.py:826-830): projected q/k/v
        as [b, h, s, d] views, before RoPE (torch ops)."""
        q = self.q_proj(hidden_states).view(hidden_shape).transpose(1, 2)
        k = self.k_proj(hidden_states).view(hidden_shape).transpose(1, 2)
        v = self.v_proj(hidden_states).view(hidden_shape).transpose(1, 2)
        return q, k, v

    def _qk_norm(self):
        """(q_norm weight, k_norm weight, eps) applied before RoPE, or Nones."""
        return None, None, 1e-6

    def _qkv_rope(self, hidden_states, hidden_shape, cos, sin, timer=None, append=None):
        """Projections, then the fused prologue kernel (optional per-head q/k
        RMSNorm + RoPE) in place on the [b, s, h, d] projection outputs; returns
        [b, h, s, d] views, the layout the attention kernels read without copies.
        append: a cache in static (one-token, device-held row) mode; the same
        launch then writes the rotated k and v into it and (q, None, None) is
        returned."""
        if hidden_states.dtype not in (torch.bfloat16, torch.float16):
            # float32 models keep the reference's float32 RoPE (torch ops); the
            # attention kernels then run in bf16 as delta_forward casts
            q, k, v = self._qkv(hidden_states, hidden_shape)
            q, k = apply_rotary_pos_emb(q, k, cos, sin)
            return q, k, v
        with region(timer, "qkv_gemm"):
            qkv = self._qkv_product(hidden_states)
            if qkv is None:
                q = self.q_proj(hidden_states).view(hidden_shape)
                k = self.k_proj(hidden_states).view(hidden_shape)
                v = self.v_proj(hidden_states).view(hidden_shape)
            else:
                # strided views of the one product: the prologue kernel and the
                # attention kernels take row strides
                nq, nk = self.q_proj.out_features, self.k_proj.out_features
                q = qkv[..., :nq].unflatten(-1, (-1, self.head_dim))
                k = qkv[..., nq:nq + nk].unflatten(-1, (-1, self.head_dim))
                v = qkv[..., nq + nk:].unflatten(-1, (-1, self.head_dim))
        with region(timer, "rope_prologue"):
            qw, kw, eps = self._qk_norm()
            if append is not None:
                ops.rope_qk_append(q, k, v, cos, sin, append.k[self.layer_idx],
                                   append.v[self.layer_idx], append.pos, q_norm_w=qw,
                                   k_norm_w=kw, eps=eps)
                return q.transpose(1, 2), None, None
            ops.rope_qk(q, k, cos, sin, q_norm_w=qw, k_norm_w=kw, eps=eps)
        return q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)

    def forward(self, hidden_states, position_embeddings, attention_mask=None,
                past_key_value=None, cache_position=None, **kwargs):
        """hidden [b, s, hidden] -> (o_proj(attention) [b, s, hidden], None)
        (llama.py:832-914); `window` routes to delta_forward."""
        input_shape = hidden_states.shape[:-1]
        hidden_shape = (*input_shape, -1, self.head_dim)
        cos, sin = position_embeddings
        timer = kwargs.get("timer")
        static = (past_key_value is not None and getattr(past_key_value, "static", False)
                  and hidden_states.dtype in (torch.bfloat16, torch.float16))
        query_states, key_states, value_states = self._qkv_rope(
            hidden_states, hidden_shape, cos, sin, timer, append=past_key_value if static else None)
        extra = {}
        if past_key_value is not None:
            if key_states is None:   # appended by the prologue launch
                key_states, value_states = past_key_value.views(self.layer_idx)
            else:
                key_states, value_states = past_key_value.update(
                    key_states, value_states, self.layer_idx,
                    {"sin": sin, "cos": cos, "cache_position": cache_position})
            if getattr(past_key_value, "static", False):
                # recorded decode step: full cache buffers, key count on the device
                extra = {"n_keys": past_key_value.n_keys,
                         "decode_anchor": bool(past_key_value.anchor)}
        impl = self.config._attn_implementation
        if impl == "window":
            interface = self.delta_forward
        elif impl == "sdpa_rectangle":       # decode steps after the prefill (sample.py:160)
            interface = self.sdpa_rectangle_forward
        else:
            raise NotImplementedError(
                f"attention implementation {impl!r} is not part of the MI355X delta path "
                "(use 'window', then 'sdpa_rectangle' for decode)")
        with region(timer, "attention_kernels"):
            attn_output, attn_weights = interface(
                self, query_states, key_states, value_states, attention_mask,
                dropout=0.0 if not self.training else self.attention_dropout, scaling=self.scaling,
                **extra)
        assert attn_output.shape[-2] == self.config.num_attention_heads, attn_output.shape
        b, s, _, _ = attn_output.size()
        attn_output = attn_output.reshape(b, s, -1)
        with region(timer, "o_gemm"):
            return self.o_proj(attn_output), attn_weights
