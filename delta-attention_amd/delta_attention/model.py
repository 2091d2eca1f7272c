"""Llama causal LM with delta attention in every layer, for the full-model
prefill (time to first token): the reference's LlamaMLP, LlamaDecoderLayer,
LlamaModel and LlamaForCausalLM (delta_attention/llama.py:195-215, 917-1004,
1006-1029, 1111-1145, 1455-1470), random-initialised as its `_init_weights`
does (normal(0, initializer_range) for every linear and embedding weight,
RMSNorm weights 1).

Compute: projections and the MLP GEMMs are torch matmuls (hipBLASLt); the
attention layer is `LlamaAttention` (fused RoPE prologue + the delta-attention
kernels); every residual add is fused into the RMSNorm that follows it
(`ops.add_rmsnorm`), and the SwiGLU gate is one element-wise kernel
(`ops.swiglu`). A decoder layer therefore hands on (branch output, residual)
and the next norm forms their sum.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

import torch
from torch import nn

from . import ops
from .llama import LlamaAttention, LlamaRMSNorm, fuse_linears, fused_params, rope_cos_sin
from .timing import Timer, region as _region


@dataclass
class LlamaConfig:
    """Llama-3.1-8B architecture plus the delta-attention pipeline knobs."""
    vocab_size: int = 128256
    hidden_size: int = 4096
    intermediate_size: int = 14336
    num_hidden_layers: int = 32
    num_attention_heads: int = 32
    num_key_value_heads: int = 8
    head_dim: int = 128
    rope_theta: float = 500000.0
    rope_scaling: Optional[dict] = field(default_factory=lambda: {
        "rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
        "original_max_position_embeddings": 8192})
    rms_norm_eps: float = 1e-5
    initializer_range: float = 0.02
    attention_bias: bool = False
    mlp_bias: bool = False
    attention_dropout: float = 0.0
    tie_word_embeddings: bool = False
    _attn_implementation: str = "window"
    mode: str = "delta"
    delta_lambda: int = 64
    sliding_window: int = 2048
    sink_tokens: int = 128
    stride_policy: str = "fixed"
    # adaptive stride (stride_policy "adaptive"), the defaults of config.Config
    gamma_min: int = 16
    gamma_max: int = 256
    adapt_chunk: int = 4096
    adapt_threshold: float = 0.95
    stride_trigger: str = "absolute"
    adapt_k: float = 2.0
    log_drift: bool = False
    decode_mode: str = "dense"
    gamma_dec: int = 32
    refresh_policy: str = "fixed"
    drift_threshold: float = 0.95
    drift_k: float = 2.0
    gamma_dec_max: int = 128


class KVCache:
    """Per-layer key/value storage preallocated as [B, max_len, Hkv, D] (the
    projection layout, so appending is one strided copy); `update` appends
    and returns [B, Hkv, len, D] views, which the kernels read in place."""

    def __init__(self, config, batch: int, max_len: int, device, dtype):
        shape = (batch, max_len, config.num_key_value_heads, config.head_dim)
        n = config.num_hidden_layers
        self.k = [torch.empty(shape, device=device, dtype=dtype) for _ in range(n)]
        self.v = [torch.empty(shape, device=device, dtype=dtype) for _ in range(n)]
        self.len = [0] * n
        self.max_len = max_len
        # static mode (decode steps recorded in a HIP graph): the appended row
        # and the key count live on the device and advance there
        self.static = False
        self.pos = None        # int64 [1]: row of the next append
        self.n_keys = None     # int32 [1]: keys after that append
        self.anchor = False    # delta decode: whether the recorded step is an anchor step

    def start_static(self):
        """Switch to device-side positions: one-token appends go to row
        `pos` and the decode rows read `n_keys` keys of the full buffers."""
        assert len(set(self.len)) == 1, self.len
        dev = self.k[0].device
        self.pos = torch.full((1,), self.len[0], dtype=torch.int64, device=dev)
        self.n_keys = torch.full((1,), self.len[0] + 1, dtype=torch.int32, device=dev)
        self.static = True

    def advance_static(self):
        """Device-side step to the next position (recorded with the step)."""
        self.pos.add_(1)
        self.n_keys.add_(1)

    def stop_static(self, n_appended: int):
        """Back to host-side lengths after n_appended one-token steps."""
        self.len = [l + n_appended for l in self.len]
        self.static, self.pos, self.n_keys, self.anchor = False, None, None, False

    def views(self, layer_idx: int):
        """Static mode: [B, Hkv, max_len, D] views of a layer's full buffers
        (the decode rows read the device-held key count of them)."""
        assert self.static
        return self.k[layer_idx].transpose(1, 2), self.v[layer_idx].transpose(1, 2)

    def update(self, key_states, value_states, layer_idx: int, cache_kwargs=None):
        s = key_states.shape[2]
        if self.static:
            assert s == 1, "static mode appends one token per step"
            self.k[layer_idx].index_copy_(1, self.pos, key_states.transpose(1, 2))
            self.v[layer_idx].index_copy_(1, self.pos, value_states.transpose(1, 2))
            return self.k[layer_idx].transpose(1, 2), self.v[layer_idx].transpose(1, 2)
        l0 = self.len[layer_idx]
        assert l0 + s <= self.max_len, (l0, s, self.max_len)
        self.k[layer_idx][:, l0:l0 + s] = key_states.transpose(1, 2)
        self.v[layer_idx][:, l0:l0 + s] = value_states.transpose(1, 2)
        self.len[layer_idx] = l0 + s
        return (self.k[layer_idx][:, :l0 + s].transpose(1, 2),
                self.v[layer_idx][:, :l0 + s].transpose(1, 2))

    def seq_len(self) -> int:
        return self.len[0]


class LlamaMLP(nn.Module):
    """down_proj(silu(gate_proj(x)) * up_proj(x)) (llama.py:195-215)."""

    def __init__(self, config):
        super().__init__()
        bias = getattr(config, "mlp_bias", False)
        self.gate_proj = nn.Linear(config.hidden_size, config.intermediate_size, bias=bias)
        self.up_proj = nn.Linear(config.hidden_size, config.intermediate_size, bias=bias)
        self.down_proj = nn.Linear(config.intermediate_size, config.hidden_size, bias=bias)
        self._gate_up_fused = None

    def fuse_projections(self):
        """gate_proj and up_proj as one product (views of one weight buffer;
        names and values unchanged; see LlamaAttention.fuse_projections)."""
        self._gate_up_fused = fuse_linears(self.gate_proj, self.up_proj)

    def forward(self, x: torch.Tensor, timer: Optional[Timer] = None) -> torch.Tensor:
        with _region(timer, "mlp_gemm"):
            w, b = fused_params(self._gate_up_fused, (self.gate_proj, self.up_proj),
                                x.numel() // x.shape[-1])
            if w is None:
                g = self.gate_proj(x)
                u = self.up_proj(x)
            else:
                gu = nn.functional.linear(x, w, b)
                n = self.gate_proj.out_features
                g, u = gu[..., :n], gu[..., n:]
        with _region(timer, "swiglu"):
            if g.dtype in (torch.bfloat16, torch.float16):
                a = ops.swiglu(g, u, out=g)     # in place over the gate
            else:
                a = nn.functional.silu(g) * u
        del u
        with _region(timer, "mlp_gemm"):
            return self.down_proj(a)


def _norm(norm: LlamaRMSNorm, x: torch.Tensor, residual: Optional[torch.Tensor], timer):
    """(norm(x + residual), x + residual) with the add fused into the norm."""
    with _region(timer, "norm"):
        if x.dtype in (torch.bfloat16, torch.float16) and x.shape[-1] in (2048, 4096, 5120, 8192):
            if residual is None:
                return ops.add_rmsnorm(x, norm.weight, norm.variance_epsilon), x
            return ops.add_rmsnorm(x, norm.weight, norm.variance_epsilon, residual=residual,
                                   residual_out=residual)
        h = x if residual is None else residual + x
        return norm(h), h


class LlamaDecoderLayer(nn.Module):
    attn_cls = LlamaAttention  # model-family hook (qwen3.py overrides)

    def __init__(self, config, layer_idx: int):
        super().__init__()
        self.self_attn = self.attn_cls(config, layer_idx)
        self.mlp = LlamaMLP(config)
        self.input_layernorm = LlamaRMSNorm(config.hidden_size, eps=config.rms_norm_eps)
        self.post_attention_layernorm = LlamaRMSNorm(config.hidden_size, eps=config.rms_norm_eps)

    def forward_fused(self, hidden_states: torch.Tensor, residual: Optional[torch.Tensor],
                      position_embeddings, timer: Optional[Timer] = None, cache=None):
        """The layer on the split residual stream: its input is
        hidden_states + residual (residual None: hidden_states alone), its
        output (mlp_out, residual) with the same meaning."""
        x, residual = _norm(self.input_layernorm, hidden_states, residual, timer)
        a, _ = self.self_attn(x, position_embeddings, past_key_value=cache, timer=timer)
        x, residual = _norm(self.post_attention_layernorm, a, residual, timer)
        return self.mlp(x, timer), residual

    def forward(self, hidden_states: torch.Tensor, position_embeddings, **kwargs):
        """(hidden_states_out,) as llama.py:917-1004 returns it."""
        out, residual = self.forward_fused(hidden_states, None, position_embeddings)
        return (residual + out,)


class LlamaModel(nn.Module):
    layer_cls = LlamaDecoderLayer  # model-family hook (qwen3.py overrides)

    def __init__(self, config):
        super().__init__()
        self.config = config
        self.embed_tokens = nn.Embedding(config.vocab_size, config.hidden_size)
        self.layers = nn.ModuleList([self.layer_cls(config, i) for i in range(config.num_hidden_layers)])
        self.norm = LlamaRMSNorm(config.hidden_size, eps=config.rms_norm_eps)

    def rotary(self, position_ids: torch.Tensor, dtype: torch.dtype):
        c = self.config
        return rope_cos_sin(position_ids, c.head_dim, c.rope_theta, dtype, c.rope_scaling)

    def forward(self, input_ids: torch.Tensor, timer: Optional[Timer] = None,
                cache: Optional[KVCache] = None) -> torch.Tensor:
        """input_ids [b, s] -> final hidden states [b, s, hidden] (llama.py:1148-1300);
        with a cache, positions continue after the cached ones."""
        with _region(timer, "embed"):
            h = self.embed_tokens(input_ids)
            if cache is not None and cache.static:
                pos = cache.pos[None]              # device-side position of this token
            else:
                start = cache.seq_len() if cache is not None else 0
                pos = torch.arange(start, start + input_ids.shape[1], device=input_ids.device)[None]
            cos, sin = self.rotary(pos, h.dtype)
        residual = None
        for layer in self.layers:
            h, residual = layer.forward_fused(h, residual, (cos, sin), timer, cache)
        out, _ = _norm(self.norm, h, residual, timer)
        return out


class LlamaForCausalLM(nn.Module):
    model_cls = LlamaModel  # model-family hook (qwen3.py overrides)

    def __init__(self, config):
        super().__init__()
        self.config = config
        self.model = self.model_cls(config)
        self.lm_head = nn.Linear(config.hidden_size, config.vocab_size, bias=False)
        self.tie_weights()

    def tie_weights(self):
        """With tie_word_embeddings, lm_head shares the embedding matrix (again
        after `to_empty` / `to`, which give each module its own copy)."""
        if getattr(self.config, "tie_word_embeddings", False):
            self.lm_head.weight = self.model.embed_tokens.weight

    @torch.inference_mode()
    def prefill_next_token(self, input_ids: torch.Tensor, timer: Optional[Timer] = None) -> torch.Tensor:
        """The prefill of generation: the whole prompt through the model, then
        lm_head on the last position only and the greedy next token
        (sample.py:144, 178-179). -> [b] token ids."""
        h = self.model(input_ids, timer)
        with _region(timer, "lm_head"):
            logits = self.lm_head(h[:, -1])
            return logits.argmax(-1)


    def reset_decode_state(self):
        """Per-prompt hygiene of the decode-delta state (sample.py:147-152)."""
        for m in self.modules():
            if isinstance(m, LlamaAttention):
                m._dec_state = None
                m._dec_drift_points = None
                m._dec_static = None

    def graph_decodable(self) -> bool:
        """Whether decode steps can be recorded once and replayed: dense and
        sparse decode always; delta decode with the fixed refresh policy and no
        drift logging (the drift policies decide on host-read cosines)."""
        cfg = self.config
        mode = getattr(cfg, "decode_mode", "dense")
        if mode in ("dense", "sparse"):
            return True
        return (mode == "delta" and getattr(cfg, "refresh_policy", "fixed") == "fixed"
                and not bool(getattr(cfg, "log_drift", False)))

    def _decode_graphed(self, cache: KVCache, tok: torch.Tensor, max_new_tokens: int,
                        step_ms: Optional[list], logits_out: Optional[list],
                        record: bool = True, eos: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Decode steps 1 .. max_new_tokens-1 as HIP graph replays. The cache
        holds the token's row and key count on the device; each step kind
        (delta decode: anchor steps every min(gamma_dec, gamma_dec_max) steps,
        starting with the first; otherwise one kind) runs eagerly once, then is
        recorded and replayed. Outside the graph per step: the greedy argmax
        (into the next step's input) and the token copy. record=False runs
        every step eagerly in the same static form (the replays' reference).
        eos: stop once every row has produced one of these ids."""
        import time
        cfg = self.config
        mode = getattr(cfg, "decode_mode", "dense")
        period = (min(int(cfg.gamma_dec), int(getattr(cfg, "gamma_dec_max", 128)))
                  if mode == "delta" else 0)
        toks = torch.empty((tok.shape[0], max_new_tokens), dtype=torch.int64, device=tok.device)
        toks[:, 0] = tok
        tok_buf = tok[:, None].clone()
        cache.start_static()
        graphs = {}

        def run_step(anchor: bool) -> torch.Tensor:
            cache.anchor = anchor
            h = self.model(tok_buf, None, cache)
            logits = self.lm_head(h[:, -1])
            cache.advance_static()
            return logits

        n = max_new_tokens - 1
        done = _finished(tok, eos)
        ran = 0
        try:
            for j in range(n):
                t0 = time.perf_counter()
                kind = period > 0 and j % period == 0
                if kind in graphs:
                    g, logits = graphs[kind]
                    g.replay()
                else:
                    logits = run_step(kind)
                    if record:
                        g = torch.cuda.CUDAGraph()
                        with torch.cuda.graph(g):
                            glogits = run_step(kind)
                        graphs[kind] = (g, glogits)
                if logits_out is not None:
                    logits_out.append(logits.float().clone())
                ran = j + 1
                torch.argmax(logits, dim=-1, keepdim=True, out=tok_buf)
                toks[:, j + 1] = tok_buf[:, 0]
                if step_ms is not None:
                    torch.cuda.synchronize()
                    step_ms.append((time.perf_counter() - t0) * 1e3)
                if done is not None:
                    done |= _finished(tok_buf[:, 0], eos)
                    if bool(done.all()):
                        return toks[:, :j + 2]
        finally:
            cache.stop_static(ran)
        return toks

    @torch.inference_mode()
    def generate_greedy(self, input_ids: torch.Tensor, max_new_tokens: int,
                        timer: Optional[Timer] = None, step_ms: Optional[list] = None,
                        graph: bool = False, logits_out: Optional[list] = None,
                        record: bool = True, eos_token_id=None) -> torch.Tensor:
        """Greedy generation as sample.py drives it: the prompt is prefilled
        with the configured attention ("window": delta attention), then each
        new token runs one decode step with `sdpa_rectangle` (dense, or the
        sparse / delta decode of config.decode_mode). -> [b, max_new_tokens].
        step_ms: receives each decode step's wall time; logits_out: each
        step's fp32 logits, the prefill's first. graph: record the decode step in
        HIP graphs and replay it (when graph_decodable(); the decode rows then
        read the key count on the device, so they agree with the eager steps
        to rounding); record=False runs those static steps eagerly.
        eos_token_id (int or ids): stop once every row has produced one (the
        result then has fewer columns; rows that finished earlier keep
        generating, the caller masks them)."""
        import time
        cfg = self.config
        eos = None
        if eos_token_id is not None:
            ids = [eos_token_id] if isinstance(eos_token_id, int) else list(eos_token_id)
            eos = torch.tensor(ids, dtype=torch.int64, device=input_ids.device)
        b, s = input_ids.shape
        cache = KVCache(cfg, b, s + max_new_tokens, input_ids.device, self.lm_head.weight.dtype)
        self.reset_decode_state()
        impl = cfg._attn_implementation
        out = []
        try:
            h = self.model(input_ids, timer, cache)
            logits = self.lm_head(h[:, -1])
            if logits_out is not None:
                logits_out.append(logits.float().clone())
            tok = logits.argmax(-1)
            out.append(tok)
            done = _finished(tok, eos)
            cfg._attn_implementation = "sdpa_rectangle"
            if done is not None and bool(done.all()):
                return torch.stack(out, dim=1)
            if graph and self.graph_decodable() and max_new_tokens > 1:
                return self._decode_graphed(cache, tok, max_new_tokens, step_ms, logits_out, record, eos)
            for _ in range(max_new_tokens - 1):
                t0 = time.perf_counter()
                h = self.model(tok[:, None], timer, cache)
                logits = self.lm_head(h[:, -1])
                if logits_out is not None:
                    logits_out.append(logits.float().clone())
                tok = logits.argmax(-1)
                out.append(tok)
                if step_ms is not None:
                    torch.cuda.synchronize()
                    step_ms.append((time.perf_counter() - t0) * 1e3)
                if done is not None:
                    done |= _finished(tok, eos)
                    if bool(done.all()):
                        break
        finally:
            cfg._attn_implementation = impl
        return torch.stack(out, dim=1)

    @torch.inference_mode()
    def generate(self, input_ids: torch.Tensor, attention_mask: Optional[torch.Tensor] = None,
                 max_new_tokens: int = 128, do_sample: bool = False, eos_token_id=None,
                 pad_token_id: Optional[int] = None, graph: bool = False, **unused) -> torch.Tensor:
        """The call model_wrapper.py:97 makes (HF `generate` with the greedy
        `_sample` loop of sample.py:25-262): -> [b, s + n] token ids, the
        prompt (with its padding) followed by the generated tokens; after a
        row's first eos token its remaining positions hold pad_token_id, and
        generation stops once every row has finished. Left-padded rows
        (attention_mask 0 on the padding) run one at a time over their real
        tokens: the attention kernels take no padding mask. Only greedy
        decoding is built (do_sample=True raises); `unused` takes the
        generation kwargs greedy decoding ignores (temperature, top_k, ...)."""
        if do_sample:
            raise NotImplementedError("only greedy decoding (do_sample=False) is built")
        if unused.get("repetition_penalty") not in (None, 1, 1.0):
            raise NotImplementedError("repetition_penalty other than 1 is not built")
        b, s = input_ids.shape
        if pad_token_id is None:
            pad_token_id = (eos_token_id if isinstance(eos_token_id, int)
                            else (list(eos_token_id)[0] if eos_token_id is not None else 0))
        if attention_mask is None or bool(attention_mask.bool().all()):
            rows = [self.generate_greedy(input_ids, max_new_tokens, graph=graph,
                                         eos_token_id=eos_token_id)]
            rows = list(rows[0].unbind(0))
        else:
            rows = []
            for i in range(b):
                keep = attention_mask[i].bool()
                if not bool(keep.any()):
                    raise ValueError(f"row {i} of the batch has no tokens (attention_mask all 0)")
                rows.append(self.generate_greedy(input_ids[i:i + 1, keep], max_new_tokens,
                                                 graph=graph, eos_token_id=eos_token_id)[0])
        ids = ([eos_token_id] if isinstance(eos_token_id, int) else list(eos_token_id)
               if eos_token_id is not None else [])
        n = max(len(r) for r in rows)
        new = torch.full((b, n), int(pad_token_id), dtype=input_ids.dtype, device=input_ids.device)
        for i, r in enumerate(rows):
            hit = (torch.isin(r, torch.tensor(ids, device=r.device)).nonzero()
                   if ids else torch.empty(0, 1))
            end = int(hit[0, 0]) + 1 if len(hit) else len(r)
            new[i, :end] = r[:end]
        return torch.cat([input_ids, new], dim=1)


def _finished(tok: torch.Tensor, eos: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
    """[b] bool: which rows' token is an eos id (None without eos ids)."""
    return None if eos is None else torch.isin(tok, eos)


def init_weights_(model: nn.Module, std: float, seed: int = 0) -> nn.Module:
    """normal(0, std) for every linear and embedding weight, zero biases, RMSNorm
    weights 1 (llama.py:1020-1029), drawn on the model's device."""
    dev = next(model.parameters()).device
    g = torch.Generator(device=dev).manual_seed(seed)
    with torch.no_grad():
        for m in model.modules():
            if isinstance(m, (nn.Linear, nn.Embedding)):
                m.weight.normal_(0.0, std, generator=g)
                if getattr(m, "bias", None) is not None:
                    m.bias.zero_()
            elif isinstance(m, LlamaRMSNorm):
                m.weight.fill_(1.0)
    return model


def random_llama(config: LlamaConfig, device="cuda", dtype=torch.bfloat16, seed: int = 0) -> LlamaForCausalLM:
    """Build on the meta device, materialise on `device` in `dtype`, initialise;
    an inference model (no gradients)."""
    with torch.device("meta"):
        model = LlamaForCausalLM(config)
    model = model.to_empty(device=device).to(dtype)
    model.tie_weights()
    model = init_weights_(model, config.initializer_range, seed).eval().requires_grad_(False)
    return fuse_model_projections(model)


def fuse_model_projections(model: nn.Module) -> nn.Module:
    """fuse_projections on every attention and MLP block (one product each for
    q/k/v and gate/up on short inputs; names and values unchanged)."""
    for m in model.modules():
        if isinstance(m, (LlamaAttention, LlamaMLP)):
            m.fuse_projections()
    return model
