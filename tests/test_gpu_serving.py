"""Generation through the user-facing entry points on the GPU: init_model
(sample.py:265-333) on small Hugging Face-format checkpoints, llama and
qwen3, and HuggingFaceModel (model_wrapper.py:86-136) text in, text out.

- the Qwen3 causal LM built by init_model (per-head q/k RMSNorm inside the
  fused prologue, GQA 5) against the same model's layers run as separate
  torch ops (projection, RMSNorm, RoPE, delta_forward, o_proj, MLP);
- process_batch's completions against greedy token generation decoded by
  the tokenizer; left-padded batches against the same prompts one by one;
  stop words and eos.
"""

import numpy as np
import pytest
import torch

from helpers import np64, write_checkpoint

pytestmark = pytest.mark.gpu

ARCH = dict(vocab_size=512, hidden_size=1280, intermediate_size=2048, num_hidden_layers=2,
            num_attention_heads=10, num_key_value_heads=2, head_dim=128)


def _config(path, **kw):
    from delta_attention.config import Config
    base = dict(model_str=str(path), delta_lambda=16, sliding_window=128, sink_tokens=8)
    base.update(kw)
    return Config(**base)


@pytest.mark.parametrize("family", ["qwen3", "llama"])
def test_loaded_model_matches_layer_ops(gpu, tmp_path, family):
    from delta_attention.llama import apply_rotary_pos_emb
    from delta_attention.sample import init_model
    write_checkpoint(tmp_path, family, seed=21, tied=(family == "qwen3"), **ARCH)
    m, _ = init_model(_config(tmp_path))
    S, D = 700, ARCH["head_dim"]
    ids = torch.randint(0, ARCH["vocab_size"], (1, S), device="cuda",
                        generator=torch.Generator(device="cuda").manual_seed(22))
    print(f"{family} S{S}", flush=True)
    with torch.inference_mode():
        got = m.model(ids)
        h = m.model.embed_tokens(ids)
        cos, sin = m.model.rotary(torch.arange(S, device="cuda")[None], h.dtype)
        for layer in m.model.layers:
            at = layer.self_attn
            residual = h
            x = layer.input_layernorm(h)
            q, k, v = at._qkv(x, (1, S, -1, D))           # qwen3: q/k RMSNorm here
            q, k = apply_rotary_pos_emb(q, k, cos, sin)
            a, _ = at.delta_forward(at, q, k, v, None, scaling=at.scaling)
            h = residual + at.o_proj(a.reshape(1, S, -1))
            residual = h
            x = layer.post_attention_layernorm(h)
            mlp = layer.mlp
            h = residual + mlp.down_proj(torch.nn.functional.silu(mlp.gate_proj(x)) * mlp.up_proj(x))
        ref = m.model.norm(h)
    torch.cuda.synchronize()
    g64, r64 = np64(got)[0], np64(ref)[0]
    cos_rows = (g64 * r64).sum(-1) / (np.linalg.norm(g64, axis=-1) * np.linalg.norm(r64, axis=-1))
    assert cos_rows.min() > 0.999, cos_rows.min()


@pytest.fixture(scope="module")
def wrapper(tmp_path_factory):
    from delta_attention.model_wrapper import HuggingFaceModel
    path = tmp_path_factory.mktemp("ckpt")
    write_checkpoint(path, "llama", seed=31, **ARCH)
    return HuggingFaceModel(_config(path, decode_mode="delta", gamma_dec=4),
                            max_new_tokens=12, stop=None)


def _prompt(n, seed):
    rng = np.random.default_rng(seed)
    return " ".join(f"w{int(i)}" for i in rng.integers(2, ARCH["vocab_size"], size=n))


def _greedy_text(w, prompt, n_new):
    tok = w.tokenizer
    ids = tok(prompt, return_tensors="pt").input_ids.cuda()
    out = w.model.generate_greedy(ids, n_new)[0].tolist()
    if tok.eos_token_id in out:
        out = out[:out.index(tok.eos_token_id) + 1]
    return tok.decode(out, skip_special_tokens=True), out


def test_wrapper_completion_is_greedy_generation(gpu, wrapper):
    prompt = _prompt(600, 1)
    print("single prompt, 600 words", flush=True)
    res = wrapper(prompt)
    assert set(res) == {"text"} and len(res["text"]) == 1
    text, toks = _greedy_text(wrapper, prompt, 12)
    assert res["text"][0].strip() == text.strip()
    assert len(toks) >= 1


def test_wrapper_left_padded_batch_equals_single_prompts(gpu, wrapper):
    prompts = [_prompt(n, 10 + n) for n in (520, 333, 700)]
    print("batch of 3 prompts, left-padded", flush=True)
    batch = wrapper.process_batch(prompts)
    single = [wrapper(p) for p in prompts]
    assert batch == single
    for p, r in zip(prompts, batch):
        assert r["text"][0].strip() == _greedy_text(wrapper, p, 12)[0].strip()


def test_wrapper_stop_words_and_eos(gpu, wrapper):
    prompt = _prompt(400, 5)
    full = wrapper(prompt)["text"][0]
    words = full.split()
    assert len(words) >= 3, full
    stop = words[2]
    wrapper.stop = [stop]
    try:
        cut = wrapper(prompt)["text"][0]
    finally:
        wrapper.stop = None
    assert cut == full.split(stop)[0]
    # with the third generated token as eos, generation ends at its first
    # occurrence (eager steps and graph-replayed steps)
    ids = wrapper.tokenizer(prompt, return_tensors="pt").input_ids.cuda()
    for graph in (False, True):
        toks = wrapper.model.generate_greedy(ids, 12, graph=graph)[0].tolist()
        eos = toks[2]
        out = wrapper.model.generate(ids, max_new_tokens=12, eos_token_id=eos, pad_token_id=0,
                                     graph=graph)
        assert out.shape[1] == ids.shape[1] + toks.index(eos) + 1
        assert out[0, ids.shape[1]:].tolist() == toks[:toks.index(eos) + 1]
    with pytest.raises(NotImplementedError):
        wrapper.model.generate(ids, max_new_tokens=2, do_sample=True)
