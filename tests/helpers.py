"""Shared helpers of the test suite (inputs, comparisons)."""

import numpy as np
import torch


def gen_qkv(B, H, Hkv, S, D, seed=0, dtype=torch.bfloat16, device="cuda", std=1.0, N=None,
            model_layout=False):
    """Seeded CPU randn (q, k, v order), rounded to `dtype`, moved to `device`.
    model_layout=True returns q/k/v as [B,H,S,D] views of [B,S,H,D] storage,
    the layout the attention module hands over after its projections."""
    N = S if N is None else N
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, S, D, generator=g) * std
    k = torch.randn(B, Hkv, N, D, generator=g) * std
    v = torch.randn(B, Hkv, N, D, generator=g) * std
    q, k, v = (x.to(dtype) for x in (q, k, v))
    if model_layout:
        q, k, v = (x.transpose(1, 2).contiguous().transpose(1, 2) for x in (q, k, v))
    return q.to(device), k.to(device), v.to(device)


def np64(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def assert_close(got, ref, cos_min=0.999, atol=2e-2, what=""):
    """Tolerance of the reference's T1 gate (tests/test_math_identities.py:85-89):
    per-row (last dim) cosine > cos_min and max |diff| < atol."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    num = (got * ref).sum(-1)
    den = np.sqrt((got * got).sum(-1) * (ref * ref).sum(-1))
    nz = den > 0
    cos = np.where(nz, num / np.where(nz, den, 1.0), 1.0)
    # rows that are zero in both are equal; a zero row against a non-zero one fails
    both_zero = (np.abs(got).sum(-1) == 0) & (np.abs(ref).sum(-1) == 0)
    cos = np.where(both_zero, 1.0, np.where(nz, cos, 0.0))
    diff = np.abs(got - ref).max() if got.size else 0.0
    print(f"{what}: cos min {cos.min():.6f} mean {cos.mean():.6f} max|diff| {diff:.5f}", flush=True)
    assert cos.min() > cos_min, f"{what}: per-row cos {cos.min():.6f} <= {cos_min}"
    assert diff < atol, f"{what}: max abs diff {diff:.4f} >= {atol}"


def workload_inputs(B, H, Hkv, S, D, theta, seed=0, qk_norm=False, q_scale=True):
    """Seeded N(0,1) q/k/v on the GPU drawn in q, k, v order; optional per-head
    RMSNorm of q/k (Qwen3), q * D^-0.5 (Llama workloads), RoPE with `theta`,
    cast to bf16. Generated in row chunks to bound the fp32 temporaries."""
    from delta_attention.llama import apply_rotary_pos_emb, rope_cos_sin
    g = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.empty(B, H, S, D, device="cuda", dtype=torch.bfloat16)
    k = torch.empty(B, Hkv, S, D, device="cuda", dtype=torch.bfloat16)
    v = torch.empty(B, Hkv, S, D, device="cuda", dtype=torch.bfloat16)
    cos, sin = rope_cos_sin(torch.arange(S, device="cuda")[None], D, theta, torch.float32)
    for c0 in range(0, S, 8192):
        c1 = min(S, c0 + 8192)
        qc = torch.randn(B, H, c1 - c0, D, device="cuda", generator=g)
        kc = torch.randn(B, Hkv, c1 - c0, D, device="cuda", generator=g)
        if qk_norm:
            qc = torch.nn.functional.rms_norm(qc, (D,), eps=1e-6)
            kc = torch.nn.functional.rms_norm(kc, (D,), eps=1e-6)
        if q_scale:
            qc = qc * D ** -0.5
        qc, kc = apply_rotary_pos_emb(qc, kc, cos[:, c0:c1], sin[:, c0:c1])
        q[:, :, c0:c1] = qc.to(torch.bfloat16)
        k[:, :, c0:c1] = kc.to(torch.bfloat16)
        v[:, :, c0:c1] = torch.randn(B, Hkv, c1 - c0, D, device="cuda", generator=g).to(torch.bfloat16)
    return q, k, v


def write_checkpoint(path, model_type="llama", seed=0, tied=False, shards=1, tokenizer=True, **cfg):
    """A small Hugging Face-format checkpoint in `path`: config.json,
    safetensors weights (one file, or `shards` files with an index; with tied
    embeddings lm_head.weight is left out, as Hugging Face saves it) and a
    word-level tokenizer over the words w2 .. w{vocab-1} with </s> (id 1) as
    eos. -> the float32 state dict written (unfused parameter names)."""
    import json
    import os
    from safetensors.torch import save_file
    from delta_attention.model import LlamaConfig, LlamaForCausalLM, init_weights_
    from delta_attention.qwen3 import Qwen3Config, Qwen3ForCausalLM
    cls, cfg_cls = (Qwen3ForCausalLM, Qwen3Config) if model_type == "qwen3" else (LlamaForCausalLM, LlamaConfig)
    arch = dict(vocab_size=64, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                num_attention_heads=4, num_key_value_heads=2, head_dim=64, tie_word_embeddings=tied)
    arch.update(cfg)
    m = init_weights_(cls(cfg_cls(**arch)), 0.02, seed)
    g = torch.Generator().manual_seed(seed + 1)
    with torch.no_grad():
        for n, p in m.named_parameters():
            if n.endswith("norm.weight"):      # non-trivial norm weights
                p.uniform_(0.5, 1.5, generator=g)
    sd = {n: p.detach().contiguous().clone() for n, p in m.named_parameters()}
    if tied:
        sd.pop("lm_head.weight", None)
    hf = dict(model_type=model_type, torch_dtype="bfloat16", **{k: v for k, v in arch.items()})
    if model_type == "qwen3":
        hf["rope_scaling"] = None
    os.makedirs(path, exist_ok=True)
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump(hf, f)
    names = sorted(sd)
    if shards == 1:
        save_file(sd, os.path.join(path, "model.safetensors"))
    else:
        wmap = {}
        for i in range(shards):
            fn = f"model-{i + 1:05d}-of-{shards:05d}.safetensors"
            part = {n: sd[n] for n in names[i::shards]}
            save_file(part, os.path.join(path, fn))
            wmap.update({n: fn for n in part})
        with open(os.path.join(path, "model.safetensors.index.json"), "w") as f:
            json.dump({"metadata": {}, "weight_map": wmap}, f)
    if tokenizer:
        from tokenizers import Tokenizer, models, pre_tokenizers
        vocab = {"<unk>": 0, "</s>": 1, **{f"w{i}": i for i in range(2, arch["vocab_size"])}}
        tok = Tokenizer(models.WordLevel(vocab, unk_token="<unk>"))
        tok.pre_tokenizer = pre_tokenizers.Whitespace()
        tok.save(os.path.join(path, "tokenizer.json"))
        with open(os.path.join(path, "tokenizer_config.json"), "w") as f:
            json.dump({"tokenizer_class": "PreTrainedTokenizerFast", "eos_token": "</s>",
                       "unk_token": "<unk>"}, f)
    return sd
