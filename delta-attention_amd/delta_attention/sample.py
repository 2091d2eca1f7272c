"""Model construction for generation: `init_model(config) -> (model, tokenizer)`
(delta_attention/sample.py:265-333).

The reference registers its attention names with Hugging Face, reads the
checkpoint with `from_pretrained`, dispatches on `model_type` (llama or dense
qwen3, anything else exits), copies the pipeline knobs onto `model.config`,
tags every attention module, optionally merges a LoRA adapter, and patches
the model's sampling loop. Here:

- the checkpoint is a local Hugging Face directory (config.json, safetensors
  weights, tokenizer files), or a model id already in the local Hugging Face
  cache; nothing is downloaded;
- weights are read with safetensors only (`pytorch_model.bin` is a pickle and
  is refused) straight onto the device, in bf16;
- the attention names are checked rather than registered: prefill runs
  "window" (the delta path), decode steps "sdpa_rectangle";
- `LlamaForCausalLM.generate` is the greedy sampling loop itself, so no
  method is patched in;
- a LoRA adapter directory (`config.checkpoint`, PEFT's file layout) is
  merged as W += (alpha / r) * B @ A (alpha / sqrt(r) with rsLoRA).
"""

from __future__ import annotations

import dataclasses
import json
import math
from pathlib import Path
from typing import Optional, Tuple

import torch
from torch import nn

from .config import PIPELINE_FIELDS
from .llama import LlamaAttention
from .model import LlamaConfig, LlamaForCausalLM, fuse_model_projections

# attention implementations the model runs (llama.py's forward dispatch):
# "window" for the prefill, "sdpa_rectangle" for the decode steps
ATTENTION_IMPLEMENTATIONS = ("window", "sdpa_rectangle")

# architecture fields read from config.json
MODEL_FIELDS = (
    "vocab_size", "hidden_size", "intermediate_size", "num_hidden_layers",
    "num_attention_heads", "num_key_value_heads", "head_dim", "rope_theta",
    "rope_scaling", "rms_norm_eps", "initializer_range", "attention_bias",
    "mlp_bias", "attention_dropout", "tie_word_embeddings",
)


def resolve_checkpoint(model_str: str) -> Path:
    """A local checkpoint directory, or a model id resolved in the local
    Hugging Face cache without network access."""
    p = Path(model_str).expanduser()
    if p.is_dir():
        return p
    try:
        from huggingface_hub import snapshot_download
        return Path(snapshot_download(model_str, local_files_only=True))
    except Exception as e:  # not cached (or no hub library): nothing to load
        raise FileNotFoundError(
            f"{model_str!r} is neither a checkpoint directory nor in the local Hugging Face "
            "cache (nothing is downloaded)") from e


def model_family(path: Path):
    """(causal-LM class, config class) for config.json's model_type
    (sample.py:275-290): llama, or dense qwen3; anything else exits."""
    hf = json.loads((path / "config.json").read_text())
    model_type = hf.get("model_type")
    if model_type == "qwen3":
        from .qwen3 import Qwen3Config, Qwen3ForCausalLM
        return Qwen3ForCausalLM, Qwen3Config
    if model_type == "llama":
        return LlamaForCausalLM, LlamaConfig
    raise SystemExit(
        f"unsupported model_type {model_type!r} for {path} (delta attention covers llama and "
        "dense qwen3; hybrid and linear-attention families have no softmax rows to correct)")


def read_model_config(path: Path, config_cls=LlamaConfig):
    """The architecture fields of config.json on a `config_cls`; absent
    fields keep the class defaults, except num_key_value_heads (defaults to
    num_attention_heads) and head_dim (hidden_size / num_attention_heads)."""
    hf = json.loads((path / "config.json").read_text())
    names = {f.name for f in dataclasses.fields(config_cls)}
    kw = {k: hf[k] for k in MODEL_FIELDS if k in hf and k in names}
    kw.setdefault("num_key_value_heads", hf["num_attention_heads"])
    if kw.get("head_dim") is None:
        kw["head_dim"] = hf["hidden_size"] // hf["num_attention_heads"]
    if "rope_scaling" in hf:
        kw["rope_scaling"] = hf["rope_scaling"]
    return config_cls(**kw)


def weight_files(path: Path) -> list:
    """The safetensors files of a checkpoint (sharded via the index, or one)."""
    index = path / "model.safetensors.index.json"
    if index.exists():
        shards = sorted(set(json.loads(index.read_text())["weight_map"].values()))
        return [path / f for f in shards]
    if (path / "model.safetensors").exists():
        return [path / "model.safetensors"]
    raise FileNotFoundError(
        f"no safetensors weights in {path} (pickle checkpoints such as pytorch_model.bin "
        "are not loaded)")


@torch.no_grad()
def load_weights_(model: nn.Module, files, device) -> nn.Module:
    """Copy every tensor of `files` into the parameter of the same name, on
    `device`, converting to the parameter's dtype. Every parameter must be
    present exactly once; rotary inv_freq buffers and, with tied embeddings,
    lm_head.weight are skipped; any other unknown name raises."""
    from safetensors import safe_open
    params = dict(model.named_parameters())
    tied = bool(getattr(model.config, "tie_word_embeddings", False))
    loaded = set()
    for f in files:
        with safe_open(str(f), framework="pt", device=str(device)) as sf:
            for name in sf.keys():
                if name.endswith("rotary_emb.inv_freq") or (tied and name == "lm_head.weight"):
                    continue
                if name not in params:
                    raise KeyError(f"unexpected tensor {name!r} in {Path(f).name}")
                if name in loaded:
                    raise KeyError(f"tensor {name!r} appears twice in the checkpoint")
                t = sf.get_tensor(name)
                p = params[name]
                if tuple(t.shape) != tuple(p.shape):
                    raise ValueError(f"{name}: checkpoint shape {tuple(t.shape)} "
                                     f"!= model shape {tuple(p.shape)}")
                p.copy_(t)
                loaded.add(name)
    missing = sorted(set(params) - loaded)
    if missing:
        raise KeyError(f"checkpoint lacks {len(missing)} parameters, e.g. {missing[:3]}")
    return model


@torch.no_grad()
def merge_lora_(model: nn.Module, adapter_dir: Path) -> nn.Module:
    """Merge a LoRA adapter (PEFT layout: adapter_config.json with r,
    lora_alpha, use_rslora; adapter_model.safetensors with
    `base_model.model.<module>.lora_A.weight` / `.lora_B.weight`) into the
    linear weights: W += s * B @ A in float32, s = alpha / r (alpha / sqrt(r)
    with rsLoRA). Every adapter tensor must name a linear of the model."""
    from safetensors import safe_open
    cfg = json.loads((adapter_dir / "adapter_config.json").read_text())
    r, alpha = int(cfg["r"]), float(cfg.get("lora_alpha", cfg["r"]))
    scale = alpha / math.sqrt(r) if cfg.get("use_rslora") else alpha / r
    mods = dict(model.named_modules())
    pairs = {}
    with safe_open(str(adapter_dir / "adapter_model.safetensors"), framework="pt", device="cpu") as sf:
        for name in sf.keys():
            base = name[len("base_model.model."):] if name.startswith("base_model.model.") else name
            for part in ("lora_A", "lora_B"):
                tag = f".{part}."
                if tag in base:
                    mod = base.split(tag)[0]
                    pairs.setdefault(mod, {})[part] = sf.get_tensor(name)
                    break
            else:
                raise KeyError(f"adapter tensor {name!r} is not a lora_A/lora_B weight")
    for mod, ab in pairs.items():
        lin = mods.get(mod)
        if not isinstance(lin, nn.Linear) or set(ab) != {"lora_A", "lora_B"}:
            raise KeyError(f"adapter module {mod!r}: no such linear, or lora_A/lora_B missing")
        w = lin.weight
        delta = ab["lora_B"].to(w.device, torch.float32) @ ab["lora_A"].to(w.device, torch.float32)
        w.copy_((w.float() + scale * delta).to(w.dtype))
    return model


def init_model(config, device="cuda", dtype: torch.dtype = torch.bfloat16) -> Tuple[nn.Module, Optional[object]]:
    """-> (model, tokenizer) for `config.model_str` with the pipeline knobs of
    `config` (sample.py:265-333). The model is built for `model_type`, loaded
    in `dtype` on `device`, its q/k/v and gate/up products fused, with
    config._attn_implementation = config.attn_implementation and the
    PIPELINE_FIELDS knobs copied onto model.config; every attention module
    gets `args` and `attention_method`. The tokenizer is the directory's
    (transformers.AutoTokenizer, local files only), or None if it has none."""
    impl = config.attn_implementation
    if impl not in ATTENTION_IMPLEMENTATIONS:
        raise NotImplementedError(
            f"attn_implementation {impl!r} is not built (built: {', '.join(ATTENTION_IMPLEMENTATIONS)})")
    path = resolve_checkpoint(config.model_str)
    cls, cfg_cls = model_family(path)
    model_config = read_model_config(path, cfg_cls)
    model_config._attn_implementation = impl
    with torch.device("meta"):
        model = cls(model_config)
    model = model.to_empty(device=device).to(dtype)
    model.tie_weights()
    load_weights_(model, weight_files(path), device)
    model.eval().requires_grad_(False)

    ckpt = getattr(config, "checkpoint", "") or ""
    if ckpt:
        merge_lora_(model, Path(ckpt))

    model.args = config
    for name in PIPELINE_FIELDS:
        setattr(model.config, name, getattr(config, name))
    model.config.attn_implementation_original = getattr(
        config, "attn_implementation_original", impl)
    for name in ("hip_attention_dense_layers", "hip_attention_last_dense"):
        if hasattr(config, name):
            setattr(model.config, name, getattr(config, name))
    for m in model.modules():
        if isinstance(m, LlamaAttention):
            m.args = config
            m.attention_method = impl
    fuse_model_projections(model)
    return model, load_tokenizer(path)


def load_tokenizer(path: Path):
    """AutoTokenizer from the checkpoint's own files (no network, no remote
    code), or None when the directory holds no tokenizer."""
    if not any((path / f).exists() for f in ("tokenizer.json", "tokenizer.model", "vocab.json")):
        return None
    import transformers
    return transformers.AutoTokenizer.from_pretrained(str(path), local_files_only=True)
