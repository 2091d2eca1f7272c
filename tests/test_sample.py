"""init_model and HuggingFaceModel construction on the CPU (sample.py:265-333,
model_wrapper.py:11-54): small Hugging Face-format checkpoints written here
(llama and qwen3, one file and sharded, tied embeddings), loaded through
safetensors with every weight equal to what was written, the pipeline knobs
copied, the model-family dispatch and its refusals, and the LoRA merge
against its closed form. Loading runs no kernel; generation is in the GPU
tests."""

import dataclasses
import json
import os

import pytest
import torch

import conftest  # noqa: F401
from helpers import write_checkpoint
from delta_attention import config as C
from delta_attention import sample
from delta_attention.model import LlamaForCausalLM
from delta_attention.qwen3 import Qwen3DeltaAttention, Qwen3ForCausalLM


def _cfg(path, **kw):
    return C.Config(model_str=str(path), **kw)


def _check_weights(model, sd):
    params = dict(model.named_parameters())
    for n, w in sd.items():
        assert torch.equal(params[n].float(), w.to(torch.bfloat16).float()), n


@pytest.mark.parametrize("family,shards,tied", [("llama", 1, False), ("llama", 3, True),
                                               ("qwen3", 1, False), ("qwen3", 2, True)])
def test_init_model_loads_checkpoint(tmp_path, family, shards, tied):
    sd = write_checkpoint(tmp_path, family, seed=3, tied=tied, shards=shards)
    cfg = _cfg(tmp_path, delta_lambda=16, sliding_window=128, sink_tokens=8, decode_mode="delta",
               gamma_dec=4, log_drift=True, mode="recompute")
    model, tok = sample.init_model(cfg, device="cpu")
    assert isinstance(model, Qwen3ForCausalLM if family == "qwen3" else LlamaForCausalLM)
    if family == "qwen3":
        assert isinstance(model.model.layers[0].self_attn, Qwen3DeltaAttention)
        assert model.config.rope_scaling is None and model.config.rms_norm_eps == 1e-6
    assert next(model.parameters()).dtype == torch.bfloat16
    _check_weights(model, sd)
    if tied:
        assert model.lm_head.weight.data_ptr() == model.model.embed_tokens.weight.data_ptr()
    for name in C.PIPELINE_FIELDS:
        assert getattr(model.config, name) == getattr(cfg, name), name
    assert model.config._attn_implementation == "window"
    assert model.config.attn_implementation_original == "window"
    assert model.args is cfg
    attn = [m for m in model.modules() if hasattr(m, "attention_method")]
    assert len(attn) == 2 and all(m.args is cfg and m.attention_method == "window" for m in attn)
    # the q/k/v products are fused into one buffer; names and values unchanged
    at = model.model.layers[0].self_attn
    assert at._qkv_fused is not None
    assert at.q_proj.weight.data_ptr() + at.q_proj.weight.numel() * 2 == at.k_proj.weight.data_ptr()
    assert tok is not None and tok.eos_token_id == 1 and tok("w3 w4").input_ids == [3, 4]


def test_init_model_head_dim_and_kv_defaults(tmp_path):
    write_checkpoint(tmp_path, "llama")
    hf = json.loads((tmp_path / "config.json").read_text())
    del hf["head_dim"], hf["num_key_value_heads"]
    (tmp_path / "config.json").write_text(json.dumps(hf))
    mc = sample.read_model_config(tmp_path)
    assert mc.head_dim == 256 // 4 and mc.num_key_value_heads == 4


def test_init_model_refusals(tmp_path):
    write_checkpoint(tmp_path / "a", "llama", tokenizer=False)
    with pytest.raises(NotImplementedError, match="hip_attention"):
        sample.init_model(_cfg(tmp_path / "a", attn_implementation="hip_attention"), device="cpu")
    with pytest.raises(FileNotFoundError, match="nothing is downloaded"):
        sample.init_model(_cfg(tmp_path / "no-such-model"), device="cpu")
    model, tok = sample.init_model(_cfg(tmp_path / "a"), device="cpu")
    assert tok is None
    # other families exit, like the reference
    hf = json.loads((tmp_path / "a" / "config.json").read_text())
    (tmp_path / "a" / "config.json").write_text(json.dumps({**hf, "model_type": "qwen3_next"}))
    with pytest.raises(SystemExit, match="qwen3_next"):
        sample.init_model(_cfg(tmp_path / "a"), device="cpu")
    # pickle checkpoints are not loaded
    write_checkpoint(tmp_path / "b", "llama", tokenizer=False)
    os.remove(tmp_path / "b" / "model.safetensors")
    (tmp_path / "b" / "pytorch_model.bin").write_bytes(b"not loaded")
    with pytest.raises(FileNotFoundError, match="pickle"):
        sample.init_model(_cfg(tmp_path / "b"), device="cpu")


def test_init_model_checks_tensor_names_and_shapes(tmp_path):
    from safetensors.torch import load_file, save_file
    write_checkpoint(tmp_path, "llama", tokenizer=False)
    f = tmp_path / "model.safetensors"
    sd = load_file(str(f))
    full = dict(sd)
    sd.pop("model.layers.1.mlp.up_proj.weight")
    save_file(sd, str(f))
    with pytest.raises(KeyError, match="lacks 1 parameters"):
        sample.init_model(_cfg(tmp_path), device="cpu")
    save_file({**full, "model.layers.0.extra.weight": torch.zeros(2)}, str(f))
    with pytest.raises(KeyError, match="unexpected tensor"):
        sample.init_model(_cfg(tmp_path), device="cpu")
    bad = dict(full)
    bad["model.norm.weight"] = torch.ones(7)
    save_file(bad, str(f))
    with pytest.raises(ValueError, match="model.norm.weight"):
        sample.init_model(_cfg(tmp_path), device="cpu")
    # rotary inv_freq buffers of older checkpoints are skipped
    save_file({**full, "model.layers.0.self_attn.rotary_emb.inv_freq": torch.ones(32)}, str(f))
    sample.init_model(_cfg(tmp_path), device="cpu")


@pytest.mark.parametrize("rslora", [False, True])
def test_lora_merge_closed_form(tmp_path, rslora):
    """W' = W + s * B @ A with s = alpha / r (alpha / sqrt(r) with rsLoRA),
    on the named linears only; from PEFT's adapter file layout."""
    from safetensors.torch import save_file
    sd = write_checkpoint(tmp_path / "base", "llama", seed=4, tokenizer=False)
    r, alpha = 4, 16
    g = torch.Generator().manual_seed(9)
    targets = {"model.layers.0.self_attn.q_proj": (256, 256), "model.layers.1.mlp.down_proj": (256, 512)}
    ad = {}
    for mod, (o, i) in targets.items():
        ad[f"base_model.model.{mod}.lora_A.weight"] = torch.randn(r, i, generator=g) * 0.05
        ad[f"base_model.model.{mod}.lora_B.weight"] = torch.randn(o, r, generator=g) * 0.05
    os.makedirs(tmp_path / "lora")
    save_file(ad, str(tmp_path / "lora" / "adapter_model.safetensors"))
    (tmp_path / "lora" / "adapter_config.json").write_text(
        json.dumps({"r": r, "lora_alpha": alpha, "use_rslora": rslora}))
    model, _ = sample.init_model(_cfg(tmp_path / "base", checkpoint=str(tmp_path / "lora")), device="cpu")
    s = alpha / (r ** 0.5) if rslora else alpha / r
    params = dict(model.named_parameters())
    for n, w in sd.items():
        mod = n[: -len(".weight")]
        exp = w.to(torch.bfloat16).float()
        if mod in targets:
            delta = ad[f"base_model.model.{mod}.lora_B.weight"] @ ad[f"base_model.model.{mod}.lora_A.weight"]
            exp = (exp + s * delta).to(torch.bfloat16).float()
            assert not torch.equal(exp, w.to(torch.bfloat16).float())
        assert torch.equal(params[n].float(), exp), n


def test_wrapper_fields_are_config_fields():
    from delta_attention.model_wrapper import WRAPPER_FIELDS
    names = {f.name for f in dataclasses.fields(C.Config)}
    assert set(WRAPPER_FIELDS) <= names


def test_wrapper_construction_and_drift_log(tmp_path, monkeypatch):
    from delta_attention.model_wrapper import HuggingFaceModel
    write_checkpoint(tmp_path / "m", "llama")
    monkeypatch.setattr(sample, "init_model",
                        lambda c, device="cuda", dtype=torch.bfloat16: _orig_init(c, device="cpu"))
    import delta_attention.model_wrapper as W
    monkeypatch.setattr(W, "init_model", sample.init_model)
    cfg = _cfg(tmp_path / "m", gamma_min=8, adapt_k=3.0, decode_mode="sparse", stop_words="")
    w = HuggingFaceModel(cfg, max_new_tokens=5, stop=["w9"])
    assert w.stop == ["w9"] and w.generation_kwargs == {"max_new_tokens": 5}
    for name in W.WRAPPER_FIELDS:
        assert getattr(w.model.config, name) == getattr(cfg, name), name
    # no pad token in the tokenizer: pad with eos on the left
    assert w.tokenizer.pad_token_id == 1 and w.tokenizer.padding_side == "left"
    args = w.generation_args(max_new_tokens=7)
    assert args == {"max_new_tokens": 7, "eos_token_id": 1, "pad_token_id": 1}
    # drift statistics go to DELTA_DRIFT_LOG sorted by layer, then are cleared
    at = [m for m in w.model.modules() if hasattr(m, "attention_method")]
    at[1]._drift_stats = {"layer": 1, "cos": 0.9}
    at[0]._stride_stats = {"layer": 0, "gamma": 32}
    at[0]._dec_drift_points = [{"step": 1, "cos": 0.99}]
    log = tmp_path / "drift.jsonl"
    monkeypatch.setenv("DELTA_DRIFT_LOG", str(log))
    w._flush_drift_stats()
    lines = [json.loads(x) for x in log.read_text().splitlines()]
    assert [x["layer"] for x in lines] == [0, 0, 1]
    assert {"kind": "decode_drift", "layer": 0, "points": [{"step": 1, "cos": 0.99}]} in lines
    assert at[1]._drift_stats is None and at[0]._dec_drift_points is None
    w._flush_drift_stats()
    assert len(log.read_text().splitlines()) == 3
    # a layer stores its summary as a deferred call (no device read inside the
    # layer); the first read runs it once and keeps the value
    calls = []
    at[1]._drift_stats = lambda: calls.append(1) or {"layer": 1, "cos": 0.5}
    assert calls == []
    assert at[1]._drift_stats == {"layer": 1, "cos": 0.5}
    assert at[1]._drift_stats["cos"] == 0.5 and calls == [1]
    at[0]._stride_stats = lambda: {"layer": 0, "gamma": 16}
    w._flush_drift_stats()
    lines = [json.loads(x) for x in log.read_text().splitlines()][3:]
    assert lines == [{"layer": 0, "gamma": 16}, {"layer": 1, "cos": 0.5}]
    assert at[1]._drift_stats is None and at[0]._stride_stats is None


_orig_init = sample.init_model
