"""Text-in / text-out generation over a delta-attention model:
`HuggingFaceModel(config, **generation_kwargs)` (delta_attention/model_wrapper.py:11-136).

Construction builds the model with `init_model` and copies the pipeline
knobs onto model.config (model_wrapper.py:22-42); `process_batch` tokenizes,
generates greedily, decodes, strips the prompt and cuts at the stop words,
returning [{"text": [completion]}] per prompt (model_wrapper.py:89-136);
after each batch the per-layer drift statistics go to the JSON-lines file
named by DELTA_DRIFT_LOG (model_wrapper.py:56-84).

`__call__(prompt)` takes one prompt string and returns its one result dict;
it hands process_batch a one-element list (a bare string would be split into
characters by the per-prompt loop).
"""

from __future__ import annotations

import json
import os
from typing import List

from .sample import init_model

# knobs copied from the config onto model.config (model_wrapper.py:22-42)
WRAPPER_FIELDS = (
    "mode", "delta_lambda", "sliding_window", "hip_attention_dense_layers",
    "hip_attention_last_dense", "log_drift", "stride_policy", "gamma_min", "gamma_max",
    "adapt_chunk", "adapt_threshold", "stride_trigger", "adapt_k", "decode_mode",
    "gamma_dec", "refresh_policy", "drift_threshold", "drift_k", "gamma_dec_max",
)


class HuggingFaceModel:
    def __init__(self, config, **generation_kwargs) -> None:
        model, tokenizer = init_model(config)
        if tokenizer is None:
            raise FileNotFoundError(f"{config.model_str}: the checkpoint has no tokenizer files")
        self.pipeline = None
        self.model = model.eval()
        cfg = self.model.config
        cfg.attn_implementation_original = getattr(
            config, "attn_implementation_original", config.attn_implementation)
        cfg._attn_implementation = config.attn_implementation
        for name in WRAPPER_FIELDS:
            setattr(cfg, name, getattr(config, name))
        self.tokenizer = tokenizer
        self.generation_kwargs = dict(generation_kwargs)
        self.stop = self.generation_kwargs.pop("stop", None)
        if self.tokenizer.pad_token is None:
            # batching pads on the left with the eos token
            self.tokenizer.padding_side = "left"
            self.tokenizer.pad_token = self.tokenizer.eos_token

    def _flush_drift_stats(self) -> None:
        """Append the per-layer drift and stride summaries (left by the
        attention modules when log_drift is on) and the decode drift points to
        the DELTA_DRIFT_LOG file, one JSON object per line sorted by layer, then
        clear them. Without DELTA_DRIFT_LOG they are only cleared."""
        collected = []
        for m in self.model.modules():
            for attr in ("_drift_stats", "_stride_stats"):
                stats = getattr(m, attr, None)
                if stats is not None:
                    collected.append(stats)
                    setattr(m, attr, None)
            pts = getattr(m, "_dec_drift_points", None)
            if pts:
                collected.append({"kind": "decode_drift", "layer": int(m.layer_idx), "points": pts})
                m._dec_drift_points = None
        path = os.environ.get("DELTA_DRIFT_LOG")
        if not collected or not path:
            return
        with open(path, "a", encoding="utf-8") as f:
            for stats in sorted(collected, key=lambda s: s["layer"]):
                f.write(json.dumps(stats) + "\n")

    def __call__(self, prompt: str, **kwargs) -> dict:
        return self.process_batch([prompt], **kwargs)[0]

    def generation_args(self, **kwargs) -> dict:
        """Stored generation kwargs overridden by the call's, with the
        tokenizer's eos and pad ids filled in where absent."""
        args = {**self.generation_kwargs, **kwargs}
        args.setdefault("eos_token_id", self.tokenizer.eos_token_id)
        args.setdefault("pad_token_id", self.tokenizer.pad_token_id)
        return args

    def process_batch(self, prompts: List[str], **kwargs) -> List[dict]:
        args = self.generation_args(**kwargs)
        device = self.model.lm_head.weight.device
        inputs = self.tokenizer(prompts, return_tensors="pt", padding=True).to(device)
        generated = self.model.generate(inputs["input_ids"], attention_mask=inputs.get("attention_mask"),
                                        **args)
        texts = self.tokenizer.batch_decode(generated, skip_special_tokens=True)
        self._flush_drift_stats()
        results = []
        for text, prompt in zip(texts, prompts):
            # the prompt as the tokenizer round-trips it (it need not reproduce
            # the original string exactly)
            ids = self.tokenizer(prompt, return_tensors="pt").input_ids[0]
            prompt = self.tokenizer.decode(ids, skip_special_tokens=True)
            if text.startswith(prompt):
                text = text[len(prompt):]
            for s in self.stop or ():
                text = text.split(s)[0]
            results.append({"text": [text]})
        return results
