"""Pipeline knobs of the delta-attention path (delta_attention/config.py:10-93).

`Config` keeps the reference's field names and defaults for every knob the
prefill path reads, plus `sink_tokens`: the reference hard-codes 1024 sink
tokens (llama.py:415, config.py:128, flex_delta.py:101); here it is a knob
with that default, and it is part of PIPELINE_FIELDS so that init code copies
it onto model.config with the others.
"""

from __future__ import annotations

import argparse
import dataclasses
from dataclasses import dataclass, field
from typing import List, Optional, Sequence


@dataclass
class Config:
    model_str: str = "meta-llama/Llama-3.1-8B-Instruct"
    attn_implementation: str = "window"   # window (delta path); hip_attention is not built here
    mode: str = "delta"                   # delta | recompute | sparse-only

    port: int = 8080
    host: str = "0.0.0.0"
    trust_remote_code: bool = True
    temperature: float = 0.0
    top_k: int = 1
    top_p: int = 1
    stop_words: str = ""
    max_new_tokens: int = 128
    repetition_penalty: int = 1

    delta_lambda: int = 64          # gamma: anchor stride of the query-sparse pass
    sliding_window: int = 2048
    sink_tokens: int = 1024         # the reference's hard-coded sink size
    delta_grad_scale: float = 1.0
    checkpoint: str = ""
    log_drift: bool = False

    stride_policy: str = "fixed"    # fixed | adaptive
    gamma_min: int = 16
    gamma_max: int = 256
    adapt_chunk: int = 4096
    adapt_threshold: float = 0.95
    stride_trigger: str = "absolute"  # absolute | relative
    adapt_k: float = 2.0

    decode_mode: str = "dense"
    gamma_dec: int = 32
    refresh_policy: str = "fixed"
    drift_threshold: float = 0.95
    drift_k: float = 2.0
    gamma_dec_max: int = 128

    hip_attention_dense_layers: List[int] = field(default_factory=lambda: [0, 1, 2])
    hip_attention_last_dense: int = 64

    @classmethod
    def from_args(cls, argv: Optional[Sequence[str]] = None) -> "Config":
        """`--field value` flags for every scalar field (booleans are
        presence flags), like the reference's argparse_dataclass parser."""
        p = argparse.ArgumentParser()
        for f in dataclasses.fields(cls):
            if f.type in ("bool", bool):
                p.add_argument(f"--{f.name}", action="store_true", default=f.default)
            elif f.type in ("int", int, "float", float, "str", str):
                typ = {"int": int, "float": float, "str": str}.get(f.type, f.type)
                p.add_argument(f"--{f.name}", type=typ, default=f.default)
        ns = p.parse_args(argv)
        return cls(**{k: v for k, v in vars(ns).items()})


# Knobs the attention modules read from model.config; init code copies exactly
# these (config.py:87-93 of the reference, plus sink_tokens).
PIPELINE_FIELDS = (
    "mode", "delta_lambda", "sliding_window", "sink_tokens", "log_drift", "delta_grad_scale",
    "stride_policy", "gamma_min", "gamma_max", "adapt_chunk",
    "adapt_threshold", "stride_trigger", "adapt_k",
    "decode_mode", "gamma_dec", "refresh_policy", "drift_threshold",
    "drift_k", "gamma_dec_max",
)


def copy_pipeline_fields(config: Config, model_config) -> None:
    """Set every PIPELINE_FIELDS knob of `config` on `model_config`."""
    for name in PIPELINE_FIELDS:
        setattr(model_config, name, getattr(config, name))
