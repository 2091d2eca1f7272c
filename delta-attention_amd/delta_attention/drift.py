"""Prefill drift telemetry over the anchor deltas (delta_attention/drift.py).

The fused path keeps the anchor deltas in a [b, n_anchors, h, d] buffer, the
same tensor the reference summarises (llama.py:742-746), so the summary runs
on it directly when `log_drift` is set.
"""

from __future__ import annotations

from typing import Any, Dict, Iterable, List

HIST_BINS = 40
HIST_RANGE = (-1.0, 1.0)


def drift_summary(dense_sparse_diff, layer_idx: int, gamma: int, seq_len: int) -> Dict[str, Any]:
    """Cosine between consecutive anchor deltas (per head, over d): mean,
    p10/p50/p90 and a HIST_BINS histogram over HIST_RANGE (drift.py:23-49).
    The cosines and the histogram come from one kernel pass over the delta
    buffer (ops.anchor_delta_cos); the mean and quantiles are taken over the
    [b, n-1, h] cosines."""
    import torch

    from . import ops

    cos, hist = ops.anchor_delta_cos(dense_sparse_diff, hist_bins=HIST_BINS, hist_range=HIST_RANGE)
    flat = cos.flatten()
    qs = torch.quantile(flat, torch.tensor([0.1, 0.5, 0.9], device=flat.device))
    mean, p10, p50, p90 = torch.cat((flat.mean()[None], qs)).tolist()   # one device sync
    return {
        "layer": int(layer_idx), "gamma": int(gamma), "seq_len": int(seq_len),
        "n": int(flat.numel()), "mean": float(mean),
        "p10": float(p10), "p50": float(p50), "p90": float(p90),
        "hist_bins": HIST_BINS, "hist_range": list(HIST_RANGE),
        "hist": [int(x) for x in hist.tolist()],
    }


def aggregate_drift(lines: Iterable[Dict[str, Any]]) -> Dict[int, Dict[str, Any]]:
    """One entry per layer: n-weighted mean, summed histograms; mismatched bins
    are an error (drift.py:52-77)."""
    out: Dict[int, Dict[str, Any]] = {}
    for s in lines:
        if s["hist_bins"] != HIST_BINS or list(s["hist_range"]) != list(HIST_RANGE):
            raise ValueError(
                f"drift sidecar bins/range {s['hist_bins']}/{s['hist_range']} do not match "
                f"{HIST_BINS}/{list(HIST_RANGE)} (mixed-version sidecar files)")
        layer = int(s["layer"])
        agg = out.setdefault(layer, {"layer": layer, "n": 0, "mean": 0.0, "requests": 0,
                                     "hist": [0] * HIST_BINS, "hist_bins": HIST_BINS,
                                     "hist_range": list(HIST_RANGE), "gamma": s["gamma"]})
        total = agg["n"] + s["n"]
        if total > 0:
            agg["mean"] = (agg["mean"] * agg["n"] + s["mean"] * s["n"]) / total
        agg["n"] = total
        agg["requests"] += 1
        agg["hist"] = [x + y for x, y in zip(agg["hist"], s["hist"])]
    return out


def hist_bin_edges() -> List[float]:
    lo, hi = HIST_RANGE
    step = (hi - lo) / HIST_BINS
    return [lo + i * step for i in range(HIST_BINS + 1)]
