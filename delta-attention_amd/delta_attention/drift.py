"""Prefill drift telemetry over the anchor deltas (delta_attention/drift.py).

The fused path keeps the anchor deltas in a [b, n_anchors, h, d] buffer, the
same tensor the reference summarises (llama.py:742-746), so the summary runs
on it directly when `log_drift` is set.
"""

from __future__ import annotations

from functools import reduce
from typing import Any, Dict, Iterable, List, Tuple

HIST_BINS = 40
HIST_RANGE = (-1.0, 1.0)


def drift_summary(dense_sparse_diff, layer_idx: int, gamma: int, seq_len: int) -> Dict[str, Any]:
    """Cosine between consecutive anchor deltas (per head, over d): mean,
    p10/p50/p90 and a HIST_BINS histogram over HIST_RANGE (drift.py:23-49).
    The cosines and the histogram come from one kernel pass over the delta
    buffer (ops.anchor_delta_cos); the mean and quantiles are taken over the
    [b, n-1, h] cosines."""
    return drift_summary_of(*drift_cosines(dense_sparse_diff), layer_idx, gamma, seq_len)


def drift_cosines(dense_sparse_diff):
    """The device half of drift_summary: the [b, n-1, h] cosines and their
    histogram, launched on the current stream, nothing read back."""
    from . import ops

    return ops.anchor_delta_cos(dense_sparse_diff, hist_bins=HIST_BINS, hist_range=HIST_RANGE)


def drift_summary_of(cos, hist, layer_idx: int, gamma: int, seq_len: int) -> Dict[str, Any]:
    """The host half of drift_summary: the summary of drift_cosines' output
    (one device sync)."""
    import torch

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


def _check_binning(summary: Dict[str, Any]) -> None:
    """A summary binned differently from this module (another version wrote
    it) cannot be summed with the others."""
    bins, rng = summary["hist_bins"], list(summary["hist_range"])
    if bins != HIST_BINS or rng != list(HIST_RANGE):
        raise ValueError(
            f"drift sidecar bins/range {bins}/{rng} do not match {HIST_BINS}/{list(HIST_RANGE)} "
            "(mixed-version sidecar files)")


def _fold_mean(acc: Tuple[float, int], summary: Dict[str, Any]) -> Tuple[float, int]:
    """Running n-weighted mean, one summary at a time in input order (the
    aggregated means of the reference's sidecar tools carry exactly these
    roundings)."""
    mean, n = acc
    total = n + int(summary["n"])
    if total > 0:
        mean = (mean * n + float(summary["mean"]) * int(summary["n"])) / total
    return mean, total


def aggregate_drift(lines: Iterable[Dict[str, Any]]) -> Dict[int, Dict[str, Any]]:
    """Per-request summaries -> one entry per layer, the reference's schema
    (drift.py:52-77): `n` and `hist` summed, `mean` the n-weighted mean (0.0
    for a layer without cosines), `requests` the number of summaries, `gamma`
    the first summary's. Pure Python; a summary with other bins or range is
    an error."""
    groups: Dict[int, List[Dict[str, Any]]] = {}
    for summary in lines:
        _check_binning(summary)
        groups.setdefault(int(summary["layer"]), []).append(summary)
    result: Dict[int, Dict[str, Any]] = {}
    for layer, group in groups.items():
        mean, n = reduce(_fold_mean, group, (0.0, 0))
        result[layer] = {
            "layer": layer, "n": n, "mean": mean, "requests": len(group),
            "hist": [sum(col) for col in zip(*(g["hist"] for g in group))],
            "hist_bins": HIST_BINS, "hist_range": list(HIST_RANGE), "gamma": group[0]["gamma"],
        }
    return result


def hist_bin_edges() -> List[float]:
    """The HIST_BINS + 1 bin edges over HIST_RANGE (torch.histc's equal bins),
    as the reference's eval tools write them: lo + i * (span / bins)."""
    lo, hi = HIST_RANGE
    width = (hi - lo) / HIST_BINS
    return [lo + i * width for i in range(HIST_BINS + 1)]
