"""Variable-stride delta correction and the adaptive-stride rules
(delta_attention/stride.py of the reference).

`apply_delta_variable` runs kernel (3) with an anchor list: every row i < s_p
gets sparse[i] + (dense_sel - sparse[idx])[owner(i)], owner(i) = the last
anchor <= i. The elementwise arithmetic is bf16 with one rounding per op, as
the reference's torch ops (stride.py:38-40), so results are bit-identical.

The stride rules and the cost model are host-side scalar formulas; they follow
the reference definitions (stride.py:23, 55-128) because callers compare
their numbers across implementations.
"""

from __future__ import annotations

from typing import List, Tuple

import numpy as np

ADAPT_MARGIN = 0.02  # hysteresis above adapt_threshold before gamma grows (stride.py:23)


def apply_delta_variable(sparse_out, dense_out_sel, idx, s_p: int):
    """sparse_out [b, >=s_p, h, d], dense_out_sel [b, n, h, d], idx [n] ascending
    anchor rows (idx[0] == 0 expected; rows before idx[0] take the last anchor's
    delta, as searchsorted(...) - 1 == -1 does in the reference).
    Returns the corrected rows [b, s_p, h, d] (stride.py:26-40)."""
    from . import ops

    assert idx.dim() == 1 and idx.numel() == dense_out_sel.shape[1], (idx.shape, dense_out_sel.shape)
    return ops.delta_add(sparse_out, s_p=int(s_p), dense_sel=dense_out_sel, anchors=idx)


def interanchor_cos(deltas, *, sparse=None, rows=None) -> Tuple[float, float]:
    """(mean, min) cosine between consecutive anchor deltas [b, n, h, d],
    per (b, pair, h) over d (stride.py:43-52), on the GPU kernel
    (ops.anchor_delta_cos). With `sparse` and `rows` given, `deltas` holds the
    dense anchor rows and the deltas rnd(dense - sparse[:, rows]) are formed
    inside the kernel. Fewer than two anchors: (1.0, 1.0)."""
    from . import ops

    if deltas.size(1) < 2:
        return 1.0, 1.0

    cos = ops.anchor_delta_cos(deltas, sparse=sparse, rows=rows)
    # one device-to-host copy of the [b, n-1, h] cosines (a few KB) instead
    # of reduction launches; the mean is taken in float64 on the host
    c = cos.cpu().numpy()
    return float(c.mean(dtype=np.float64)), float(c.min())


def next_gamma(cos_mean: float, gamma_c: int, *, threshold: float,
               gamma_min: int, gamma_max: int) -> int:
    """Halve gamma when the chunk's mean delta cosine is below `threshold`,
    double it above threshold + ADAPT_MARGIN, else keep it (stride.py:55-62)."""
    if cos_mean < threshold:
        return max(gamma_c // 2, gamma_min)
    if cos_mean > threshold + ADAPT_MARGIN:
        return min(gamma_c * 2, gamma_max)
    return gamma_c


def next_gamma_relative(cos_mean: float, history: List[float], gamma_c: int, *,
                        k: float, gamma_min: int, gamma_max: int) -> int:
    """Relative trigger (stride.py:65-86): compare to mean -/+ k * std of the
    history (population std); needs at least two history entries."""
    if len(history) < 2:
        return gamma_c
    n = len(history)
    mu = sum(history) / n
    sd = (sum((x - mu) ** 2 for x in history) / n) ** 0.5
    if cos_mean < mu - k * sd:
        return max(gamma_c // 2, gamma_min)
    if cos_mean > mu + k * sd:
        return min(gamma_c * 2, gamma_max)
    return gamma_c


def _sparse_pass_cost(s: int, window: int, sink: int) -> int:
    """Key count of a causal pass where row i reads min(i+1, window+sink) keys
    (stride.py:89-96)."""
    w = min(window + sink, s)
    return w * (w - 1) // 2 + (s - (w - 1)) * w


def effective_sparsity(anchor_idx, s: int, window: int, sink: int = 1024) -> float:
    """1 - (sparse pass + sum over dense rows of (i+1)) / (s^2 / 2) (stride.py:99-108)."""
    dense_cost = int(anchor_idx.sum().item()) + anchor_idx.numel()
    return 1.0 - (_sparse_pass_cost(s, window, sink) + dense_cost) / (s * s / 2.0)


def plan_chunks(s_p: int, chunk: int) -> List[Tuple[int, int]]:
    """[start, end) row chunks of the adaptive pass (stride.py:111-112)."""
    return [(a, min(a + chunk, s_p)) for a in range(0, s_p, chunk)]


def uniform_effective_sparsity(s: int, gamma: int, window: int, sink: int = 1024) -> float:
    """effective_sparsity of the fixed-stride layout in closed form (stride.py:115-128)."""
    cut_n = s % gamma + max(128, gamma)
    s_p = s - cut_n
    n = (s_p + gamma - 1) // gamma
    anchor_cost = gamma * n * (n - 1) // 2 + n
    tail_cost = (s * (s + 1) - s_p * (s_p + 1)) // 2
    return 1.0 - (_sparse_pass_cost(s, window, sink) + anchor_cost + tail_cost) / (s * s / 2.0)
