"""Delta decode: when a decode step refreshes its correction.

A delta decode layer (semantics: llama.py:551-634) carries, between decode
steps, the difference between the dense and the sparse attention row of its
last *anchor* step, and outputs sparse + that difference on the steps in
between. `RefreshRule` decides which steps anchor:

* every policy anchors the first step (there is no difference yet) and any
  step `gamma_dec_max` steps after the last anchor;
* ``fixed`` anchors every `gamma_dec` steps;
* ``drift`` anchors when the cosine between this step's sparse row and the
  previous step's falls below `drift_threshold`;
* ``drift_rel`` anchors when that cosine falls below the mean of the recent
  cosines minus `drift_k` of their (population) standard deviations, once
  `WARMUP` cosines are recorded; it records every cosine it tests and keeps
  the last `WINDOW`.

The per-layer state is a plain dict, ``_dec_state``, with the keys the
reference's tools and tests read: ``last_delta`` (the correction),
``steps`` (steps since the anchor), ``last_sparse`` (the previous sparse row)
and ``cos_hist`` (the recorded cosines).
"""

from __future__ import annotations

import statistics
from dataclasses import dataclass

import torch

POLICIES = ("fixed", "drift", "drift_rel")


def new_state() -> dict:
    return {"last_delta": None, "steps": 0, "last_sparse": None, "cos_hist": []}


def row_cos(a: torch.Tensor, b: torch.Tensor, eps: float = 1e-8) -> float:
    """Cosine of two rows flattened, in float32 (one read-back for the three
    reductions)."""
    a, b = a.reshape(-1).float(), b.reshape(-1).float()
    ab, aa, bb = torch.stack((a @ b, a @ a, b @ b)).tolist()
    return ab / max(aa ** 0.5, eps) / max(bb ** 0.5, eps)


@dataclass(frozen=True)
class RefreshRule:
    policy: str = "fixed"
    gamma_dec: int = 8
    gamma_dec_max: int = 128
    drift_threshold: float = 0.95
    drift_k: float = 2.0

    WARMUP = 8     # drift_rel: recorded cosines before the first test
    WINDOW = 16    # drift_rel: cosines kept

    @classmethod
    def of(cls, config) -> "RefreshRule":
        rule = cls(policy=getattr(config, "refresh_policy", "fixed"),
                   gamma_dec=int(getattr(config, "gamma_dec", 8)),
                   gamma_dec_max=int(getattr(config, "gamma_dec_max", 128)),
                   drift_threshold=float(getattr(config, "drift_threshold", 0.95)),
                   drift_k=float(getattr(config, "drift_k", 2.0)))
        assert rule.policy in POLICIES, rule.policy
        return rule

    @property
    def needs_sparse_history(self) -> bool:
        """Whether decisions read the previous step's sparse row."""
        return self.policy != "fixed"

    def count_due(self, since: int) -> bool:
        """Anchors owed to the step count alone (`since` steps after the last)."""
        return since >= self.gamma_dec_max or (self.policy == "fixed" and since >= self.gamma_dec)

    def drifted(self, cos: float, recorded) -> bool:
        if self.policy == "drift":
            return cos < self.drift_threshold
        if len(recorded) < self.WARMUP:
            return False
        mean = statistics.fmean(recorded)
        return cos < mean - self.drift_k * statistics.pstdev(recorded, mean)

    def decide(self, state: dict, sparse: torch.Tensor) -> tuple[bool, int]:
        """(anchor?, steps since the last anchor counting this one) for the
        step whose sparse row is `sparse`; records the tested cosine
        (drift_rel) in `state`."""
        if state["last_delta"] is None:
            return True, 0
        since = state["steps"] + 1
        if self.count_due(since):
            return True, since
        if not self.needs_sparse_history or state["last_sparse"] is None:
            return False, since
        cos = row_cos(sparse, state["last_sparse"])
        hit = self.drifted(cos, state["cos_hist"])
        if self.policy == "drift_rel":
            state["cos_hist"] = (state["cos_hist"] + [cos])[-self.WINDOW:]
        return hit, since


def commit(state: dict, anchor: bool, since: int, sparse: torch.Tensor,
           dense: torch.Tensor | None, out: torch.Tensor) -> None:
    """State after a step: an anchor stores its correction dense - sparse and
    restarts the count."""
    if anchor:
        state["last_delta"] = dense - sparse
    state["steps"] = 0 if anchor else since
    state["last_sparse"] = sparse


def drift_point(state: dict, since: int, anchor: bool, sparse: torch.Tensor,
                dense: torch.Tensor, out: torch.Tensor) -> dict:
    """One record of the drift log (the sidecar schema of
    model_wrapper._flush_drift_stats): the cached correction against this
    step's true one, and the output against the dense row."""
    return {"steps_since_anchor": int(since), "anchor": bool(anchor),
            "drift_cos": row_cos(dense - sparse, state["last_delta"]),
            "applied_vs_true_cos": row_cos(out, dense)}
