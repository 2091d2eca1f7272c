"""GPU region timing from HIP event pairs on the current stream."""

from __future__ import annotations

import contextlib
from typing import Dict, List, Optional, Tuple

import torch


class Timer:
    """Named GPU time totals (ms) from event pairs recorded on the current
    stream; nothing synchronises until `totals`."""

    def __init__(self):
        self._pairs: Dict[str, List[Tuple[torch.cuda.Event, torch.cuda.Event]]] = {}

    @contextlib.contextmanager
    def region(self, name: str):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        yield
        e1.record()
        self._pairs.setdefault(name, []).append((e0, e1))

    def totals(self) -> Dict[str, float]:
        torch.cuda.synchronize()
        return {k: sum(a.elapsed_time(b) for a, b in v) for k, v in self._pairs.items()}


def region(timer: Optional[Timer], name: str):
    """timer.region(name), or a no-op without a timer."""
    return timer.region(name) if timer is not None else contextlib.nullcontext()
