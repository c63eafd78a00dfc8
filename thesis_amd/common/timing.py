"""Step timers (common/timing.py:16-47 semantics): HIP events on the current stream, read lazily."""

from __future__ import annotations

import time
from typing import Optional

import torch


class Interval:
    """One measured interval.  start() / stop() enqueue events; `ms` synchronises on the stop event."""

    def __init__(self, device: torch.device):
        self.device = device
        self.cuda = device.type == "cuda"
        self._t0: Optional[float] = None
        self._t1: Optional[float] = None
        if self.cuda:
            self._e0 = torch.cuda.Event(enable_timing=True)
            self._e1 = torch.cuda.Event(enable_timing=True)

    def start(self) -> "Interval":
        if self.cuda:
            self._e0.record()
        else:
            self._t0 = time.perf_counter()
        return self

    def stop(self) -> "Interval":
        if self.cuda:
            self._e1.record()
        else:
            self._t1 = time.perf_counter()
        return self

    @property
    def ms(self) -> float:
        if self.cuda:
            self._e1.synchronize()
            return float(self._e0.elapsed_time(self._e1))
        return (self._t1 - self._t0) * 1000.0


def sync(device: torch.device) -> None:
    if device.type == "cuda":
        torch.cuda.synchronize(device)
