"""Device-side time spans for the engines' step records.

A span marks two points in the work queued on the current stream: on the GPU two timing events (recording
them does not block the host), on the CPU two wall-clock readings.  The elapsed time is read on demand; on
the GPU that first waits for the closing event, so engines keep spans and read them after the step's own
host synchronisation (the semantics of the reference's common/timing.py:16-47 step timers).
"""

from __future__ import annotations

import time

import torch


class DeviceSpan:
    __slots__ = ("_gpu", "_marks", "_cached")

    def __init__(self, device: torch.device):
        self._gpu = torch.device(device).type == "cuda"
        self._marks: list = []
        self._cached = None

    def _mark(self):
        if not self._gpu:
            return time.perf_counter()
        ev = torch.cuda.Event(enable_timing=True)
        ev.record()
        return ev

    def open(self) -> "DeviceSpan":
        self._marks = [self._mark()]
        self._cached = None
        return self

    def close(self) -> "DeviceSpan":
        if len(self._marks) != 1:
            raise RuntimeError("DeviceSpan.close() without a matching open()")
        self._marks.append(self._mark())
        return self

    @property
    def ms(self) -> float:
        """Milliseconds between open() and close() (waits for the closing GPU event the first time)."""
        if self._cached is None:
            first, last = self._marks
            if self._gpu:
                last.synchronize()
                self._cached = float(first.elapsed_time(last))
            else:
                self._cached = (last - first) * 1e3
        return self._cached


def sync(device: torch.device) -> None:
    """Wait for all queued work of a GPU device (no-op on the CPU)."""
    if torch.device(device).type == "cuda":
        torch.cuda.synchronize(device)
