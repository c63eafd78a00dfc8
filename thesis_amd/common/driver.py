"""Request drivers shared by the engines.

An engine exposes its slots through four calls (`SlotOps`); the drivers decide which request enters which slot
and when a measurement ends:

  run_pool      the prompt pool once ("static") or cyclically ("cyclic": a finished slot is refilled with the next
                prompt, round robin), under a MeasureWindow
  run_arrivals  open loop: requests arrive at wall-clock times drawn from a Poisson process and wait in FIFO
                order for a free slot; the run ends after a fixed number of completions

The measurement rules are the reference's (common/engine.py:143-230 and solutions/engine.py:544-673): a number of
warm-up completions is excluded; a cyclic run stops when the running throughput has stayed within a relative
threshold of an anchor for a window of consecutive completions (after a minimum count), or at a maximum count.
"""

from __future__ import annotations

import math
import time
from collections import deque
from typing import Callable, Optional, Protocol

import numpy as np


class SlotOps(Protocol):
    n_slots: int

    def admit(self, slot: int, index: int, prompt) -> bool:
        """Start `prompt` (pool index `index`) in a free slot; True if it already finished (its first token)."""

    def advance(self) -> list:
        """One engine step; the slots whose request finished in it."""

    def release(self, slot: int) -> None:
        """Record the finished request of `slot` and free the slot."""

    def busy(self) -> bool:
        """Whether any slot still has work (decoding or a pending prefill)."""


class MeasureWindow:
    """Which completions are measured, and when a replay has measured enough.

    warmup      completions before measuring starts (0: measure from the first step)
    min_eval    measured completions before the convergence test applies
    max_eval    measured completions that end the run ("max_eval_samples"); None: no cap
    threshold   relative distance from the anchor throughput that counts as stable
    window      consecutive stable completions that end the run ("converged")
    per_step    a completion counts as measured by the window's state when its step began (the DecodeEngine
                rule, common/engine.py:224-247: requests finishing in the step where warm-up ends are not
                evaluated); False: by the state when it is accounted (the EESD rule, solutions/engine.py:588-600)
    A throughput callable that returns None (no measured time yet) skips the convergence test.
    """

    def __init__(self, warmup: int = 0, min_eval: int = 0, max_eval: Optional[int] = None, threshold: float = 0.01,
                 window: int = 4, converge: bool = True, on_start: Optional[Callable[[], None]] = None,
                 per_step: bool = False):
        self.warmup, self.min_eval, self.max_eval = warmup, min_eval, max_eval
        self.threshold, self.window, self.converge = threshold, window, converge
        self.on_start = on_start
        self.per_step = per_step
        self.measuring = False
        self.step_measured = False
        self.warm_done = 0
        self.evaluated = 0
        self._anchor: Optional[float] = None
        self._stable = 0
        self.t_start: Optional[float] = None
        if warmup <= 0:
            self._start()
        self.step_measured = self.measuring

    def begin_step(self) -> None:
        """Snapshot the measuring state for the completions of the step about to be accounted."""
        self.step_measured = self.measuring

    def _start(self) -> None:
        self.measuring = True
        if self.on_start is not None:
            self.on_start()
        self.t_start = time.perf_counter()

    def completed(self, throughput: Callable[[], float]) -> Optional[str]:
        """Account one finished request; returns the stop reason when the window is full."""
        if not (self.step_measured if self.per_step else self.measuring):
            if not self.measuring:
                self.warm_done += 1
                if self.warm_done >= self.warmup:
                    self._start()
            return None
        self.evaluated += 1
        thr = throughput() if self.converge and self.evaluated >= self.min_eval else None
        if thr is not None:
            if self._anchor is not None and abs(thr - self._anchor) < self.threshold * max(self._anchor, 1e-9):
                self._stable += 1
            else:
                self._anchor, self._stable = thr, 0
            if self._stable >= self.window:
                return "converged"
        if self.max_eval is not None and self.evaluated >= self.max_eval:
            return "max_eval_samples"
        return None


class PromptPool:
    """Prompts handed out in order, once (static) or round robin without end (cyclic)."""

    def __init__(self, prompts: list, cyclic: bool):
        self.prompts, self.cyclic, self.cursor = prompts, cyclic, 0

    def has_next(self) -> bool:
        return bool(self.prompts) and (self.cyclic or self.cursor < len(self.prompts))

    def take(self) -> tuple:
        i = self.cursor % len(self.prompts)
        self.cursor += 1
        return i, self.prompts[i]


def run_pool(ops: SlotOps, prompts: list, cyclic: bool, window: MeasureWindow,
             throughput: Callable[[], Optional[float]], max_steps: Optional[int] = None,
             drain_after_stop: bool = True) -> str:
    """Drive `ops` over the pool until it is exhausted, the window stops the run or `max_steps` engine steps
    ran; returns the stop reason.  Requests finished by their first token are released without a step.
    drain_after_stop: the step's remaining finished requests are still released and accounted after the stop
    reason is set (the EESD rule, solutions/engine.py:582-604); False: they are left unrecorded (the
    DecodeEngine rule, common/engine.py:226-229)."""
    pool = PromptPool(prompts, cyclic)
    finished: deque = deque()
    for slot in range(ops.n_slots):
        if not pool.has_next():
            break
        if ops.admit(slot, *pool.take()):
            finished.append(slot)
    steps, stop = 0, None
    while stop is None:
        window.begin_step()
        if not finished:
            if not ops.busy():
                return "pool_exhausted"
            finished.extend(ops.advance())
            steps += 1
        while finished:
            if stop is not None and not drain_after_stop:
                break
            slot = finished.popleft()
            ops.release(slot)
            reason = window.completed(throughput)
            stop = stop or reason
            if stop is None and pool.has_next() and ops.admit(slot, *pool.take()):
                finished.append(slot)
        if stop is None and max_steps is not None and steps >= max_steps:
            stop = "max_steps"
    return stop


class PoissonArrivals:
    """Arrival times t_0 + e_1, t_0 + e_1 + e_2, ... with e_i ~ Exp(rate), drawn from default_rng(seed)."""

    def __init__(self, rate_per_s: float, seed: int, t0: float):
        self.rng = np.random.default_rng(seed)
        self.scale = 1.0 / rate_per_s
        self.next_t = t0 + self.rng.exponential(self.scale)

    def due(self, now: float) -> list:
        """Arrival times up to `now` not yet returned."""
        out = []
        while self.next_t <= now:
            out.append(self.next_t)
            self.next_t += self.rng.exponential(self.scale)
        return out


def run_arrivals(ops: SlotOps, free_slots: Callable[[], list], make_request: Callable[[int, float], object],
                 admit_request: Callable[[int, object], bool], arrivals: PoissonArrivals, n_total: int,
                 on_release: Callable[[], None]) -> int:
    """Open-loop driver: arriving requests queue FIFO and take free slots; idle waits sleep until the next
    arrival (at most 10 ms at a time).  Ends after n_total releases; returns the queue length left."""
    queue: deque = deque()
    released, arrived = 0, 0
    while released < n_total:
        for t in arrivals.due(time.perf_counter()):
            queue.append(make_request(arrived, t))
            arrived += 1
        finished = []
        for slot in free_slots():
            if not queue:
                break
            if admit_request(slot, queue.popleft()):
                finished.append(slot)
        if not finished:
            if not ops.busy():
                time.sleep(max(0.0, min(arrivals.next_t - time.perf_counter(), 0.01)))
                continue
            finished = ops.advance()
        for slot in finished:
            ops.release(slot)
            released += 1
            on_release()
    return len(queue)


def warmup_count(samples: int, per_slot: float, n_slots: int) -> int:
    """Warm-up completions of a cyclic run: max(samples, ceil(per_slot * slots)), 0 when samples is 0."""
    return max(samples, math.ceil(per_slot * n_slots)) if samples else 0
