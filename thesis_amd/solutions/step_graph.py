"""HIP-graph replay of fixed-shape shallow steps (the shallow-step glue of solutions/engine.py:308-354).

A shallow-only step (no verification, probe or prefill chunk) issues the same launches with the same launch
dimensions whenever its shape key repeats: packed tokens, blocks, attention work items, combine groups,
partial slots, schedule items and slots, drafts and the exit layer.  Only the packed metadata and the index
arrays change from step to step.  Those live here in per-key device buffers at fixed addresses, refreshed by
one host-to-device copy per step, so the step's launches (embedding, k layers, exit-state copy, draft head)
replay as one captured graph.

* A key is captured the second time it is seen: the first, eager run sizes every reusable model buffer, so
  the capture allocates only the intermediates it owns (its private memory pool).
* Every graph is dropped when the model reallocates a reusable buffer, its cache or its native handle
  (`LayerSkipLlama.buf_epoch`), and a capture that itself grew a buffer is discarded unreplayed.
* The graph holds no memset node: every kernel overwrites its outputs.
* Profiling launches (`_lsk.Profiler`) are never captured; the caller runs such steps eagerly.
"""

from __future__ import annotations

from typing import Callable, Optional

import numpy as np
import torch

_ALIGN = 256
_NP_TO_TORCH = {np.dtype(np.int32): torch.int32, np.dtype(np.int64): torch.int64}


class _Entry:
    """Fixed-address staging (pinned host + device) for one shape key, and its graph once captured."""

    def __init__(self, arrays: list, device: torch.device):
        self.offs, total = [], 0
        for a in arrays:
            total = (total + _ALIGN - 1) // _ALIGN * _ALIGN
            self.offs.append(total)
            total += a.nbytes
        self.host = torch.empty(max(total, _ALIGN), dtype=torch.uint8, pin_memory=True)
        self.dev = torch.empty(max(total, _ALIGN), dtype=torch.uint8, device=device)
        hv = self.host.numpy()
        self.host_views = [hv[o:o + a.nbytes].view(a.dtype) for a, o in zip(arrays, self.offs)]
        self.dev_views = [self.dev[o:o + a.nbytes].view(_NP_TO_TORCH[a.dtype]) for a, o in zip(arrays, self.offs)]
        self.copied = torch.cuda.Event()      # the last copy out of `host` has been read by the device
        self.copied.record()
        self.graph: Optional[torch.cuda.CUDAGraph] = None
        self.epoch = -1
        self.seen = 0


class ShallowGraphs:
    def __init__(self, device: torch.device, max_keys: int = 64):
        self.dev = torch.device(device)
        self.max_keys = max_keys
        self.entries: dict = {}
        self.replays = 0
        self.captures = 0

    def stage(self, key: tuple, arrays: list) -> tuple:
        """Copy `arrays` (int32 / int64, shapes fixed by `key`) into the key's fixed device buffers; returns
        (device views in order, entry)."""
        e = self.entries.get(key)
        if e is None:
            if len(self.entries) >= self.max_keys:
                self.entries.pop(next(iter(self.entries)))
            e = self.entries[key] = _Entry(arrays, self.dev)
        e.copied.synchronize()                # the previous step's copy has left the pinned buffer
        for v, a in zip(e.host_views, arrays):
            v[...] = a
        e.dev.copy_(e.host, non_blocking=True)
        e.copied.record()
        return e.dev_views, e

    def run(self, e: _Entry, epoch: Callable[[], int], step: Callable[[], None]) -> str:
        """Run one step of entry `e`: replay its graph, capture it (second sighting) or run it eagerly.
        `epoch()` reads the model's buffer epoch.  Returns "replay", "capture" or "eager"."""
        if e.graph is not None and e.epoch != epoch():
            e.graph, e.seen = None, 0         # a buffer it writes or reads was reallocated
        if e.graph is not None:
            e.graph.replay()
            self.replays += 1
            return "replay"
        e.seen += 1
        if e.seen < 2:
            step()
            return "eager"
        before = epoch()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            step()
        if epoch() != before:                 # the capture allocated a model buffer: never replay it
            step()
            return "eager"
        e.graph, e.epoch = g, before
        self.captures += 1
        g.replay()
        self.replays += 1
        return "capture"

    def clear(self) -> None:
        self.entries.clear()
