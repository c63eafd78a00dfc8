"""Packed (ragged) forward over an arbitrary set of request token blocks (solutions/packed.py surface).

Every block r contributes T_r consecutive tokens at positions pos0_r .. pos0_r + T_r - 1 of KV cache
row `row_r`; the blocks are concatenated into one token axis (qo_indptr = cumsum(T_r)).  A query at
position p of row r attends to cached positions <= p of row r, after this call's K/V were appended
(solutions/packed.py:3-8).  Shallow-draft rows, deep-verify rows and prefill chunks with different
layer ranges are expressed as separate packed segments over the same cache.

Kept from the reference API: `upload`, `Block`, `Bucket`, `PackedBatch` (blocks, offsets, pos, rows,
cos, sin, buckets, n_tokens, kv_read, kv_read_padded, kv_gathered, block_slice), `build_packed`
(same block order: bucket-major by T then (row, pos0) for "exact", one (row, pos0)-sorted group for
"pad", ValueError otherwise), `packed_layer`, `packed_layers`, `qo_indptr`.

What changes: the attention metadata is a per-block ragged description consumed by one kernel
(lsk_ragged_attn) instead of per-bucket dense masks and KV gathers, so `Bucket.mask` is None and
no KV is copied for non-contiguous rows.  The buckets are still computed on the host for the
reference's accounting (kv_read_padded / kv_gathered keep the reference's definitions).  All
metadata of a segment travels in one pinned, non_blocking H2D copy: no device->host sync here.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

import numpy as np
import torch

from .. import _lsk


def upload(arr, device: torch.device, dtype=torch.long) -> torch.Tensor:
    """CPU numpy/list -> device tensor without a stream synchronisation (pinned + non_blocking)."""
    t = torch.as_tensor(np.asarray(arr), dtype=dtype)
    if torch.device(device).type == "cuda":
        return t.pin_memory().to(device, non_blocking=True)
    return t


def qo_indptr(lengths) -> np.ndarray:
    """cumsum of per-request token counts with a leading 0 (solutions/packed.py:199-201)."""
    return np.concatenate([[0], np.cumsum(np.asarray(lengths, dtype=np.int64))]).astype(np.int64)


@dataclass
class Block:
    row: int
    pos0: int
    T: int
    tag: object = None


@dataclass
class Bucket:
    start: int
    end: int
    b: int
    T: int
    L: int
    rows: Optional[torch.Tensor]
    b0: int
    mask: Optional[torch.Tensor] = None            # never built: the ragged kernel applies the causal rule
    pad_index: Optional[torch.Tensor] = None


@dataclass
class PackedBatch:
    blocks: list
    offsets: np.ndarray
    pos_h: np.ndarray                 # [N] positions (host)
    rows_h: np.ndarray                # [N] cache rows (host)
    buckets: list = field(default_factory=list)
    n_tokens: int = 0
    kv_read: int = 0
    kv_read_padded: int = 0
    kv_gathered: int = 0
    # kernel metadata (device int32): [rows N][pos N][blocks nb*4][works nw*8][groups ng*8]
    meta: Optional[torch.Tensor] = None
    nb: int = 0
    n_works: int = 0
    n_groups: int = 0
    n_parts: int = 0
    attn_bytes: float = 0.0
    attn_flops: float = 0.0
    _model: object = None

    def block_slice(self, i: int) -> slice:
        return slice(int(self.offsets[i]), int(self.offsets[i + 1]))

    @property
    def pos(self) -> torch.Tensor:
        return torch.as_tensor(self.pos_h).to(self._model.device)

    @property
    def rows(self) -> torch.Tensor:
        return torch.as_tensor(self.rows_h).to(self._model.device)

    @property
    def cos(self) -> torch.Tensor:
        m = self._model
        return m.rope_cos[self.pos].to(m.dtype).unsqueeze(1)

    @property
    def sin(self) -> torch.Tensor:
        m = self._model
        return m.rope_sin[self.pos].to(m.dtype).unsqueeze(1)


def _validate(model, blocks) -> None:
    cache = model.cache
    if cache is None:
        raise ValueError("allocate_cache() first")
    for b in blocks:
        if not (0 <= b.row < cache.max_batch):
            raise ValueError(f"block row {b.row} outside the cache's {cache.max_batch} rows")
        if b.T < 1 or b.pos0 < 0 or b.pos0 + b.T > cache.max_seq:
            raise ValueError(f"block positions [{b.pos0}, {b.pos0 + b.T}) outside max_seq={cache.max_seq}")
    if blocks and max(b.pos0 + b.T for b in blocks) > model.rope_cos.shape[0]:
        raise ValueError("positions beyond the RoPE table")


def pack_blocks(model, ordered: list, groups: Optional[list] = None, bucketing: str = "exact") -> PackedBatch:
    """Build the packed batch for blocks already in packed order (groups = bucket partition)."""
    _validate(model, ordered)
    nb = len(ordered)
    Ts = np.fromiter((b.T for b in ordered), dtype=np.int64, count=nb)
    pos0 = np.fromiter((b.pos0 for b in ordered), dtype=np.int64, count=nb)
    rws = np.fromiter((b.row for b in ordered), dtype=np.int64, count=nb)
    offsets = qo_indptr(Ts)
    N = int(offsets[-1])
    within = np.arange(N, dtype=np.int64) - np.repeat(offsets[:-1], Ts)
    pos_h = np.repeat(pos0, Ts) + within
    rows_h = np.repeat(rws, Ts)
    blk = np.stack([offsets[:-1], pos0, Ts, rws], axis=1).astype(np.int32) if nb else np.zeros((0, 4), np.int32)
    split = model.cache.attn_split
    works, grps, n_parts = _lsk.attn_plan(blk, model.group, split) if nb else (np.zeros((0, 8), np.int32),) * 2 + (0,)
    meta = np.concatenate([rows_h.astype(np.int32), pos_h.astype(np.int32), blk.ravel(), works.ravel(),
                           grps.ravel()]).astype(np.int32)
    pb = PackedBatch(list(ordered), offsets, pos_h, rows_h, n_tokens=N, nb=nb, n_works=len(works),
                     n_groups=len(grps), n_parts=n_parts, _model=model)
    # algorithmic work of one attention launch (per layer): K+V of every attended position read once per
    # (block, KV head), Q read and O written once; flops = 4 Hq D per (query, attended position)
    c = model.cfg
    es = model.dtype.itemsize
    pb.attn_bytes = float((pos0 + Ts).sum()) * c.n_kv_heads * c.head_dim * 2 * es + N * c.n_heads * c.head_dim * 2 * es
    pb.attn_flops = 4.0 * c.n_heads * c.head_dim * float((Ts * pos0 + Ts * (Ts + 1) // 2).sum())
    pb.meta = upload(meta, model.device, dtype=torch.int32) if N else None
    # ---- reference bucket bookkeeping (solutions/packed.py:109-138), host only
    if groups is None:
        groups = [ordered] if ordered else []
    max_seq = model.cache.max_seq
    first = 0
    for g in groups:
        n = len(g)
        start, end = int(offsets[first]), int(offsets[first + n])
        Tm = max(b.T for b in g)
        L = min((max(b.pos0 + b.T - 1 for b in g) + 1 + 63) // 64 * 64, max_seq)
        rl = [b.row for b in g]
        contiguous = rl == list(range(rl[0], rl[0] + n))
        pad = None
        if bucketing == "pad" and any(b.T != Tm for b in g):
            pad = torch.full((n, Tm), -1, dtype=torch.long)
            for j in range(n):
                pad[j, :g[j].T] = torch.arange(int(offsets[first + j]), int(offsets[first + j + 1]))
        pb.buckets.append(Bucket(start, end, n, Tm, L, None if contiguous else torch.tensor(rl), rl[0], None, pad))
        pb.kv_read += sum(b.pos0 + b.T for b in g)
        pb.kv_read_padded += n * L
        if not contiguous:
            pb.kv_gathered += n * L
        first += n
    return pb


def build_packed(model, blocks: list, bucketing: str = "exact") -> PackedBatch:
    """Order the blocks bucket-major (by T, then row) and build all attention metadata
    (solutions/packed.py:81-139)."""
    key = lambda b: (b.row, b.pos0)  # noqa: E731
    if bucketing == "exact":
        by_T: dict = {}
        for b in blocks:
            by_T.setdefault(b.T, []).append(b)
        groups = [sorted(by_T[T], key=key) for T in sorted(by_T)]
    elif bucketing == "pad":
        groups = [sorted(blocks, key=key)] if blocks else []
    else:
        raise ValueError(bucketing)
    ordered = [b for g in groups for b in g]
    return pack_blocks(model, ordered, groups, bucketing)


def packed_layers(model, x: torch.Tensor, pb: PackedBatch, start: int, end: int, capture: Optional[dict] = None,
                  capture_layers: tuple = ()) -> torch.Tensor:
    """Run layers [start, end) on packed tokens x [N, dim] (one native call).  capture[k] = hidden state
    entering exit layer k (output of layer k-1) for every k in capture_layers with start < k <= end."""
    N = pb.n_tokens
    if x.shape != (N, model.cfg.dim) or x.dtype != model.dtype or x.device != model.device:
        raise ValueError(f"x must be [{N}, {model.cfg.dim}] {model.dtype} on {model.device}")
    x = x.contiguous()
    out = torch.empty_like(x)
    if N == 0 or start == end:
        out.copy_(x)
        if capture is not None:
            for k in capture_layers:
                if start < k <= end:
                    capture[k] = out
        return out
    cap_ptrs = None
    if capture is not None:
        cap_ptrs = [None] * model.n_layers
        for k in capture_layers:
            if start < k <= end:
                t = out if k == end else torch.empty_like(x)
                capture[k] = t
                if k != end:
                    cap_ptrs[k - 1] = t.data_ptr()
    ws = model.workspace(model.native.workspace_bytes(N, pb.n_parts))
    model.native.forward_layers(x, out, N, start, end, pb.meta, pb.nb, pb.n_works, pb.n_groups, pb.n_parts, ws,
                                cap_ptrs, pb.attn_bytes, pb.attn_flops)
    return out


def packed_layer(model, i: int, x: torch.Tensor, pb: PackedBatch) -> torch.Tensor:
    """One decoder layer on packed tokens x [N, dim]; writes this call's K/V into the cache."""
    return packed_layers(model, x, pb, i, i + 1)
