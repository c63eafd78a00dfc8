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


_NP_TO_TORCH = {np.dtype(np.int32): torch.int32, np.dtype(np.int64): torch.int64}


def upload_many(arrays: list, device: torch.device) -> list:
    """Several int32 / int64 numpy arrays -> device tensors through ONE pinned staging buffer and ONE
    non_blocking copy (each array 8-byte aligned in the buffer); returns the device views in order."""
    offs, total = [], 0
    for a in arrays:
        total = (total + 7) // 8 * 8
        offs.append(total)
        total += a.nbytes
    host = torch.empty(max(total, 8), dtype=torch.uint8, pin_memory=True)
    hv = host.numpy()
    for a, o in zip(arrays, offs):
        hv[o:o + a.nbytes] = np.ascontiguousarray(a).view(np.uint8).reshape(-1)
    dev = host.to(device, non_blocking=True)
    return [dev[o:o + a.nbytes].view(_NP_TO_TORCH[a.dtype]) for a, o in zip(arrays, offs)]


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
    """Packed segment metadata.  Per-block arrays are in packed order; `blocks` lists them as Block
    objects (built on first access when the batch came from arrays).  `order[j]` is the caller's index
    of packed block j."""
    offsets: np.ndarray
    pos_h: np.ndarray                 # [N] positions (host)
    rows_h: np.ndarray                # [N] cache rows (host)
    blk_rows: np.ndarray = None
    blk_pos0: np.ndarray = None
    blk_T: np.ndarray = None
    order: np.ndarray = None
    n_tokens: int = 0
    kv_read: int = 0
    kv_read_padded: int = 0
    kv_gathered: int = 0
    # kernel metadata (device int32): [rows N][pos N][blocks nb*4][works nw*8][groups ng*8]
    # [schedule records n_slots*n_rounds*8]
    meta: Optional[torch.Tensor] = None
    meta_host: Optional[np.ndarray] = None
    nb: int = 0
    n_works: int = 0
    n_groups: int = 0
    n_parts: int = 0
    n_rounds: int = 0
    n_slots: int = 0
    rows_cap: int = 48                     # query rows per attention work item (lsk_attn_rows_cap)
    attn_bytes: float = 0.0
    attn_flops: float = 0.0
    _model: object = None
    _blocks: Optional[list] = None
    _tags: Optional[list] = None
    _buckets: Optional[list] = None
    _bounds: Optional[np.ndarray] = None
    _bucketing: str = "exact"

    @property
    def buckets(self) -> list:
        """The reference's bucket bookkeeping (solutions/packed.py:109-138), built on first access."""
        if self._buckets is None:
            self._buckets = _buckets(self.blk_rows, self.blk_pos0, self.blk_T, self.offsets, self._bounds,
                                     self._bucketing, self._model.cache.max_seq)
        return self._buckets

    @property
    def blocks(self) -> list:
        if self._blocks is None:
            tags = self._tags
            self._blocks = [Block(int(r), int(p), int(t), tags[j] if tags is not None else None)
                            for j, (r, p, t) in enumerate(zip(self.blk_rows, self.blk_pos0, self.blk_T))]
        return self._blocks

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


def _validate(model, rows: np.ndarray, pos0: np.ndarray, T: np.ndarray) -> None:
    cache = model.cache
    if cache is None:
        raise ValueError("allocate_cache() first")
    if len(rows) == 0:
        return
    bad = (rows < 0) | (rows >= cache.max_batch)
    if bad.any():
        raise ValueError(f"block row {int(rows[bad][0])} outside the cache's {cache.max_batch} rows")
    bad = (T < 1) | (pos0 < 0) | (pos0 + T > cache.max_seq)
    if bad.any():
        j = int(np.flatnonzero(bad)[0])
        raise ValueError(f"block positions [{int(pos0[j])}, {int(pos0[j] + T[j])}) outside max_seq={cache.max_seq}")
    if int((pos0 + T).max()) > model.rope_cos.shape[0]:
        raise ValueError("positions beyond the RoPE table")


def packed_order(rows, pos0, T, bucketing: str = "exact") -> np.ndarray:
    """Packed block order of solutions/packed.py:95-101: "exact" groups by T ascending, each group by
    (row, pos0); "pad" is one (row, pos0)-ordered group.  Stable, like the reference's sorted()."""
    if bucketing == "exact":
        return np.lexsort((pos0, rows, T))
    if bucketing == "pad":
        return np.lexsort((pos0, rows))
    raise ValueError(bucketing)


def build_packed_arrays(model, rows, pos0, T, bucketing: str = "exact", tags: Optional[list] = None,
                        upload_meta: bool = True) -> PackedBatch:
    """build_packed over per-block arrays (row, pos0, T) in caller order.  With upload_meta=False the
    kernel metadata stays in `meta_host` for the caller to upload (e.g. with upload_many) into `meta`."""
    rows = np.asarray(rows, dtype=np.int64)
    pos0 = np.asarray(pos0, dtype=np.int64)
    T = np.asarray(T, dtype=np.int64)
    order = packed_order(rows, pos0, T, bucketing)
    rws, p0, Ts = rows[order], pos0[order], T[order]
    cache = model.cache
    if cache is None:
        raise ValueError("allocate_cache() first")
    n_slots = _lsk.cu_count(model.device)
    meta, cnt = _lsk.pack_segment(rws, p0, Ts, model.group, cache.attn_split, model.cfg.n_kv_heads,
                                  model.cfg.head_dim, n_slots, 0 if bucketing == "exact" else 1, cache.max_batch,
                                  cache.max_seq, model.rope_cos.shape[0])
    N, nw, ng, n_parts, n_rounds, _, kv_read, kv_padded, kv_gathered, pairs, rows_cap = cnt
    nb = len(Ts)
    offsets = qo_indptr(Ts)
    pb = PackedBatch(offsets, meta[N:2 * N].astype(np.int64), meta[:N].astype(np.int64), rws, p0, Ts, n_tokens=N,
                     nb=nb, n_works=nw, n_groups=ng, n_parts=n_parts, n_rounds=n_rounds, n_slots=n_slots,
                     rows_cap=rows_cap, _model=model, meta_host=meta, kv_read=kv_read, kv_read_padded=kv_padded,
                     kv_gathered=kv_gathered, _bucketing=bucketing)
    if bucketing == "exact" and nb and Ts[0] != Ts[-1]:            # (Ts ascending: equal ends = one bucket)
        pb._bounds = np.concatenate([[0], np.flatnonzero(np.diff(Ts)) + 1, [nb]])
    else:
        pb._bounds = np.array([0, nb]) if nb else np.array([0])
    _attn_work(pb, model, kv_read, pairs)
    if upload_meta and N:
        pb.meta = upload(meta, model.device, dtype=torch.int32)
    pb.order = order
    pb._tags = [tags[i] for i in order] if tags is not None else None
    return pb


def _attn_work(pb: PackedBatch, model, kv_read: int, pairs: int) -> None:
    """Algorithmic work of one attention launch (per layer): K+V of every attended position read once per
    (block, KV head), Q read and O written once; flops = 4 Hq D per (query, attended position)."""
    c = model.cfg
    es = model.dtype.itemsize
    pb.attn_bytes = float(kv_read) * c.n_kv_heads * c.head_dim * 2 * es + pb.n_tokens * c.n_heads * c.head_dim * 2 * es
    pb.attn_flops = 4.0 * c.n_heads * c.head_dim * float(pairs)


def _buckets(rws, pos0, Ts, offsets, bounds, bucketing: str, max_seq: int) -> list:
    out = []
    for gi in range(len(bounds) - 1):
        a, b = int(bounds[gi]), int(bounds[gi + 1])
        n = b - a
        gr, gp, gt = rws[a:b], pos0[a:b], Ts[a:b]
        start, end = int(offsets[a]), int(offsets[b])
        Tm = int(gt.max())
        L = min((int((gp + gt).max()) + 63) // 64 * 64, max_seq)
        contiguous = bool((gr == np.arange(gr[0], gr[0] + n)).all())
        pad = None
        if bucketing == "pad" and (gt != Tm).any():
            pad = torch.full((n, Tm), -1, dtype=torch.long)
            for j in range(n):
                pad[j, :int(gt[j])] = torch.arange(int(offsets[a + j]), int(offsets[a + j + 1]))
        out.append(Bucket(start, end, n, Tm, L, None if contiguous else torch.as_tensor(gr), int(gr[0]), None, pad))
    return out


def _pack(model, rws: np.ndarray, pos0: np.ndarray, Ts: np.ndarray, bounds: np.ndarray, bucketing: str,
          upload_meta: bool) -> PackedBatch:
    """Blocks already in packed order with a caller-given bucket partition (pack_blocks)."""
    _validate(model, rws, pos0, Ts)
    nb = len(Ts)
    offsets = qo_indptr(Ts)
    N = int(offsets[-1])
    within = np.arange(N, dtype=np.int64) - np.repeat(offsets[:-1], Ts)
    pos_h = np.repeat(pos0, Ts) + within
    rows_h = np.repeat(rws, Ts)
    blk = np.stack([offsets[:-1], pos0, Ts, rws], axis=1).astype(np.int32) if nb else np.zeros((0, 4), np.int32)
    split = model.cache.attn_split
    n_slots = _lsk.cu_count(model.device)
    cap = _lsk.attn_rows_cap(blk, model.group, split, model.cfg.n_kv_heads, model.cfg.head_dim, n_slots)
    works, grps, n_parts = (_lsk.attn_plan(blk, model.group, split, cap) if nb
                            else (np.zeros((0, 8), np.int32),) * 2 + (0,))
    recs, n_rounds = _lsk.attn_schedule(works, model.cfg.n_kv_heads, n_slots)
    meta = np.concatenate([rows_h.astype(np.int32), pos_h.astype(np.int32), blk.ravel(), works.ravel(),
                           grps.ravel(), recs]).astype(np.int32)
    pb = PackedBatch(offsets, pos_h, rows_h, rws, pos0, Ts, n_tokens=N, nb=nb, n_works=len(works),
                     n_groups=len(grps), n_parts=n_parts, n_rounds=n_rounds, n_slots=n_slots, rows_cap=cap,
                     _model=model,
                     meta_host=meta, _bounds=bounds, _bucketing=bucketing)
    _attn_work(pb, model, int((pos0 + Ts).sum()), int((Ts * pos0 + Ts * (Ts + 1) // 2).sum()))
    if upload_meta and N:
        pb.meta = upload(meta, model.device, dtype=torch.int32)
    pb.kv_read = int((pos0 + Ts).sum())
    for bk in pb.buckets:
        pb.kv_read_padded += bk.b * bk.L
        if bk.rows is not None:
            pb.kv_gathered += bk.b * bk.L
    return pb


def pack_blocks(model, ordered: list, groups: Optional[list] = None, bucketing: str = "exact") -> PackedBatch:
    """Build the packed batch for blocks already in packed order (groups = bucket partition)."""
    nb = len(ordered)
    rws = np.fromiter((b.row for b in ordered), dtype=np.int64, count=nb)
    pos0 = np.fromiter((b.pos0 for b in ordered), dtype=np.int64, count=nb)
    Ts = np.fromiter((b.T for b in ordered), dtype=np.int64, count=nb)
    if groups is None:
        bounds = np.array([0, nb]) if nb else np.array([0])
    else:
        bounds = np.concatenate([[0], np.cumsum([len(g) for g in groups])]).astype(np.int64)
    pb = _pack(model, rws, pos0, Ts, bounds, bucketing, True)
    pb._blocks = list(ordered)
    pb.order = np.arange(nb)
    return pb


def build_packed(model, blocks: list, bucketing: str = "exact") -> PackedBatch:
    """Order the blocks bucket-major (by T, then row) and build all attention metadata
    (solutions/packed.py:81-139)."""
    nb = len(blocks)
    rows = np.fromiter((b.row for b in blocks), dtype=np.int64, count=nb)
    pos0 = np.fromiter((b.pos0 for b in blocks), dtype=np.int64, count=nb)
    T = np.fromiter((b.T for b in blocks), dtype=np.int64, count=nb)
    pb = build_packed_arrays(model, rows, pos0, T, bucketing)
    pb._blocks = [blocks[i] for i in pb.order]
    return pb


def packed_layers(model, x: torch.Tensor, pb: PackedBatch, start: int, end: int, capture: Optional[dict] = None,
                  capture_layers: tuple = (), out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Run layers [start, end) on packed tokens x [N, dim] (one native call).  capture[k] = hidden state
    entering exit layer k (output of layer k-1) for every k in capture_layers with start < k <= end.
    `out` (optional, contiguous [N, dim], not aliasing x) receives the result."""
    N = pb.n_tokens
    if x.shape != (N, model.cfg.dim) or x.dtype != model.dtype or x.device != model.device:
        raise ValueError(f"x must be [{N}, {model.cfg.dim}] {model.dtype} on {model.device}")
    x = x.contiguous()
    if out is None:
        out = torch.empty_like(x)
    elif out.shape != x.shape or out.dtype != x.dtype or not out.is_contiguous() or out.data_ptr() == x.data_ptr():
        raise ValueError("out must be a contiguous tensor shaped like x that does not alias it")
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
    model.native.forward_layers(x, out, N, start, end, pb.meta, pb.nb, pb.n_works, pb.n_groups, pb.n_parts,
                                pb.n_rounds, pb.n_slots, pb.rows_cap, ws, cap_ptrs, pb.attn_bytes, pb.attn_flops)
    return out


def packed_layer(model, i: int, x: torch.Tensor, pb: PackedBatch) -> torch.Tensor:
    """One decoder layer on packed tokens x [N, dim]; writes this call's K/V into the cache."""
    return packed_layers(model, x, pb, i, i + 1)
