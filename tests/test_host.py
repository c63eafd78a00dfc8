"""Host-side logic and the C ABI without a GPU (CPU only).

  * liblsk.so loads and exports every entry point include/lsk.h declares; argument errors are reported
    on the host with negative codes before any launch
  * the attention planner (a host function of the ABI): every query row's KV range [0, pos + 1) is
    covered exactly once, split boundaries are absolute, siblings sit 8 launch slots apart
  * the GEMM plan depends on the weight shape only
  * the product's build_packed equals the oracle's (block order, offsets, buckets, accounting) on
    random block sets, and rejects bad bucketing / out-of-range blocks
  * schedulers / cost model against brute force and the reference's unit cases
  * model config parsing, the product never importing the oracle, bench.py refusing --gpus > 1
"""

from __future__ import annotations

import ctypes
import re
import subprocess
import sys
from pathlib import Path
from types import SimpleNamespace

import numpy as np
import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]


def _lsk():
    from thesis_amd import _lsk

    _lsk.load()
    return _lsk


def test_library_exports_every_declared_entry_point():
    lsk = _lsk()
    header = (ROOT / "include" / "lsk.h").read_text()
    declared = set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(lsk_[a-z_0-9]+)\s*\(", header, re.M))
    assert len(declared) >= 20
    lib = ctypes.CDLL(str(lsk.LIB_PATH))
    missing = [n for n in sorted(declared) if not hasattr(lib, n)]
    assert not missing, missing
    assert declared == set(lsk.EXPORTS), declared ^ set(lsk.EXPORTS)
    assert lsk.load().lsk_abi_version() == lsk.ABI_VERSION


def test_argument_errors_are_reported_on_the_host():
    lsk = _lsk()
    lib = lsk.load()
    assert lib.lsk_gemm(1, None, 64, None, 64, None, 64, None, 0, 4, 64, 64, 0, 0, None) == -1
    rc = lib.lsk_gemm(1, 8, 64, 8, 64, 8, 64, None, 0, 4, 64, 63, 0, 0, None)       # K % 32 != 0
    assert rc == -2 and b"K" in lib.lsk_last_error()
    assert lib.lsk_gemm(1, 8, 64, 8, 64, 8, 64, None, 0, 4, 64, 64, 7, 0, None) == -1  # bad epilogue
    assert lib.lsk_gemm(5, 8, 64, 8, 64, 8, 64, None, 0, 4, 64, 64, 0, 0, None) == -3  # bad dtype
    assert lib.lsk_gemm(1, 8, 64, 8, 128, 8, 64, None, 0, 4, 64, 64, 0, 0, None) == -2  # bf16 W not packed (ldw != K)
    assert lib.lsk_pack_weight(None, 64, 8, 64, 64, None) == -1
    assert lib.lsk_pack_weight(8, 64, 16, 40, 64, None) == -2                          # N % 16 != 0
    assert lib.lsk_unpack_weight(8, 16, 64, 64, 48, None) == -2                        # K % 32 != 0
    assert lib.lsk_rmsnorm(1, 8, 8, 8, 4, 7, 1e-5, 7, 7, None) == -2                 # dim % 8 != 0
    # fused qkv + RoPE + KV append: pointers, head shapes and cache shape are checked before any launch
    q = lib.lsk_gemm_qkv_rope
    assert q(None, 8, 4, 32, 8, 128, 4096, 8, 8, 8, 8, 8, 64, 8, 8, 2, 64, None) == -1         # null A
    assert q(8, 8, 4, 32, 8, 128, 4096, 8, 8, 8, 8, 8, 64, None, 8, 2, 64, None) == -1         # null rows
    assert q(8, 8, 4, 32, 8, 80, 4096, 8, 8, 8, 8, 8, 64, 8, 8, 2, 64, None) == -2             # head_dim % 32
    assert q(8, 8, 4, 0, 8, 128, 4096, 8, 8, 8, 8, 8, 64, 8, 8, 2, 64, None) == -2             # no q heads
    assert q(8, 8, 4, 32, 8, 128, 4010, 8, 8, 8, 8, 8, 64, 8, 8, 2, 64, None) == -2           # K % 32
    assert q(8, 8, 4, 32, 8, 128, 4096, 8, 8, 8, 8, 8, 64, 8, 8, 2, 48, None) == -2           # max_seq % 32
    assert q(8, 8, 4, 32, 8, 128, 4096, 8, 8, 8, 8, 8, 0, 8, 8, 2, 64, None) == -2            # empty RoPE table
    assert q(8, 8, 0, 32, 8, 128, 4096, 8, 8, 8, 8, 8, 64, 8, 8, 2, 64, None) == 0            # M = 0: no launch
    assert lib.lsk_pack_weight_qkv(8, 4096, 8, 32, 8, 80, 4096, None) == -2                   # head_dim % 32
    assert lib.lsk_unpack_weight_qkv(8, 8, 4096, 32, 0, 128, 4096, None) == -2                 # no kv heads
    assert lib.lsk_ragged_attn(1, 8, 8, 8, 8, 8, 1, None, 0, 0, 8, 1, 1, 48, 8, 32, 8, 96, 64, 0.1, None, 0,
                               None) == -3                                            # head_dim 96
    assert lib.lsk_ragged_attn(1, 8, 8, 8, 8, 8, 1, None, 0, 0, None, 0, 0, 48, 8, 32, 8, 128, 64, 0.1, None, 0,
                               None) == -1                                            # bf16 without a schedule
    assert lib.lsk_ragged_attn(1, 8, 8, 8, 8, 8, 1, None, 0, 0, 8, 1, 1, 24, 8, 32, 8, 128, 64, 0.1, None, 0,
                               None) == -1                                            # rows per item not 16/32/48
    assert lib.lsk_model_create(1, 0, 64, 4, 2, 16, 128, 64, 1e-5, *([None] * 8), 1, 64, None, None, 1) < 0
    # one-call final norm + head: pointers, dtype, shape and workspace are checked before any launch
    hn = lib.lsk_head_norm_argmax
    assert hn(1, None, 64, 8, 1e-5, 8, 64, 4, 128, 64, None, 0, 8, None, 8, 1 << 20, None) == -1     # null h
    assert hn(5, 8, 64, 8, 1e-5, 8, 64, 4, 128, 64, None, 0, 8, None, 8, 1 << 20, None) == -3        # not bf16
    assert hn(1, 8, 64, 8, 1e-5, 8, 64, 4, 100, 64, None, 0, 8, None, 8, 1 << 20, None) == -2        # N % 64
    assert hn(1, 8, 64, 8, 1e-5, 8, 128, 4, 128, 64, None, 0, 8, None, 8, 1 << 20, None) == -2       # W not packed
    need = lib.lsk_head_norm_workspace_bytes(4, 128, 64)
    assert need == 2048 + lib.lsk_head_workspace_bytes(4, 128)     # 16 rows x 64 x bf16, then the head's
    assert hn(1, 8, 64, 8, 1e-5, 8, 64, 4, 128, 64, None, 0, 8, None, 8, need - 1, None) == -4       # workspace
    assert hn(1, 8, 64, 8, 1e-5, 8, 64, 0, 128, 64, None, 0, 8, None, 8, 0, None) == 0               # M = 0


@pytest.mark.parametrize("D", [64, 128])
def test_k_fragment_layout(D):
    """k_to_frag follows the documented lane order (computed here element by element) and inverts exactly."""
    lsk = _lsk()
    S = 64
    k = torch.arange(2 * S * D, dtype=torch.float32).view(2, S, D)
    kf = lsk.k_to_frag(k)
    assert kf.shape == (2, S // 32, D // 16, 64, 8)
    for blk, a, j, lane, e in [(0, 0, 0, 0, 0), (1, 1, D // 32 - 1, 63, 7), (0, 1, 0, 21, 3), (1, 0, 1, 42, 5)]:
        l16, lg = lane % 16, lane // 16
        p = 32 * blk + 8 * (l16 // 4) + 4 * a + l16 % 4
        d = 32 * j + 8 * lg + e
        assert kf[1, blk, a * (D // 32) + j, lane, e] == k[1, p, d]
    assert torch.equal(lsk.k_from_frag(kf), k)


def _plan(blocks, G, split):
    return _lsk().attn_plan(np.asarray(blocks, dtype=np.int32), G, split)


@pytest.mark.parametrize("G,split", [(4, 1024), (1, 1024), (4, 64), (8, 512)])
def test_attention_plan_covers_every_row_once(G, split):
    rng = np.random.default_rng(G + split)
    nb = 40
    T = rng.integers(1, 20, nb)
    pos0 = rng.integers(0, 3000, nb)
    q_start = np.concatenate([[0], np.cumsum(T)[:-1]])
    blocks = np.stack([q_start, pos0, T, rng.integers(0, 8, nb)], axis=1)
    works, groups, n_parts = _plan(blocks, G, split)
    R = _lsk().ATTN_ROWS
    by_start = {int(qs): b for b, qs in enumerate(q_start)}
    cover = {}
    parts_seen = []
    for w in works:
        qs, row0, nrows, lo, hi, part, p0, row = (int(v) for v in w)
        if nrows == 0:
            continue                                       # padding slot of the XCD order
        b = by_start[qs]                                   # the record carries its block's fields
        assert (p0, row) == (pos0[b], blocks[b][3])
        assert lo % split == 0 and hi - lo <= split and lo < hi and nrows <= R
        for r in range(row0, row0 + nrows):
            cover.setdefault((b, r), []).append((lo, hi))
        if part >= 0:
            parts_seen.append(part)
    assert len(parts_seen) == len(set(parts_seen)) == n_parts
    for b in range(nb):
        for r in range(T[b] * G):
            ivs = sorted(cover[(b, r)])
            tile = r // R
            t_last = min(tile * R + R - 1, T[b] * G - 1) // G
            end = pos0[b] + t_last + 1                     # the row tile's KV range
            assert ivs[0][0] == 0 and ivs[-1][1] == end
            assert all(ivs[i][1] == ivs[i + 1][0] for i in range(len(ivs) - 1))
    for gp in groups:
        assert gp[4] >= 2 and gp[3] + gp[4] <= n_parts


@pytest.mark.parametrize("n_slots", [1, 7, 256])
def test_attention_schedule_covers_every_item_once_longest_first(n_slots):
    lsk = _lsk()
    rng = np.random.default_rng(n_slots)
    nb = 60
    T = rng.integers(1, 12, nb)
    pos0 = rng.integers(0, 9000, nb)
    blocks = np.stack([np.concatenate([[0], np.cumsum(T)[:-1]]), pos0, T, rng.integers(0, 8, nb)], axis=1)
    works, _, _ = _plan(blocks, 4, 4096)
    Hkv = 8
    recs, R = lsk.attn_schedule(works, Hkv, n_slots)
    recs = recs.reshape(n_slots, R, 8)
    real = [w for w in range(len(works)) if works[w][2] > 0]
    per_slot = []
    for sl in range(n_slots):
        ids = []
        for r in range(R):
            rec = recs[sl, r]
            if rec[2] & 255 == 0:
                assert not rec.any() and not recs[sl, r:].any()      # padding only after the slot's items
                break
            kvh = rec[2] >> 8
            # the record is the work record with the KV head folded into field 2
            w = next(i for i in real if np.array_equal(np.delete(works[i], 2), np.delete(rec, 2))
                     and works[i][2] == rec[2] & 255)
            ids.append(w * Hkv + kvh)
        per_slot.append(ids)
    assert max(len(x) for x in per_slot) == R
    flat = [i for x in per_slot for i in x]
    assert sorted(flat) == sorted(w * Hkv + h for w in real for h in range(Hkv))

    def cost(i):
        w = works[i // Hkv]
        steps, nq = -(-(w[4] - w[3]) // 256), (w[2] + 15) // 16
        return steps * (12 if nq == 3 else 10) + 20 + 12 * (nq - 1)
    loads = [sum(cost(i) for i in x) for x in per_slot]
    # greedy longest-first bound: no slot exceeds the mean by more than the largest item
    assert max(loads) <= sum(loads) / n_slots + max(cost(i) for i in flat)
    again, R2 = lsk.attn_schedule(works, Hkv, n_slots)
    assert R2 == R and np.array_equal(again.reshape(n_slots, R, 8), recs)   # deterministic


def test_attention_rows_per_item_policy():
    """Few (block, KV head) pairs: rows split over more workgroups; a full chip: 48-row items (KV read once)."""
    lsk = _lsk()
    few = np.array([(9 * i, 700, 9, i) for i in range(4)], dtype=np.int32)          # 4 verify blocks, 36 rows
    assert lsk.attn_rows_cap(few, 4, lsk.ATTN_SPLIT, 8, 128, 256) == 16
    many = np.array([(9 * i, 1500, 9, i) for i in range(256)], dtype=np.int32)      # 2048 pairs on 256 CUs
    assert lsk.attn_rows_cap(many, 4, lsk.ATTN_SPLIT, 8, 128, 256) == 48
    # every block fits 16 rows: all caps give the same items, so the one-tile kernel (no per-item overhead) wins
    decode = np.array([(i, 700, 1, i) for i in range(32)], dtype=np.int32)
    assert lsk.attn_rows_cap(decode, 4, lsk.ATTN_SPLIT, 8, 128, 256) == 16
    # the cap is one of the kernel's tile multiples, whatever the shape
    rng = np.random.default_rng(1)
    for _ in range(20):
        nb = int(rng.integers(1, 80))
        T = rng.integers(1, 13, nb)
        blk = np.stack([np.concatenate([[0], np.cumsum(T)[:-1]]), rng.integers(0, 6000, nb), T, np.arange(nb)], 1)
        cap = lsk.attn_rows_cap(blk.astype(np.int32), int(rng.choice([1, 4, 8])), lsk.ATTN_SPLIT, 8, 128, 256)
        assert cap in (16, 32, 48)
    assert lsk.attn_rows_cap(np.zeros((0, 4), np.int32), 4, lsk.ATTN_SPLIT, 8, 128, 256) in (16, 32, 48)
    with pytest.raises(lsk.LskError):
        lsk.attn_rows_cap(decode, 4, lsk.ATTN_SPLIT, 8, 128, 0)                   # no workgroups


@pytest.mark.parametrize("cap", [16, 32, 48])
def test_attention_plan_items_respect_the_rows_cap(cap):
    """Every work item holds <= cap rows of one block, and the items of a block cover its rows once."""
    lsk = _lsk()
    blocks = np.array([(0, 100, 9, 0), (9, 5000, 12, 1), (21, 30, 1, 2)], dtype=np.int32)
    works, _, _ = lsk.attn_plan(blocks, 4, 4096, cap)
    for b, (qs, p0, T, row) in enumerate(blocks):
        mine = [w for w in works if w[2] > 0 and w[0] == qs]
        assert all(w[2] <= cap for w in mine)
        per_split = {}
        for w in mine:
            per_split.setdefault(int(w[3]), []).extend(range(int(w[1]), int(w[1]) + int(w[2])))
        assert all(sorted(r) == list(range(4 * T)) for r in per_split.values()), (cap, b)
    with pytest.raises(lsk.LskError):
        lsk.attn_plan(blocks, 4, 4096, 24)


def test_attention_plan_places_sibling_tiles_eight_slots_apart():
    R = _lsk().ATTN_ROWS
    T = (2 * R + 4) // 4                                     # G = 4: 2 R + 4 rows -> 3 sibling tiles
    blocks = [(T * i, 50 * i, T, i) for i in range(16)]      # KV < 1024: 1 split
    works, _, _ = _plan(blocks, 4, 1024)
    where = {}
    for idx, w in enumerate(works):
        if w[2] > 0:
            where.setdefault(int(w[0]), []).append(idx)
    for b, idxs in where.items():
        assert len(idxs) == 3 and all((j - idxs[0]) % 8 == 0 for j in idxs), (b, idxs)


def test_gemm_plan_depends_on_shape_only():
    lsk = _lsk()
    assert lsk.gemm_plan(28672, 4096) == (4, 1)       # w13 of the 8B shape: wide tiles, whole K
    assert lsk.gemm_plan(128256, 4096) == (4, 1)      # LM head
    ns, ks = lsk.gemm_plan(4096, 14336)               # w2: split K
    assert ns == 2 and ks >= 2 and 14336 % ks == 0 and (14336 // ks) % 128 == 0
    ns, ks = lsk.gemm_plan(6144, 4096)
    assert ns == 2 and 4096 % ks == 0


# ----------------------------------------------------------------------------- packed metadata

def _stub_model(max_batch=8, max_seq=4096, dtype=torch.bfloat16, G=4):
    from thesis_amd.common.model import ModelConfig

    cfg = ModelConfig(vocab_size=64, dim=64, n_layers=2, n_heads=G, n_kv_heads=1, head_dim=128,
                      intermediate_size=128)
    rope = torch.zeros(max_seq, 128)
    return SimpleNamespace(device=torch.device("cpu"), dtype=dtype, group=G, cfg=cfg, rope_cos=rope,
                           rope_sin=rope, cache=SimpleNamespace(max_batch=max_batch, max_seq=max_seq,
                                                                      attn_split=1024))


@pytest.mark.parametrize("bucketing", ["exact", "pad"])
def test_build_packed_matches_oracle(bucketing):
    import oracle.model as om
    from thesis_amd.solutions.packed import Block, build_packed

    rng = np.random.default_rng(1)
    ocfg = om.OracleConfig(64, 64, 1, 4, 1, 16, 64)
    orc = om.OracleLlama(ocfg, om.random_weights(ocfg), dtype=torch.float32, max_seq=4096)
    orc.allocate_cache(8, 4096)
    stub = _stub_model()
    for trial in range(20):
        n = int(rng.integers(1, 9))
        rows = rng.choice(8, n, replace=False)
        spec = [(int(r), int(rng.integers(0, 3000)), int(rng.integers(1, 10))) for r in rows]
        pb = build_packed(stub, [Block(*s) for s in spec], bucketing)
        ob = om.build_packed(orc, [om.OBlock(*s) for s in spec], bucketing)
        assert [(b.row, b.pos0, b.T) for b in pb.blocks] == [(b.row, b.pos0, b.T) for b in ob.blocks]
        assert list(pb.offsets) == list(ob.offsets) and pb.n_tokens == ob.n_tokens
        assert pb.pos_h.tolist() == ob.pos.tolist() and pb.rows_h.tolist() == ob.rows.tolist()
        assert (pb.kv_read, pb.kv_read_padded, pb.kv_gathered) == (ob.kv_read, ob.kv_read_padded, ob.kv_gathered)
        assert [(x.start, x.end, x.b, x.T, x.L, x.b0, x.rows is None) for x in pb.buckets] == \
               [(x.start, x.end, x.b, x.T, x.L, x.b0, x.rows is None) for x in ob.buckets]
        for x, y in zip(pb.buckets, ob.buckets):
            assert (x.pad_index is None) == (y.pad_index is None)
            if x.pad_index is not None:
                assert torch.equal(x.pad_index, y.pad_index)


@pytest.mark.parametrize("bucketing", ["exact", "pad"])
def test_build_packed_arrays_matches_block_path(bucketing):
    """The engine's array path gives the block path's order, metadata and accounting; `order` maps
    packed blocks back to the caller's indices and tags follow their blocks."""
    from thesis_amd.solutions.packed import Block, build_packed, build_packed_arrays

    rng = np.random.default_rng(7)
    stub = _stub_model()
    for trial in range(20):
        n = int(rng.integers(1, 12))
        rows = rng.integers(0, 8, n)                  # repeated rows: ties broken by pos0, then input order
        pos0 = rng.integers(0, 3000, n)
        T = rng.integers(1, 10, n)
        tags = [("t", j) for j in range(n)]
        ref = build_packed(stub, [Block(int(r), int(p), int(t), g) for r, p, t, g in zip(rows, pos0, T, tags)],
                           bucketing)
        got = build_packed_arrays(stub, rows, pos0, T, bucketing, tags=tags, upload_meta=False)
        assert [(b.row, b.pos0, b.T, b.tag) for b in got.blocks] == [(b.row, b.pos0, b.T, b.tag) for b in ref.blocks]
        assert [tags[j] for j in got.order] == [b.tag for b in ref.blocks]
        assert np.array_equal(got.meta_host, ref.meta.numpy()) and got.meta is None
        assert (got.kv_read, got.kv_read_padded, got.kv_gathered) == (ref.kv_read, ref.kv_read_padded, ref.kv_gathered)
        assert [(x.start, x.end, x.b, x.T, x.L, x.b0) for x in got.buckets] == \
               [(x.start, x.end, x.b, x.T, x.L, x.b0) for x in ref.buckets]


@pytest.mark.parametrize("bucketing", ["exact", "pad"])
def test_native_segment_packer_equals_plan_plus_schedule(bucketing):
    """lsk_pack_segment (one host call) writes exactly the metadata of lsk_attn_plan + lsk_attn_schedule plus the
    token expansion, and the reference's bucket accounting, that the step-by-step path (pack_blocks) builds."""
    from thesis_amd.solutions.packed import Block, build_packed_arrays, pack_blocks

    rng = np.random.default_rng(11)
    for G, split in ((4, 1024), (1, 2048), (8, 512)):
        stub = _stub_model(G=G)
        stub.cache.attn_split = split
        for trial in range(15):
            n = int(rng.integers(1, 40))
            rows = rng.integers(0, 8, n)
            pos0 = rng.integers(0, 3500, n)
            T = rng.integers(1, 60 if trial % 3 == 0 else 9, n)
            got = build_packed_arrays(stub, rows, pos0, T, bucketing, upload_meta=False)
            ordered = [Block(int(r), int(p), int(t)) for r, p, t in zip(got.blk_rows, got.blk_pos0, got.blk_T)]
            if bucketing == "exact":
                cut = np.flatnonzero(np.diff(got.blk_T)) + 1
                groups = [list(g) for g in np.split(np.arange(len(ordered)), cut)]
            else:
                groups = [list(range(len(ordered)))]
            ref = pack_blocks(stub, ordered, [[ordered[i] for i in g] for g in groups], bucketing)
            assert np.array_equal(got.meta_host, ref.meta.numpy())
            assert (got.n_works, got.n_groups, got.n_parts, got.n_rounds) == \
                   (ref.n_works, ref.n_groups, ref.n_parts, ref.n_rounds)
            assert (got.kv_read, got.kv_read_padded, got.kv_gathered) == \
                   (ref.kv_read, ref.kv_read_padded, ref.kv_gathered)
            assert (got.attn_bytes, got.attn_flops) == (ref.attn_bytes, ref.attn_flops)
            assert np.array_equal(got.pos_h, ref.pos_h) and np.array_equal(got.rows_h, ref.rows_h)


def test_build_packed_rejects_bad_input():
    from thesis_amd.solutions.packed import Block, build_packed

    stub = _stub_model(max_batch=2, max_seq=128)
    with pytest.raises(ValueError):
        build_packed(stub, [Block(0, 0, 1)], "ragged")
    with pytest.raises(ValueError):
        build_packed(stub, [Block(2, 0, 1)])
    with pytest.raises(ValueError):
        build_packed(stub, [Block(0, 120, 9)])


def test_packed_metadata_layout():
    from thesis_amd.solutions.packed import Block, build_packed

    stub = _stub_model()
    pb = build_packed(stub, [Block(3, 10, 2), Block(1, 700, 1)])
    meta = pb.meta.numpy()
    N = pb.n_tokens
    assert meta[:N].tolist() == pb.rows_h.tolist() and meta[N:2 * N].tolist() == pb.pos_h.tolist()
    blk = meta[2 * N:2 * N + 4 * pb.nb].reshape(-1, 4)
    assert blk.tolist() == [[0, 700, 1, 1], [1, 10, 2, 3]]
    assert meta.size == 2 * N + 4 * pb.nb + 8 * (pb.n_works + pb.n_groups) + 8 * pb.n_slots * pb.n_rounds
    assert pb.n_rounds == 1 and pb.n_slots >= 2                      # 2 (work, KV head) items over the slots
    works = meta[2 * N + 4 * pb.nb:2 * N + 4 * pb.nb + 8 * pb.n_works].reshape(-1, 8)
    recs = meta[2 * N + 4 * pb.nb + 8 * (pb.n_works + pb.n_groups):].reshape(pb.n_slots, pb.n_rounds, 8)
    live = recs[recs[:, 0, 2] != 0, 0]
    assert sorted(map(tuple, live.tolist())) == sorted(map(tuple, works[works[:, 2] > 0].tolist()))  # kvh = 0
    # algorithmic attention work of one launch: K+V of every attended position, Q read and O written
    assert pb.attn_bytes == (701 + 12) * 1 * 128 * 2 * 2 + N * 4 * 128 * 2 * 2


# ----------------------------------------------------------------------------- host policies

def test_expected_token_targets_match_brute_force():
    from thesis_amd.solutions.schedulers import best_gamma_expected, expected_token_targets

    rng = np.random.default_rng(0)
    a = rng.uniform(0.05, 0.97, 300)
    c = rng.uniform(0.02, 0.6, 300)
    got = expected_token_targets(a, c, 1, 12)
    ref = np.array([max(1, best_gamma_expected(ai, ci, 12)) for ai, ci in zip(a, c)])
    assert (np.abs(got - ref) <= 1).mean() > 0.97 and (got == ref).mean() > 0.8


def test_m1_rule_direction():
    from thesis_amd.common.model import PRESETS
    from thesis_amd.solutions.cost_model import synthetic_cost_model
    from thesis_amd.solutions.schedulers import make_scheduler

    cm = synthetic_cost_model(PRESETS["llama3-8b"])
    B = 16
    d, ctx, dec = np.full(B, 2), np.full(B, 1000), np.ones(B, dtype=bool)
    s = make_scheduler("m1", B, cm, 3, d_max=16)
    s.tracker.rate[:] = 0.98                  # drafts almost always accepted: drafting once more pays
    assert not s.decide(d, ctx, dec, 2).any()
    s.tracker.rate[:] = 0.05                  # drafts almost always rejected: verify now
    assert s.decide(d, ctx, dec, 2).all()
    d2 = d.copy()
    d2[0] = 16
    s.tracker.rate[:] = 0.98
    assert s.decide(d2, ctx, dec, 2).all()    # a slot at d_max forces the deep step
    assert s.decide(d, ctx, dec, 32).all()    # so does the idle-step limit (sla_steps)


def test_feedback_policies_and_acceptance_tracker():
    """fsm-sync moves one batch-wide gamma by +-1 on the majority of full accepts (history kept every round);
    aspire-fsm moves each verifying slot's target; the tracker's rate follows rate <- w rate + (1 - w) acc /
    min(acc + 1, d) on verified slots only (solutions/schedulers.py:35-51, 156-197)."""
    from thesis_amd.common.model import PRESETS
    from thesis_amd.solutions.cost_model import synthetic_cost_model
    from thesis_amd.solutions.schedulers import make_scheduler

    cm = synthetic_cost_model(PRESETS["llama3-8b"])
    f = make_scheduler("fsm-sync", 4, cm, 3, gamma=3, d_max=6, omega=0.5, alpha0=0.9)
    v = np.array([True, True, True, False])
    f.observe(v, np.array([3, 3, 1, 0]), np.array([3, 3, 3, 0]))          # 2 of 3 verifiers fully accepted
    assert f.gamma == 4
    f.observe(v, np.array([0, 3, 1, 0]), np.array([3, 3, 3, 0]))          # 1 of 3
    assert f.gamma == 3
    f.observe(np.zeros(4, dtype=bool), np.zeros(4, dtype=int), np.zeros(4, dtype=int))
    assert f.gamma_hist == [3, 4, 3, 3]
    rate = f.tracker.rate
    # slot 0: 0.9 -> 0.5 * 0.9 + 0.5 * 3 / min(4, 3) = 0.95 -> 0.5 * 0.95 + 0.5 * 0 = 0.475; slot 3 never verified
    assert np.isclose(rate[0], 0.475) and rate[3] == 0.9 and f.tracker.cold.tolist() == [False, False, False, True]
    a = make_scheduler("aspire-fsm", 3, cm, 3, d_max=5, initial_draft=2)
    a.observe(np.array([True, True, False]), np.array([2, 0, 0]), np.array([2, 2, 0]))
    assert a.targets.tolist() == [3, 1, 2]
    assert a.decide(np.array([3, 1, 1]), np.full(3, 10), np.ones(3, dtype=bool), 0).tolist() == [True, True, False]
    a.reset(0)
    assert a.targets[0] == 2 and a.tracker.cold[0]


def test_fixed_and_aspire_schedulers():
    from thesis_amd.common.model import PRESETS
    from thesis_amd.solutions.cost_model import mi355x_cost_model
    from thesis_amd.solutions.schedulers import make_scheduler

    cm = mi355x_cost_model(PRESETS["llama3-8b"])
    f = make_scheduler("fixed", 4, cm, 8, gamma=3, d_max=8)
    dec = np.ones(4, dtype=bool)
    d = np.array([0, 1, 3, 8])
    assert f.decide(d, d * 0 + 100, dec, 1).tolist() == [False, False, False, True]
    assert f.decide(d, d * 0 + 100, dec, 3).tolist() == [False, True, True, True]
    a = make_scheduler("aspire", 4, cm, 8, d_max=8, min_draft=2, initial_draft=3)
    v = a.decide(np.array([1, 2, 3, 8]), np.full(4, 500), dec, 0)
    assert not v[0] and v[3]                             # below the [2, 8] floor never verifies; d_max forces
    with pytest.raises(ValueError):
        make_scheduler("nope", 4, cm, 8)


def test_cost_model_formula():
    from thesis_amd.common.model import ModelConfig
    from thesis_amd.solutions.cost_model import GPUParams, ModelDims, RooflineCostModel

    cfg = ModelConfig(vocab_size=1000, dim=64, n_layers=4, n_heads=4, n_kv_heads=2, head_dim=16,
                      intermediate_size=128)
    dims = ModelDims.from_config(cfg)
    gpu = GPUParams(bw=1e6, flops=1e8, t_op=0.01, n_op_layer=50, n_op_bucket=10, n_op_head=8, n_op_segment=5)
    cm = RooflineCostModel(gpu, dims, n_max=64)
    W, P = dims.layer_bytes, dims.layer_params
    for n in (1, 10, 64, 200):
        assert np.isclose(cm.layer_gemm_ms(n), max(W / gpu.bw, 2 * P * n / gpu.flops))
    t = cm.t_segment(3, 10, 500, buckets=2)
    manual = 3 * (max(W / gpu.bw, 2 * P * 10 / gpu.flops) + 500 * dims.kv_bytes_per_pos / gpu.bw + 60 * 0.01) + 0.05
    assert np.isclose(t, manual)


def test_hinge_knee_recovers_a_planted_knee():
    from thesis_amd.solutions.calibrate import N_GRID, hinge_knee

    n = np.array(N_GRID, dtype=np.float64)
    for knee, a, b in ((96.0, 0.5, 0.004), (32.0, 0.12, 0.01), (256.0, 2.0, 0.02)):
        t = a + b * np.maximum(n - knee, 0.0)
        kn, coef = hinge_knee(N_GRID, t)
        assert kn == knee and np.allclose(coef, [a, b])
    # a falling line has no knee with a non-negative slope
    with pytest.raises(ValueError):
        hinge_knee(N_GRID, 1.0 - 1e-3 * n)


def test_linear_fit_recovers_planted_coefficients():
    from thesis_amd.solutions.calibrate import ape_summary, fit_linear

    rng = np.random.default_rng(0)
    rows = [{"n": int(nn), "kv": int(kv), "ms": 0.3 + 0.002 * nn + 5e-6 * kv}
            for nn, kv in zip(rng.integers(1, 600, 40), rng.integers(100, 200000, 40))]
    heads = [{"n": nn, "ms": 0.25 + 0.001 * nn} for nn in (1, 8, 64, 256)]
    fit = fit_linear(rows, heads)
    assert np.allclose([fit["a"], fit["b"], fit["c"], fit["head_a"], fit["head_b"]],
                       [0.3, 0.002, 5e-6, 0.25, 0.001])
    val = [{"kind": "deep", "n": 100, "ms": 2.0, "m": 2.2}, {"kind": "shallow", "n": 8, "ms": 1.0, "m": 0.9}]
    s = ape_summary(val, ["m"])
    assert np.isclose(s["m_all"]["mape"], 0.1) and np.isclose(s["m_deep"]["max_ape"], 0.1)
    assert s["m_n64_256"]["n"] == 1 and "m_prefill" not in s


def test_calibration_record_loads_as_cost_models(tmp_path):
    from thesis_amd.common.model import PRESETS
    from thesis_amd.solutions.cost_model import (GPUParams, LinearCostModel, RooflineCostModel, load_cost_model,
                                                 save_json)

    cfg = PRESETS["llama3-8b"]
    gpu = GPUParams(bw=5.5e9, flops=1.6e12, t_op=0.003, n_op_layer=8, n_op_bucket=0, n_op_head=3, n_op_segment=1,
                    meta={"host": "x"}, flops_eff=9e11, knee_measured=120.0)
    p = tmp_path / "c.json"
    save_json(p, {"model": "llama3-8b", "gpu": gpu,
                  "linear": {"a": 0.09, "b": 1e-4, "c": 2e-8, "head_a": 0.2, "head_b": 1e-3}})
    cm = load_cost_model(p, cfg)
    assert isinstance(cm, RooflineCostModel) and cm.F == 9e11 and cm.knee() == 120.0
    assert load_cost_model(p, cfg, "roofline-peak").F == 1.6e12
    lin = load_cost_model(p, cfg, "linear")
    assert isinstance(lin, LinearCostModel) and np.isclose(lin.layer_gemm_ms(10), 0.09 + 1e-3)


def test_committed_mi355x_calibration_is_the_default_and_fits_its_measurements():
    import csv

    from thesis_amd.common.model import PRESETS
    from thesis_amd.solutions.cost_model import RooflineCostModel, calibration_path, default_cost_model

    cfg = PRESETS["llama3-8b"]
    cm, src = default_cost_model(cfg)
    assert isinstance(cm, RooflineCostModel) and "calibrated" in src
    # the measured single-layer times of the knee grid (128 cached positions per request)
    grid = cm.gpu.meta["knee_layer_grid"]
    for r in grid:
        pred = float(cm.t_segment(1, r["n"], 128 * r["n"])) - cm.segment_ops_ms()
        assert abs(pred - r["ms"]) / r["ms"] < 0.5, (r, pred)
    # the validation steps written beside it: the roofline model within 40 % of every measured step
    with open(calibration_path("llama3-8b").with_name("llama3-8b_mi355x_validation.csv")) as f:
        rows = list(csv.DictReader(f))
    assert len(rows) >= 90
    assert max(abs(float(r["roofline"]) - float(r["ms"])) / float(r["ms"]) for r in rows) < 0.4
    # the other committed shapes load as their presets' defaults too; their linear fits (the ASPIRE 3-parameter
    # model) stay within 25 % of every validation step
    for name in ("llama2-7b", "llama3.2-1b"):
        cm, src = default_cost_model(PRESETS[name])
        assert isinstance(cm, RooflineCostModel) and f"calibrated on MI355X ({name})" in src
        with open(calibration_path(name).with_name(f"{name}_mi355x_validation.csv")) as f:
            rows = list(csv.DictReader(f))
        assert len(rows) >= 90
        assert max(abs(float(r["linear"]) - float(r["ms"])) / float(r["ms"]) for r in rows) < 0.25


def test_config_parsing_old_and_new_formats(tmp_path):
    import json

    from thesis_amd.common.model import ModelConfig

    d = tmp_path / "old"
    d.mkdir()
    (d / "config.json").write_text(json.dumps({
        "vocab_size": 10, "hidden_size": 8, "num_hidden_layers": 2, "num_attention_heads": 2,
        "intermediate_size": 16, "rope_theta": 500000.0,
        "rope_scaling": {"rope_type": "llama3", "factor": 32.0}, "eos_token_id": [5, 6]}))
    c = ModelConfig.from_hf_dir(d)
    assert c.rope_theta == 500000.0 and c.rope_scaling["factor"] == 32.0 and c.eos_token_ids == (5, 6)
    d2 = tmp_path / "new"
    d2.mkdir()
    (d2 / "config.json").write_text(json.dumps({
        "vocab_size": 10, "hidden_size": 8, "num_hidden_layers": 2, "num_attention_heads": 2,
        "intermediate_size": 16, "rope_parameters": {"rope_type": "default", "rope_theta": 1234.0}}))
    c2 = ModelConfig.from_hf_dir(d2)
    assert c2.rope_theta == 1234.0 and c2.rope_scaling is None


def test_rope_tables_equal_the_oracle_tables():
    import oracle.model as om
    from thesis_amd.common.model import PRESETS, build_rope_cache

    c = PRESETS["llama3.2-1b"]
    cos, sin = build_rope_cache(c, 300, "cpu")
    oc = om.OracleConfig(c.vocab_size, c.dim, c.n_layers, c.n_heads, c.n_kv_heads, c.head_dim, c.intermediate_size,
                         rope_theta=c.rope_theta, rope_scaling=c.rope_scaling)
    ocos, osin = om.rope_tables(oc, 300)
    assert torch.equal(cos, ocos) and torch.equal(sin, osin)


def test_product_does_not_import_the_oracle():
    for p in (ROOT / "thesis_amd").rglob("*.py"):
        src = p.read_text()
        assert not re.search(r"^\s*(from|import)\s+oracle\b", src, re.M), p


def test_model_refuses_cpu():
    from thesis_amd import _lsk
    from thesis_amd.common.model import LayerSkipLlama, ModelConfig

    cfg = ModelConfig(vocab_size=64, dim=64, n_layers=1, n_heads=4, n_kv_heads=2, head_dim=16, intermediate_size=128)
    with pytest.raises(_lsk.LskError):
        LayerSkipLlama(cfg, None, [], None, None, "cpu", torch.float32, 64)


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 2 and "one GPU" in r.stderr


def test_rocprof_summary_counts_after_the_calibration_copy(tmp_path, capsys):
    from thesis_amd import prof_summary as ps

    hdr = ["Correlation_Id", "Dispatch_Id", "Agent_Id", "Queue_Id", "Process_Id", "Thread_Id", "Grid_Size",
           "Kernel_Id", "Kernel_Name", "Workgroup_Size", "LDS_Block_Size", "Scratch_Size", "VGPR_Count",
           "Accum_VGPR_Count", "SGPR_Count", "Counter_Name", "Counter_Value", "Start_Timestamp", "End_Timestamp"]

    def write(path, counter, rows):
        import csv

        with open(path, "w", newline="") as f:
            w = csv.writer(f)
            w.writerow(hdr)
            for d, (name, grid, val) in enumerate(rows, 1):
                w.writerow([d, d, "Agent 1", 1, 1, 1, grid, 1, name, 256, 0, 0, 0, 0, 0, counter, val, 0, 1])

    gemm = "void gemm_bf16_kernel<2, 2, 2>(unsigned short const*, long)"
    copy = "void copy_rows_kernel(unsigned char*, long const*)"
    big = 65536 * 256
    # before the marker: ignored; the marker copy of 1024 MiB reads 512 MiB on FETCH_SIZE (factor 2)
    write(tmp_path / "f.csv", "FETCH_SIZE", [(gemm, 448 * 256, 1.0), (copy, big, 512 * 1024.0),
                                             (gemm, 448 * 256, 100.0), (gemm, 448 * 256, 300.0)])
    write(tmp_path / "w.csv", "WRITE_SIZE", [(copy, big, 1024 * 1024.0), (gemm, 448 * 256, 8.0),
                                             (gemm, 448 * 256, 8.0)])
    ps.main(["pmc", str(tmp_path / "f.csv"), str(tmp_path / "w.csv"), "--calib-mib", "1024"])
    out = capsys.readouterr().out
    (tmp_path / "t.md").write_text(out)
    # fetch: mean 200 KiB x 2; write: 8 KiB x 1
    assert ps.read_traffic(tmp_path / "t.md", "gemm_w13") == 200 * 1024 * 2 + 8 * 1024
    assert ps.short_name(gemm) == "gemm_bf16_kernel<2, 2, 2>"
    assert ps.classify("gemm_bf16_kernel<2, 2, 3>", 192 * 256) == "gemm_qkv"
    assert ps.classify("gemm_bf16_kernel<2, 2, 3>", 128 * 256) == "gemm_o_w2"
    assert ps.classify("attn_bf16_kernel<128>") == "attention"
    # the fragment-major-activation flag is a bool template argument
    assert ps.classify("gemm_bf16_kernel<2, 2, 3, 4, true>", 192 * 256) == "gemm_qkv"
    assert ps.classify("gemm_bf16_kernel<4, 3, 2, 2, false>") == "gemm_w13"


def test_method_registry():
    from thesis_amd.common.methods import METHODS, MethodSpec, load_plugins, register

    assert load_plugins(["no_such_module_here"]) == ["thesis_amd.solutions"]
    assert {"autoregressive", "sync_layerskip", "eesd"} <= set(METHODS)
    with pytest.raises(ValueError):
        register(MethodSpec("eesd", "again", lambda g: None, lambda *a: None))
    spec = METHODS["sync_layerskip"]
    a = SimpleNamespace(exit_layer=8, gamma=4)
    assert spec.tag(a) == "-k8-g4" and spec.step_tokens(a) == 5 and spec.params(a) == {"exit_layer": 8, "gamma": 4}


def test_sample_tokens_semantics():
    from thesis_amd.common.engine import sample_tokens

    logits = torch.tensor([[0.0, 3.0, 3.0, 1.0], [5.0, 0.0, 0.0, 0.0]])
    assert sample_tokens(logits, 0.0, 0, 1.0).tolist() == [1, 0]            # greedy: first index on ties
    g = torch.Generator().manual_seed(0)
    draws = torch.stack([sample_tokens(logits, 1.0, 1, 1.0, g) for _ in range(50)])
    assert set(draws[:, 1].tolist()) == {0} and set(draws[:, 0].tolist()) <= {1, 2}   # top-1 keeps the maxima
    draws = torch.stack([sample_tokens(logits, 1.0, 0, 0.5, g) for _ in range(50)])
    assert set(draws[:, 0].tolist()) <= {1, 2}                              # nucleus 0.5 drops the tail


def test_decode_engine_driver_on_a_stub_model():
    """Cyclic replay bookkeeping of DecodeEngine.run (warm-up completions, refill, static pass) with a
    CPU stub: every step commits one token per active slot."""
    from thesis_amd.common.data import Prompt
    from thesis_amd.common.engine import DecodeEngine, RunConfig, StepRecord

    class Stub:
        device = torch.device("cpu")

        def allocate_cache(self, b, s):
            self.cache = SimpleNamespace(max_seq=s)

        def prefill(self, tokens, slot, capture_exits=False):
            return torch.nn.functional.one_hot(torch.tensor(len(tokens) % 7), 7).float(), None

    class Counting(DecodeEngine):
        def _iteration(self, measured):
            c = 0
            for i in self._active():
                s = self.slots[i]
                s.pos += 1
                c += self._commit(i, [s.pos % 7])
            self.records.append(StepRecord("ar", 1.0, len(self._active()), 0, 0, 0, measured))
            return c

    prompts = [Prompt(f"p{i}", list(range(3 + i))) for i in range(5)]
    eng = Counting(Stub(), 2, 16, 4, (), ignore_eos=True)
    res = eng.run(prompts, RunConfig(mode="static", keep_outputs=True))
    assert res["metrics"]["stop_reason"] == "pool_exhausted"
    assert sorted(c["pid"] for c in res["completions"]) == [f"p{i}" for i in range(5)]
    assert all(c["generated"] == 4 and c["finish_reason"] == "length" for c in res["completions"])
    assert res["metrics"]["measured_tokens"] == 5 * 3                    # first tokens come from prefill
    eng = Counting(Stub(), 2, 16, 4, (), ignore_eos=True)
    res = eng.run(prompts, RunConfig(mode="cyclic", warmup_samples=2, warmup_per_slot=1.0, converge=False,
                                     max_eval_samples=6, converge_min_samples=1, min_eval_per_slot=0.0))
    assert res["metrics"]["stop_reason"] == "max_eval_samples"
    assert res["metrics"]["evaluated_completions"] == 6
    assert sum(1 for c in res["completions"] if not c["measured"]) == 2


# ----------------------------------------------------------------------------- M2 / M3 policies (host)

def test_m3_budget_respects_the_knee():
    """c == 0 or (c + shallow tokens and c + deep tokens stay within knee * safety) (tests/test_eesd.py:357-363)."""
    from thesis_amd.common.model import PRESETS
    from thesis_amd.solutions.cost_model import synthetic_cost_model
    from thesis_amd.solutions.prefill import M3Planner

    cm = synthetic_cost_model(PRESETS["llama3.2-1b"])
    cm.gpu.knee_measured = 12.0
    for safety in (0.5, 0.9):
        p = M3Planner(cm, knee_safety=safety)
        bound = 12.0 * safety
        for n_sh in range(0, 14):
            for n_dp in range(0, 14):
                c = p.chunk_budget(n_sh, n_dp, 0)
                assert c == 0 or (c + n_sh <= bound and c + n_dp <= bound)
    # admission: the refusal reasons of solutions/prefill.py:46-57, in their order
    p = M3Planner(cm, max_wait=2, knee_safety=1.0)
    assert p.admission(100, 12, 12, 4, 500.0) == (False, "no_room_below_knee")
    assert p.admission(100, 2, 2, 4, 500.0) == (False, "exceeds_max_wait")      # 10-token pieces: 10 > 2 pieces
    ok, why = p.admission(8, 2, 2, 4, 500.0)
    assert why == ("piggyback" if ok else "not_cheaper_than_separate")
    assert ok == (p.extra_cost(8, 4, 2, 2, 500.0) < float(cm.t_prefill(8, 8)))


def test_exit_controller_probe_cadence_ema_and_switch():
    from thesis_amd.common.model import PRESETS
    from thesis_amd.solutions.cost_model import synthetic_cost_model
    from thesis_amd.solutions.exit_select import ExitController

    cm = synthetic_cost_model(PRESETS["llama3.2-1b"])
    ec = ExitController(cm, 4, [2, 6], probe_every=3, margin=0.05, omega=0.5)
    assert ec.cands == [2, 4, 6]
    wants = []
    for _ in range(6):
        wants.append(ec.probe_due())
        ec.deep_step_done()
    assert wants == [False, False, True, False, False, True]
    assert ec.propose(8, 800.0, True) is None                # no probe yet
    ec.absorb_probe([1, 4, 8], 8)
    assert ec.alpha == {2: 0.125, 4: 0.5, 6: 1.0}
    ec.absorb_probe([3, 4, 8], 8)
    assert ec.alpha[2] == 0.5 * 0.125 + 0.5 * 0.375            # EMA with omega = 0.5
    ec.absorb_probe([0, 0, 0], 0)                              # no correct-prefix position: ignored
    assert ec.n_probes == 2
    new = ec.propose(8, 800.0, True)
    rates = ec.last_rates
    best = max(rates, key=rates.get)
    assert new == (best if best != 4 and rates[best] > 1.05 * rates[4] else None)
    assert ec.propose(8, 800.0, False) is None             # a half-done prefill blocks switches
    cyc = ExitController(cm, 4, [2, 6], probe_every=1, force="cycle")
    cyc.deep_step_done()
    cyc.absorb_probe([1, 1, 1], 2)
    assert cyc.propose(8, 800.0, True) == 6 and cyc.timeline == [(0, 4), (1, 6)]


def test_decoded_cache_views_refuse_writes():
    """cache.k[i] / cache.v[i] (and k_all / v_all) of the bf16 cache are decoded copies of the kernels' storage;
    a reference-style write into them (solutions/packed.py:180-181) raises instead of being lost, reads and
    out-of-place results stay ordinary tensors, and the fp32 K cache (stored in the reference layout) stays a
    writable view of the storage."""
    from thesis_amd import _lsk
    from thesis_amd.common.model import KVCache, ModelConfig

    cfg = ModelConfig(vocab_size=64, dim=64, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=32, intermediate_size=128)
    c = KVCache(cfg, 3, 64, torch.bfloat16, "cpu")
    k = torch.randn(2, 2, 32).to(torch.bfloat16)
    rows, pos = torch.tensor([0, 2]), torch.tensor([5, 9])
    for view in (c.k[1], c.v[0], c.k_all, c.v_all[1]):
        with pytest.raises(_lsk.LskError, match="decoded KV-cache view"):
            view[rows, :, pos] = k
        with pytest.raises(_lsk.LskError):
            view[0].zero_()
        with pytest.raises(_lsk.LskError):
            view.index_put_((rows[:1],), torch.zeros_like(view[rows[:1]]))
        assert type(view.clone()) is torch.Tensor and float((view + 1).sum()) == view.numel()
    assert (c.kf_all == 0).all() and (c.vb_all == 0).all()
    c32 = KVCache(cfg, 3, 64, torch.float32, "cpu")
    c32.k[1][rows, :, pos] = k.float()
    assert torch.equal(c32.kstore[1][rows, :, pos], k.float())
    with pytest.raises(_lsk.LskError):
        c32.v[1][rows, :, pos] = k.float()


def test_measure_window_convergence_and_caps():
    """Warm-up completions are not measured; the run stops once `window` consecutive completions keep the
    throughput within `threshold` of the anchor (a completion outside re-anchors), or at max_eval
    (solutions/engine.py:594-606, common/engine.py:198-216)."""
    from thesis_amd.common.driver import MeasureWindow

    started = []
    w = MeasureWindow(warmup=2, min_eval=3, max_eval=50, threshold=0.01, window=2, on_start=lambda: started.append(1))
    rates = iter([100.0, 150.0, 150.5, 150.2])
    reasons = [w.completed(lambda: next(rates)) for _ in range(2)]         # warm-up: no rate read
    assert reasons == [None, None] and w.measuring and started == [1]
    reasons = [w.completed(lambda: next(rates)) for _ in range(6)]
    # measured 1-2: below min_eval (no rate read); 3 anchors at 100; 4 (150) re-anchors; 5, 6 stable -> converged
    assert reasons == [None, None, None, None, None, "converged"]
    capped = MeasureWindow(warmup=0, max_eval=3, converge=False)
    assert [capped.completed(lambda: 1.0) for _ in range(3)] == [None, None, "max_eval_samples"]


def test_open_loop_driver_on_a_stub_engine():
    """run_arrivals: requests arrive by a seeded Poisson clock, queue FIFO for free slots, idle waits sleep until
    the next arrival; every request is admitted once, in arrival order, and the run ends after n_total
    releases."""
    import time as _time

    from thesis_amd.common.driver import PoissonArrivals, run_arrivals

    class Stub:
        n_slots = 2

        def __init__(self):
            self.slots, self.order, self.released = [None, None], [], 0

        def advance(self):
            done = [i for i, r in enumerate(self.slots) if r is not None]
            return done[:1]                                   # one request finishes per step

        def release(self, slot):
            self.slots[slot] = None
            self.released += 1

        def busy(self):
            return any(r is not None for r in self.slots)

    eng = Stub()

    def admit(slot, req):
        eng.slots[slot] = req
        eng.order.append(req)
        return False

    arr = PoissonArrivals(200.0, seed=3, t0=_time.perf_counter())
    left = run_arrivals(eng, lambda: [i for i, r in enumerate(eng.slots) if r is None],
                        lambda i, t: (i, t), admit, arr, 6, lambda: None)
    assert eng.released == 6 and [r[0] for r in eng.order[:6]] == list(range(6))
    assert all(a[1] <= b[1] for a, b in zip(eng.order, eng.order[1:])) and left >= 0


def test_graph_capture_runs_with_the_cyclic_collector_disabled(monkeypatch):
    """ShallowGraphs.run captures a step with Python's cyclic garbage collector off (a collected object holding a
    pinned buffer or an event can issue a stream operation from its destructor, which a capturing stream refuses)
    and restores the collector afterwards, also when the step raises; a collector the caller had disabled stays
    disabled.  torch.cuda.graph / CUDAGraph are replaced by recording stand-ins, so this runs on the CPU."""
    import contextlib
    import gc

    from thesis_amd.solutions import step_graph

    events = []

    class FakeGraph:
        def replay(self):
            events.append("replay")

    @contextlib.contextmanager
    def fake_capture(g):
        events.append("capture-begin")
        yield
        events.append("capture-end")

    monkeypatch.setattr(torch.cuda, "CUDAGraph", FakeGraph)
    monkeypatch.setattr(torch.cuda, "graph", fake_capture)
    sg = step_graph.ShallowGraphs("cpu")

    def entry():
        return SimpleNamespace(graph=None, epoch=-1, seen=0, out=None)

    seen_gc = []

    def step():
        seen_gc.append(gc.isenabled())
        return "out"

    was = gc.isenabled()
    try:
        gc.enable()
        e = entry()
        assert sg.run(e, lambda: 0, step) == "eager" and seen_gc == [True]       # first sighting: eager
        assert sg.run(e, lambda: 0, step) == "capture" and seen_gc == [True, False]
        assert gc.isenabled() and events == ["capture-begin", "capture-end", "replay"]
        assert sg.run(e, lambda: 0, step) == "replay" and len(seen_gc) == 2

        def boom():
            seen_gc.append(gc.isenabled())
            raise RuntimeError("step failed")

        e2 = entry()
        e2.seen = 1
        with pytest.raises(RuntimeError, match="step failed"):
            sg.run(e2, lambda: 0, boom)
        assert seen_gc[-1] is False and gc.isenabled() and e2.graph is None

        gc.disable()
        e3 = entry()
        e3.seen = 1
        sg.run(e3, lambda: 0, step)
        assert seen_gc[-1] is False and not gc.isenabled()
    finally:
        if was:
            gc.enable()
        else:
            gc.disable()


def test_bf16_runner_refuses_a_wqkv_without_the_rope_paired_packing():
    """The bf16 layer runner's fused qkv + RoPE launch reads wqkv packed RoPE-paired for the model's heads; a plain
    packing (or another head split) is refused before any device work, instead of permuting q / k rows."""
    from thesis_amd import _lsk

    w = torch.zeros(3 * 64, 64, dtype=torch.bfloat16)
    for bad in (w, SimpleNamespace(qkv_heads=None), SimpleNamespace(qkv_heads=(2, 1, 32))):
        lw = SimpleNamespace(wqkv=bad)
        with pytest.raises(_lsk.LskError, match="RoPE|qkv_heads"):
            _lsk.NativeModel(torch.bfloat16, 1, 64, 1, 1, 64, 128, 16, 1e-5, [lw], [], [], None, None)


class _FakeSlots:
    """SlotOps over a scripted sequence of steps: step i finishes the slots listed in finishes[i]."""

    def __init__(self, n_slots, finishes):
        self.n_slots, self.finishes, self.i = n_slots, list(finishes), 0
        self.released, self.admitted = [], []

    def admit(self, slot, index, prompt):
        self.admitted.append((slot, index))
        return False

    def advance(self):
        out = self.finishes[self.i] if self.i < len(self.finishes) else []
        self.i += 1
        return list(out)

    def release(self, slot):
        self.released.append(slot)

    def busy(self):
        return self.i < len(self.finishes)


def test_measure_window_rules_of_the_two_engines():
    """DecodeEngine rule (common/engine.py:224-247): a request finishing in the step where warm-up ends is not
    evaluated, and after the stop reason the step's other completions are left unrecorded.  EESD rule
    (solutions/engine.py:582-604): completions count by the state when they are accounted, and the step's other
    completions are still released and counted.  A throughput of None (no measured time) skips the convergence
    test."""
    from thesis_amd.common.driver import MeasureWindow, run_pool

    # warm-up of 2; the first step finishes 3 requests, the second 2, the third 3
    script = [[0, 1, 2], [3, 0], [1, 2, 3]]
    w = MeasureWindow(warmup=2, max_eval=3, converge=False, per_step=True)
    ops = _FakeSlots(4, script)
    stop = run_pool(ops, list(range(8)), True, w, lambda: 1.0, drain_after_stop=False)
    # step 1: two warm-up completions, the third finishes in the warm-up step (not evaluated); step 2: 2 evaluated;
    # step 3: the 3rd evaluated completion stops the run and the remaining two are not released
    assert (w.warm_done, w.evaluated, stop) == (2, 3, "max_eval_samples")
    assert ops.released == [0, 1, 2, 3, 0, 1]
    w = MeasureWindow(warmup=2, max_eval=3, converge=False)
    ops = _FakeSlots(4, script)
    stop = run_pool(ops, list(range(8)), True, w, lambda: 1.0)
    # step 1: the third completion is already evaluated; step 2 reaches 3 with its last completion
    assert (w.warm_done, w.evaluated, stop) == (2, 3, "max_eval_samples")
    assert ops.released == [0, 1, 2, 3, 0]
    # no measured time: the convergence test waits (no anchor); then a constant rate converges after `window`
    rates = iter([None, None, 5.0, 5.0, 5.0, 5.0])
    w = MeasureWindow(warmup=0, window=3)
    got = [w.completed(lambda: next(rates)) for _ in range(6)]
    assert got == [None] * 5 + ["converged"]


def test_fused_qkv_token_counts_reach_every_wide_configuration():
    """The token counts of the fused qkv GPU test reach both wide-tier tile widths (32- and 64-row tiles, ns 2 / 4)
    with one to three token groups per wave (every pair the tier instantiates for qkv) over the GQA shape and the
    64-dim MHA shape together, by the library's own configuration rule (lsk_gemm_wide_config)."""
    from thesis_amd import _lsk
    from test_kernels_gpu import FUSED_QKV_MS

    _lsk.load()
    for heads, need in (((32, 8, 128), {(2, 1), (4, 1), (4, 2), (4, 3)}),
                        ((8, 8, 64), {(2, 2), (2, 3), (4, 2), (4, 3)})):
        N = (heads[0] + 2 * heads[1]) * heads[2]
        got = {(c[0], c[3]) for c in (_lsk.gemm_wide_config(_lsk.EPI_QKV_ROPE, M, N, 1024) for M in FUSED_QKV_MS)
               if c[0]}
        assert need <= got, (heads, sorted(got))
        assert _lsk.gemm_wide_config(_lsk.EPI_QKV_ROPE, 64, N, 1024)[0] == 0       # <= 64 rows: decode tier


class _ToyTokenizer:
    """decode(ids): one character per id; ids in `nl` decode to a newline."""

    def __init__(self, nl):
        self.nl = set(nl)

    def decode(self, ids, skip_special_tokens=False):
        return "".join("\n" if i in self.nl else chr(65 + i % 26) for i in ids)


def test_stop_checker_cuts_after_the_token_completing_the_first_stop():
    """The cut keeps the token that completes the first stop string (tests/test_engine.py:98-105 of the reference):
    a stop spanning two tokens, one completed inside a multi-token commit, and a stop made of the commit alone."""
    from thesis_amd.common.data import StopChecker

    sc = StopChecker(_ToyTokenizer({9}), ("\nB",))              # "\n" (id 9) followed by id 1 ("B")
    out = [3, 4, 9, 5, 9, 1, 7, 9, 1]
    assert sc(out[:4], 4) is None
    assert sc(out[:6], 2) == 6
    assert sc(out[:5], 1) is None
    assert sc(out[:7], 7) == 6
    assert StopChecker(_ToyTokenizer({9}), ("\n",))([1, 2, 9, 9], 3) == 3
    assert not StopChecker(_ToyTokenizer(set()), ())


def test_empty_inputs_return_before_any_launch():
    """Every launching entry point accepts an empty input (no tokens, rows, verifiers or work items) and returns
    0 without launching or touching memory: this container has no GPU, so a launch would fail, and the pointers
    passed are not valid addresses."""
    lib = _lsk().load()
    P = 16                       # a non-null pointer that must never be dereferenced
    assert lib.lsk_rmsnorm(1, P, P, P, 0, 64, 1e-5, 64, 64, None) == 0
    assert lib.lsk_rope_append(1, P, P, P, P, P, P, 64, P, P, 0, 4, 2, 64, 2, 64, None) == 0
    assert lib.lsk_kv_append(1, P, P, P, P, P, P, 0, 2, 64, 2, 64, None) == 0
    assert lib.lsk_rope_append_partial(1, P, 2, P, P, P, P, P, 64, P, P, 0, 4, 2, 64, 2, 64, None) == 0
    assert lib.lsk_ragged_attn(1, P, P, P, P, P, 0, P, 0, 0, P, 1, 1, 16, P, 4, 2, 64, 64, 0.125, P, 0, None) == 0
    assert lib.lsk_gemm(1, P, 64, P, 64, P, 64, None, 0, 0, 64, 64, 0, 0, None) == 0
    assert lib.lsk_gemm(0, P, 64, P, 64, P, 64, None, 0, 0, 64, 64, 0, 0, None) == 0
    assert lib.lsk_gemm_partial(P, 64, P, 64, P, 0, 64, 64, 2, None) == 0
    assert lib.lsk_gemm_partial_frag(P, P, P, 0, 64, 64, 2, None) == 0
    assert lib.lsk_gemm_silu_frag(P, P, P, 1, 0, 64, 64, None) == 0
    assert lib.lsk_head_argmax(1, P, 64, P, 64, 0, 128, 64, None, 0, P, None, P, 0, None) == 0
    assert lib.lsk_add_rmsnorm(1, P, 64, P, 2, P, 1e-5, P, 64, P, 64, 0, 64, None) == 0
    assert lib.lsk_embed(P, 100, 128, P, 8, P, P, P, 0, None) == 0
    assert lib.lsk_copy_rows(P, P, 4, P, P, 4, 128, 0, None) == 0
    assert lib.lsk_argmax(1, P, 128, 0, 128, P, None, None) == 0
    assert lib.lsk_greedy_accept(P, P, 8, P, P, P, None, 0, P, P, P, None) == 0
    assert lib.lsk_kv_rollback(P, P, P, 0, None) == 0
    assert lib.lsk_shift_segment_positions(P, 4, 1, 1, 0, 1, 4, P, P, P, 0, None) == 0
    assert lib.lsk_gemm_qkv_rope(P, P, 0, 32, 8, 128, 4096, P, P, P, P, P, 64, P, P, 2, 64, None) == 0
