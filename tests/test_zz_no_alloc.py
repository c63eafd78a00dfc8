"""The allocation-free attention entry point (lsk_ragged_attn_static) against lsk_ragged_attn.

lsk_ragged_attn_static keeps the split partials in a static per-GPU device array instead of a caller workspace.
Called through the C ABI here, twice in a row on plans that use split partials (the second smaller, so it
reuses the array with the first call's contents left in it), it must give bitwise the outputs of lsk_ragged_attn
with a workspace; plans whose partials exceed the array are rejected on the host before any launch.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

BF16 = torch.bfloat16


def _lsk():
    from thesis_amd import _lsk

    _lsk.load()
    return _lsk


def _case(lsk, cuda, seed, n_req, ctx_hi, split):
    """n_req requests with contexts up to ctx_hi, 1-9 query rows each, on an 8-KV-head cache (D = 128)."""
    rng = np.random.default_rng(seed)
    Hq, Hkv, D = 32, 8, 128
    ctx = rng.integers(64, ctx_hi, size=n_req)
    T = rng.integers(1, 10, size=n_req)
    S = int(math.ceil((ctx + T).max() / 64) * 64)
    offs = np.concatenate([[0], np.cumsum(T)[:-1]])
    blocks = np.stack([offs, ctx, T, np.arange(n_req)], axis=1).astype(np.int32)
    g = torch.Generator(device=cuda).manual_seed(seed)
    kc = torch.empty(n_req, Hkv, S // 32, D // 16, 64, 8, dtype=BF16, device=cuda).normal_(generator=g)
    vc = torch.empty(n_req, Hkv, S // 32, D, 32, dtype=BF16, device=cuda).normal_(generator=g)
    q = torch.empty(int(T.sum()), Hq, D, dtype=BF16, device=cuda).normal_(generator=g)
    n_slots = lsk.cu_count(cuda)
    cap = lsk.attn_rows_cap(blocks, Hq // Hkv, split, Hkv, D, n_slots)
    works, groups, n_parts = lsk.attn_plan(blocks, Hq // Hkv, split, cap)
    recs, n_rounds = lsk.attn_schedule(works, Hkv, n_slots)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(cuda)  # noqa: E731
    return dict(q=q, kc=kc, vc=vc, blk=dev(blocks), wk=dev(works), nw=len(works), gr=dev(groups), ng=len(groups),
                n_parts=n_parts, recs=dev(recs), n_rounds=n_rounds, n_slots=n_slots, cap=cap, Hq=Hq, Hkv=Hkv, D=D,
                S=S, N=int(T.sum()))


def _with_workspace(lsk, cuda, c):
    out = torch.empty(c["N"], c["Hq"] * c["D"], dtype=BF16, device=cuda)
    ws = torch.empty(max(lsk.attn_workspace_bytes(c["n_parts"], c["Hkv"], c["D"]), 1), dtype=torch.uint8, device=cuda)
    lsk.ragged_attn(c["q"], c["kc"], c["vc"], c["blk"], c["wk"], c["nw"], c["gr"], c["ng"], c["n_parts"], out,
                    c["Hq"], 1.0 / math.sqrt(c["D"]), ws, c["recs"], c["n_rounds"], c["n_slots"], c["cap"])
    return out


def _static(lsk, cuda, c):
    """Direct C-ABI call of lsk_ragged_attn_static (no workspace argument) on torch's current stream."""
    out = torch.full((c["N"], c["Hq"] * c["D"]), float("nan"), dtype=BF16, device=cuda)
    p = lambda t: t.data_ptr()  # noqa: E731
    rc = lsk.load().lsk_ragged_attn_static(
        lsk.DTYPE_BF16, p(c["q"]), p(c["kc"]), p(c["vc"]), p(c["blk"]), p(c["wk"]), c["nw"], p(c["gr"]), c["ng"],
        c["n_parts"], p(c["recs"]), c["n_rounds"], c["n_slots"], c["cap"], p(out), c["Hq"], c["Hkv"], c["D"], c["S"],
        1.0 / math.sqrt(c["D"]), torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lsk.load().lsk_last_error().decode()
    return out


@pytest.mark.gpu
def test_static_scratch_attention_equals_the_workspace_entry_point(cuda):
    lsk = _lsk()
    first = _case(lsk, cuda, seed=1, n_req=40, ctx_hi=5000, split=1024)
    second = _case(lsk, cuda, seed=2, n_req=6, ctx_hi=2500, split=1024)
    assert first["n_parts"] > second["n_parts"] > 0                       # both use the scratch array
    got1 = _static(lsk, cuda, first)
    got2 = _static(lsk, cuda, second)                                     # reuses the array after call one
    ref1 = _with_workspace(lsk, cuda, first)
    ref2 = _with_workspace(lsk, cuda, second)
    torch.cuda.synchronize()
    assert torch.equal(got1, ref1)
    assert torch.equal(got2, ref2)
    assert not torch.isnan(got2.float()).any()


def test_static_scratch_attention_rejects_plans_beyond_the_array():
    """Checked on the host before any launch (also without a GPU): more partial slots than the static array holds
    -> LSK_EWORKSPACE with a message naming the limit."""
    from thesis_amd import _lsk

    lib = _lsk.load()
    cap = int(lib.lsk_ragged_attn_static_scratch_bytes())
    assert cap == 32 << 20
    per_part = _lsk.attn_workspace_bytes(1, 8, 128)
    too_many = cap // per_part + 1
    assert _lsk.attn_workspace_bytes(too_many, 8, 128) > cap
    rc = lib.lsk_ragged_attn_static(_lsk.DTYPE_BF16, 1, 1, 1, 1, 1, 1, 1, 1, too_many, 1, 1, 1, 48, 1, 32, 8, 128,
                                    128, 0.1, None)
    assert rc == -4, rc                                                   # LSK_EWORKSPACE
    assert b"static" in lib.lsk_last_error()
