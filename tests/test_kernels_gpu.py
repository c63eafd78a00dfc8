"""Kernel-level parity of liblsk against the CPU oracle / fp64 references (GPU).

Bars: bit-exact for data movement and index work (KV append, RoPE, embed, row copies, argmax,
acceptance); tolerance for reductions (GEMM, RMSNorm, attention), written in each test.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle.model import brute_attention, rms_norm as o_rms_norm, rope as o_rope

pytestmark = pytest.mark.gpu

BF16, F32 = torch.bfloat16, torch.float32


def _lsk():
    from thesis_amd import _lsk

    _lsk.load()
    return _lsk


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _kstore(lsk, k):
    """K cache storage the kernels read: fragment-major for bf16, row-major for fp32."""
    return lsk.k_to_frag(k) if k.dtype == BF16 else k


def _kview(lsk, kstore):
    return lsk.k_from_frag(kstore) if kstore.dtype == BF16 else kstore


# ----------------------------------------------------------------------------- GEMM

@pytest.mark.parametrize("M,N,K", [(1, 64, 64), (5, 128, 256), (16, 64, 96), (17, 256, 512), (33, 128, 4160),
                                   (64, 4096, 256), (65, 256, 512), (100, 320, 1024), (128, 1024, 256),
                                   (129, 128, 512), (288, 512, 2048)])
def test_gemm_bf16_none_matches_fp32_reference(cuda, M, N, K):
    lsk = _lsk()
    g = _gen(M * 7 + N)
    a = torch.randn(M, K, generator=g).to(BF16)
    w = torch.randn(N, K, generator=g).to(BF16)
    ref = a.float() @ w.float().t()                      # exact products, fp32 accumulation
    got = lsk.gemm(a.to(cuda), lsk.PackedWeight(w.to(cuda))).cpu().float()
    # bf16 output rounding (2^-8 relative) + fp32 accumulation-order error
    tol = 2.0 ** -8 * ref.abs() + 1e-3 * math.sqrt(K)
    assert ((got - ref).abs() <= tol).all(), (got - ref).abs().max()


@pytest.mark.parametrize("K,N", [(1024, 384), (4096, 256)])
def test_gemm_bf16_is_batch_invariant(cuda, K, N):
    """Every row's result is bitwise independent of M and of which rows share a tile (16- to 128-token tiles,
    one or several token tiles, the wide-M tier above 64 / 128 rows, every epilogue)."""
    lsk = _lsk()
    g = _gen(3)
    M = 300
    a = torch.randn(M, K, generator=g).to(BF16).to(cuda)
    w = lsk.PackedWeight(torch.randn(N, K, generator=g).to(BF16).to(cuda))
    w13 = lsk.PackedWeight(torch.randn(2 * N, K, generator=g).to(BF16).to(cuda))
    r = torch.randn(M, N, generator=g).to(BF16).to(cuda)
    full = lsk.gemm(a, w)
    full_r = lsk.gemm(a, w, residual=r, epilogue=lsk.EPI_RESIDUAL)
    full_s = lsk.gemm(a, w13, epilogue=lsk.EPI_SILU_MUL)
    ns, ks = lsk.gemm_plan(N, K)
    full_p = lsk.gemm_partial(a, w, ks)
    for lo, hi in [(0, 1), (7, 8), (3, 19), (150, 200), (0, 33), (40, 104), (10, 130), (0, 65), (20, 149),
                   (0, 300)]:
        sub = a[lo:hi].contiguous()
        assert torch.equal(lsk.gemm(sub, w), full[lo:hi]), (lo, hi)
        assert torch.equal(lsk.gemm(sub, w, residual=r[lo:hi].contiguous(), epilogue=lsk.EPI_RESIDUAL),
                           full_r[lo:hi]), (lo, hi)
        assert torch.equal(lsk.gemm(sub, w13, epilogue=lsk.EPI_SILU_MUL), full_s[lo:hi]), (lo, hi)
        assert torch.equal(lsk.gemm_partial(sub, w, ks), full_p[:, lo:hi]), (lo, hi)
    # the wide tier against fp32 math (its own check, independent of the decode kernel)
    ref = (a.float() @ w.unpack().float().t()).to(BF16)
    assert ((full.float() - ref.float()).abs() <= 2.0 ** -7 * ref.float().abs() + 2e-2).all()


@pytest.mark.parametrize("big", [0, 1])
def test_gemm_bf16_epilogues_match_reference_rounding(cuda, big):
    """RESIDUAL: rnd(R + rnd(acc)); SILU_MUL: rnd(rnd(silu(rnd(g))) * rnd(u))  (solutions/packed.py:182-185)."""
    lsk = _lsk()
    g = _gen(11)
    M, K, F_ = 37 + 64 * big, 512, 256
    a = torch.randn(M, K, generator=g).to(BF16)
    w13 = (torch.randn(2 * F_, K, generator=g) * 0.05).to(BF16)
    r = torch.randn(M, 2 * F_, generator=g).to(BF16)
    acc = (a.float() @ w13.float().t())
    # residual: compare with the same formula on the CPU from the fp32 accumulation
    w13p = lsk.PackedWeight(w13.to(cuda))
    got_r = lsk.gemm(a.to(cuda), w13p, residual=r.to(cuda), epilogue=lsk.EPI_RESIDUAL).cpu()
    ref_r = (r.float() + acc.to(BF16).float()).to(BF16)
    close = (got_r.float() - ref_r.float()).abs() <= 2.0 ** -7 * ref_r.float().abs() + 1e-2
    assert close.all()
    got_s = lsk.gemm(a.to(cuda), w13p, epilogue=lsk.EPI_SILU_MUL).cpu()
    gg, uu = acc.to(BF16).chunk(2, dim=-1)
    ref_s = F.silu(gg) * uu                               # torch bf16 ops: the reference's rounding points
    assert ((got_s.float() - ref_s.float()).abs() <= 2.0 ** -6 * ref_s.float().abs() + 2e-3).all()


@pytest.mark.parametrize("N,K,ld", [(16, 32, 32), (48, 96, 128), (6144, 4096, 4096)])
def test_pack_weight_layout_and_round_trip(cuda, N, K, ld):
    """Packed storage follows the documented fragment order (computed here in numpy) and unpacks bit-exact."""
    lsk = _lsk()
    g = _gen(N + K)
    full = torch.randn(N, ld, generator=g).to(BF16)
    w = full[:, :K]
    wp = lsk.PackedWeight(w.to(cuda))
    # fragment (g, j) = rows 16g.., k 32j..; lane l holds row 16g + l % 16, k 32j + 8 (l // 16) .. +7
    gi, j, l, e = np.meshgrid(np.arange(N // 16), np.arange(K // 32), np.arange(64), np.arange(8), indexing="ij")
    rows = 16 * gi + l % 16
    cols = 32 * j + 8 * (l // 16) + e
    want = w.view(torch.int16).numpy()[rows.reshape(-1), cols.reshape(-1)]
    assert np.array_equal(wp.data.cpu().view(torch.int16).numpy(), want)
    assert torch.equal(wp.unpack().cpu(), w)


def test_bf16_gemm_rejects_unpacked_weights(cuda):
    lsk = _lsk()
    a = torch.zeros(4, 64, dtype=BF16, device=cuda)
    with pytest.raises(lsk.LskError):
        lsk.gemm(a, torch.zeros(64, 64, dtype=BF16, device=cuda))


@pytest.mark.parametrize("M,N,K", [(1, 8, 16), (7, 64, 64), (33, 100, 130)])
def test_gemm_f32(cuda, M, N, K):
    lsk = _lsk()
    g = _gen(5)
    a, w = torch.randn(M, K, generator=g), torch.randn(N, K, generator=g)
    got = lsk.gemm(a.to(cuda), w.to(cuda)).cpu()
    assert torch.allclose(got, a.double().mm(w.double().t()).float(), rtol=1e-5, atol=1e-5)
    r = torch.randn(M, N, generator=g)
    got = lsk.gemm(a.to(cuda), w.to(cuda), residual=r.to(cuda), epilogue=lsk.EPI_RESIDUAL).cpu()
    assert torch.allclose(got, r + a @ w.t(), rtol=1e-5, atol=1e-5)
    w13 = torch.randn(2 * N, K, generator=g)
    got = lsk.gemm(a.to(cuda), w13.to(cuda), epilogue=lsk.EPI_SILU_MUL).cpu()
    gg, uu = (a @ w13.t()).chunk(2, dim=-1)
    assert torch.allclose(got, F.silu(gg) * uu, rtol=1e-4, atol=1e-5)


# ----------------------------------------------------------------------------- RMSNorm

@pytest.mark.parametrize("dtype", [BF16, F32])
def test_rmsnorm(cuda, dtype):
    lsk = _lsk()
    g = _gen(1)
    x = (torch.randn(19, 4096, generator=g) * 3).to(dtype)
    w = (1 + 0.1 * torch.randn(4096, generator=g)).to(dtype)
    got = lsk.rmsnorm(x.to(cuda), w.to(cuda), 1e-5).cpu()
    ref = o_rms_norm(x, w, 1e-5)
    if dtype == F32:
        assert torch.allclose(got, ref, rtol=2e-6, atol=1e-6)
    else:
        # the mean's summation order differs; after the bf16 cast almost every element is identical
        # and the rest differ by one bf16 ulp
        diff = (got.float() - ref.float()).abs()
        assert (diff <= 2.0 ** -7 * ref.float().abs() + 1e-6).all()
        assert (got == ref).float().mean() > 0.98


# ----------------------------------------------------------------------------- RoPE + append

@pytest.mark.parametrize("dtype,D", [(BF16, 128), (BF16, 64), (F32, 16)])
def test_rope_append_is_bit_exact(cuda, dtype, D):
    """q_out and the appended K are bitwise the oracle's rope(); V is copied bitwise; nothing else in
    the cache changes (solutions/packed.py:176-181)."""
    lsk = _lsk()
    from oracle.model import OracleConfig, rope_tables

    g = _gen(D)
    Hq, Hkv, B, S, N = 8, 2, 3, 256, 11
    cfg = OracleConfig(64, 64, 1, Hq, Hkv, D, 64, rope_theta=500000.0)
    cos, sin = rope_tables(cfg, S)
    qkv = torch.randn(N, (Hq + 2 * Hkv) * D, generator=g).to(dtype)
    rows = torch.randint(0, B, (N,), generator=g)
    pos = torch.randperm(S, generator=g)[:N]             # distinct (row, pos) slots
    kc = torch.zeros(B, Hkv, S, D, dtype=dtype)
    vc = torch.zeros_like(kc)
    kd = _kstore(lsk, kc).to(cuda)                                          # fragment-major for bf16
    vd = torch.zeros(B, Hkv, S // 32, D, 32, dtype=dtype, device=cuda)      # blocked-transposed V storage
    q_out = torch.empty(N, Hq, D, dtype=dtype, device=cuda)
    lsk.rope_append(qkv.to(cuda), q_out, kd, vd, cos.to(cuda), sin.to(cuda),
                    rows.to(torch.int32).to(cuda), pos.to(torch.int32).to(cuda), Hq, Hkv, D)
    vd = lsk.v_from_blocked(vd)
    c = cos[pos].to(dtype).unsqueeze(1)
    s = sin[pos].to(dtype).unsqueeze(1)
    q_ref = o_rope(qkv[:, :Hq * D].view(N, Hq, D), c, s)
    k_ref = o_rope(qkv[:, Hq * D:(Hq + Hkv) * D].view(N, Hkv, D), c, s)
    v_ref = qkv[:, (Hq + Hkv) * D:].view(N, Hkv, D)
    assert torch.equal(q_out.cpu(), q_ref)
    kc[rows, :, pos] = k_ref
    vc[rows, :, pos] = v_ref
    assert torch.equal(_kview(lsk, kd.cpu()), kc)
    assert torch.equal(vd.cpu(), vc)


def test_kv_append_is_bit_exact(cuda):
    lsk = _lsk()
    g = _gen(2)
    B, Hkv, S, D, N = 4, 8, 128, 128, 9
    k = torch.randn(N, Hkv, D, generator=g).to(BF16)
    v = torch.randn(N, Hkv, D, generator=g).to(BF16)
    rows = torch.randint(0, B, (N,), generator=g)
    pos = torch.randperm(S, generator=g)[:N]
    kc = torch.randn(B, Hkv, S, D, generator=g).to(BF16)
    vc = torch.randn(B, Hkv, S, D, generator=g).to(BF16)
    kd, vd = lsk.k_to_frag(kc).to(cuda), lsk.v_to_blocked(vc).to(cuda)
    lsk.kv_append(k.to(cuda), v.to(cuda), kd, vd, rows.to(torch.int32).to(cuda), pos.to(torch.int32).to(cuda))
    kc[rows, :, pos] = k
    vc[rows, :, pos] = v
    assert torch.equal(lsk.k_from_frag(kd.cpu()), kc) and torch.equal(lsk.v_from_blocked(vd).cpu(), vc)


# ----------------------------------------------------------------------------- attention

def _attn_case(seed, dtype, B, Hq, Hkv, D, S, blocks):
    """blocks: list of (row, pos0, T); returns q, caches, host block table and reference output."""
    g = _gen(seed)
    N = sum(T for _, _, T in blocks)
    q = torch.randn(N, Hq, D, generator=g).to(dtype)
    kc = torch.randn(B, Hkv, S, D, generator=g).to(dtype)
    vc = torch.randn(B, Hkv, S, D, generator=g).to(dtype)
    rows, pos, tab, off = [], [], [], 0
    for (r, p0, T) in blocks:
        tab.append((off, p0, T, r))
        rows += [r] * T
        pos += list(range(p0, p0 + T))
        off += T
    ref = brute_attention(q, kc, vc, rows, pos, Hq // Hkv)
    return q, kc, vc, np.array(tab, dtype=np.int32), ref


def _run_attn(lsk, cuda, q, kc, vc, tab, split, rows_cap=None):
    """rows_cap None: the launch policy's choice (lsk_attn_rows_cap)."""
    Hq, D = q.shape[1], q.shape[2]
    Hkv = kc.shape[1]
    n_slots = lsk.cu_count(cuda)
    if rows_cap is None:
        rows_cap = lsk.attn_rows_cap(tab, Hq // Hkv, split, Hkv, D, n_slots)
    works, groups, n_parts = lsk.attn_plan(tab, Hq // Hkv, split, rows_cap)
    out = torch.empty(q.shape[0], Hq * D, dtype=q.dtype, device=cuda)
    ws = torch.empty(max(lsk.attn_workspace_bytes(n_parts, Hkv, D), 1), dtype=torch.uint8, device=cuda)
    gdev = torch.from_numpy(groups).to(cuda) if len(groups) else None
    recs, n_rounds = lsk.attn_schedule(works, Hkv, n_slots)
    lsk.ragged_attn(q.to(cuda), _kstore(lsk, kc).to(cuda), lsk.v_to_blocked(vc).to(cuda), torch.from_numpy(tab).to(cuda),
                    torch.from_numpy(works).to(cuda), len(works), gdev, len(groups), n_parts, out, Hq,
                    1.0 / math.sqrt(D), ws, torch.from_numpy(recs).to(cuda), n_rounds, n_slots, rows_cap)
    return out.cpu()


ATTN_TEST_SPLIT = 1024   # KV positions per split in these cases (block ranges cross split boundaries)

ATTN_CASES = [
    # (B, Hq, Hkv, D, S, blocks)
    (3, 32, 8, 128, 1024, [(0, 5, 1), (1, 100, 4), (2, 63, 9)]),
    (4, 32, 8, 128, 2048, [(1, 700, 1), (3, 1500, 7), (0, 511, 2), (2, 1023, 9)]),  # split boundaries
    (2, 32, 32, 128, 512, [(0, 10, 3), (1, 300, 5)]),                                 # MHA (7B shape)
    (3, 32, 8, 64, 1024, [(0, 0, 40), (2, 200, 6), (1, 64, 1)]),                       # D = 64, prefill chunk
]


@pytest.mark.parametrize("case", range(len(ATTN_CASES)))
def test_ragged_attention_bf16_matches_brute_force(cuda, case):
    lsk = _lsk()
    B, Hq, Hkv, D, S, blocks = ATTN_CASES[case]
    q, kc, vc, tab, ref = _attn_case(case, BF16, B, Hq, Hkv, D, S, blocks)
    got = _run_attn(lsk, cuda, q, kc, vc, tab, ATTN_TEST_SPLIT).double()
    # bf16 inputs are exact in the fp64 reference; the kernel rounds P to bf16 and the output to bf16
    err = (got - ref).abs()
    assert err.max() < 2e-2, err.max()
    assert err.mean() < 3e-3, err.mean()


@pytest.mark.parametrize("case", range(len(ATTN_CASES)))
def test_ragged_attention_rows_per_item_never_changes_the_output(cuda, case):
    """16-row items (one-tile kernel, Q in registers), 32- and 48-row items (three-tile kernel, Q in LDS):
    bitwise equal outputs, with splits, in every shape."""
    lsk = _lsk()
    B, Hq, Hkv, D, S, blocks = ATTN_CASES[case]
    q, kc, vc, tab, _ = _attn_case(40 + case, BF16, B, Hq, Hkv, D, S, blocks)
    outs = {cap: _run_attn(lsk, cuda, q, kc, vc, tab, ATTN_TEST_SPLIT, cap) for cap in (16, 32, 48)}
    assert torch.equal(outs[16], outs[48]) and torch.equal(outs[32], outs[48])


def _blocked_oracle(q, kc, vc, tab, split):
    from oracle import ordered as O

    rows = np.concatenate([[r] * T for (_, _, T, r) in tab])
    pos = np.concatenate([np.arange(p0, p0 + T) for (_, p0, T, _) in tab])
    G = q.shape[1] // kc.shape[1]
    out = O.attend_bf16_blocked(q.float().numpy(), kc.float().numpy(), vc.float().numpy(), rows, pos, G, split)
    return torch.from_numpy(out.reshape(q.shape[0], -1))


LONG_ATTN_CASES = [
    # (B, Hq, Hkv, D, S, blocks, split): contexts up to 4500+ positions, blocks straddling 2048-position splits
    (4, 32, 8, 128, 4608, [(0, 4090, 9), (1, 2046, 4), (2, 100, 1), (3, 4500, 2)], 2048),
    (3, 32, 8, 64, 4608, [(0, 2040, 12), (1, 4095, 3), (2, 777, 5)], 2048),
]


@pytest.mark.parametrize("case", range(len(ATTN_CASES) + len(LONG_ATTN_CASES)))
def test_ragged_attention_bf16_matches_the_blocked_oracle(cuda, case):
    """The bf16 kernel against oracle/ordered.py's restatement of its softmax blocking (32-position steps dealt to
    8 waves, P rounded to bf16 at each step's running max, waves then position splits merged in order): relative
    L2 <= 1e-4 with 16- and 48-row items, single and multi-split contexts.  What remains is the MFMA's fp32
    summation order (q . k and the P.V step sums) and the exp2 instruction's last bit, which move an occasional
    bf16 rounding of P or of the output; a wrong merge, rescale or rounding point is ~1e-3 or more away."""
    lsk = _lsk()
    if case < len(ATTN_CASES):
        B, Hq, Hkv, D, S, blocks = ATTN_CASES[case]
        split = ATTN_TEST_SPLIT
    else:
        B, Hq, Hkv, D, S, blocks, split = LONG_ATTN_CASES[case - len(ATTN_CASES)]
    q, kc, vc, tab, ref = _attn_case(70 + case, BF16, B, Hq, Hkv, D, S, blocks)
    want = _blocked_oracle(q, kc, vc, tab, split)
    d_exact = float((want.double() - ref).norm() / ref.norm())
    for cap in (16, 48):
        got = _run_attn(lsk, cuda, q, kc, vc, tab, split, cap).float()
        rel = float((got - want).norm() / want.norm())
        differ = float((got != want).float().mean())
        print(f"case {case} cap {cap}: relL2 to the blocked oracle {rel:.2e}, elements differing {differ:.2e} "
              f"(oracle to fp64 exact {d_exact:.2e})")
        assert rel <= 1e-4 and differ <= 1e-2, (cap, rel, differ)


def test_ragged_attention_f32_matches_brute_force(cuda):
    lsk = _lsk()
    q, kc, vc, tab, ref = _attn_case(9, F32, 3, 4, 2, 16, 256, [(0, 3, 1), (1, 30, 5), (2, 100, 9)])
    got = _run_attn(lsk, cuda, q, kc, vc, tab, 1 << 30).double()
    assert (got - ref).abs().max() < 1e-5


def test_ragged_attention_bf16_is_batch_invariant(cuda):
    """A query's output is bitwise the same alone (T = 1) and inside a verify block that crosses a
    split boundary."""
    lsk = _lsk()
    B, Hq, Hkv, D, S = 2, 32, 8, 128, 2048
    blocks = [(0, 505, 9), (1, 1020, 8)]
    q, kc, vc, tab, _ = _attn_case(21, BF16, B, Hq, Hkv, D, S, blocks)
    full = _run_attn(lsk, cuda, q, kc, vc, tab, ATTN_TEST_SPLIT)
    off = 0
    for (r, p0, T) in blocks:
        for t in range(T):
            one = np.array([(0, p0 + t, 1, r)], dtype=np.int32)
            got = _run_attn(lsk, cuda, q[off + t:off + t + 1].contiguous(), kc, vc, one, ATTN_TEST_SPLIT)
            assert torch.equal(got[0], full[off + t]), (r, p0, t)
        off += T


def test_ragged_attention_is_invariant_to_launch_size(cuda):
    """A block gives bitwise the same output inside a launch of hundreds of workgroups (several per CU) as
    alone."""
    lsk = _lsk()
    B, Hq, Hkv, D, S = 40, 32, 8, 128, 1024
    rng = np.random.default_rng(5)
    blocks = [(r, int(rng.integers(0, 900)), int(rng.integers(1, 9))) for r in range(B)]
    q, kc, vc, tab, _ = _attn_case(33, BF16, B, Hq, Hkv, D, S, blocks)
    works, _, _ = lsk.attn_plan(tab, Hq // Hkv, lsk.ATTN_SPLIT)
    assert len(works) * Hkv > 256                                  # the large-launch kernel
    full = _run_attn(lsk, cuda, q, kc, vc, tab, lsk.ATTN_SPLIT)
    off = 0
    for i, (r, p0, T) in enumerate(blocks[:6]):
        one = np.array([(0, p0, T, r)], dtype=np.int32)
        got = _run_attn(lsk, cuda, q[off:off + T].contiguous(), kc, vc, one, lsk.ATTN_SPLIT)
        assert torch.equal(got, full[off:off + T]), (r, p0, T)
        off += T


# ----------------------------------------------------------------------------- glue

def test_argmax_first_index_on_ties(cuda):
    lsk = _lsk()
    x = torch.zeros(4, 1000, dtype=BF16)
    x[0, 17] = x[0, 900] = 3.0
    x[1, :] = -1.0
    x[2, 999] = 1.0
    x[3] = torch.randn(1000, generator=_gen(0)).to(BF16)
    out = torch.empty(4, dtype=torch.long, device=cuda)
    lsk.argmax(x.to(cuda), out)
    assert out.cpu().tolist() == x.float().argmax(-1).tolist() == [17, 0, 999, int(x[3].float().argmax())]


def test_embed_and_copy_rows(cuda):
    lsk = _lsk()
    g = _gen(4)
    table = torch.randn(50, 64, generator=g).to(BF16)
    seq = torch.tensor([[5, 6, 7], [8, 9, 10]], dtype=torch.long)
    sel = torch.tensor([0, -1, 4, 2, -1], dtype=torch.long)
    alt = torch.tensor([0, 33, 0, 0, 49], dtype=torch.long)
    out = torch.empty(5, 64, dtype=BF16, device=cuda)
    lsk.embed(table.to(cuda), alt.to(cuda), out, seq.to(cuda).view(-1), sel.to(cuda))
    ids = [5, 33, 9, 7, 49]
    assert torch.equal(out.cpu(), table[ids])
    dst = torch.zeros(6, 64, dtype=BF16, device=cuda)
    lsk.copy_rows(dst, torch.tensor([5, 0], device=cuda), out, torch.tensor([1, 3], device=cuda), 2)
    assert torch.equal(dst.cpu()[5], table[33]) and torch.equal(dst.cpu()[0], table[7])
    assert (dst.cpu()[1:5] == 0).all()


def test_greedy_accept_matches_closed_form(cuda):
    """acc = min{j : Y_j != draft_{j+1}} <= d; forced: min(draw, d) and drafts[0..a-1] + Y[a]."""
    lsk = _lsk()
    rng = np.random.default_rng(0)
    Dm1, B = 6, 5
    seq = rng.integers(0, 9, size=(B, Dm1))
    slots = np.array([3, 0, 4])
    Ts = np.array([4, 1, 6])
    starts = np.concatenate([[0], np.cumsum(Ts)[:-1]])
    Y = rng.integers(0, 9, size=int(Ts.sum()))
    Y[starts[0]:starts[0] + 2] = seq[3, 1:3]            # first two drafts of slot 3 accepted
    forced = np.array([-1, -1, 2])
    dev = lambda a, dt=torch.int32: torch.as_tensor(a, dtype=dt).to(cuda)  # noqa: E731
    sb = dev(seq.reshape(-1), torch.long)
    acc = torch.empty(3, dtype=torch.long, device=cuda)
    yo = torch.empty(len(Y), dtype=torch.long, device=cuda)
    kvl = dev(np.full(B, 100), torch.long)
    lsk.greedy_accept(dev(Y, torch.long), sb, Dm1, dev(slots), dev(starts), dev(Ts), dev(forced), 3, acc, yo, kvl)
    acc_h, yo_h, sb_h = acc.cpu().numpy(), yo.cpu().numpy(), sb.cpu().numpy().reshape(B, Dm1)
    for j in range(3):
        i, s, T = slots[j], starts[j], Ts[j]
        nat = next((jj for jj in range(T - 1) if Y[s + jj] != seq[i, jj + 1]), T - 1)
        a = min(forced[j], T - 1) if forced[j] >= 0 else nat
        assert acc_h[j] == a
        toks = list(seq[i, 1:1 + a]) + [Y[s + a]] if forced[j] >= 0 else list(Y[s:s + a + 1])
        assert list(yo_h[s:s + a + 1]) == toks
        assert sb_h[i, 0] == Y[s + a]
        assert kvl.cpu()[i] == 100 + a + 1
    assert acc_h[0] == 2


# ----------------------------------------------------------------------------- split-K partials + fused consumers

@pytest.mark.parametrize("M,N,K", [(32, 4096, 4096), (7, 512, 256), (100, 6144, 4096)])
def test_gemm_partial_slices(cuda, M, N, K):
    """Slice partials add up (in slice order) to the fp32 product; rows are bitwise batch invariant."""
    lsk = _lsk()
    ns, ks = lsk.gemm_plan(N, K)
    g = _gen(M + N)
    a = torch.randn(M, K, generator=g).to(BF16)
    w = torch.randn(N, K, generator=g).to(BF16)
    wp = lsk.PackedWeight(w.to(cuda))
    P = lsk.gemm_partial(a.to(cuda), wp, ks).cpu()
    assert P.shape == (ks, M, N)
    ref = a.float() @ w.float().t()
    tot = P[0].clone()
    for s in range(1, ks):
        tot = tot + P[s]
    assert torch.allclose(tot, ref, rtol=1e-4, atol=1e-3 * math.sqrt(K))
    sub = lsk.gemm_partial(a[3:5].contiguous().to(cuda), wp, ks).cpu()
    assert torch.equal(sub, P[:, 3:5])


def test_add_rmsnorm_rounding_points(cuda):
    """x_new = rnd(x + rnd(sum_s P[s])) bitwise; the norm of x_new as the plain kernel computes it."""
    lsk = _lsk()
    g = _gen(8)
    n, dim, ks = 13, 4096, 4
    x = torch.randn(n, dim, generator=g).to(BF16)
    P = torch.randn(ks, n, dim, generator=g)
    w = (1 + 0.1 * torch.randn(dim, generator=g)).to(BF16)
    xd, xo, xn = x.to(cuda), torch.empty(n, dim, dtype=BF16, device=cuda), torch.empty(n, dim, dtype=BF16, device=cuda)
    lsk.add_rmsnorm(xd, P.to(cuda), w.to(cuda), 1e-5, x_out=xo, out=xn)
    acc = P[0].clone()
    for s in range(1, ks):
        acc = acc + P[s]
    x_new = (x.float() + acc.to(BF16).float()).to(BF16)
    assert torch.equal(xo.cpu(), x_new)
    plain = lsk.rmsnorm(xo, w.to(cuda), 1e-5).cpu()
    assert torch.equal(xn.cpu(), plain)
    ref = o_rms_norm(x_new, w, 1e-5)
    assert ((xn.cpu().float() - ref.float()).abs() <= 2.0 ** -7 * ref.float().abs() + 1e-6).all()


def test_rope_append_partial_is_bit_exact(cuda):
    lsk = _lsk()
    from oracle.model import OracleConfig, rope_tables

    g = _gen(31)
    Hq, Hkv, D, B, S, N, ks = 8, 2, 128, 2, 128, 5, 2
    cfg = OracleConfig(64, 64, 1, Hq, Hkv, D, 64, rope_theta=500000.0)
    cos, sin = rope_tables(cfg, S)
    P = torch.randn(ks, N, (Hq + 2 * Hkv) * D, generator=g)
    qkv = (P[0] + P[1]).to(BF16)
    rows = torch.tensor([0, 1, 1, 0, 1])
    pos = torch.tensor([3, 9, 10, 4, 11])
    kd = lsk.k_to_frag(torch.zeros(B, Hkv, S, D, dtype=BF16)).to(cuda)
    vd = torch.zeros(B, Hkv, S // 32, D, 32, dtype=BF16, device=cuda)
    q_out = torch.empty(N, Hq, D, dtype=BF16, device=cuda)
    lsk.rope_append_partial(P.to(cuda), q_out, kd, vd, cos.to(cuda), sin.to(cuda), rows.to(torch.int32).to(cuda),
                            pos.to(torch.int32).to(cuda), Hq, Hkv, D)
    vd = lsk.v_from_blocked(vd)
    c, s = cos[pos].to(BF16).unsqueeze(1), sin[pos].to(BF16).unsqueeze(1)
    assert torch.equal(q_out.cpu(), o_rope(qkv[:, :Hq * D].view(N, Hq, D), c, s))
    kref = o_rope(qkv[:, Hq * D:(Hq + Hkv) * D].view(N, Hkv, D), c, s)
    assert torch.equal(lsk.k_from_frag(kd.cpu())[rows, :, pos], kref)
    assert torch.equal(vd.cpu()[rows, :, pos], qkv[:, (Hq + Hkv) * D:].view(N, Hkv, D))


@pytest.mark.parametrize("M", [37, 100, 150])
def test_head_argmax_matches_logits_argmax(cuda, M):
    """Fused head + pick == argmax over the materialised bf16 logits (first index on ties)."""
    lsk = _lsk()
    g = _gen(12)
    V, K = 4096 + 64, 512
    a = torch.randn(M, K, generator=g).to(BF16).to(cuda)
    w = torch.randn(V, K, generator=g).to(BF16)
    w[3000] = w[100]                      # duplicate rows -> exact ties, the first index must win
    w[4100] = w[100]
    wd = lsk.PackedWeight(w.to(cuda))
    logits = lsk.gemm(a, wd)
    ref = logits.float().argmax(-1)
    out = torch.empty(M, dtype=torch.long, device=cuda)
    lo2 = torch.empty(M, V, dtype=BF16, device=cuda)
    lsk.head_argmax(a, wd, out, logits=lo2)
    assert torch.equal(out, ref)
    assert torch.equal(lo2, logits)
    # scatter into a destination index map
    dst = torch.arange(M, device=cuda) * 2
    big = torch.full((2 * M,), -1, dtype=torch.long, device=cuda)
    lsk.head_argmax(a, wd, big, dst_idx=dst)
    assert torch.equal(big[::2], ref) and (big[1::2] == -1).all()


@pytest.mark.parametrize("M", [1, 17, 40, 64, 100])
def test_head_norm_argmax_equals_norm_then_head(cuda, M):
    """One-call final norm + head + pick (fragment-major normalised rows up to 64, row-major above) is bitwise
    the RMSNorm followed by the fused head: ids, logits, and the scatter through dst_idx."""
    lsk = _lsk()
    g = _gen(13)
    V, K = 4096 + 64, 512
    h = (torch.randn(M, K, generator=g) * 3).to(BF16).to(cuda)
    nw = (1 + 0.1 * torch.randn(K, generator=g)).to(BF16).to(cuda)
    w = torch.randn(V, K, generator=g).to(BF16)
    w[3000] = w[100]
    wd = lsk.PackedWeight(w.to(cuda))
    xn = torch.empty(M, K, dtype=BF16, device=cuda)
    lsk.rmsnorm(h, nw, 1e-5, out=xn)
    ref_ids = torch.empty(M, dtype=torch.long, device=cuda)
    ref_lo = torch.empty(M, V, dtype=BF16, device=cuda)
    lsk.head_argmax(xn, wd, ref_ids, logits=ref_lo)
    ids = torch.empty(M, dtype=torch.long, device=cuda)
    lo = torch.empty(M, V, dtype=BF16, device=cuda)
    lsk.head_norm_argmax(h, nw, 1e-5, wd, ids, logits=lo)
    assert torch.equal(ids, ref_ids) and torch.equal(lo, ref_lo)
    dst = torch.arange(M, device=cuda) * 2
    big = torch.full((2 * M,), -1, dtype=torch.long, device=cuda)
    lsk.head_norm_argmax(h, nw, 1e-5, wd, big, dst_idx=dst)
    assert torch.equal(big[::2], ref_ids) and (big[1::2] == -1).all()


def test_add_rmsnorm_without_partials_stores_x_out(cuda):
    """ks = 0: x_new = x is stored to x_out whenever x_out is given (also in place, x_out == x), and the norm
    of x is the plain RMSNorm's."""
    lsk = _lsk()
    g = _gen(9)
    n, dim = 7, 1024
    x = torch.randn(n, dim, generator=g).to(BF16).to(cuda)
    w = (1 + 0.1 * torch.randn(dim, generator=g)).to(BF16).to(cuda)
    xo = torch.full((n, dim), 7.0, dtype=BF16, device=cuda)
    xn = torch.empty(n, dim, dtype=BF16, device=cuda)
    lsk.add_rmsnorm(x, None, w, 1e-5, x_out=xo, out=xn)
    assert torch.equal(xo, x)
    assert torch.equal(xn, lsk.rmsnorm(x, w, 1e-5))
    xi = x.clone()
    lsk.add_rmsnorm(xi, None, None, 1e-5, x_out=xi)              # in place, no norm output
    assert torch.equal(xi, x)


@pytest.mark.parametrize("dtype", [BF16, F32])
@pytest.mark.parametrize("ks,dim", [(1, 512), (2, 2056), (3, 4096), (8, 8192), (4, 2048)])
def test_add_rmsnorm_slice_counts_and_widths(cuda, dtype, ks, dim):
    """Every launch shape of the add + RMSNorm kernel (compile-time slice counts 1 / 2 / 4 / 8 and the run-time
    count, one to four passes including a partly filled last pass): x_new = rnd(x + rnd(sum_s P[s])) bitwise,
    the norm equal to the plain RMSNorm of x_new bitwise (same per-row order), and within one rounding of
    common/model.py:153-156 evaluated by the oracle."""
    lsk = _lsk()
    g = _gen(100 + ks)
    n = 11
    x = torch.randn(n, dim, generator=g).to(dtype)
    P = torch.randn(ks, n, dim, generator=g)
    w = (1 + 0.1 * torch.randn(dim, generator=g)).to(dtype)
    xd, wd = x.to(cuda), w.to(cuda)
    xo, xn = torch.empty(n, dim, dtype=dtype, device=cuda), torch.empty(n, dim, dtype=dtype, device=cuda)
    lsk.add_rmsnorm(xd, P.to(cuda), wd, 1e-5, x_out=xo, out=xn)
    acc = P[0].clone()
    for s in range(1, ks):
        acc = acc + P[s]
    x_new = (x.float() + acc.to(dtype).float()).to(dtype)
    assert torch.equal(xo.cpu(), x_new)
    assert torch.equal(xn, lsk.rmsnorm(xo, wd, 1e-5))
    ref = o_rms_norm(x_new, w, 1e-5)
    ulp = 2.0 ** -7 if dtype == BF16 else 2.0 ** -20
    assert ((xn.cpu().float() - ref.float()).abs() <= ulp * ref.float().abs() + 1e-6).all()
    xi = xd.clone()                                              # x_out only, in place: the residual update
    lsk.add_rmsnorm(xi, P.to(cuda), None, 1e-5, x_out=xi)
    assert torch.equal(xi.cpu(), x_new)


@pytest.mark.parametrize("nc,nblk", [(1, 3), (5, 40), (7, 64)])
def test_probe_matches_equal_the_closed_form(cuda, nc, nblk):
    """M2 agreement counts (solutions/engine.py:491-514): out[c] = #{t : pred[c, t] == Y[t] and jl[t] <= acc[blk[t]]},
    out[nc] = #{t : jl[t] <= acc[blk[t]]}, computed here by a plain loop over the tokens.  Verify blocks of 1-9
    tokens (several hundred tokens in the larger cases, more than one pass of the 256-thread count), predictions
    that agree with Y often, and accepted counts at both ends (0 and T - 1) so the boundary jl == acc is hit."""
    lsk = _lsk()
    rng = np.random.default_rng(nc * 100 + nblk)
    T = rng.integers(1, 10, size=nblk)
    T[-1] = max(T[-1], 3)                               # its tokens 1.. lie beyond acc = 0: some are not counted
    acc = np.array([rng.integers(0, t) if t > 1 else 0 for t in T], dtype=np.int64)
    acc[0] = T[0] - 1
    acc[-1] = 0
    nvt = int(T.sum())
    blk = np.repeat(np.arange(nblk), T)
    jl = np.concatenate([np.arange(t) for t in T])
    Y = rng.integers(0, 50, size=nvt)
    pred = np.where(rng.random((nc, nvt)) < 0.6, Y[None, :], rng.integers(0, 50, size=(nc, nvt)))
    want = [0] * (nc + 1)
    for t in range(nvt):
        if jl[t] <= acc[blk[t]]:
            want[nc] += 1
            for c in range(nc):
                want[c] += int(pred[c, t] == Y[t])
    dev = lambda a, dt: torch.as_tensor(np.ascontiguousarray(a), dtype=dt).to(cuda)  # noqa: E731
    out = torch.full((nc + 1,), -1, dtype=torch.long, device=cuda)
    lsk.probe_matches(dev(pred.reshape(-1), torch.long), dev(Y, torch.long), dev(acc, torch.long),
                      dev(blk, torch.int32), dev(jl, torch.int32), nc, nvt, out)
    assert out.cpu().tolist() == want
    assert 0 < want[nc] < nvt


@pytest.mark.parametrize("M", [66, 150, 200, 288, 300, 400, 600, 800])
def test_gemm_wide_tier_is_bitwise_the_decode_kernel(cuda, M):
    """Above 64 rows the wide tier (weights staged in LDS) takes every row: token groups dealt to one or more
    blocks and, within a block, evenly to the 8 waves (1 to 3 groups each), with 64-row tiles or, for silu-mul,
    32 + 32-row tiles, as its cost model picks.  These M reach every configuration at these shapes: 1, 2 and 3
    groups per wave in one block, 2 and 3 in several blocks, both silu-mul tiles (66: 1 group; 150, 200: 2; 288,
    300: 3; 400, 600: several blocks; 800: the 32 + 32 silu-mul tile in several blocks).  Every epilogue -- plain,
    residual, silu-mul, split-K partials, LM-head argmax with its logits -- gives bitwise what the decode kernel
    gives row chunk by row chunk (<= 48 rows, one token tile), so a token's result never depends on the batch it is
    packed in."""
    lsk = _lsk()
    g = _gen(M)
    K = 512
    a = torch.randn(M, K, generator=g).to(BF16).to(cuda)
    w = lsk.PackedWeight(torch.randn(12288, K, generator=g).to(BF16).to(cuda))            # 192 row tiles
    w13 = lsk.PackedWeight(torch.randn(2 * 14336, K, generator=g).to(BF16).to(cuda))       # 224 row tiles
    wo = torch.randn(4096, 4096, generator=g).to(BF16)
    wop = lsk.PackedWeight(wo.to(cuda))
    a4 = torch.randn(M, 4096, generator=g).to(BF16).to(cuda)
    r = torch.randn(M, 12288, generator=g).to(BF16).to(cuda)
    head = torch.randn(16384, K, generator=g).to(BF16)
    head[9000] = head[77]                                                                   # exact ties
    headp = lsk.PackedWeight(head.to(cuda))
    ns, ks = lsk.gemm_plan(4096, 4096)
    ids_full = torch.empty(M, dtype=torch.long, device=cuda)
    logit_full = torch.empty(M, 16384, dtype=BF16, device=cuda)
    lsk.head_argmax(a, headp, ids_full, logits=logit_full)
    full = {"none": lsk.gemm(a, w), "residual": lsk.gemm(a, w, residual=r, epilogue=lsk.EPI_RESIDUAL),
            "silu": lsk.gemm(a, w13, epilogue=lsk.EPI_SILU_MUL), "partial": lsk.gemm_partial(a4, wop, ks)}
    for lo in range(0, M, 48):
        hi = min(M, lo + 48)
        sub, sub4 = a[lo:hi].contiguous(), a4[lo:hi].contiguous()
        assert torch.equal(lsk.gemm(sub, w), full["none"][lo:hi]), ("none", lo)
        assert torch.equal(lsk.gemm(sub, w, residual=r[lo:hi].contiguous(), epilogue=lsk.EPI_RESIDUAL),
                           full["residual"][lo:hi]), ("residual", lo)
        assert torch.equal(lsk.gemm(sub, w13, epilogue=lsk.EPI_SILU_MUL), full["silu"][lo:hi]), ("silu", lo)
        assert torch.equal(lsk.gemm_partial(sub4, wop, ks), full["partial"][:, lo:hi]), ("partial", lo)
        ids = torch.empty(hi - lo, dtype=torch.long, device=cuda)
        lg = torch.empty(hi - lo, 16384, dtype=BF16, device=cuda)
        lsk.head_argmax(sub, headp, ids, logits=lg)
        assert torch.equal(ids, ids_full[lo:hi]) and torch.equal(lg, logit_full[lo:hi]), ("head", lo)
    # and against fp32 arithmetic: logits within bf16 rounding, ids = argmax of the returned logits (first on ties)
    ref = a.float() @ head.to(cuda).float().t()
    assert ((logit_full.float() - ref).abs() <= 2.0 ** -7 * ref.abs() + 1e-2).all()
    assert torch.equal(ids_full, logit_full.float().argmax(-1))


@pytest.mark.parametrize("M", [5, 40, 100, 288])
def test_fragment_major_gemms_are_bitwise_the_row_major_ones(cuda, M):
    """lsk_gemm_partial_frag / lsk_gemm_silu_frag -- the layer loop's launches, A fragment-major in whole
    16-token groups (lsk_pack_weight's layout of the same values) -- give bitwise the row-major entry points'
    results, in the decode tier (<= 64 rows) and in the wide tier (above); the silu variant's
    fragment-major h holds the row-major h's values."""
    lsk = _lsk()
    g = _gen(1000 + M)
    K = 1024
    m16 = lsk.frag_rows(M)
    a = torch.randn(m16, K, generator=g).to(BF16).to(cuda)                 # rows >= M: the padding group
    af = lsk.PackedWeight(a).data                                          # same values, fragment-major
    w = lsk.PackedWeight(torch.randn(12288, K, generator=g).to(BF16).to(cuda))          # 192 row tiles
    w13 = lsk.PackedWeight(torch.randn(2 * 12288, K, generator=g).to(BF16).to(cuda))     # 192 row tiles
    ns, ks = lsk.gemm_plan(12288, K)
    want = lsk.gemm_partial(a[:M].contiguous(), w, ks)
    assert torch.equal(lsk.gemm_partial_frag(af, M, w, ks), want)
    h_row = lsk.gemm(a[:M].contiguous(), w13, epilogue=lsk.EPI_SILU_MUL)
    h1 = torch.empty(M, 12288, dtype=BF16, device=cuda)
    assert torch.equal(lsk.gemm_silu_frag(af, M, w13, h1, False), h_row)
    h2 = torch.full((m16 * 12288,), float("nan"), dtype=BF16, device=cuda)
    lsk.gemm_silu_frag(af, M, w13, h2, True)
    back = lsk.PackedWeight.__new__(lsk.PackedWeight)                      # view h2 as packed [m16, 12288]
    back.shape, back.dtype, back.device, back.data = (m16, 12288), BF16, h2.device, h2
    assert torch.equal(back.unpack()[:M], h_row)


@pytest.mark.parametrize("split", [4096, 128])
def test_shifted_segment_metadata_equals_a_plan_at_the_actual_positions(cuda, split):
    """A decode segment planned at its verifiers' upper-bound positions (all drafts accepted) and moved back on the
    device by lsk_shift_segment_positions holds the metadata of a plan made at the actual positions: the same
    tokens, positions and blocks, the same work records, and schedule records that are those works once per KV
    head (the slots they land on may differ: the schedule was costed at the bound).  With 128-position splits the
    blocks span several KV splits and only the last one's end moves."""
    lsk = _lsk()
    rng = np.random.default_rng(split)
    B, Hkv, group, D, n_slots = 24, 8, 4, 128, 256
    rows = np.arange(B, dtype=np.int64)
    base = rng.integers(100, 1500, size=B).astype(np.int64)
    vs = np.sort(rng.choice(B, size=10, replace=False))
    dr = rng.integers(1, 9, size=len(vs)).astype(np.int64)            # drafts held by each verifier
    acc = np.array([rng.integers(0, d + 1) for d in dr], dtype=np.int64)
    if split == 128:                                                   # keep every verifier inside one split count
        for j, i in enumerate(vs):
            lo, hi = base[i] + 2, base[i] + dr[j] + 2
            if (lo + split - 1) // split != (hi + split - 1) // split:
                base[i] = base[i] // split * split + 5                  # KV ends base + 7 .. base + 15
    est = base + 1
    est[vs] += dr                                                       # upper bound: all drafts accepted
    actual = est.copy()
    actual[vs] -= dr - acc
    T = np.ones(B, dtype=np.int64)
    args = (group, split, Hkv, D, n_slots, 0, B, 4096, 4096)
    meta_e, cnt_e = lsk.pack_segment(rows, est, T, *args)
    meta_a, cnt_a = lsk.pack_segment(rows, actual, T, *args)
    N, nw, ng = cnt_e[0], cnt_e[1], cnt_e[2]
    assert (N, nw, ng) == tuple(cnt_a[:3])
    dev = torch.as_tensor(meta_e).to(cuda)
    acc_t = torch.as_tensor(acc).to(cuda)
    lsk.shift_segment_positions(dev, N, B, nw, ng, n_slots * cnt_e[4], group, acc_t,
                                torch.as_tensor(vs.astype(np.int32)).to(cuda),
                                torch.as_tensor(dr.astype(np.int32)).to(cuda), len(vs))
    got = dev.cpu().numpy()
    head = 2 * N + 4 * B
    assert np.array_equal(got[:head], meta_a[:head])                  # rows, positions, blocks
    w_got = got[head:head + 8 * nw].reshape(-1, 8)
    w_ref = meta_a[head:head + 8 * nw].reshape(-1, 8)
    key = lambda a: sorted(map(tuple, a.tolist()))                    # noqa: E731
    assert key(w_got) == key(w_ref)
    if split == 128:
        assert nw > B                                                 # several splits per block
    r_got = got[head + 8 * nw + 8 * ng:].reshape(-1, 8)
    r_ref = meta_a[head + 8 * nw + 8 * ng:].reshape(-1, 8)
    live = lambda r: r[(r[:, 2] & 255) > 0]                           # noqa: E731
    assert key(live(r_got)) == key(live(r_ref))


FUSED_QKV_MS = [5, 32, 48, 64, 100, 160, 288, 600, 1200, 1600, 2000, 2100]   # wide tier: every (ns, msw) it picks for qkv


@pytest.mark.parametrize("M", FUSED_QKV_MS)
@pytest.mark.parametrize("heads", [(32, 8, 128), (8, 8, 64)])
def test_fused_qkv_rope_writes_what_the_unfused_path_writes(cuda, M, heads):
    """lsk_gemm_qkv_rope -- the qkv projection with RoPE and the KV append in its epilogue, the weight's q / k row
    groups RoPE-paired -- writes bitwise what the qkv GEMM without a K split (lsk_gemm_partial, ks = 1) followed by
    lsk_rope_append_partial writes: the rotated q, the K cache and the V cache (every other cache slot untouched),
    in the decode tier (<= 64 rows) and in the wide tier (every tile width and groups-per-wave count it picks for
    these shapes, up to 2100-token prefill sizes: test_fused_qkv_token_counts_reach_every_wide_configuration);
    unpacking the paired storage gives the weight back."""
    lsk = _lsk()
    Hq, Hkv, D = heads
    g = _gen(2000 + M + D)
    K, N, B, S = 1024, (Hq + 2 * Hkv) * D, 4, 1024
    m16 = lsk.frag_rows(M)
    a = torch.randn(m16, K, generator=g).to(BF16).to(cuda)
    af = lsk.PackedWeight(a).data                                          # fragment-major A, same values
    wd = (torch.randn(N, K, generator=g) * 0.05).to(BF16).to(cuda)
    wp = lsk.PackedWeight(wd, qkv_heads=heads)
    assert torch.equal(wp.unpack(), wd)
    with pytest.raises(lsk.LskError):
        lsk.gemm_partial(a[:M].contiguous(), wp, 1)                        # paired storage: fused GEMM only
    cos = torch.randn(S, D, generator=g).to(cuda)
    sin = torch.randn(S, D, generator=g).to(cuda)
    perm = torch.randperm(B * S, generator=g)[:M]                         # distinct (row, position) per token
    rows = (perm // S).to(torch.int32).to(cuda)
    pos = (perm % S).to(torch.int32).to(cuda)
    k0 = lsk.k_to_frag(torch.randn(B, Hkv, S, D, generator=g).to(BF16)).to(cuda)
    v0 = lsk.v_to_blocked(torch.randn(B, Hkv, S, D, generator=g).to(BF16)).to(cuda)
    k1, v1, k2, v2 = k0.clone(), v0.clone(), k0.clone(), v0.clone()
    q1 = torch.empty(M, Hq, D, dtype=BF16, device=cuda)
    q2 = torch.empty(M, Hq, D, dtype=BF16, device=cuda)
    P = lsk.gemm_partial(a[:M].contiguous(), lsk.PackedWeight(wd), 1)
    lsk.rope_append_partial(P, q1, k1, v1, cos, sin, rows, pos, Hq, Hkv, D)
    lsk.gemm_qkv_rope(af, wp, M, q2, k2, v2, cos, sin, rows, pos)
    torch.cuda.synchronize()
    assert torch.equal(q2.view(torch.int16), q1.view(torch.int16))
    assert torch.equal(k2.view(torch.int16), k1.view(torch.int16))
    assert torch.equal(v2.view(torch.int16), v1.view(torch.int16))
    assert not torch.equal(k2, k0) and not torch.equal(v2, v0)
