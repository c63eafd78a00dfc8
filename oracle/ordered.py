"""Ordered fp32 restatement of the reference's reductions (TEST INFRASTRUCTURE ONLY).

Only tests/ (and, through OracleLlama(ordered=True), the checks built on it) use this module; the product path
never imports it.

The reference leaves the summation order of its fp32 reductions to torch (F.linear, mean, SDPA, exp).  These
functions evaluate the same mathematics in one fixed order -- the order the fp32 kernels use -- with every step
a single IEEE fp32 operation, so the fp32 engine can be compared bit for bit:

  exp_f32    Cody and Waite's range reduction + degree-7 Taylor polynomial (common/model.py's softmax and
             F.silu use exp); results below 2^-124 flush to 0
  silu_f32   x / (1 + exp(-x))                                  (solutions/packed.py:185, F.silu)
  linear     y[m, n] = 64-lane xor butterfly (32, 16, ..., 1) of the lane sums over k = lane, lane + 64, ...
                                                                (F.linear, solutions/packed.py:175-185)
  rms_norm   thread t sums x[j]^2 over j = (256 p + t) 8 + i (p, then i, in order), a 64-lane butterfly per
             wave, the 4 waves added in order; w * (x * (1 / sqrt(mean + eps)))   (common/model.py:153-156)
  attend     per query and head: 64-position chunks, scores as sequential dot products times the scale,
             online softmax (max, alpha = exp(m_old - m_new), p = exp(s - m_new), butterfly sum of p),
             o = o * alpha + sum_j p_j v_j in position order, o / l at the end  (solutions/packed.py:142-166)

Pinned by tests/test_oracle.py: the same HF golden logits as the default oracle (atol 1e-4), the default
oracle's fp32 forward (1e-5), exp_f32 against numpy's exp (2 ulp), and planted mistakes (a lane order that
skips the butterfly, a Taylor term dropped) that the bitwise GPU checks reject.

The bf16 attention (solutions/packed.py:142-166 evaluated in bf16) has its own restatement here,
attend_bf16_blocked: the bf16 kernel's softmax blocking (32-position steps dealt to 8 waves, P rounded to bf16 at
each step's running max, waves and then position splits merged in order).  Pinned by a known answer on inputs where
every step is exact (bit-equal to the base-2 textbook softmax, with planted mistakes that change it), and on random
bf16 inputs by its distance to an fp64 brute force, which matches that of torch's bf16 SDPA.
"""

from __future__ import annotations

import math

import numpy as np
import torch

F32 = np.float32
_LOG2E = F32("1.4426950216293335")
_LN2_HI = F32("0.693145751953125")           # 16 significant bits: n * _LN2_HI is exact for |n| <= 128
_LN2_LO = F32("1.428606765330187e-06")
_TAYLOR = [F32(c) for c in ("0.00019841270113829523", "0.0013888889225199819", "0.008333333767950535",
                            "0.0416666679084301", "0.1666666716337204", "0.5", "1.0", "1.0")]  # 1/7! .. 1/0!


def exp_f32(x) -> np.ndarray:
    x = np.asarray(x, dtype=F32)
    with np.errstate(over="ignore", invalid="ignore"):
        n = np.rint(x * _LOG2E)
        n = np.where(np.isfinite(n), n, F32(0)).astype(F32)
        r = (x - n * _LN2_HI) - n * _LN2_LO
        p = np.full_like(r, _TAYLOR[0])
        for c in _TAYLOR[1:]:
            p = p * r + c
        out = np.ldexp(p, np.clip(n, -200, 200).astype(np.int32)).astype(F32)
    out = np.where(x < F32(-86.0), F32(0.0), out)
    out = np.where(x > F32(89.0), F32(np.inf), out)
    return np.where(np.isnan(x), x, out).astype(F32)


def silu_f32(x) -> np.ndarray:
    x = np.asarray(x, dtype=F32)
    with np.errstate(over="ignore"):
        return (x / (F32(1.0) + exp_f32(-x))).astype(F32)


def butterfly_sum(v: np.ndarray) -> np.ndarray:
    """xor butterfly over the last axis (64 lanes): v[l] += v[l ^ o] for o = 32, 16, ..., 1."""
    idx = np.arange(v.shape[-1])
    o = v.shape[-1] // 2
    while o >= 1:
        v = v + v[..., idx ^ o]
        o //= 2
    return v


def linear(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    """x [M, K] @ w[N, K]^T in the fp32 GEMM kernel's order."""
    x = np.asarray(x, dtype=F32)
    w = np.asarray(w, dtype=F32)
    M, K = x.shape
    N = w.shape[0]
    acc = np.zeros((M, N, 64), dtype=F32)
    for j in range(0, K, 64):
        L = min(64, K - j)
        acc[:, :, :L] = acc[:, :, :L] + x[:, None, j:j + L] * w[None, :, j:j + L]
    return butterfly_sum(acc)[..., 0]


def rms_norm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = np.asarray(x, dtype=F32)
    M, dim = x.shape
    ss = np.zeros((M, 256), dtype=F32)
    t = np.arange(256)
    for p in range(4):
        for i in range(8):
            j = (p * 256 + t) * 8 + i
            ok = np.nonzero(j < dim)[0]
            if len(ok):
                v = x[:, j[ok]]
                ss[:, ok] = ss[:, ok] + v * v
    wsum = butterfly_sum(ss.reshape(M, 4, 64))[..., 0]
    tot = ((wsum[:, 0] + wsum[:, 1]) + wsum[:, 2]) + wsum[:, 3]
    mean = tot / F32(dim)
    r = F32(1.0) / np.sqrt(mean + F32(eps))
    return (np.asarray(w, dtype=F32)[None, :] * (x * r[:, None])).astype(F32)


def attend(q: np.ndarray, kc: np.ndarray, vc: np.ndarray, rows, pos, group: int) -> np.ndarray:
    """q [N, Hq, D] (RoPE applied) over the cache [B, Hkv, S, D]; token t attends cache[rows[t], :, 0..pos[t]]."""
    q = np.asarray(q, dtype=F32)
    N, Hq, D = q.shape
    scale = F32(1.0 / math.sqrt(D))
    heads = np.arange(Hq) // group
    out = np.zeros((N, Hq, D), dtype=F32)
    for t in range(N):
        r, p = int(rows[t]), int(pos[t])
        K = np.asarray(kc[r], dtype=F32)[heads]          # [Hq, S, D]
        V = np.asarray(vc[r], dtype=F32)[heads]
        m_run = np.full(Hq, -np.inf, dtype=F32)
        l_run = np.zeros(Hq, dtype=F32)
        o = np.zeros((Hq, D), dtype=F32)
        for base in range(0, p + 1, 64):
            nv = min(64, p + 1 - base)
            acc = np.zeros((Hq, nv), dtype=F32)
            for d in range(D):
                acc = acc + q[t, :, d:d + 1] * K[:, base:base + nv, d]
            s = np.full((Hq, 64), -np.inf, dtype=F32)
            s[:, :nv] = acc * scale
            m_new = np.maximum(m_run, s.max(axis=1))
            alpha = np.where(m_new == m_run, F32(1.0), exp_f32(m_run - m_new)).astype(F32)
            pr = np.where(s == -np.inf, F32(0.0), exp_f32(s - m_new[:, None])).astype(F32)
            rs = butterfly_sum(pr)[:, 0]
            l_run = l_run * alpha + rs
            m_run = m_new
            acc_o = o * alpha[:, None]
            for j in range(nv):
                acc_o = acc_o + pr[:, j:j + 1] * V[:, base + j, :]
            o = acc_o
        out[t] = o / l_run[:, None]
    return out


def bf16_round(x) -> np.ndarray:
    """fp32 -> bf16 -> fp32, round to nearest even, NaN -> the bf16 quiet NaN (the store rule of torch and of the
    bf16 kernels)."""
    x = np.ascontiguousarray(x, dtype=F32)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    r = np.where(np.isnan(x), np.uint32(0x7FC00000), r).astype(np.uint32)
    return r.view(F32)


def exp2_f32(x) -> np.ndarray:
    """2^x rounded to fp32 (the bf16 attention's exp2 instruction, specified to 1 ulp of this)."""
    x = np.asarray(x, dtype=F32)
    with np.errstate(over="ignore", under="ignore", invalid="ignore"):
        return np.exp2(x.astype(np.float64)).astype(F32)


def attn_scale_log2(head_dim: int) -> np.float32:
    """The bf16 attention's score multiplier: fp32(1 / sqrt(D)) * fp32(log2 e), one fp32 product."""
    return F32(F32(1.0 / math.sqrt(head_dim)) * F32(1.4426950408889634))


def attend_bf16_blocked(q, kc, vc, rows, pos, group: int, split: int, scale_log2=None, step: int = 32,
                        waves: int = 8, rescale: bool = True, weigh_waves: bool = True) -> np.ndarray:
    """bf16 attention in the blocking of the bf16 kernel (softmax(q K^T / sqrt(D)) V, solutions/packed.py:142-166).

    q [N, Hq, D] (RoPE applied, bf16 values), kc / vc [B, Hkv, S, D] (bf16 values); token t attends positions
    0..pos[t] of cache row rows[t].  Per (token, head):
      * positions are cut into splits at absolute multiples of `split`, each split into `step`-position steps;
        step i of a split belongs to wave i % waves, and every wave takes its steps in order;
      * a step's scores are fp32(q . k) * scale_log2 (log2 units); with the wave's running max m and the step's
        max mt: m' = max(m, mt), alpha = 1 if m' == m else 2^(m - m'), p = 2^(s - m') (0 when masked),
        l = l * alpha + ((g0 + g1) + (g2 + g3)) where g_j sums p over positions 8j .. 8j + 7 in order,
        o = o * alpha + sum_pos bf16(p) v  (the P.V product takes p rounded to bf16 at the running max);
      * the waves are merged in wave order: M = max m_w, e_w = 0 (empty wave), 1 (m_w == M) or 2^(m_w - M),
        L = sum e_w l_w, O = sum e_w o_w (fp32, from 0);
      * the splits are merged in split order with the same weights; out = bf16(O / L).
    Sums of exact products (q . k, the P.V step sum) are rounded to fp32 once; every other step is one fp32
    operation.  `rescale` / `weigh_waves` = False plant mistakes for the tests: no alpha rescale of o, or the
    waves and splits summed without their weights."""
    if step != 32 or split % (step * waves):
        raise ValueError("the bf16 kernel's steps are 32 positions (4 lane groups of 8); splits are whole rounds")
    q = np.asarray(q, dtype=F32)
    N, Hq, D = q.shape
    Hkv = Hq // group
    sl2 = attn_scale_log2(D) if scale_log2 is None else F32(scale_log2)
    ninf = F32(-np.inf)
    out = np.zeros((N, Hq, D), dtype=F32)
    for t in range(N):
        r, p = int(rows[t]), int(pos[t])
        n = p + 1
        K = np.asarray(kc[r, :, :n], dtype=np.float64)               # [Hkv, n, D]
        V = np.asarray(vc[r, :, :n], dtype=np.float64)
        qh = q[t].reshape(Hkv, group, D).astype(np.float64)
        S = (np.einsum("hgd,hnd->hgn", qh, K).astype(F32) * sl2).astype(F32)   # [Hkv, G, n]
        parts = []
        for s0 in range(0, n, split):
            ls = min(split, n - s0)
            nst = (ls + step - 1) // step
            rounds = (nst + waves - 1) // waves
            tot = rounds * waves * step
            Sp = np.full((Hkv, group, tot), ninf, dtype=F32)
            Sp[:, :, :ls] = S[:, :, s0:s0 + ls]
            Vp = np.zeros((Hkv, tot, D), dtype=np.float64)
            Vp[:, :ls] = V[:, s0:s0 + ls]
            Sp = Sp.reshape(Hkv, group, rounds, waves, step)
            Vp = Vp.reshape(Hkv, rounds, waves, step, D)
            m = np.full((Hkv, group, waves), ninf, dtype=F32)
            lsum = np.zeros((Hkv, group, waves), dtype=F32)
            o = np.zeros((Hkv, group, waves, D), dtype=F32)
            with np.errstate(invalid="ignore"):
                for i in range(rounds):
                    sv = Sp[:, :, i]                                          # [Hkv, G, W, step]
                    m_new = np.maximum(m, sv.max(axis=-1))
                    alpha = np.where(m_new == m, F32(1.0), exp2_f32(m - m_new)).astype(F32)
                    pe = np.where(sv == ninf, F32(0.0), exp2_f32(sv - m_new[..., None])).astype(F32)
                    g = pe.reshape(Hkv, group, waves, 4, 8)
                    acc = g[..., 0]
                    for e in range(1, 8):
                        acc = acc + g[..., e]
                    rs = (acc[..., 0] + acc[..., 1]) + (acc[..., 2] + acc[..., 3])
                    lsum = (lsum * alpha + rs).astype(F32)
                    pv = np.einsum("hgws,hwsd->hgwd", bf16_round(pe).astype(np.float64), Vp[:, i])
                    if rescale:
                        o = (o * alpha[..., None]).astype(F32)
                    o = (o.astype(np.float64) + pv).astype(F32)
                    m = m_new
            parts.append(_merge(m, lsum, o, weigh_waves))
        ms = np.stack([pm for pm, _, _ in parts], axis=-1)                     # [Hkv, G, n_split]
        ls_ = np.stack([pl for _, pl, _ in parts], axis=-1)
        os_ = np.stack([po for _, _, po in parts], axis=-2)                    # [Hkv, G, n_split, D]
        _, L, Ov = _merge(ms, ls_, os_, weigh_waves)
        out[t] = bf16_round((Ov / L[..., None]).astype(F32)).reshape(Hq, D)
    return out


def _merge(m, l, o, weigh: bool = True):
    """Merge partial softmax states along the last axis of m / l (o: the axis before D), in index order:
    M = max m_i, e_i = 0 if m_i = -inf, 1 if m_i == M, else 2^(m_i - M); L = sum e_i l_i, O = sum e_i o_i (fp32)."""
    M = m.max(axis=-1)
    with np.errstate(invalid="ignore"):
        e = np.where(m == F32(-np.inf), F32(0.0),
                     np.where(m == M[..., None], F32(1.0), exp2_f32(m - M[..., None]))).astype(F32)
    if not weigh:
        e = np.where(m == F32(-np.inf), F32(0.0), F32(1.0)).astype(F32)
    L = np.zeros(l.shape[:-1], dtype=F32)
    O = np.zeros(o.shape[:-2] + o.shape[-1:], dtype=F32)
    for i in range(m.shape[-1]):
        L = (L + e[..., i] * l[..., i]).astype(F32)
        O = (O + e[..., i, None] * o[..., i, :]).astype(F32)
    return M, L, O


def t2n(x: torch.Tensor) -> np.ndarray:
    return x.detach().to(torch.float32).numpy()


def n2t(x: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(x, dtype=F32))
