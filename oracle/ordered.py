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


def t2n(x: torch.Tensor) -> np.ndarray:
    return x.detach().to(torch.float32).numpy()


def n2t(x: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(x, dtype=F32))
