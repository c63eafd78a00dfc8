"""When to run the deep layers (solutions/schedulers.py surface; host-only NumPy, no GPU access).

Each scheduler sees the decoding slots' state before a step and returns the verifying set V (deep
step iff V is non-empty); the other decoding slots draft one token in the same step.

  fixed       a deep step every gamma shallow steps (solutions/schedulers.py:77-89)
  aspire      per-request target draft length from an EMA acceptance and the homogeneous-batch cost
              ratio t_sh / t_deep (solutions/schedulers.py:92-111; targets by
              common/policies.py:54-68).  `min_draft` is exposed so the [2, 8] draft range of the
              Llama3-8B configuration can be expressed (the reference's make_scheduler cannot).
  m1          batch-level trigger R(s+1) <= R(s) (solutions/schedulers.py:114-153)
  fsm-sync    one batch-wide gamma, +-1 by the majority of full accepts (solutions/schedulers.py:156-171)
  aspire-fsm  per-request targets, +-1 after each round (solutions/schedulers.py:174-197)
Acceptance estimate: a <- omega a + (1 - omega) acc / min(acc + 1, d) (solutions/schedulers.py:35-51).
"""

from __future__ import annotations

import numpy as np


def expected_tokens(alpha, d) -> np.ndarray:
    a = np.clip(np.asarray(alpha, dtype=np.float64), 0.0, 1 - 1e-6)
    return (1 - a ** (np.asarray(d, dtype=np.float64) + 1)) / (1 - a)


_G_COLS: dict = {}


def expected_token_targets(alphas, cost_ratios, min_draft: int, max_draft: int) -> np.ndarray:
    """Largest gamma with a positive marginal gain of E[tokens]/E[time] = ((1 - a^(g+1)) / (1 - a)) / (1 + c g):
    a^g ((1 - a) c (g - 1) + c + (1 - a)) > c  (common/policies.py:54-68)."""
    a = np.minimum(np.maximum(np.asarray(alphas, dtype=np.float64), 0.0), 1.0)
    c = np.asarray(cost_ratios, dtype=np.float64)
    if max_draft < 1:
        return np.full(a.shape, min_draft, dtype=np.int64)
    g = _G_COLS.get(max_draft)
    if g is None:
        g = _G_COLS[max_draft] = np.arange(1, max_draft + 1, dtype=np.int64)[:, None]
    om = 1 - a
    gain = a ** g * (om * c * (g - 1) + c + om) > c
    last = (max_draft - 1) - np.argmax(gain[::-1], axis=0)
    t = np.where(gain.any(axis=0), last + 1, min_draft)
    t = np.where(a >= 1 - 1e-7, max_draft, t)
    return np.minimum(np.maximum(t, min_draft), max_draft).astype(np.int64)


def best_gamma_expected(alpha: float, c: float, gmax: int) -> int:
    """Brute-force argmax_g ((1 - a^(g+1)) / (1 - a)) / (1 + c g) (checker for expected_token_targets)."""
    g = np.arange(0, gmax + 1)
    a = min(max(alpha, 1e-6), 1 - 1e-6)
    return int(g[np.argmax((1 - a ** (g + 1)) / (1 - a) / (1 + c * g))])


class _EMA:
    def __init__(self, B: int, omega: float, alpha0: float):
        self.omega, self.alpha0 = omega, alpha0
        self.alpha = np.full(B, alpha0)
        self.fresh = np.ones(B, dtype=bool)

    def observe(self, verify, accepted, drafts) -> None:
        ok = verify & (drafts > 0)
        if ok.any():
            a = accepted[ok].astype(np.float64)
            d = drafts[ok].astype(np.float64)
            self.alpha[ok] = self.omega * self.alpha[ok] + (1 - self.omega) * (a / np.minimum(a + 1.0, d))
            self.fresh[ok] = False

    def reset(self, slot: int, alpha=None) -> None:
        self.alpha[slot] = self.alpha0 if alpha is None else alpha
        self.fresh[slot] = True


class Scheduler:
    name = "base"

    def __init__(self, B: int, cost_model, k: int, d_max: int = 16, omega: float = 0.8, alpha0: float = 0.9):
        self.B, self.cm, self.k, self.d_max = B, cost_model, k, d_max
        self.ema = _EMA(B, omega, alpha0)

    def decide(self, d, ctx, dec, steps_since_deep) -> np.ndarray:
        raise NotImplementedError

    def observe(self, verify, accepted, drafts) -> None:
        self.ema.observe(verify, accepted, drafts)

    def reset(self, slot: int) -> None:
        self.ema.reset(slot)

    def set_exit(self, k: int, alpha=None) -> None:
        self.k = k
        if alpha is not None:
            self.ema.alpha[:] = alpha


class FixedScheduler(Scheduler):
    name = "fixed"

    def __init__(self, B, cost_model, k, gamma: int, **kw):
        super().__init__(B, cost_model, k, **kw)
        if not 1 <= gamma <= self.d_max:
            raise ValueError("gamma must be in [1, d_max]")
        self.gamma = gamma

    def decide(self, d, ctx, dec, steps_since_deep):
        if steps_since_deep >= self.gamma:
            return dec & (d >= 1)
        return dec & (d >= self.d_max)


class AspireScheduler(Scheduler):
    name = "aspire"

    def __init__(self, B, cost_model, k, initial_draft: int = 3, min_draft: int = 1, **kw):
        super().__init__(B, cost_model, k, **kw)
        self.initial_draft, self.min_draft = initial_draft, min_draft

    def decide(self, d, ctx, dec, steps_since_deep):
        n = int(dec.sum())
        if n == 0:
            return np.zeros_like(dec)
        C = float(ctx[dec].sum())
        t_sh = float(self.cm.t_sh(n, self.k, C))
        t_v = self.cm.t_deep(n * (d + 1), self.k, C, n)
        ratio = np.minimum(np.maximum(t_sh / np.maximum(t_v, 1e-9), 1e-4), 1.0)
        tgt = expected_token_targets(self.ema.alpha, ratio, self.min_draft, self.d_max)
        floor = np.where(self.ema.fresh, max(self.min_draft, self.initial_draft), self.min_draft)
        tgt = np.minimum(np.maximum(tgt, floor), self.d_max)
        return dec & (d >= 1) & ((d >= tgt) | (d >= self.d_max))


class M1Scheduler(Scheduler):
    name = "m1"

    def __init__(self, B, cost_model, k, sla_steps: int = 32, **kw):
        super().__init__(B, cost_model, k, **kw)
        self.sla_steps = sla_steps

    def rates(self, d, ctx, dec, s):
        dd = d[dec]
        cc = ctx[dec].astype(np.float64)
        al = self.ema.alpha[dec]
        n = len(dd)
        C = float(cc.sum())
        t_sh = float(self.cm.t_sh(n, self.k, C))
        ver = dd >= 1
        e_now = float(expected_tokens(al, dd)[ver].sum())
        t_now = s * t_sh + float(self.cm.t_deep(int((dd[ver] + 1).sum()), self.k, C, n, C_deep=float(cc[ver].sum())))
        e_next = float(expected_tokens(al, dd + 1).sum())
        t_next = (s + 1) * t_sh + float(self.cm.t_deep(int((dd + 2).sum()), self.k, C + n, n, C_deep=C + n))
        return e_now / max(t_now, 1e-9), e_next / max(t_next, 1e-9)

    def decide(self, d, ctx, dec, steps_since_deep):
        ver = dec & (d >= 1)
        if not ver.any():
            return ver
        if (d[dec] >= self.d_max).any() or steps_since_deep >= self.sla_steps:
            return ver
        r_now, r_next = self.rates(d, ctx, dec, steps_since_deep)
        return ver if r_next <= r_now else np.zeros_like(ver)


class SyncFSMScheduler(FixedScheduler):
    name = "fsm-sync"

    def __init__(self, *a, **kw):
        super().__init__(*a, **kw)
        self.gamma_hist = [self.gamma]

    def observe(self, verify, accepted, drafts) -> None:
        super().observe(verify, accepted, drafts)
        ver = verify & (drafts > 0)
        if ver.any():
            full = int((accepted[ver] >= drafts[ver]).sum())
            self.gamma = int(np.clip(self.gamma + (1 if full > 0.5 * int(ver.sum()) else -1), 1, self.d_max))
        self.gamma_hist.append(self.gamma)


class AspireFSMScheduler(Scheduler):
    name = "aspire-fsm"

    def __init__(self, B, cost_model, k, initial_draft: int = 3, **kw):
        super().__init__(B, cost_model, k, **kw)
        self.initial_draft = initial_draft
        self.targets = np.full(B, initial_draft, dtype=np.int64)

    def decide(self, d, ctx, dec, steps_since_deep):
        return dec & (d >= 1) & ((d >= self.targets) | (d >= self.d_max))

    def observe(self, verify, accepted, drafts) -> None:
        super().observe(verify, accepted, drafts)
        ids = np.flatnonzero(verify & (drafts > 0))
        if ids.size:
            full = accepted[ids] >= drafts[ids]
            self.targets[ids] = np.clip(np.where(full, self.targets[ids] + 1, self.targets[ids] - 1), 1, self.d_max)

    def reset(self, slot: int) -> None:
        super().reset(slot)
        self.targets[slot] = self.initial_draft


SCHEDULERS = ("fixed", "aspire", "m1", "fsm-sync", "aspire-fsm")


def make_scheduler(name: str, B: int, cost_model, k: int, *, gamma: int = 4, d_max: int = 16, sla_steps: int = 32,
                   initial_draft: int = 3, omega: float = 0.8, alpha0: float = 0.9, min_draft: int = 1, ref=None):
    kw = dict(d_max=d_max, omega=omega, alpha0=alpha0)
    if name == "fixed":
        return FixedScheduler(B, cost_model, k, gamma, **kw)
    if name == "aspire":
        return AspireScheduler(B, cost_model, k, initial_draft=initial_draft, min_draft=min_draft, **kw)
    if name == "m1":
        return M1Scheduler(B, cost_model, k, sla_steps=sla_steps, **kw)
    if name == "fsm-sync":
        return SyncFSMScheduler(B, cost_model, k, gamma, **kw)
    if name == "aspire-fsm":
        return AspireFSMScheduler(B, cost_model, k, initial_draft=initial_draft, **kw)
    raise ValueError(f"unknown scheduler {name!r}; known: {SCHEDULERS}")
