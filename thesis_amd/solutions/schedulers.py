"""Deep-step policies: which decoding slots verify in the next step (host-only NumPy, no GPU access).

Before every engine step the policy sees, for each slot, how many drafts it holds (d), how many KV positions it
reads (context) and whether it is decoding (live), plus the number of shallow-only steps since the last deep step
(idle).  It returns the verifying set V; the step is deep iff V is non-empty, and every live slot outside V drafts
one more token in the same step.  The decision rules are the reference's methods (solutions/schedulers.py:29-197,
targets by common/policies.py:54-68); a different rule would be a different method.

  fixed       verify everyone holding drafts every `gamma` idle steps (a slot at d_max verifies earlier)
  aspire      per-slot target draft length: the largest gamma whose marginal expected-tokens-per-time gain is
              positive, with the cost ratio c = t_shallow / t_deep(d + 1) of a homogeneous batch; a slot verifies
              as soon as it reaches its target.  `min_draft` bounds targets from below (the Llama3-8B
              configuration's [2, 8] range), fresh slots start at `initial_draft`
  m1          batch trigger: verify now iff the expected throughput of verifying now is at least that of
              drafting one more step, R(s) >= R(s + 1); forced at d_max or after `sla_steps` idle steps
  fsm-sync    `fixed` with one batch-wide gamma moved by +-1 after each round (majority of full accepts)
  aspire-fsm  per-slot targets moved by +-1 after each round (full accept: +1)

Acceptance rate per slot (all policies): rate <- w rate + (1 - w) acc / min(acc + 1, d) after each round in which
the slot verified d >= 1 drafts and accepted acc of them.
"""

from __future__ import annotations

import numpy as np

POLICIES = ("fixed", "aspire", "m1", "fsm-sync", "aspire-fsm")
SCHEDULERS = POLICIES


def expected_tokens(alpha, d) -> np.ndarray:
    """Expected tokens committed by verifying d drafts at per-token acceptance alpha: sum_{j<=d} alpha^j."""
    a = np.clip(np.asarray(alpha, dtype=np.float64), 0.0, 1 - 1e-6)
    return (1 - a ** (np.asarray(d, dtype=np.float64) + 1)) / (1 - a)


_TARGET_GRID: dict = {}


def expected_token_targets(alphas, cost_ratios, min_draft: int, max_draft: int) -> np.ndarray:
    """Per slot, the largest gamma in [1, max_draft] at which one more draft still raises
    E[tokens] / E[time] = ((1 - a^(g+1)) / (1 - a)) / (1 + c g), i.e. a^g ((1 - a) c (g - 1) + c + (1 - a)) > c;
    min_draft when no gamma qualifies; max_draft at a = 1; clipped to [min_draft, max_draft]."""
    a = np.clip(np.asarray(alphas, dtype=np.float64), 0.0, 1.0)
    c = np.asarray(cost_ratios, dtype=np.float64)
    if max_draft < 1:
        return np.full(a.shape, min_draft, dtype=np.int64)
    g = _TARGET_GRID.setdefault(max_draft, np.arange(1, max_draft + 1, dtype=np.int64)[:, None])
    miss = 1 - a
    rising = a ** g * (miss * c * (g - 1) + c + miss) > c            # [gamma, slot]
    top = max_draft - np.argmax(rising[::-1], axis=0)               # largest rising gamma (1-based)
    target = np.where(rising.any(axis=0), top, min_draft)
    target = np.where(a >= 1 - 1e-7, max_draft, target)
    return np.clip(target, min_draft, max_draft).astype(np.int64)


def best_gamma_expected(alpha: float, c: float, gmax: int) -> int:
    """Brute force over gamma = 0..gmax of ((1 - a^(g+1)) / (1 - a)) / (1 + c g) (checks the closed form)."""
    a = min(max(alpha, 1e-6), 1 - 1e-6)
    g = np.arange(gmax + 1)
    return int(g[np.argmax((1 - a ** (g + 1)) / (1 - a) / (1 + c * g))])


class AcceptanceTracker:
    """Exponentially weighted per-slot acceptance rate; `cold` marks slots without a verified round yet."""

    def __init__(self, n_slots: int, weight: float, prior: float):
        self.weight, self.prior = weight, prior
        self.rate = np.full(n_slots, prior, dtype=np.float64)
        self.cold = np.ones(n_slots, dtype=bool)

    def update(self, verified: np.ndarray, accepted: np.ndarray, drafts: np.ndarray) -> None:
        hit = verified & (drafts > 0)
        if not hit.any():
            return
        acc, d = accepted[hit].astype(np.float64), drafts[hit].astype(np.float64)
        self.rate[hit] = self.weight * self.rate[hit] + (1 - self.weight) * acc / np.minimum(acc + 1.0, d)
        self.cold[hit] = False

    def restart(self, slot: int, rate=None) -> None:
        self.rate[slot] = self.prior if rate is None else rate
        self.cold[slot] = True


class DraftPolicy:
    """One engine's deep-step policy (see the module docstring for the rules).

    decide(d, ctx, live, idle) -> bool[B]   verifying set of the next step
    observe(verified, accepted, drafts)     feedback after a deep step
    reset(slot)                             a new request took the slot
    set_exit(k, rate)                       the exit layer moved (M2): costs change, rates restart at `rate`
    """

    def __init__(self, kind: str, n_slots: int, cost_model, exit_layer: int, *, gamma: int = 4, d_max: int = 16,
                 sla_steps: int = 32, initial_draft: int = 3, min_draft: int = 1, omega: float = 0.8,
                 alpha0: float = 0.9):
        if kind not in POLICIES:
            raise ValueError(f"unknown scheduler {kind!r}; known: {POLICIES}")
        if kind in ("fixed", "fsm-sync") and not 1 <= gamma <= d_max:
            raise ValueError("gamma must be in [1, d_max]")
        self.name = kind
        self.B, self.cm, self.k, self.d_max = n_slots, cost_model, exit_layer, d_max
        self.sla_steps, self.initial_draft, self.min_draft = sla_steps, initial_draft, min_draft
        self.tracker = AcceptanceTracker(n_slots, omega, alpha0)
        self.gamma = gamma if kind in ("fixed", "fsm-sync") else None
        self.gamma_hist = [gamma] if kind == "fsm-sync" else None
        self.targets = np.full(n_slots, initial_draft, dtype=np.int64) if kind == "aspire-fsm" else None
        self._rule = {"fixed": self._by_round, "fsm-sync": self._by_round, "aspire": self._by_target_cost,
                      "aspire-fsm": self._by_target_feedback, "m1": self._by_rate}[kind]

    @property
    def alpha(self) -> np.ndarray:
        return self.tracker.rate

    # ------------------------------------------------------------------ engine calls
    def decide(self, d, ctx, dec, steps_since_deep) -> np.ndarray:
        ready = dec & (d >= 1)
        if not ready.any():
            return ready
        return self._rule(d, ctx, dec, ready, steps_since_deep)

    def observe(self, verify, accepted, drafts) -> None:
        self.tracker.update(verify, accepted, drafts)
        rounds = verify & (drafts > 0)
        full = accepted >= drafts
        if self.gamma_hist is not None:                                   # fsm-sync: one batch-wide gamma
            if rounds.any():
                step = 1 if int((full & rounds).sum()) > 0.5 * int(rounds.sum()) else -1
                self.gamma = int(np.clip(self.gamma + step, 1, self.d_max))
            self.gamma_hist.append(self.gamma)
        if self.targets is not None and rounds.any():                    # aspire-fsm: per-slot targets
            self.targets = np.where(rounds, np.clip(self.targets + np.where(full, 1, -1), 1, self.d_max),
                                    self.targets)

    def reset(self, slot: int) -> None:
        self.tracker.restart(slot)
        if self.targets is not None:
            self.targets[slot] = self.initial_draft

    def set_exit(self, k: int, alpha=None) -> None:
        self.k = k
        if alpha is not None:
            self.tracker.rate[:] = alpha

    # ------------------------------------------------------------------ rules
    def _by_round(self, d, ctx, dec, ready, idle):
        return ready if idle >= self.gamma else ready & (d >= self.d_max)

    def _by_target_cost(self, d, ctx, dec, ready, idle):
        n = int(dec.sum())
        C = float(ctx[dec].sum())
        t_sh = float(self.cm.t_sh(n, self.k, C))
        ratio = np.clip(t_sh / np.maximum(self.cm.t_deep(n * (d + 1), self.k, C, n), 1e-9), 1e-4, 1.0)
        target = expected_token_targets(self.tracker.rate, ratio, self.min_draft, self.d_max)
        lowest = np.where(self.tracker.cold, max(self.min_draft, self.initial_draft), self.min_draft)
        return ready & (d >= np.minimum(np.maximum(target, lowest), self.d_max))

    def _by_target_feedback(self, d, ctx, dec, ready, idle):
        return ready & (d >= np.minimum(self.targets, self.d_max))

    def _by_rate(self, d, ctx, dec, ready, idle):
        if (d[dec] >= self.d_max).any() or idle >= self.sla_steps:
            return ready
        now, later = self.rates(d, ctx, dec, idle)
        return ready if later <= now else np.zeros_like(ready)

    def rates(self, d, ctx, dec, s) -> tuple:
        """(R(s), R(s + 1)): expected tokens per expected time of verifying now (the slots holding drafts read the
        deep layers) and after one more draft for everyone (all live slots verify, contexts one token longer)."""
        dl = d[dec]
        cl = ctx[dec].astype(np.float64)
        rate = self.tracker.rate[dec]
        n, C = len(dl), float(cl.sum())
        t_sh = float(self.cm.t_sh(n, self.k, C))
        holding = dl >= 1
        tokens_now = float(expected_tokens(rate, dl)[holding].sum())
        time_now = s * t_sh + float(self.cm.t_deep(int((dl[holding] + 1).sum()), self.k, C, n,
                                                   C_deep=float(cl[holding].sum())))
        tokens_later = float(expected_tokens(rate, dl + 1).sum())
        time_later = (s + 1) * t_sh + float(self.cm.t_deep(int((dl + 2).sum()), self.k, C + n, n, C_deep=C + n))
        return tokens_now / max(time_now, 1e-9), tokens_later / max(time_later, 1e-9)


def make_scheduler(name: str, B: int, cost_model, k: int, *, gamma: int = 4, d_max: int = 16, sla_steps: int = 32,
                   initial_draft: int = 3, omega: float = 0.8, alpha0: float = 0.9, min_draft: int = 1) -> DraftPolicy:
    """The policy `name` for B slots at exit layer k (the reference's --sched values)."""
    return DraftPolicy(name, B, cost_model, k, gamma=gamma, d_max=d_max, sla_steps=sla_steps,
                       initial_draft=initial_draft, min_draft=min_draft, omega=omega, alpha0=alpha0)
