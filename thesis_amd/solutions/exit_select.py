"""M2: one exit layer for the whole batch, moved at run time by probe measurements (rules of the reference's
solutions/exit_select.py:28-72).

Every `probe_every`-th deep step probes: the verifiers run all of their d + 1 tokens through the shallow layers
again, the hidden state entering every candidate exit layer is captured (shallow candidates in the shallow
segment, deeper ones in the deep segment), the shared final norm + LM head turns each into a greedy token, and
the device counts agreement with the full model's token Y on the positions with a correct prefix (j <= accepted).
The fraction per candidate feeds an exponentially weighted estimate alpha(k).

After each deep step (never while a prompt is half piggybacked) the candidate with the best cost-model rate
max_s B E(alpha, s) / (s t_sh(B, k) + t_deep(B (s + 1), k)) becomes the exit when it beats the current one by
more than `margin`.  Drafts in flight are dropped at a switch; they are guesses, so outputs stay lossless.
Host-only; the match counts arrive with the deep step's single readback.
"""

from __future__ import annotations

from typing import Optional


class ExitController:
    def __init__(self, cost_model, k0: int, cands, probe_every: int = 20, margin: float = 0.05, omega: float = 0.8,
                 d_max: int = 16, force: Optional[str] = None):
        self.cm, self.k, self.d_max = cost_model, int(k0), d_max
        self.cands = sorted({int(c) for c in cands} | {self.k})
        self.period, self.margin, self.weight = probe_every, margin, omega
        self.force = force                     # "cycle": step to the next candidate at every probe (tests)
        self.alpha: dict = dict.fromkeys(self.cands)
        self.n_deep = 0
        self.n_probes = 0
        self.timeline = [(0, self.k)]          # (deep step index, exit layer)
        self.last_rates: dict = {}

    def probe_due(self) -> bool:
        """Whether the coming deep step is a probe."""
        return (self.n_deep + 1) % self.period == 0

    def deep_step_done(self) -> None:
        self.n_deep += 1

    def absorb_probe(self, matches, total: int) -> None:
        """matches[i]: correct-prefix positions (of `total`) on which candidate cands[i] agreed with Y."""
        if total <= 0:
            return
        self.n_probes += 1
        for c, m in zip(self.cands, matches):
            frac = float(m) / float(total)
            old = self.alpha[c]
            self.alpha[c] = frac if old is None else self.weight * old + (1.0 - self.weight) * frac

    def _pick(self, n_live: int, ctx_sum: float) -> Optional[int]:
        if self.force == "cycle":
            if self.n_deep % self.period:
                return None
            return self.cands[(self.cands.index(self.k) + 1) % len(self.cands)]
        measured = {c: a for c, a in self.alpha.items() if a is not None}
        if self.k not in measured or n_live <= 0:
            return None
        self.last_rates = {c: self.cm.best_rate(a, n_live, c, ctx_sum, self.d_max) for c, a in measured.items()}
        best = max(self.last_rates, key=self.last_rates.get)
        if best == self.k or self.last_rates[best] <= (1.0 + self.margin) * self.last_rates[self.k]:
            return None
        return best

    def propose(self, n_live: int, ctx_sum: float, allowed: bool) -> Optional[int]:
        """After a deep step: the new exit layer (the controller switches to it), or None to keep the current."""
        if not allowed or self.n_probes == 0:
            return None
        new = self._pick(n_live, ctx_sum)
        if new is not None:
            self.k = new
            self.timeline.append((self.n_deep, new))
        return new
