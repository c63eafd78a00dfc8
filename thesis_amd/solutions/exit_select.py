"""M2: a batch-shared exit layer chosen at run time from probe measurements (solutions/exit_select.py surface).

Every `probe_every`-th deep step is a probe: the verifying requests run all of their d + 1 tokens through the
shallow layers again, the hidden state entering every candidate exit layer is captured (shallow candidates in the
shallow segment, deeper ones in the deep segment), the shared final norm + LM head is applied to each, and its
greedy token is compared with the full model's token Y at the positions whose prefix is correct (j <= accepted).
The per-candidate match fraction feeds an EMA alpha(k).  After each deep step without a half-done prefill, the
candidate with the best cost-model rate max_s B E(alpha, s) / (s t_sh(B, k) + t_deep(B (s + 1), k)) replaces the
current exit when it beats it by more than `margin` (solutions/exit_select.py:28-72).  A switch drops the drafts in
flight (they are guesses; outputs stay lossless).

Host-only; the probe's match counts come back in the deep step's single readback.
"""

from __future__ import annotations

from typing import Optional


class ExitController:
    def __init__(self, cost_model, k0: int, cands, probe_every: int = 20, margin: float = 0.05, omega: float = 0.8,
                 d_max: int = 16, force: Optional[str] = None):
        self.cm, self.k = cost_model, int(k0)
        self.cands = sorted({int(c) for c in cands} | {int(k0)})
        self.probe_every, self.margin, self.omega, self.d_max = probe_every, margin, omega, d_max
        self.alpha = {c: None for c in self.cands}
        self.deep_steps = 0
        self.probes = 0
        self.timeline = [(0, self.k)]        # (deep step index, exit layer)
        self.force = force                   # "cycle": move to the next candidate at every probe (tests)
        self.last_rates: dict = {}

    def want_probe(self) -> bool:
        return (self.deep_steps + 1) % self.probe_every == 0

    def after_deep_step(self) -> None:
        self.deep_steps += 1

    def observe_probe(self, matches, total: int) -> None:
        """matches[i]: tokens on which candidate cands[i] agrees with Y among `total` correct-prefix positions."""
        if total <= 0:
            return
        self.probes += 1
        for c, m in zip(self.cands, matches):
            a = float(m) / float(total)
            prev = self.alpha[c]
            self.alpha[c] = a if prev is None else self.omega * prev + (1.0 - self.omega) * a

    def maybe_switch(self, B: int, C: float, can_switch: bool) -> Optional[int]:
        """After a deep step: the new exit layer, or None to keep the current one."""
        if not can_switch or self.probes == 0:
            return None
        if self.force == "cycle":
            if self.deep_steps % self.probe_every:
                return None
            new = self.cands[(self.cands.index(self.k) + 1) % len(self.cands)]
        else:
            known = {c: a for c, a in self.alpha.items() if a is not None}
            if self.k not in known or B <= 0:
                return None
            per_req = C / max(B, 1)
            self.last_rates = {c: self.cm.best_rate(a, B, c, B * per_req, self.d_max) for c, a in known.items()}
            new = max(self.last_rates, key=self.last_rates.get)
            if new == self.k or self.last_rates[new] <= (1.0 + self.margin) * self.last_rates[self.k]:
                return None
        self.k = new
        self.timeline.append((self.deep_steps, new))
        return new
