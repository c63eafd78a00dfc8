"""Prefill policies (solutions/prefill.py surface).

separate  the batch pauses while a new prompt runs through all layers in chunks of `prefill_chunk` tokens.
m3        depth-split piggybacking: a chunk of a pending prompt rides on a step's shallow segment (layers [0, k);
          its layer-k hidden state is kept) and on the deep segment of the next deep step (layers [k, L)), writing
          KV in every layer as it passes; later chunks attend to earlier ones.  The last chunk's deep pass gives the
          first generated token.
          chunk size  c = min(remaining, knee * s - shallow tokens, knee * s - expected deep tokens - pending deep
          tokens), knee = the cost model's knee, s = knee_safety; at assignment a prompt piggybacks only when
          c > 0, it needs at most `max_wait` deep steps and the marginal cost of carrying c tokens in both segments
          is below a separate pass (solutions/prefill.py:28-64).

Host-only (cost-model queries).
"""

from __future__ import annotations

import math
from typing import Optional


class M3Planner:
    def __init__(self, cost_model, max_wait: int = 3, chunk_cap: Optional[int] = None, no_knee_chunk: int = 512,
                 knee_safety: float = 0.9):
        self.cm, self.max_wait, self.chunk_cap = cost_model, max_wait, chunk_cap
        self.no_knee_chunk = no_knee_chunk   # cost models without a knee (linear) cap the chunk here instead
        self.knee_safety = knee_safety

    def knee(self) -> float:
        return self.cm.knee() * self.knee_safety

    def budget(self, n_sh: int, n_deep_est: int, pending_deep: int) -> int:
        knee = self.knee()
        if not math.isfinite(knee):
            knee = self.no_knee_chunk + max(n_sh, n_deep_est + pending_deep)
        c = int(min(knee - n_sh, knee - n_deep_est - pending_deep))
        if self.chunk_cap is not None:
            c = min(c, self.chunk_cap)
        return max(c, 0)

    def admit(self, prompt_len: int, n_sh: int, n_deep_est: int, k: int, C: float) -> tuple:
        """(piggyback?, reason) for a prompt assigned while n_sh slots decode (C cached positions)."""
        c = min(self.budget(n_sh, n_deep_est, 0), prompt_len)
        if c <= 0:
            return False, "no_room_below_knee"
        if math.ceil(prompt_len / c) > self.max_wait:
            return False, "exceeds_max_wait"
        if not self.worth_it(c, k, n_sh, C, n_deep_est, C, float(c)):
            return False, "not_cheaper_than_separate"
        return True, "piggyback"

    def worth_it(self, c: int, k: int, n_sh: int, C_sh: float, n_dp: int, C_dp: float, C_chunk: float) -> bool:
        """Marginal time of c more tokens in both segments < time of a separate pass over them."""
        L = self.cm.dims.n_layers
        seg = self.cm.t_segment
        dt = (float(seg(k, n_sh + c, C_sh + C_chunk)) - float(seg(k, n_sh, C_sh))
              + float(seg(L - k, n_dp + c, C_dp + C_chunk)) - float(seg(L - k, n_dp, C_dp)))
        return dt < float(self.cm.t_prefill(c, C_chunk))


def chunk_kv_positions(pos0: int, c: int) -> float:
    """Cached positions a causal chunk [pos0, pos0 + c) reads per layer (the prefix once per query block)."""
    return float(pos0 + c)


def split_separate(prompt_len: int, chunk: int) -> list:
    """(start, length) chunks of a separate chunked prefill."""
    return [(s, min(chunk, prompt_len - s)) for s in range(0, prompt_len, chunk)] or [(0, 0)]
