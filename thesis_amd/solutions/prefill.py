"""Prefill placement (the engine's `prefill` option; rules of the reference's solutions/prefill.py:28-77).

separate  a new prompt runs through all layers at once, in pieces of `prefill_chunk` tokens, while the batch waits.
m3        depth-split piggybacking: pieces of a waiting prompt ride on the decode steps.  A piece goes through the
          shallow layers [0, k) in one step's shallow segment (its layer-k states are kept on the device) and
          through [k, L) in the next deep segment, writing its KV in every layer on the way; later pieces attend to
          earlier ones.  The deep pass of the last piece yields the request's first token.

Piece size: the room below the cost model's knee (scaled by `knee_safety`) left by the tokens already in the
shallow segment and by those expected (plus already pending) in the deep segment, capped by `chunk_cap`.
A prompt is piggybacked only if a piece fits, the prompt needs at most `max_wait` pieces and carrying one piece
in both segments costs less than a separate pass over it; otherwise it is prefilled separately and the reason
is counted ("no_room_below_knee", "exceeds_max_wait", "not_cheaper_than_separate").
Host-only (cost-model queries).
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional


@dataclass
class M3Planner:
    cm: object                          # cost model (t_segment, t_prefill, knee, dims)
    max_wait: int = 3
    chunk_cap: Optional[int] = None
    no_knee_chunk: int = 512            # piece size cap when the cost model has no knee (linear models)
    knee_safety: float = 0.9

    def room(self) -> float:
        """Tokens a segment may hold: knee x safety (inf for models without a knee)."""
        return self.cm.knee() * self.knee_safety

    def chunk_budget(self, shallow_tokens: int, deep_tokens_est: int, pending_deep: int) -> int:
        """Largest piece that keeps both segments within the room (>= 0)."""
        cap = self.room()
        if not math.isfinite(cap):
            cap = self.no_knee_chunk + max(shallow_tokens, deep_tokens_est + pending_deep)
        size = int(min(cap - shallow_tokens, cap - deep_tokens_est - pending_deep))
        if self.chunk_cap is not None:
            size = min(size, self.chunk_cap)
        return max(size, 0)

    def admission(self, prompt_len: int, shallow_tokens: int, deep_tokens_est: int, k: int, ctx_sum: float) -> tuple:
        """(piggyback?, reason) for a prompt arriving while `shallow_tokens` slots decode over ctx_sum cached
        positions."""
        piece = min(self.chunk_budget(shallow_tokens, deep_tokens_est, 0), prompt_len)
        if piece <= 0:
            return False, "no_room_below_knee"
        if math.ceil(prompt_len / piece) > self.max_wait:
            return False, "exceeds_max_wait"
        if self.extra_cost(piece, k, shallow_tokens, deep_tokens_est, ctx_sum) >= float(self.cm.t_prefill(piece, piece)):
            return False, "not_cheaper_than_separate"
        return True, "piggyback"

    def extra_cost(self, piece: int, k: int, shallow_tokens: int, deep_tokens: int, ctx_sum: float) -> float:
        """Added time of `piece` prompt tokens in a step's shallow segment (layers [0, k)) and in the next deep
        segment ([k, L)); the piece reads piece cached positions per layer."""
        seg, L = self.cm.t_segment, self.cm.dims.n_layers
        shallow = float(seg(k, shallow_tokens + piece, ctx_sum + piece)) - float(seg(k, shallow_tokens, ctx_sum))
        deep = (float(seg(L - k, deep_tokens + piece, ctx_sum + piece))
                - float(seg(L - k, deep_tokens, ctx_sum)))
        return shallow + deep


def chunk_kv_positions(pos0: int, c: int) -> float:
    """Cached positions one layer's attention reads for the causal piece [pos0, pos0 + c): its prefix once."""
    return float(pos0 + c)


def split_separate(prompt_len: int, chunk: int) -> list:
    """(start, length) pieces of a separate prefill."""
    return [(s, min(chunk, prompt_len - s)) for s in range(0, prompt_len, chunk)] or [(0, 0)]
