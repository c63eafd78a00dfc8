"""Prompts (common/data.py: Prompt), the seeded synthetic prompt pools of the benchmark configurations (token ids
uniform over the vocabulary; no dataset download) and the stop-string rule of a request (StopChecker)."""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np


@dataclass
class Prompt:
    pid: str
    tokens: list


def synthetic_prompts(n: int, vocab: int, min_len: int, max_len: int, seed: int = 0, lo: int = 0) -> list:
    """n prompts, lengths uniform in [min_len, max_len], ids uniform in [lo, vocab)."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        L = int(rng.integers(min_len, max_len + 1))
        out.append(Prompt(pid=f"p{i}", tokens=rng.integers(lo, vocab, size=L).tolist()))
    return out


class StopChecker:
    """Stop strings over a request's generated tokens (the stop rule of common/data.py:289-313).

    checker(output, n_new) -> the length to cut `output` to, or None: the shortest prefix that ends inside the
    `n_new` tokens just committed and whose decoded text contains a stop string (the token that completes it is
    kept, as an autoregressive run with this rule would stop there).  Only the last `window` tokens before the
    commit, plus the commit, are decoded, so a check costs the same however long the output is."""

    def __init__(self, tokenizer, stops, window: int = 24):
        self.tokenizer = tokenizer
        self.stops = tuple(s for s in stops if s)
        self.window = window

    def __bool__(self) -> bool:
        return bool(self.stops)

    def _has_stop(self, ids: list) -> bool:
        text = self.tokenizer.decode(ids, skip_special_tokens=False)
        return any(s in text for s in self.stops)

    def __call__(self, output: list, n_new: int):
        first_new = len(output) - n_new
        if not self._has_stop(output[max(first_new - self.window, 0):]):
            return None
        for end in range(first_new + 1, len(output) + 1):
            if self._has_stop(output[max(end - n_new - self.window, 0):end]):
                return end
        return len(output)
