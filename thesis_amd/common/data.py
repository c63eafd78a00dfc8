"""Prompts (common/data.py: Prompt) and the seeded synthetic prompt pools of the benchmark
configurations (token ids uniform over the vocabulary; no dataset download)."""

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
