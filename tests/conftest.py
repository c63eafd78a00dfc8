"""Shared test setup.  `-m gpu` tests need a HIP device and the built liblsk.so; everything else runs
on the CPU (oracle vs golden vectors, host logic, C-ABI loading and argument validation)."""

from __future__ import annotations

import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built liblsk.so")
    config.addinivalue_line("markers", "slow: long-running")


@pytest.fixture(scope="session")
def cuda():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    return torch.device("cuda:0")


# Small configurations used across tests.  TINY mirrors the reference's test checkpoint
# (tests/conftest.py:19-31 of the reference: 6 layers, vocab 64, hidden 64, FFN 128, 4 q / 2 kv heads);
# SMALL has head_dim 64 so the bf16 MFMA attention path is exercised.
def tiny_cfg(**kw):
    from oracle.model import OracleConfig

    base = dict(vocab_size=64, dim=64, n_layers=6, n_heads=4, n_kv_heads=2, head_dim=16, intermediate_size=128,
                norm_eps=1e-5, rope_theta=10000.0, max_position_embeddings=512)
    base.update(kw)
    return OracleConfig(**base)


def small_cfg(**kw):
    from oracle.model import OracleConfig

    base = dict(vocab_size=512, dim=256, n_layers=4, n_heads=4, n_kv_heads=2, head_dim=64, intermediate_size=512,
                norm_eps=1e-5, rope_theta=10000.0, max_position_embeddings=1024)
    base.update(kw)
    return OracleConfig(**base)


def to_model_config(ocfg):
    from thesis_amd.common.model import ModelConfig

    return ModelConfig(vocab_size=ocfg.vocab_size, dim=ocfg.dim, n_layers=ocfg.n_layers, n_heads=ocfg.n_heads,
                       n_kv_heads=ocfg.n_kv_heads, head_dim=ocfg.head_dim, intermediate_size=ocfg.intermediate_size,
                       norm_eps=ocfg.norm_eps, rope_theta=ocfg.rope_theta,
                       max_position_embeddings=ocfg.max_position_embeddings,
                       tie_word_embeddings=ocfg.tie_word_embeddings, rope_scaling=ocfg.rope_scaling)
