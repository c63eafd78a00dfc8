"""M2 (run-time exit layer from probe steps) and M3 (prefill chunks piggybacked on decode steps) on the MI355X
engine: losslessness of every scheduler x exit x prefill combination and the mechanisms' own invariants
(tests/test_eesd.py:55-97, 174-196, 340-363 of the reference).

fp32 runs compare against the CPU oracle's autoregressive tokens; bf16 runs against this engine's own
autoregressive tokens (the batch-invariant kernels make speculation lossless in bf16 as well).
"""

from __future__ import annotations

import itertools

import pytest
import torch

from conftest import small_cfg, tiny_cfg, to_model_config

pytestmark = pytest.mark.gpu

MAX_NEW = 30
BASE = dict(k=2, d_max=6, gamma=3, probe_every=2, k_cands=(1, 2, 3, 4, 5), max_wait=100, m3_chunk_cap=3)


def _prompts(n, vocab, seed=3):
    from thesis_amd.common.data import synthetic_prompts

    return synthetic_prompts(n, vocab, 5, 20, seed=seed)


def _gpu_model(ocfg, dtype, seed=0):
    from oracle.model import random_weights
    from thesis_amd.common.model import LayerSkipLlama

    w = random_weights(ocfg, seed=seed, std=0.1)
    return LayerSkipLlama.from_weights(to_model_config(ocfg), w, device="cuda", dtype=dtype, max_seq=512), w


def _engine(g, cm=None, B=3, **kw):
    from thesis_amd.solutions.cost_model import synthetic_cost_model
    from thesis_amd.solutions.engine import EESDEngine, EngineConfig

    cfg = EngineConfig(**{**BASE, **kw})
    return EESDEngine(g, B, 24, MAX_NEW, (), cfg, cm if cm is not None else synthetic_cost_model(g.cfg))


def _outputs(res):
    return {c["pid"]: c["tokens"] for c in res["completions"]}


@pytest.fixture(scope="module")
def fp32_setup(cuda):
    from oracle.engine import OracleEngine
    from oracle.model import OracleLlama

    ocfg = tiny_cfg()
    g, w = _gpu_model(ocfg, torch.float32)
    o = OracleLlama(ocfg, w, dtype=torch.float32, max_seq=512)
    prompts = _prompts(7, ocfg.vocab_size)
    ref = OracleEngine(o, 3, 24, MAX_NEW, mode="ar").run_static([(p.pid, p.tokens) for p in prompts])
    return g, prompts, ref


@pytest.fixture(scope="module")
def bf16_setup(cuda):
    ocfg = small_cfg(n_layers=6)
    g, _ = _gpu_model(ocfg, torch.bfloat16, seed=1)
    prompts = _prompts(7, ocfg.vocab_size, seed=4)
    ref = _outputs(_engine(g, mode="ar").run(prompts, "static", keep_outputs=True))
    return g, prompts, ref


COMBOS = list(itertools.product(["fixed", "aspire", "m1"], ["fixed", "m2"], ["separate", "m3"]))


@pytest.mark.parametrize("sched,exit_,prefill", COMBOS)
def test_every_combination_is_lossless_fp32(fp32_setup, sched, exit_, prefill):
    g, prompts, ref = fp32_setup
    res = _engine(g, sched=sched, exit=exit_, prefill=prefill,
                  m2_force="cycle" if exit_ == "m2" else None).run(prompts, "static", keep_outputs=True)
    assert _outputs(res) == ref


@pytest.mark.parametrize("sched,exit_,prefill", [("aspire", "m2", "m3"), ("m1", "m2", "separate"),
                                                 ("fixed", "fixed", "m3")])
def test_mechanisms_are_lossless_bf16(bf16_setup, sched, exit_, prefill):
    g, prompts, ref = bf16_setup
    res = _engine(g, sched=sched, exit=exit_, prefill=prefill,
                  m2_force="cycle" if exit_ == "m2" else None).run(prompts, "static", keep_outputs=True)
    assert _outputs(res) == ref


def test_exit_switch_keeps_outputs(fp32_setup):
    g, prompts, ref = fp32_setup
    res = _engine(g, sched="m1", exit="m2", m2_force="cycle").run(prompts, "static", keep_outputs=True)
    ks = {k for _, k in res["metrics"]["k_timeline"]}
    assert len(ks) >= 3, "the forced cycle must actually switch the exit layer"
    assert _outputs(res) == ref


def test_m2_probe_estimates_are_probabilities(fp32_setup):
    g, prompts, _ = fp32_setup
    res = _engine(g, sched="fixed", exit="m2").run(prompts, "static")
    alpha = res["metrics"]["k_alpha"]
    assert res["metrics"]["probe_steps"] > 0
    assert all(a is None or 0.0 <= a <= 1.0 for a in alpha.values())
    assert any(a is not None for a in alpha.values())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_piggyback_prefill_writes_the_same_kv_as_a_normal_prefill(cuda, dtype):
    """A prompt carried in 3-token chunks through the shallow and deep segments leaves the same KV in every
    layer as a separate prefill of the same prompt, and its first token is the prefill's greedy token
    (bitwise in bf16 too: every kernel's result is independent of how tokens are grouped)."""
    from thesis_amd.solutions.engine import DECODE, PREFILL, Request

    ocfg = tiny_cfg() if dtype == torch.float32 else small_cfg(n_layers=6)
    g, _ = _gpu_model(ocfg, dtype, seed=2)
    prompts = _prompts(5, ocfg.vocab_size, seed=8)
    eng = _engine(g, sched="m1", prefill="m3", m3_chunk_cap=3)
    eng.assign(0, Request(prompts[0].pid, list(prompts[0].tokens)))       # decoding slot (separate prefill)
    p = max(prompts[1:], key=lambda q: len(q.tokens))
    eng.assign(1, Request(p.pid, list(p.tokens)))
    assert eng.state[1] == PREFILL, "the request must be piggybacked"
    n_steps = 0
    while eng.state[1] == PREFILL:
        eng.step()
        n_steps += 1
        assert n_steps < 60
    assert eng.req[1].piggybacked == len(p.tokens) > 3
    logits, _ = g.prefill(list(p.tokens), 2)                              # reference into the free row 2
    n = len(p.tokens)
    for layer in range(g.n_layers):
        k1, k2 = g.cache.k[layer][1, :, :n], g.cache.k[layer][2, :, :n]
        v1, v2 = g.cache.v[layer][1, :, :n], g.cache.v[layer][2, :, :n]
        if dtype == torch.float32:
            assert torch.allclose(k1, k2, atol=1e-5) and torch.allclose(v1, v2, atol=1e-5)
        else:
            assert torch.equal(k1, k2) and torch.equal(v1, v2)
    assert eng.req[1].out[0] == int(logits.float().argmax())
    assert eng.state[1] == DECODE


@pytest.mark.parametrize("safety", [0.5, 0.9])
def test_m3_chunks_respect_measured_knee(fp32_setup, safety):
    """Every step carrying a chunk keeps its shallow segment within knee * safety tokens (flush steps without a
    decoding slot are exempt), and outputs stay lossless (tests/test_eesd.py:340-363)."""
    from thesis_amd.solutions.cost_model import synthetic_cost_model

    g, prompts, ref = fp32_setup
    cm = synthetic_cost_model(g.cfg)
    cm.gpu.knee_measured = 12.0
    eng = _engine(g, cm=cm, sched="m1", prefill="m3", m3_chunk_cap=None, knee_safety=safety)
    res = eng.run(prompts, "static", keep_outputs=True)
    assert _outputs(res) == ref
    carried = [r for r in eng.records if r.n_chunk > 0 and r.kind != "prefill"]
    assert carried, "some chunk must actually be piggybacked"
    bound = 12.0 * safety
    dec_only = [r for r in carried if r.n_sh - r.n_chunk > 0]
    assert all(r.n_sh <= bound for r in dec_only), [(r.n_sh, r.n_chunk) for r in dec_only]
