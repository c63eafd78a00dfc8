"""The method registry's engines on the GPU (common/methods.py, common/engine.py surface).

ARBatchEngine / SyncSpecEngine step through the padded per-call path (make_ctx / forward_layers) of the
native model; "eesd" is the packed EESDEngine behind the DecodeEngine contract.  fp32: tokens equal to
the oracle's AR decode; bf16: every method produces the AR tokens (greedy speculation is lossless).
"""

from __future__ import annotations

import argparse

import pytest
import torch

from conftest import small_cfg, tiny_cfg, to_model_config

pytestmark = pytest.mark.gpu


def _model(ocfg, dtype, std=0.1):
    from oracle.model import OracleLlama, random_weights
    from thesis_amd.common.model import LayerSkipLlama

    w = random_weights(ocfg, seed=0, std=std)
    return OracleLlama(ocfg, w, dtype=dtype, max_seq=1024), \
        LayerSkipLlama.from_weights(to_model_config(ocfg), w, device="cuda", dtype=dtype, max_seq=1024)


def _prompts(n, vocab, seed=3):
    from thesis_amd.common.data import synthetic_prompts

    return synthetic_prompts(n, vocab, 5, 20, seed=seed)


def _args(**kw):
    base = dict(max_new_tokens=24, ignore_eos=True, temperature=0.0, top_k=0, top_p=1.0, seed=0, exit_layer=2,
                gamma=3, sched="fixed", k=None, d_max=6, min_draft=1, eesd_gamma=3, cost_model=None,
                forced_accept_p=None)
    base.update(kw)
    return argparse.Namespace(**base)


def _run(name, g, prompts, B, **kw):
    from thesis_amd.common.engine import RunConfig
    from thesis_amd.common.methods import METHODS, load_plugins

    load_plugins()
    eng = METHODS[name].build(g, _args(**kw), B, 24, ())
    res = eng.run(prompts, RunConfig(mode="static", keep_outputs=True))
    return {c["pid"]: c["tokens"] for c in res["completions"]}, res


@pytest.mark.parametrize("which", ["tiny", "small"])
def test_registry_engines_fp32_match_oracle(cuda, which):
    from oracle.engine import OracleEngine

    ocfg = tiny_cfg() if which == "tiny" else small_cfg()
    o, g = _model(ocfg, torch.float32)
    prompts = _prompts(5, ocfg.vocab_size)
    ref = OracleEngine(o, 3, 24, 24, mode="ar").run_static([(p.pid, p.tokens) for p in prompts])
    ar, res = _run("autoregressive", g, prompts, 3)
    assert ar == ref
    sp, res_sp = _run("sync_layerskip", g, prompts, 3)
    assert sp == ref
    m = res_sp["metrics"]
    assert m["evaluated_completions"] == 5 and m["stop_reason"] == "pool_exhausted"
    assert 0.0 <= m["spec"]["acceptance_rate"] <= 1.0 and m["spec"]["tokens_per_verify"] >= 1.0


def test_registry_methods_are_lossless_in_bf16(cuda):
    ocfg = small_cfg()
    _, g = _model(ocfg, torch.bfloat16)
    prompts = _prompts(6, ocfg.vocab_size, seed=4)
    ar, res = _run("autoregressive", g, prompts, 3)
    sp, _ = _run("sync_layerskip", g, prompts, 3, gamma=4)
    ee, res_e = _run("eesd", g, prompts, 3, sched="aspire")
    assert sp == ar
    assert ee == ar
    m = res_e["metrics"]
    for key in ("throughput_tok_s", "wall_throughput_tok_s", "mean_tpot_ms", "evaluated_completions",
                "stop_reason"):
        assert key in m
    assert m["throughput_tok_s"] > 0 and m["spec"]["tokens_per_verify"] >= 1.0
    for c in res_e["completions"]:
        assert c["generated"] == 24 and c["finish_reason"] == "length"
