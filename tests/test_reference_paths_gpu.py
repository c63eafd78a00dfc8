"""Token identity with the reference path and the reference's stop rules on the MI355X engine (GPU).

  * config 1 (Llama3.2-1B shape, fp32, B = 4, prompts U[16, 128], 64 new tokens, exit 4, draft 4): the GPU
    engine's speculative and autoregressive tokens equal the CPU oracle engine's autoregressive tokens (the
    reference's lossless gate, solutions/check_lossless.py:102-105: fp32 tokens identical)
  * EOS inside a multi-token commit (tests/test_engine.py:72-82 of the reference)
  * a stop string completed inside a speculative commit (tests/test_engine.py:108-125)
  * pad bucketing with the cyclic driver (tests/test_eesd.py:71-78)
fp32 runs compare with oracle.engine.OracleEngine's autoregressive tokens (the stop-string expectation is those
tokens cut after the first stop token, the rule's closed form); bf16 runs compare speculation with this engine's
own autoregressive decoding.
"""

from __future__ import annotations

import gc

import pytest
import torch

from conftest import small_cfg, tiny_cfg, to_model_config

pytestmark = pytest.mark.gpu

F32, BF16 = torch.float32, torch.bfloat16
MAX_NEW = 30
BASE = dict(k=2, d_max=6, gamma=3)


@pytest.fixture(autouse=True)
def _free_models():
    yield
    gc.collect()
    torch.cuda.empty_cache()


def _prompts(n, vocab, lo=5, hi=20, seed=3):
    from thesis_amd.common.data import synthetic_prompts

    return synthetic_prompts(n, vocab, lo, hi, seed=seed)


def _outputs(res):
    return {c["pid"]: c["tokens"] for c in res["completions"]}


def _eesd(g, B, max_prompt, max_new, eos=(), stop_for=None, **kw):
    from thesis_amd.solutions.cost_model import synthetic_cost_model
    from thesis_amd.solutions.engine import EESDEngine, EngineConfig

    return EESDEngine(g, B, max_prompt, max_new, eos, EngineConfig(**{**BASE, **kw}), synthetic_cost_model(g.cfg),
                      stop_for=stop_for)


def _oracle_ar(o, prompts, B, max_prompt, max_new, eos=()):
    from oracle.engine import OracleEngine

    return OracleEngine(o, B, max_prompt, max_new, mode="ar", eos=eos).run_static([(p.pid, p.tokens) for p in prompts])


@pytest.fixture(scope="module")
def tiny_fp32(cuda):
    from oracle.model import OracleLlama, random_weights
    from thesis_amd.common.model import LayerSkipLlama

    ocfg = tiny_cfg()
    w = random_weights(ocfg, seed=0, std=0.1)
    g = LayerSkipLlama.from_weights(to_model_config(ocfg), w, device="cuda", dtype=F32, max_seq=512)
    o = OracleLlama(ocfg, w, dtype=F32, max_seq=512)
    prompts = _prompts(7, ocfg.vocab_size)
    return g, o, prompts, _oracle_ar(o, prompts, 3, 24, MAX_NEW)


# ----------------------------------------------------------------------------- config 1 against the oracle

def _hf_weights(g) -> dict:
    """The GPU model's fp32 weights as HF-named CPU tensors (q / k / v and gate / up split back out)."""
    c = g.cfg
    qd, kvd = c.n_heads * c.head_dim, c.n_kv_heads * c.head_dim
    w = {"model.embed_tokens.weight": g.embed_w.cpu(), "model.norm.weight": g.norm_w.cpu(),
         "lm_head.weight": g.lm_head_w.cpu()}
    for i, lw in enumerate(g.layers):
        p = f"model.layers.{i}."
        qkv = lw.wqkv.cpu()
        w[p + "self_attn.q_proj.weight"] = qkv[:qd]
        w[p + "self_attn.k_proj.weight"] = qkv[qd:qd + kvd]
        w[p + "self_attn.v_proj.weight"] = qkv[qd + kvd:]
        w[p + "self_attn.o_proj.weight"] = lw.wo.cpu()
        w13 = lw.w13.cpu()
        w[p + "mlp.gate_proj.weight"] = w13[:c.intermediate_size]
        w[p + "mlp.up_proj.weight"] = w13[c.intermediate_size:]
        w[p + "mlp.down_proj.weight"] = lw.w2.cpu()
        w[p + "input_layernorm.weight"] = lw.attn_norm.cpu()
        w[p + "post_attention_layernorm.weight"] = lw.ffn_norm.cpu()
    return w


def test_config1_llama32_1b_fp32_tokens_equal_the_oracle_engine(cuda):
    """Config 1 at its real shape: 1B fp32 random init (HF-style N(0, 0.02)), B = 4, prompts U[16, 128], 64 new
    tokens, exit layer 4, draft length 4.  The CPU oracle engine decodes autoregressively on the host; the GPU
    engine's autoregressive and speculative (fixed, gamma 4) runs give the same tokens, as does the registry's
    synchronous LayerSkip engine."""
    from oracle.model import OracleConfig, OracleLlama
    from thesis_amd.common.engine import RunConfig, SyncSpecEngine
    from thesis_amd.common.model import PRESETS, LayerSkipLlama

    c = PRESETS["llama3.2-1b"]
    g = LayerSkipLlama.random(c, seed=0, dtype=F32, max_seq=256)
    ocfg = OracleConfig(vocab_size=c.vocab_size, dim=c.dim, n_layers=c.n_layers, n_heads=c.n_heads,
                        n_kv_heads=c.n_kv_heads, head_dim=c.head_dim, intermediate_size=c.intermediate_size,
                        norm_eps=c.norm_eps, rope_theta=c.rope_theta, max_position_embeddings=c.max_position_embeddings,
                        tie_word_embeddings=c.tie_word_embeddings, rope_scaling=c.rope_scaling)
    o = OracleLlama(ocfg, _hf_weights(g), dtype=F32, max_seq=256)
    prompts = _prompts(4, c.vocab_size, 16, 128, seed=11)
    ref = _oracle_ar(o, prompts, 4, 128, 64)
    print("oracle engine done:", {k: v[:6] for k, v in ref.items()}, flush=True)
    del o
    gc.collect()
    ar = _outputs(_eesd(g, 4, 128, 64, mode="ar", k=4).run(prompts, "static", keep_outputs=True))
    sp_eng = _eesd(g, 4, 128, 64, sched="fixed", k=4, gamma=4, d_max=4)
    sp = _outputs(sp_eng.run(prompts, "static", keep_outputs=True))
    sync = _outputs(SyncSpecEngine(g, 4, 128, 64, (), exit_layer=4, gamma=4).run(
        prompts, RunConfig(mode="static", keep_outputs=True)))
    assert all(len(v) == 64 for v in ref.values())
    assert ar == ref
    assert sp == ref and sp_eng.stats["deep_steps"] > 0
    assert sync == ref


# ----------------------------------------------------------------------------- EOS inside a commit

def test_eos_inside_a_speculative_commit(tiny_fp32):
    """An EOS id that the speculative run commits inside a multi-token commit ends the request there, as the
    autoregressive run does (tests/test_engine.py:72-82): EESD, SyncSpec and AR on the GPU against the oracle
    engine decoding with the same EOS."""
    from thesis_amd.common.engine import ARBatchEngine, RunConfig, SyncSpecEngine

    g, o, prompts, ref = tiny_fp32
    eos = ref["p0"][5]
    want = _oracle_ar(o, prompts, 3, 24, MAX_NEW, eos=(eos,))
    assert want["p0"][-1] == eos and len(want["p0"]) <= 6
    assert want != ref
    cfg = RunConfig(mode="static", keep_outputs=True)
    ee = _outputs(_eesd(g, 3, 24, MAX_NEW, eos=(eos,), sched="fixed", gamma=4).run(prompts, "static",
                                                                                  keep_outputs=True))
    ar = _outputs(ARBatchEngine(g, 3, 24, MAX_NEW, (eos,)).run(prompts, cfg))
    sp = _outputs(SyncSpecEngine(g, 3, 24, MAX_NEW, (eos,), exit_layer=3, gamma=4).run(prompts, cfg))
    assert ee == want and ar == want and sp == want


def test_eos_inside_a_speculative_commit_bf16(cuda):
    from oracle.model import random_weights
    from thesis_amd.common.model import LayerSkipLlama

    ocfg = small_cfg()
    g = LayerSkipLlama.from_weights(to_model_config(ocfg), random_weights(ocfg, seed=1, std=0.1), device="cuda",
                                    dtype=BF16, max_seq=512)
    prompts = _prompts(7, ocfg.vocab_size, seed=5)
    base = _outputs(_eesd(g, 3, 24, MAX_NEW, mode="ar").run(prompts, "static", keep_outputs=True))
    eos = base["p0"][4]
    ar = _outputs(_eesd(g, 3, 24, MAX_NEW, eos=(eos,), mode="ar").run(prompts, "static", keep_outputs=True))
    sp = _outputs(_eesd(g, 3, 24, MAX_NEW, eos=(eos,), sched="aspire").run(prompts, "static", keep_outputs=True))
    assert ar["p0"][-1] == eos and len(ar["p0"]) <= 5
    assert sp == ar


# ----------------------------------------------------------------------------- stop strings

class _ToyTokenizer:
    """decode(ids): one character per id; ids in `nl` decode to a newline."""

    def __init__(self, nl):
        self.nl = set(nl)

    def decode(self, ids, skip_special_tokens=False):
        return "".join("\n" if i in self.nl else chr(65 + i % 26) for i in ids)


@pytest.mark.parametrize("k,gamma", [(2, 3), (4, 6)])
def test_stop_string_inside_a_speculative_commit(tiny_fp32, k, gamma):
    """A stop string completed inside a multi-token commit truncates the speculative output exactly where the
    autoregressive run stops (tests/test_engine.py:108-125): with "\\n" the output ends at its first newline token,
    which it keeps.  EESD (per-request checker), SyncSpec and AR (the DecodeEngine's checker) on the GPU."""
    from thesis_amd.common.data import StopChecker
    from thesis_amd.common.engine import ARBatchEngine, RunConfig, SyncSpecEngine

    g, o, prompts, ref = tiny_fp32
    nl = {ref["p0"][7], ref["p2"][11]}
    sc = StopChecker(_ToyTokenizer(nl), ("\n",))
    want = {}
    for pid, toks in ref.items():
        cut = next((i + 1 for i, t in enumerate(toks) if t in nl), len(toks))
        want[pid] = toks[:cut]
    assert len(want["p0"]) <= 8 and want != ref
    res = _eesd(g, 3, 24, MAX_NEW, stop_for=lambda pid: sc, sched="fixed", k=k, gamma=gamma).run(
        prompts, "static", keep_outputs=True)
    assert _outputs(res) == want
    assert any(c["finish_reason"] == "stop" for c in res["completions"])
    cfg = RunConfig(mode="static", keep_outputs=True)
    ar = ARBatchEngine(g, 3, 24, MAX_NEW, ())
    ar.stop_checker = sc
    sp = SyncSpecEngine(g, 3, 24, MAX_NEW, (), exit_layer=k, gamma=gamma)
    sp.stop_checker = sc
    assert _outputs(ar.run(prompts, cfg)) == want
    assert _outputs(sp.run(prompts, cfg)) == want


# ----------------------------------------------------------------------------- pad bucketing + cyclic driver

@pytest.mark.parametrize("sched", ["fixed", "aspire", "m1"])
def test_pad_bucketing_and_cyclic_driver_are_lossless(tiny_fp32, sched):
    """build_packed's "pad" accounting and the cyclic driver (refilled slots, warm-up, measured window) with M3
    prefill chunks (tests/test_eesd.py:71-78): every completion of the replay equals the oracle engine's tokens."""
    g, _, prompts, ref = tiny_fp32
    res = _eesd(g, 3, 24, MAX_NEW, sched=sched, bucketing="pad", prefill="m3", max_wait=100, m3_chunk_cap=3,
                probe_every=2).run(prompts, "cyclic", warmup_samples=2, warmup_per_slot=0, min_eval=4,
                                   min_eval_per_slot=0, max_eval=10, keep_outputs=True)
    out = res["completions"]
    assert len(out) >= 10
    assert all(c["tokens"] == ref[c["pid"]] for c in out)


def test_pad_bucketing_and_cyclic_driver_are_lossless_bf16(cuda):
    from oracle.model import random_weights
    from thesis_amd.common.model import LayerSkipLlama

    ocfg = small_cfg()
    g = LayerSkipLlama.from_weights(to_model_config(ocfg), random_weights(ocfg, seed=2, std=0.1), device="cuda",
                                    dtype=BF16, max_seq=512)
    prompts = _prompts(7, ocfg.vocab_size, seed=6)
    ar = _outputs(_eesd(g, 3, 24, MAX_NEW, mode="ar").run(prompts, "static", keep_outputs=True))
    res = _eesd(g, 3, 24, MAX_NEW, sched="aspire", bucketing="pad", prefill="m3", max_wait=100, m3_chunk_cap=3).run(
        prompts, "cyclic", warmup_samples=2, warmup_per_slot=0, min_eval=4, min_eval_per_slot=0, max_eval=10,
        keep_outputs=True)
    assert len(res["completions"]) >= 10
    assert all(c["tokens"] == ar[c["pid"]] for c in res["completions"])
