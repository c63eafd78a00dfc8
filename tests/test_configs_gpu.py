"""The engine at the benchmark configurations' real model shapes (random init, synthetic prompts): speculation
is lossless token for token against autoregressive decoding of the same model, in every configuration.

  config 1  Llama3.2-1B shape, fp32, B = 4, prompts U[16, 128], 64 new tokens, exit 4, draft 4
  config 3  Llama3.2-1B shape, bf16, B = 64, prompts of 512, exit 6, draft 6 (32 new tokens here; the forced
            geometric acceptance run's tokens are checked against a teacher-forced prefill)
  config 4  Llama3-8B shape, bf16, B = 32, prompts U[128, 1024], exit 8, aspire drafts in [2, 8] (24 new tokens);
            with the benchmark's forced acceptance (p = 0.3) every committed token is checked against a
            teacher-forced prefill
  config 2  isolated verify attention + KV append + rollback at the microbenchmark's exact inputs: 256
            requests, GQA 32/8, head_dim 128, bf16 cache, lognormal contexts (median 1500, sigma 0.5, clipped to
            [64, 8192]), 1-9 query rows each, the production split (bench.AttentionInputs) and 4096-position splits
  config 5  Llama2-7B shape (MHA, vocab 32000), bf16, exit 8, draft 4, 256-token prefill chunks piggybacked on
            the decode steps (M3); 16 slots and 24 requests of U[256, 1024] prompt tokens, 16 new tokens each,
            and the open-loop driver at B = 128 with Poisson arrivals at 8 requests/s
The reference's own check for these paths is spec == AR (tests/test_eesd.py:55-97); the oracle comparisons of
the same code paths run at small shapes in the other test files.
"""

from __future__ import annotations

import gc
import math

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _free_models():
    yield
    gc.collect()
    torch.cuda.empty_cache()


def _model(preset: str, dtype, max_seq: int, seed: int = 0):
    from thesis_amd.common.model import PRESETS, LayerSkipLlama

    return LayerSkipLlama.random(PRESETS[preset], seed=seed, dtype=dtype, max_seq=max_seq)


def _prompts(n, vocab, lo, hi, seed):
    from thesis_amd.common.data import synthetic_prompts

    return synthetic_prompts(n, vocab, lo, hi, seed=seed)


def _run(model, prompts, B, max_prompt, max_new, cost_model=None, **kw):
    from thesis_amd.solutions.cost_model import default_cost_model
    from thesis_amd.solutions.engine import EESDEngine, EngineConfig

    cm = cost_model if cost_model is not None else default_cost_model(model.cfg)[0]
    eng = EESDEngine(model, B, max_prompt, max_new, (), EngineConfig(**kw), cm)
    res = eng.run(prompts, "static", keep_outputs=True)
    return {c["pid"]: c["tokens"] for c in res["completions"]}, eng, res


def test_config1_llama32_1b_fp32_spec_equals_ar(cuda):
    m = _model("llama3.2-1b", torch.float32, 256)
    prompts = _prompts(4, m.cfg.vocab_size, 16, 128, seed=11)
    ar, _, _ = _run(m, prompts, 4, 128, 64, mode="ar", k=4)
    sp, eng, res = _run(m, prompts, 4, 128, 64, sched="fixed", k=4, gamma=4, d_max=4)
    assert sp == ar
    assert all(len(v) == 64 for v in sp.values())
    assert eng.stats["deep_steps"] > 0


def test_config3_llama32_1b_bf16_b64(cuda):
    m = _model("llama3.2-1b", torch.bfloat16, 640)
    prompts = _prompts(64, m.cfg.vocab_size, 512, 512, seed=12)
    ar, _, _ = _run(m, prompts, 64, 512, 32, mode="ar", k=6)
    sp, _, _ = _run(m, prompts, 64, 512, 32, sched="fixed", k=6, gamma=6, d_max=6)
    assert sp == ar
    # forced geometric acceptance (p = 0.3): ragged verify rows and rollbacks; every request finishes with its
    # 32 tokens and its cache pointer at prompt + generated - 1
    fo, eng, _ = _run(m, prompts, 64, 512, 32, sched="fixed", k=6, gamma=6, d_max=6, forced_accept_p=0.3,
                      forced_seed=3)
    assert all(len(v) == 32 for v in fo.values())
    assert eng.stats["accepted"] < eng.stats["drafted"]          # drafts were rejected and rolled back
    # every forced-run token is the exit head's or the full model's greedy token after its own prefix
    _check_forced_tokens(m, prompts, fo, 6)


def test_config4_llama3_8b_bf16_aspire(cuda):
    m = _model("llama3-8b", torch.bfloat16, 1152)
    prompts = _prompts(32, m.cfg.vocab_size, 128, 1024, seed=13)
    ar, _, _ = _run(m, prompts, 32, 1024, 24, mode="ar", k=8)
    sp, eng, _ = _run(m, prompts, 32, 1024, 24, sched="aspire", k=8, d_max=8, min_draft=2, initial_draft=3)
    assert sp == ar
    assert eng.stats["deep_steps"] > 0


def _teacher_forced_argmax(m, seqs, k):
    """Greedy tokens after every prefix of each sequence, from one prefill per sequence (cache row i, positions
    0..len-1): (exit layer k through the shared final norm + LM head, the full model).  Entry j of both arrays is
    the token predicted for position j + 1."""
    from thesis_amd.solutions.packed import Block, pack_blocks, packed_layers

    m.allocate_cache(len(seqs), m.cache.max_seq)
    out = []
    for i, s in enumerate(seqs):
        pb = pack_blocks(m, [Block(i, 0, len(s))])
        x = m.embed(torch.tensor(s, dtype=torch.long))
        cap = {}
        h = packed_layers(m, x, pb, 0, m.n_layers, cap, (k,))
        out.append((m.head_argmax(cap[k]).cpu().numpy(), m.head_argmax(h).cpu().numpy()))
    return out


def _check_forced_tokens(m, prompts, fo, k):
    """Every generated token of a forced-acceptance run (fo: pid -> tokens) is the exit-k head's greedy token (an
    accepted draft) or the full model's (a correction) after its own prefix, and both kinds occur."""
    ptok = {p.pid: list(p.tokens) for p in prompts}
    pids = sorted(fo)
    seqs = [ptok[i] + list(fo[i]) for i in pids]
    n_draft_only = n_full_only = 0
    for i, (s, (ex, full)) in zip(pids, zip(seqs, _teacher_forced_argmax(m, seqs, k))):
        P = len(ptok[i])
        tok = np.asarray(s[P:])
        e, f = ex[P - 1:len(s) - 1], full[P - 1:len(s) - 1]
        assert ((tok == e) | (tok == f)).all(), (i, np.flatnonzero((tok != e) & (tok != f))[:5])
        n_draft_only += int(((tok == e) & (tok != f)).sum())
        n_full_only += int(((tok == f) & (tok != e)).sum())
    assert n_draft_only > 0 and n_full_only > 0


def test_config4_forced_acceptance_commits_only_model_tokens(cuda):
    """The benchmark's own mode at config 4's shape: aspire drafts in [2, 8] with acceptance forced by the seeded
    geometric draw (p = 0.3), so drafts the full model disagrees with are committed and rejected ones rolled back.
    Checked against a teacher-forced prefill of each request's final sequence with the same weights: every AR token
    is the full model's greedy token after its prefix (prefill and incremental decode give the same bits), and every
    token of the forced run is the exit head's greedy token (an accepted draft) or the full model's (a correction)
    after its own prefix, with both kinds present; any error in the rollback, the positions or the KV kept would
    change the prefixes and break the match from there on."""
    m = _model("llama3-8b", torch.bfloat16, 1152)
    prompts = _prompts(32, m.cfg.vocab_size, 128, 1024, seed=13)
    k = 8
    ar, _, _ = _run(m, prompts, 32, 1024, 24, mode="ar", k=k)
    fo, eng, _ = _run(m, prompts, 32, 1024, 24, sched="aspire", k=k, d_max=8, min_draft=2, initial_draft=3,
                      forced_accept_p=0.3, forced_seed=7)
    assert all(len(v) == 24 for v in fo.values())
    assert eng.stats["deep_steps"] > 0 and 0 < eng.stats["accepted"] < eng.stats["drafted"]
    ptok = {p.pid: list(p.tokens) for p in prompts}
    pids = sorted(ar)
    seqs_ar = [ptok[i] + list(ar[i]) for i in pids]
    for i, (s, (_, full)) in zip(pids, zip(seqs_ar, _teacher_forced_argmax(m, seqs_ar, k))):
        P = len(ptok[i])
        assert np.array_equal(np.asarray(s[P:]), full[P - 1:len(s) - 1]), i
    _check_forced_tokens(m, prompts, fo, k)


def test_config5_llama2_7b_bf16_m3_chunks(cuda):
    from thesis_amd.solutions.cost_model import GPUParams, ModelDims, RooflineCostModel

    m = _model("llama2-7b", torch.bfloat16, 1152)
    prompts = _prompts(24, m.cfg.vocab_size, 256, 1024, seed=14)
    # a cost model whose knee admits 256-token chunks next to 16 decode rows
    gpu = GPUParams(bw=6.6e9, flops=1.2e12, t_op=0.007, n_op_layer=9, n_op_bucket=0, n_op_head=3, n_op_segment=1,
                    flops_eff=4.2e11, knee_measured=600.0)
    cm = RooflineCostModel(gpu, ModelDims.from_config(m.cfg))
    ar, _, _ = _run(m, prompts, 16, 1024, 16, cost_model=cm, mode="ar", k=8)
    sp, eng, _ = _run(m, prompts, 16, 1024, 16, cost_model=cm, sched="fixed", k=8, gamma=4, d_max=4, prefill="m3",
                      m3_chunk_cap=256, prefill_chunk=256, max_wait=100)
    assert sp == ar
    assert eng.stats["piggyback_tokens"] > 0


def test_config5_llama2_7b_poisson_b128_spec_equals_ar(cuda):
    """Open loop (solutions/engine.py:625-673): Poisson arrivals at 8 requests/s into B = 128 slots, 256-token
    prompt chunks piggybacked on the decode steps.  Whatever packing the arrival times produce, every request's
    tokens equal its autoregressive tokens, and the M3 chunks wrote the KV the deep segments read."""
    from thesis_amd.solutions.cost_model import GPUParams, ModelDims, RooflineCostModel
    from thesis_amd.solutions.engine import EESDEngine, EngineConfig

    m = _model("llama2-7b", torch.bfloat16, 1152)
    prompts = _prompts(24, m.cfg.vocab_size, 256, 1024, seed=15)
    gpu = GPUParams(bw=6.6e9, flops=1.2e12, t_op=0.007, n_op_layer=9, n_op_bucket=0, n_op_head=3, n_op_segment=1,
                    flops_eff=4.2e11, knee_measured=600.0)
    cm = RooflineCostModel(gpu, ModelDims.from_config(m.cfg))
    ar, _, _ = _run(m, prompts, 24, 1024, 32, cost_model=cm, mode="ar", k=8)
    eng = EESDEngine(m, 128, 1024, 32, (), EngineConfig(sched="fixed", k=8, gamma=4, d_max=4, prefill="m3",
                                                        m3_chunk_cap=256, prefill_chunk=256, max_wait=100), cm)
    res = eng.run_poisson(prompts, 8.0, len(prompts), warm_requests=0, seed=4, keep_outputs=True)
    sp = {c["pid"]: c["tokens"] for c in res["completions"]}
    assert sp == ar
    assert res["metrics"]["poisson_rate_per_s"] == 8.0 and res["metrics"]["evaluated_completions"] == len(prompts)
    assert eng.stats["piggyback_tokens"] > 0, "arrivals during decoding must ride the decode steps"
    assert res["metrics"]["wall_throughput_tok_s"] > 0


# ----------------------------------------------------------------------------- config 2: the microbenchmark

def _ubench_sample(a) -> list:
    """Requests checked against the fp64 brute force: the longest context, the shortest, every one whose
    block crosses a split boundary (up to 4), the largest and smallest query blocks, and a seeded spread."""
    ctx, T, split = a.ctx, a.T, a.split
    end = ctx + T
    crossing = [int(r) for r in np.flatnonzero((ctx // split) != ((end - 1) // split))][:4]
    multi = [int(r) for r in np.flatnonzero(end > split)][:3]
    picks = [int(np.argmax(ctx)), int(np.argmin(ctx)), int(np.argmax(T)), int(np.argmin(T))] + crossing + multi
    picks += [int(r) for r in np.random.default_rng(7).choice(a.B, 6, replace=False)]
    return sorted(set(picks))


@pytest.mark.parametrize("split", [None, 4096])
def test_config2_verify_attention_microbench_matches_brute_force(cuda, split):
    """The microbenchmark's attention launch (256 requests, contexts up to 8192, the rows cap and schedule the
    benchmark uses) after its KV append, at the production split of this cache (8192 positions: every context
    unsplit) and at 4096-position splits (two-split requests and the combine): the appended rows equal the
    inputs bitwise, the cached prefix [0, ctx) is untouched, sampled requests (longest, multi-split,
    split-crossing, ragged) match the fp64 brute force at the kernel tests' bounds, and the rollback gives
    kv_len = ctx + accepted + 1."""
    import bench
    from oracle.model import brute_attention
    from thesis_amd import _lsk

    a = bench.AttentionInputs(0, cuda, split)
    Hq, Hkv, D = a.Hq, a.Hkv, a.D
    if split is None:
        assert a.split == _lsk.ATTN_SPLIT and a.ctx.max() + a.T.max() <= a.split and a.n_parts == 0
    else:
        assert a.ctx.max() > a.split and a.n_parts > 0          # two-split requests, combine groups in the plan
    sample = _ubench_sample(a)
    assert len(sample) >= 8
    before = {r: (a.kc[r:r + 1].clone(), a.vc[r:r + 1].clone()) for r in sample[:4]}
    a.append()
    a.attn()
    torch.cuda.synchronize()
    got = a.out.float().cpu()
    k_new, v_new = a.k_new.cpu(), a.v_new.cpu()
    worst_max, worst_mean = 0.0, 0.0
    for r in sample:
        c, t, o = int(a.ctx[r]), int(a.T[r]), int(a.offs[r])
        kh = _lsk.k_from_frag(a.kc[r:r + 1].cpu())
        vh = _lsk.v_from_blocked(a.vc[r:r + 1].cpu())
        assert torch.equal(kh[0, :, c:c + t].transpose(0, 1), k_new[o:o + t]), f"request {r}: appended K"
        assert torch.equal(vh[0, :, c:c + t].transpose(0, 1), v_new[o:o + t]), f"request {r}: appended V"
        if r in before:
            k0 = _lsk.k_from_frag(before[r][0].cpu())
            v0 = _lsk.v_from_blocked(before[r][1].cpu())
            assert torch.equal(kh[..., :c, :], k0[..., :c, :]) and torch.equal(vh[..., :c, :], v0[..., :c, :])
        ref = brute_attention(a.q[o:o + t].cpu(), kh, vh, [0] * t, list(range(c, c + t)), Hq // Hkv)
        err = (got[o:o + t].double() - ref).abs()
        worst_max, worst_mean = max(worst_max, float(err.max())), max(worst_mean, float(err.mean()))
        assert err.max() < 2e-2 and err.mean() < 3e-3, (r, c, t, float(err.max()), float(err.mean()))
    print(f"config 2: {len(sample)} requests (contexts {sorted(int(a.ctx[r]) for r in sample)}), split {a.split}, "
          f"rows cap {a.rows_cap}: max |err| {worst_max:.3e}, worst mean {worst_mean:.3e}")
    a.rollback()
    assert torch.equal(a.kv_len.cpu(), torch.from_numpy(a.ctx + a.acc + 1))
    assert (a.acc <= a.T - 1).all() and (a.acc >= 0).all()
