"""The CPU oracle is pinned before it is trusted (CPU only).

  * golden vectors from HF transformers' LlamaForCausalLM (tests/golden/hf_tiny.npz; default RoPE,
    tied embeddings, llama3 RoPE scaling): last-position logits, every exit hidden state, and a cached
    decode step (the reference's test_matches_hf, tests/test_model.py:9-36, atol 1e-4)
  * planted mistakes in the oracle (RoPE sign, norm epsilon, missing llama3 smoothing, softmax scale)
    must break those golden checks: the checks have teeth
  * packed attention against an fp64 brute-force per-token loop
  * packed forward == per-block forward (tests/test_eesd.py:120-142 of the reference)
  * build_packed against the reference's hand-written cases (tests/test_eesd.py:99-117, 534-546)
  * losslessness of the oracle engine (spec == AR) and the acceptance closed form
  * the ordered fp32 mode (oracle/ordered.py): the same golden vectors, the default oracle, exp against
    float64 exp, and planted order / term mistakes that change the bits the bitwise GPU checks compare
"""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle.model as om
from oracle.engine import ForcedAcceptance, OracleEngine

GOLDEN = Path(__file__).resolve().parent / "golden" / "hf_tiny.npz"


def _golden_model(name, ordered=False):
    import importlib.util

    spec = importlib.util.spec_from_file_location("mkg", GOLDEN.with_name("make_hf_golden.py"))
    mkg = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mkg)
    v = mkg.VARIANTS[name]
    cfg = mkg.oracle_cfg(v)
    w = om.random_weights(cfg, seed=mkg.SEED, std=mkg.STD)
    m = om.OracleLlama(cfg, w, dtype=torch.float32, max_seq=512, ordered=ordered)
    m.allocate_cache(2, 256)
    return m


def _check_golden(name, atol=1e-4, ordered=False):
    g = np.load(GOLDEN)
    m = _golden_model(name, ordered)
    ids = g["ids"].tolist()
    with torch.inference_mode():
        logits, hidden = m.prefill(ids, slot=1, capture=True)
        ok = np.allclose(logits.numpy(), g[f"{name}/logits_last"], atol=atol)
        hid = g[f"{name}/hidden_last"]
        for k in range(1, m.n_layers):          # HF hidden_states[k] = after layer k-1 (the exit-k input)
            ok &= np.allclose(hidden[k - 1].numpy(), hid[k - 1], atol=atol)
        nxt = int(g[f"{name}/next_token"])
        assert int(logits.argmax()) == nxt or not ok
        pb = om.build_packed(m, [om.OBlock(1, len(ids), 1)])
        h = om.packed_layers(m, m.embed(torch.tensor([nxt])), pb, 0, m.n_layers)
        step = m.head(h)[0]
        ok &= np.allclose(step.numpy(), g[f"{name}/decode_logits"], atol=atol)
    return bool(ok)


@pytest.mark.parametrize("name", ["default", "tied", "llama3_rope"])
def test_oracle_matches_hf_golden(name):
    assert _check_golden(name)


@pytest.mark.parametrize("name", ["default", "llama3_rope"])
def test_oracle_matches_live_transformers(name, tmp_path):
    """The same comparison against transformers run now (guards the committed fixture itself)."""
    pytest.importorskip("transformers")
    import importlib.util
    import json

    from safetensors.torch import save_file
    from transformers import LlamaForCausalLM

    spec = importlib.util.spec_from_file_location("mkg", GOLDEN.with_name("make_hf_golden.py"))
    mkg = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mkg)
    v = mkg.VARIANTS[name]
    w = om.random_weights(mkg.oracle_cfg(v), seed=mkg.SEED, std=mkg.STD)
    (tmp_path / "config.json").write_text(json.dumps(mkg.hf_config(v)))
    save_file({k: t.contiguous() for k, t in w.items()}, str(tmp_path / "model.safetensors"))
    hf = LlamaForCausalLM.from_pretrained(tmp_path, dtype=torch.float32).eval()
    ids = torch.from_numpy(np.load(GOLDEN)["ids"]).unsqueeze(0)
    with torch.inference_mode():
        ref = hf(ids).logits[0, -1]
    m = _golden_model(name)
    got, _ = m.prefill(ids[0].tolist(), slot=0)
    assert torch.allclose(got, ref, atol=1e-4)


@pytest.mark.parametrize("mistake", ["rope_sign", "norm_eps", "no_llama3_smoothing", "attn_scale", "rope_half"])
def test_golden_checks_catch_planted_mistakes(mistake, monkeypatch):
    """A plausible mistake planted in the oracle must fail the golden comparison."""
    name = "llama3_rope" if mistake == "no_llama3_smoothing" else "default"
    if mistake == "rope_sign":
        def bad(x, cos, sin):
            half = x.shape[-1] // 2
            return x * cos + torch.cat([x[..., half:], -x[..., :half]], dim=-1) * sin
        monkeypatch.setattr(om, "rope", bad)
    elif mistake == "rope_half":
        def bad(x, cos, sin):
            half = x.shape[-1] // 2
            return x * cos + torch.cat([-x[..., :half], x[..., half:]], dim=-1) * sin
        monkeypatch.setattr(om, "rope", bad)
    elif mistake == "norm_eps":
        real = om.rms_norm
        monkeypatch.setattr(om, "rms_norm", lambda x, w, eps: real(x, w, 1e-1))
    elif mistake == "no_llama3_smoothing":
        def bad(cfg):
            exps = torch.arange(0, cfg.head_dim, 2, dtype=torch.int64).float() / cfg.head_dim
            return 1.0 / (cfg.rope_theta ** exps)
        monkeypatch.setattr(om, "rope_inv_freq", bad)
    elif mistake == "attn_scale":
        real = torch.nn.functional.scaled_dot_product_attention
        monkeypatch.setattr(om.F, "scaled_dot_product_attention",
                            lambda q, k, v, attn_mask=None: real(q, k, v, attn_mask=attn_mask, scale=1.0))
    assert not _check_golden(name)


# ----------------------------------------------------------------------------- attention / packing

def _tiny(dtype=torch.float32, **kw):
    cfg = om.OracleConfig(vocab_size=64, dim=64, n_layers=3, n_heads=4, n_kv_heads=2, head_dim=16,
                          intermediate_size=128, **kw)
    return om.OracleLlama(cfg, om.random_weights(cfg, seed=3, std=0.1), dtype=dtype, max_seq=256)


def test_packed_attention_matches_brute_force():
    m = _tiny()
    m.allocate_cache(3, 128)
    g = torch.Generator().manual_seed(0)
    for i in range(m.n_layers):
        m.cache.k[i].copy_(torch.randn(m.cache.k[i].shape, generator=g))
        m.cache.v[i].copy_(torch.randn(m.cache.v[i].shape, generator=g))
    blocks = [om.OBlock(0, 5, 1), om.OBlock(1, 30, 4), om.OBlock(2, 0, 7), om.OBlock(0, 70, 2)]
    pb = om.build_packed(m, blocks)
    q = torch.randn(pb.n_tokens, 4, 16, generator=g)
    got = om.attend(m, 1, q, pb)
    ref = om.brute_attention(q, m.cache.k[1], m.cache.v[1], pb.rows, pb.pos, m.group)
    assert torch.allclose(got.double(), ref, atol=1e-5)


def test_brute_force_reduces_to_single_position_value():
    """Special case with a closed form: a query at position 0 returns V[row, head, 0] exactly."""
    kc = torch.randn(2, 2, 8, 4)
    vc = torch.randn(2, 2, 8, 4)
    q = torch.randn(1, 4, 4)
    out = om.brute_attention(q, kc, vc, [1], [0], 2).view(4, 4)
    for h in range(4):
        assert torch.allclose(out[h], vc[1, h // 2, 0].double())


def test_packed_forward_matches_per_block_forward():
    m = _tiny()
    m.allocate_cache(3, 64)
    g = torch.Generator().manual_seed(0)
    for row in range(3):
        m.prefill(torch.randint(3, 60, (8,), generator=g).tolist(), row)
    blocks = [om.OBlock(0, 8, 1), om.OBlock(1, 8, 4), om.OBlock(2, 8, 2)]
    x = torch.randn(7, 64, generator=g)
    pb = om.build_packed(m, blocks)
    order = [blocks.index(b) for b in pb.blocks]
    starts = np.concatenate([[0], np.cumsum([b.T for b in blocks])])
    xp = torch.cat([x[starts[i]:starts[i + 1]] for i in order])
    snap_k = [t.clone() for t in m.cache.k]
    snap_v = [t.clone() for t in m.cache.v]
    yp = om.packed_layers(m, xp, pb, 0, m.n_layers)
    for j, i in enumerate(order):
        for l in range(m.n_layers):
            m.cache.k[l].copy_(snap_k[l])
            m.cache.v[l].copy_(snap_v[l])
        b = blocks[i]
        ref = om.packed_layers(m, x[starts[i]:starts[i + 1]], om.build_packed(m, [b]), 0, m.n_layers)
        assert torch.allclose(yp[pb.offsets[j]:pb.offsets[j + 1]], ref, atol=1e-5)


def test_build_packed_reference_cases():
    """tests/test_eesd.py:99-117 and 534-546 of the reference."""
    m = _tiny()
    m.allocate_cache(4, 128)
    blocks = [om.OBlock(2, 10, 3, "a"), om.OBlock(0, 5, 1, "b"), om.OBlock(1, 7, 2, "c"), om.OBlock(3, 9, 1, "d")]
    pb = om.build_packed(m, blocks, "exact")
    assert pb.n_tokens == 7
    assert list(pb.offsets) == list(om.qo_indptr([b.T for b in pb.blocks]))
    assert [b.T for b in pb.blocks] == [1, 1, 2, 3]
    assert [bk.T for bk in pb.buckets] == [1, 2, 3]
    pos = pb.pos.tolist()
    for i, b in enumerate(pb.blocks):
        assert pos[pb.offsets[i]:pb.offsets[i + 1]] == list(range(b.pos0, b.pos0 + b.T))
    assert pb.buckets[0].rows is not None
    pad = om.build_packed(m, blocks, "pad")
    assert len(pad.buckets) == 1 and pad.buckets[0].T == 3
    assert sorted(i for i in pad.buckets[0].pad_index.view(-1).tolist() if i >= 0) == list(range(7))
    pb2 = om.build_packed(m, [om.OBlock(0, 10, 1), om.OBlock(2, 70, 1), om.OBlock(1, 5, 3)], "exact")
    assert pb2.kv_read_padded == 2 * 128 + 64 and pb2.kv_gathered == 2 * 128
    with pytest.raises(ValueError):
        om.build_packed(m, blocks, "nope")


# ----------------------------------------------------------------------------- engine

def _prompts(n, seed=3):
    g = torch.Generator().manual_seed(seed)
    out = []
    for i in range(n):
        L = int(torch.randint(5, 21, (1,), generator=g))
        out.append((f"p{i}", [1] + torch.randint(3, 64, (L - 1,), generator=g).tolist()))
    return out


@pytest.mark.parametrize("k,gamma,B", [(1, 3, 2), (2, 4, 3), (2, 1, 1)])
def test_oracle_engine_is_lossless(k, gamma, B):
    m = _tiny()
    prompts = _prompts(5)
    ar = OracleEngine(m, 2, 24, 20, mode="ar").run_static(prompts)
    sp = OracleEngine(m, B, 24, 20, mode="spec", k=k, gamma=gamma, d_max=6).run_static(prompts)
    assert ar == sp and all(len(v) == 20 for v in ar.values())


def test_forced_acceptance_is_seeded_and_bounded():
    fa, fb = ForcedAcceptance(0.3, seed=4), ForcedAcceptance(0.3, seed=4)
    a = [fa.draw(j) for j in range(3) for _ in range(50)]
    b = [fb.draw(j) for j in range(3) for _ in range(50)]
    assert a == b and min(a) >= 0
    # P(a == 0) = p for a geometric draw minus one
    draws = [ForcedAcceptance(0.3, seed=s).draw(0) for s in range(2000)]
    assert abs(np.mean(np.array(draws) == 0) - 0.3) < 0.05


def test_acceptance_closed_form_in_oracle_engine():
    """acc = min{j : Y_j != draft_{j+1}}: with all-matching drafts the whole block is accepted."""
    m = _tiny()
    prompts = _prompts(2, seed=9)
    eng = OracleEngine(m, 2, 24, 30, mode="spec", k=2, gamma=3, d_max=6)
    out = eng.run_static(prompts)
    ar = OracleEngine(m, 2, 24, 30, mode="ar").run_static(prompts)
    assert out == ar and eng.n_deep > 0


# ----------------------------------------------------------------------------- ordered fp32 mode

@pytest.mark.parametrize("name", ["default", "tied", "llama3_rope"])
def test_ordered_oracle_matches_hf_golden(name):
    assert _check_golden(name, ordered=True)


def test_ordered_oracle_matches_the_default_oracle():
    import oracle.ordered as O
    from conftest import small_cfg

    cfg = small_cfg()
    w = om.random_weights(cfg, seed=4, std=0.05)
    a = om.OracleLlama(cfg, w, dtype=torch.float32, max_seq=256)
    b = om.OracleLlama(cfg, w, dtype=torch.float32, max_seq=256, ordered=True)
    for m in (a, b):
        m.allocate_cache(3, 128)
    blocks = [om.OBlock(0, 0, 40), om.OBlock(1, 0, 7), om.OBlock(2, 0, 70)]
    ids = torch.randint(0, cfg.vocab_size, (117,), generator=torch.Generator().manual_seed(0))
    ya = om.packed_layers(a, a.embed(ids), om.build_packed(a, blocks), 0, a.n_layers)
    yb = om.packed_layers(b, b.embed(ids), om.build_packed(b, blocks), 0, b.n_layers)
    assert torch.allclose(ya, yb, atol=1e-5, rtol=1e-5)
    assert torch.allclose(a.head(ya), b.head(yb), atol=1e-5, rtol=1e-5)
    assert not torch.equal(ya, yb)          # the orders differ, so the bits do: the bitwise checks can tell
    assert O.exp_f32(np.float32(0)) == 1


def test_exp_f32_is_within_two_ulp_of_exp():
    import oracle.ordered as O

    x = np.concatenate([np.linspace(-85.9, 88.5, 200001, dtype=np.float32),
                        np.random.default_rng(0).normal(0, 4, 100000).astype(np.float32)])
    got = O.exp_f32(x).astype(np.float64)
    ref = np.exp(x.astype(np.float64))
    ulp = np.spacing(ref.astype(np.float32)).astype(np.float64)
    assert (np.abs(got - ref) / ulp).max() <= 2.0
    assert O.exp_f32(np.float32(-np.inf)) == 0 and O.exp_f32(np.float32(-87)) == 0
    assert np.isinf(O.exp_f32(np.float32(90))) and np.isnan(O.exp_f32(np.float32(np.nan)))
    sil = O.silu_f32(np.float32([-100, -3, 0, 2.5, 100]))
    assert np.allclose(sil, np.array([-100, -3, 0, 2.5, 100]) / (1 + np.exp(-np.array([-100, -3, 0, 2.5, 100.]))),
                       rtol=1e-6, atol=1e-30)                     # silu(-100) = -0: exp(100) is inf in fp32


def test_ordered_checks_catch_planted_mistakes(monkeypatch):
    """A dropped Taylor term breaks the exp bound; a plain left-to-right sum instead of the lane / butterfly
    order gives different bits for the same products (what the GPU's bitwise comparison would flag)."""
    import oracle.ordered as O

    x = np.linspace(-20, 20, 10001, dtype=np.float32)
    ref = np.exp(x.astype(np.float64))
    bad = list(O._TAYLOR)
    bad[2] = np.float32(0.0)                                     # drop the r^5 / 5! term
    monkeypatch.setattr(O, "_TAYLOR", bad)
    got = O.exp_f32(x).astype(np.float64)
    monkeypatch.undo()
    assert (np.abs(got - ref) / np.spacing(ref.astype(np.float32))).max() > 2.0
    rng = np.random.default_rng(1)
    a = rng.normal(size=(8, 700)).astype(np.float32)
    w = rng.normal(size=(16, 700)).astype(np.float32)
    ordered = O.linear(a, w)
    plain = np.zeros((8, 16), np.float32)
    for k in range(700):
        plain = plain + a[:, k:k + 1] * w[None, :, k]
    assert np.allclose(ordered, plain, atol=1e-3) and not np.array_equal(ordered, plain)
    nrm = O.rms_norm(a, np.ones(700, np.float32), 1e-5)
    plain_ms = np.float32(1) / np.sqrt((a * a).sum(axis=1, dtype=np.float32) / np.float32(700) + np.float32(1e-5))
    assert np.allclose(nrm, a * plain_ms[:, None], rtol=1e-5) and not np.array_equal(nrm, a * plain_ms[:, None])


# ----------------------------------------------------------------------------- blocked bf16 attention

def _exact_attention_case(seed=0, D=64, G=4, Hkv=2, split=512, ctx=(37, 300, 700, 1100, 1535)):
    """Inputs on which every step of the blocked bf16 softmax is exact: with scale_log2 = 1 and one-hot queries a
    score is one integer K entry in [-6, 0], so every p, alpha and merge weight is a power of two 2^-k (k <= 6, bf16
    exact) and every partial O / L is a multiple of 2^-6 below 2^13 (exact in fp32).  The scores rise within a wave
    (round 0 in [-6, -3], later rounds in [-6, -2]), one wave per split sees -1, and one position of the second
    split scores 0, so the running-max rescale, the wave merge weights and the split merge weights all matter."""
    rng = np.random.default_rng(seed)
    n = max(ctx)
    S = ((n + 63) // 64 + 1) * 64
    K = rng.integers(-6, -2, size=(1, Hkv, S, D)).astype(np.float32)
    pos_in = np.arange(S) % split
    later = pos_in >= 256
    K[:, :, later] = rng.integers(-6, -1, size=(1, Hkv, int(later.sum()), D))
    wave = (pos_in // 32) % 8
    hot = later & (wave == (np.arange(S) // split) % 8)
    K[:, :, hot] = rng.integers(-6, 0, size=(1, Hkv, int(hot.sum()), D))
    K[:, :, split + 300] = 0.0
    V = rng.integers(-4, 5, size=(1, Hkv, S, D)).astype(np.float32)
    N = len(ctx)
    q = np.zeros((N, Hkv * G, D), np.float32)
    hot_dim = rng.integers(0, D, size=(N, Hkv * G))
    q[np.arange(N)[:, None], np.arange(Hkv * G)[None, :], hot_dim] = 1.0
    pos = np.array(ctx) - 1
    return q, K, V, np.zeros(N, np.int64), pos, G, split


def _exact_base2(q, K, V, rows, pos, G):
    """Textbook softmax in base 2 over the scores q . k (scale_log2 = 1), fp64, then rounded fp32 -> bf16."""
    import oracle.ordered as O

    N, Hq, D = q.shape
    out = np.zeros((N, Hq, D), np.float64)
    for t in range(N):
        for h in range(Hq):
            s = K[rows[t], h // G, :pos[t] + 1].astype(np.float64) @ q[t, h].astype(np.float64)
            w = np.exp2(s - s.max())
            out[t, h] = (w @ V[rows[t], h // G, :pos[t] + 1].astype(np.float64)) / w.sum()
    return O.bf16_round(out.astype(np.float32))


def test_blocked_bf16_attention_is_exact_where_every_step_is_exact():
    """Known answer: on the exact inputs the blocked softmax (several waves, rounds and position splits) equals the
    base-2 textbook result bit for bit, for a single-split and a four-split context alike.  Planted mistakes -- no
    alpha rescale of the running output, waves and splits summed without their weights -- change the result."""
    import oracle.ordered as O

    q, K, V, rows, pos, G, split = _exact_attention_case()
    want = _exact_base2(q, K, V, rows, pos, G)
    got = O.attend_bf16_blocked(q, K, V, rows, pos, G, split, scale_log2=1.0)
    assert np.array_equal(got, want)
    for kw in (dict(rescale=False), dict(weigh_waves=False)):
        bad = O.attend_bf16_blocked(q, K, V, rows, pos, G, split, scale_log2=1.0, **kw)
        assert not np.array_equal(bad, want), kw
        assert (bad != want).mean() > 0.05, kw
    # the same inputs with no split at all (one wave chain over the whole context) agree too
    assert np.array_equal(O.attend_bf16_blocked(q, K, V, rows, pos, G, 1 << 20, scale_log2=1.0), want)


def _random_attention_case(seed, D, G=4, Hkv=2, ctx=(1, 9, 64, 257, 600, 2100, 4500)):
    rng = np.random.default_rng(seed)
    S = (max(ctx) + 63) // 64 * 64
    bf = lambda a: torch.from_numpy(a.astype(np.float32)).to(torch.bfloat16)  # noqa: E731
    K = bf(rng.normal(size=(2, Hkv, S, D)))
    V = bf(rng.normal(size=(2, Hkv, S, D)))
    q = bf(rng.normal(size=(len(ctx), Hkv * G, D)))
    rows = np.arange(len(ctx)) % 2
    pos = np.array(ctx) - 1
    return q, K, V, rows, pos, G


@pytest.mark.parametrize("D", [64, 128])
def test_blocked_bf16_attention_sits_at_the_bf16_rounding_floor(D):
    """Random bf16 inputs, contexts of 1 to 4500 positions (up to three 2048-position splits): the blocked form is
    as far from the fp64 brute force as the reference's eager bf16 SDPA is (within [0.75, 1.25] x: both round the
    softmax weights to bf16), and within 3e-3 of it.  Planted mistakes land outside: weights kept in fp32 (no bf16
    rounding of P or of the output) sit far closer to exact, a dropped rescale or unweighted merges far above."""
    import torch.nn.functional as F

    import oracle.ordered as O

    q, K, V, rows, pos, G = _random_attention_case(3, D)
    exact = om.brute_attention(q.float(), K.float(), V.float(), rows, pos, G).view(len(pos), -1, D).numpy()
    sdpa = np.zeros_like(exact)
    for t in range(len(pos)):
        kk = K[rows[t], :, :pos[t] + 1].repeat_interleave(G, 0)
        vv = V[rows[t], :, :pos[t] + 1].repeat_interleave(G, 0)
        sdpa[t] = F.scaled_dot_product_attention(q[t][:, None], kk, vv)[:, 0].float().numpy()
    args = (q.float().numpy(), K.float().numpy(), V.float().numpy(), rows, pos, G, 2048)
    got = O.attend_bf16_blocked(*args)
    rel = lambda a: float(np.linalg.norm(a - exact) / np.linalg.norm(exact))  # noqa: E731
    d_blk, d_sdpa = rel(got), rel(sdpa)
    assert 0.75 * d_sdpa <= d_blk <= 1.25 * d_sdpa, (d_blk, d_sdpa)
    assert float(np.linalg.norm(got - sdpa) / np.linalg.norm(sdpa)) <= 3e-3
    assert rel(O.attend_bf16_blocked(*args, rescale=False)) > 10 * d_sdpa
    assert rel(O.attend_bf16_blocked(*args, weigh_waves=False)) > 10 * d_sdpa
    import unittest.mock as um
    with um.patch.object(O, "bf16_round", lambda x: np.asarray(x, np.float32)):
        assert rel(O.attend_bf16_blocked(*args)) < 0.1 * d_sdpa
