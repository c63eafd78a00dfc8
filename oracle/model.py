"""CPU oracle of the packed ragged LayerSkip-Llama forward (TEST INFRASTRUCTURE ONLY).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package, and
only as the reference for parity tests / CPU baseline: the product path (thesis_amd) never calls it.

This is a from-scratch torch-CPU restatement of the reference's math, with the dtype rounding
points of its eager ops kept in place (so a bf16 oracle rounds where the reference rounds):

  rms_norm         common/model.py:153-156   fp32 normalise, cast, then `weight * x`
  RoPE table       common/model.py:113-140   inv_freq on CPU in fp32, llama3 smoothing, cat(f, f)
  apply_rope       common/model.py:143-150   x*cos + rotate_half(x)*sin (3 roundings)
  fused weights    common/model.py:259-276   wqkv = [q;k;v], w13 = [gate;up], tied lm_head
  KV cache         common/model.py:171-183   [max_batch, Hkv, max_seq, D] per layer, zeros
  embed / head     common/model.py:325-330
  build_packed     solutions/packed.py:81-139  (block order, buckets, masks, accounting)
  _attend          solutions/packed.py:142-166 (per-bucket masked SDPA)
  packed_layer(s)  solutions/packed.py:169-196
  qo_indptr        solutions/packed.py:199-201

OracleLlama(ordered=True) (fp32) evaluates the reductions in the fixed order of oracle/ordered.py, the
fp32 kernels' order, so the fp32 engine is compared with it bit for bit.  OracleLlama(attention="blocked")
(bf16) runs attention in the bf16 kernel's softmax blocking (ordered.attend_bf16_blocked: 32-position steps dealt
to 8 waves, P rounded to bf16 at each step's running max, waves then position splits merged in order); every
other op keeps the reference's eager bf16 rounding points.

Pinned by (tests/test_oracle.py): HF transformers LlamaForCausalLM golden logits / hidden states
(tests/golden/hf_tiny.npz), fp64 brute-force per-token attention, packed == per-block forward,
and the reference's own hand-written build_packed cases (tests/test_eesd.py:99-117, 534-546).
"""

from __future__ import annotations

import json
import math
from dataclasses import dataclass, field
from pathlib import Path
from typing import Optional

import numpy as np
import torch
import torch.nn.functional as F

from oracle import ordered as O


# ----------------------------------------------------------------------------- config

@dataclass
class OracleConfig:
    vocab_size: int
    dim: int
    n_layers: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    intermediate_size: int
    norm_eps: float = 1e-5
    rope_theta: float = 10000.0
    max_position_embeddings: int = 4096
    tie_word_embeddings: bool = False
    rope_scaling: Optional[dict] = None

    @classmethod
    def from_hf_dir(cls, path) -> "OracleConfig":
        """config.json of an HF Llama checkpoint (old `rope_theta`/`rope_scaling` or new
        `rope_parameters` format; common/model.py:57-91)."""
        c = json.loads((Path(path) / "config.json").read_text())
        rp = c.get("rope_parameters") or {}
        scaling = c.get("rope_scaling")
        if scaling is None and rp.get("rope_type", "default") != "default":
            scaling = rp
        nh = c["num_attention_heads"]
        return cls(vocab_size=c["vocab_size"], dim=c["hidden_size"], n_layers=c["num_hidden_layers"], n_heads=nh,
                   n_kv_heads=c.get("num_key_value_heads", nh), head_dim=c.get("head_dim") or c["hidden_size"] // nh,
                   intermediate_size=c["intermediate_size"], norm_eps=c.get("rms_norm_eps", 1e-5),
                   rope_theta=c.get("rope_theta", rp.get("rope_theta", 10000.0)),
                   max_position_embeddings=c.get("max_position_embeddings", 4096),
                   tie_word_embeddings=c.get("tie_word_embeddings", False), rope_scaling=scaling)


# ----------------------------------------------------------------------------- math

def rope_inv_freq(cfg: OracleConfig) -> torch.Tensor:
    """1 / theta^(2i/D) in fp32 on the CPU, with llama3 frequency smoothing when configured."""
    exps = torch.arange(0, cfg.head_dim, 2, dtype=torch.int64).float() / cfg.head_dim
    inv = 1.0 / (cfg.rope_theta ** exps)
    sc = cfg.rope_scaling or {}
    kind = sc.get("rope_type", sc.get("type"))
    if kind in (None, "default"):
        return inv
    if kind != "llama3":
        raise NotImplementedError(kind)
    factor, lo, hi = sc["factor"], sc["low_freq_factor"], sc["high_freq_factor"]
    old = sc["original_max_position_embeddings"]
    wavelen = 2 * math.pi / inv
    scaled = torch.where(wavelen > old / lo, inv / factor, inv)
    t = (old / wavelen - lo) / (hi - lo)
    blended = (1 - t) * scaled / factor + t * scaled
    medium = ~(wavelen < old / hi) & ~(wavelen > old / lo)
    return torch.where(medium, blended, scaled)


def rope_tables(cfg: OracleConfig, n_pos: int) -> tuple[torch.Tensor, torch.Tensor]:
    """fp32 cos/sin tables [n_pos, D] in the rotate-half layout (frequencies repeated twice)."""
    ang = torch.outer(torch.arange(n_pos, dtype=torch.float32), rope_inv_freq(cfg))
    ang = torch.cat([ang, ang], dim=-1)
    return ang.cos(), ang.sin()


def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    xf = x.float()
    r = torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return w * (xf * r).to(x.dtype)


def rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    half = x.shape[-1] // 2
    rot = torch.cat([-x[..., half:], x[..., :half]], dim=-1)
    return x * cos + rot * sin


# ----------------------------------------------------------------------------- weights / cache

@dataclass
class OracleLayer:
    wqkv: torch.Tensor
    wo: torch.Tensor
    w13: torch.Tensor
    w2: torch.Tensor
    attn_norm: torch.Tensor
    ffn_norm: torch.Tensor


class OracleCache:
    def __init__(self, cfg: OracleConfig, max_batch: int, max_seq: int, dtype):
        shape = (max_batch, cfg.n_kv_heads, max_seq, cfg.head_dim)
        self.max_batch, self.max_seq = max_batch, max_seq
        self.k = [torch.zeros(shape, dtype=dtype) for _ in range(cfg.n_layers)]
        self.v = [torch.zeros(shape, dtype=dtype) for _ in range(cfg.n_layers)]


def random_weights(cfg: OracleConfig, seed: int = 0, std: float = 0.02) -> dict:
    """Seeded HF-style init: N(0, std) matrices, unit norm weights; fp32 on the CPU.
    Keys follow the HF checkpoint names so the same dict feeds both the oracle and the GPU model."""
    g = torch.Generator().manual_seed(seed)
    qd, kvd = cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim

    def mat(r, c):
        return torch.randn(r, c, generator=g) * std

    w = {"model.embed_tokens.weight": mat(cfg.vocab_size, cfg.dim), "model.norm.weight": torch.ones(cfg.dim)}
    for i in range(cfg.n_layers):
        p = f"model.layers.{i}."
        w[p + "self_attn.q_proj.weight"] = mat(qd, cfg.dim)
        w[p + "self_attn.k_proj.weight"] = mat(kvd, cfg.dim)
        w[p + "self_attn.v_proj.weight"] = mat(kvd, cfg.dim)
        w[p + "self_attn.o_proj.weight"] = mat(cfg.dim, qd)
        w[p + "mlp.gate_proj.weight"] = mat(cfg.intermediate_size, cfg.dim)
        w[p + "mlp.up_proj.weight"] = mat(cfg.intermediate_size, cfg.dim)
        w[p + "mlp.down_proj.weight"] = mat(cfg.dim, cfg.intermediate_size)
        w[p + "input_layernorm.weight"] = torch.ones(cfg.dim)
        w[p + "post_attention_layernorm.weight"] = torch.ones(cfg.dim)
    if not cfg.tie_word_embeddings:
        w["lm_head.weight"] = mat(cfg.vocab_size, cfg.dim)
    return w


def load_hf_weights(path) -> dict:
    from safetensors import safe_open

    path = Path(path)
    idx = path / "model.safetensors.index.json"
    files = sorted(set(json.loads(idx.read_text())["weight_map"].values())) if idx.exists() else ["model.safetensors"]
    out = {}
    for f in files:
        with safe_open(str(path / f), framework="pt", device="cpu") as fh:
            for k in fh.keys():
                out[k] = fh.get_tensor(k)
    return out


class OracleLlama:
    """CPU LayerSkip-Llama; same attributes as the reference model object where the packed path reads them."""

    def __init__(self, cfg: OracleConfig, weights: dict, dtype=torch.float32, max_seq: int = 512,
                 ordered: bool = False, attention: str = "sdpa"):
        """ordered=True (fp32 only): the reductions run in the fixed order of oracle/ordered.py.
        attention="blocked" (bf16 only): attention in the bf16 kernel's softmax blocking
        (ordered.attend_bf16_blocked); "sdpa": torch's scaled_dot_product_attention, as the reference."""
        if ordered and dtype != torch.float32:
            raise ValueError("the ordered oracle is fp32 only")
        if attention not in ("sdpa", "blocked") or (attention == "blocked" and dtype != torch.bfloat16):
            raise ValueError(f"attention={attention!r} (sdpa, or blocked for bf16)")
        self.cfg, self.dtype, self.device = cfg, dtype, torch.device("cpu")
        self.ordered = ordered
        self.attention = attention
        self.attn_split = 2048
        self.group = cfg.n_heads // cfg.n_kv_heads
        self.q_size = cfg.n_heads * cfg.head_dim
        self.kv_size = cfg.n_kv_heads * cfg.head_dim

        def t(k):
            return weights[k].to(dtype)

        self.layers = []
        for i in range(cfg.n_layers):
            p = f"model.layers.{i}."
            self.layers.append(OracleLayer(
                wqkv=torch.cat([weights[p + "self_attn.q_proj.weight"], weights[p + "self_attn.k_proj.weight"],
                                weights[p + "self_attn.v_proj.weight"]]).to(dtype),
                wo=t(p + "self_attn.o_proj.weight"),
                w13=torch.cat([weights[p + "mlp.gate_proj.weight"], weights[p + "mlp.up_proj.weight"]]).to(dtype),
                w2=t(p + "mlp.down_proj.weight"),
                attn_norm=t(p + "input_layernorm.weight"), ffn_norm=t(p + "post_attention_layernorm.weight")))
        self.embed_w = t("model.embed_tokens.weight")
        self.norm_w = t("model.norm.weight")
        self.lm_head_w = t("lm_head.weight") if "lm_head.weight" in weights else self.embed_w
        self.rope_cos, self.rope_sin = rope_tables(cfg, max_seq)
        self.cache: Optional[OracleCache] = None

    @classmethod
    def synthetic(cls, cfg: OracleConfig, dtype=torch.bfloat16, seed: int = 0, std: float = 0.02,
                  max_seq: int = 2048, pool_elems: int = 1 << 26) -> "OracleLlama":
        """Full-size model for CPU timing: every weight matrix is its own allocation, filled from one
        seeded N(0, std) pool at random offsets (drawing 8e9 fresh normals on the CPU would take minutes;
        the cost of the forward does not depend on the values)."""
        g = torch.Generator().manual_seed(seed)
        pool = (torch.randn(pool_elems, generator=g) * std).to(dtype)
        offs = iter(torch.randint(0, pool_elems, (1 << 16,), generator=g).tolist())

        def fill(r, c):
            t = torch.empty(r * c, dtype=dtype)
            pos, o = 0, next(offs)
            while pos < t.numel():
                n = min(t.numel() - pos, pool_elems - o)
                t[pos:pos + n] = pool[o:o + n]
                pos, o = pos + n, 0
            return t.view(r, c)

        self = cls.__new__(cls)
        self.cfg, self.dtype, self.device = cfg, dtype, torch.device("cpu")
        self.group = cfg.n_heads // cfg.n_kv_heads
        self.q_size = cfg.n_heads * cfg.head_dim
        self.kv_size = cfg.n_kv_heads * cfg.head_dim
        ones = torch.ones(cfg.dim, dtype=dtype)
        self.layers = [OracleLayer(fill(self.q_size + 2 * self.kv_size, cfg.dim), fill(cfg.dim, self.q_size),
                                   fill(2 * cfg.intermediate_size, cfg.dim), fill(cfg.dim, cfg.intermediate_size),
                                   ones, ones) for _ in range(cfg.n_layers)]
        self.embed_w = fill(cfg.vocab_size, cfg.dim)
        self.norm_w = ones
        self.lm_head_w = self.embed_w if cfg.tie_word_embeddings else fill(cfg.vocab_size, cfg.dim)
        self.rope_cos, self.rope_sin = rope_tables(cfg, max_seq)
        self.cache = None
        return self

    @property
    def n_layers(self) -> int:
        return self.cfg.n_layers

    def allocate_cache(self, max_batch: int, max_seq: int) -> OracleCache:
        max_seq = (max_seq + 63) // 64 * 64
        if max_seq > self.rope_cos.shape[0]:
            self.rope_cos, self.rope_sin = rope_tables(self.cfg, max_seq)
        self.cache = OracleCache(self.cfg, max_batch, max_seq, self.dtype)
        # the bf16 kernel's position splits: 8192 positions once the cache holds >= 1024 (row, KV head) stripes
        self.attn_split = 8192 if max_batch * self.cfg.n_kv_heads >= 1024 else 2048
        return self.cache

    def embed(self, ids: torch.Tensor) -> torch.Tensor:
        return F.embedding(ids, self.embed_w)

    def head(self, h: torch.Tensor) -> torch.Tensor:
        if getattr(self, "ordered", False):
            return O.n2t(O.linear(O.rms_norm(O.t2n(h), O.t2n(self.norm_w), self.cfg.norm_eps), O.t2n(self.lm_head_w)))
        return F.linear(rms_norm(h, self.norm_w, self.cfg.norm_eps), self.lm_head_w)

    # ---- whole-sequence forward of one request (used against HF and as the AR reference)
    def prefill(self, tokens: list, slot: int, capture: bool = False):
        pb = build_packed(self, [OBlock(slot, 0, len(tokens))])
        cap = {} if capture else None
        h = packed_layers(self, self.embed(torch.tensor(tokens)), pb, 0, self.n_layers, cap,
                          tuple(range(1, self.n_layers)))
        logits = self.head(h[-1:])[0]
        hidden = [cap[k][-1] for k in range(1, self.n_layers)] if capture else None
        return logits, hidden


# ----------------------------------------------------------------------------- packed batches

@dataclass
class OBlock:
    row: int
    pos0: int
    T: int
    tag: object = None


@dataclass
class OBucket:
    start: int
    end: int
    b: int
    T: int
    L: int
    rows: Optional[torch.Tensor]
    b0: int
    mask: torch.Tensor
    pad_index: Optional[torch.Tensor] = None


@dataclass
class OPacked:
    blocks: list
    offsets: np.ndarray
    pos: torch.Tensor
    rows: torch.Tensor
    cos: torch.Tensor
    sin: torch.Tensor
    buckets: list = field(default_factory=list)
    n_tokens: int = 0
    kv_read: int = 0
    kv_read_padded: int = 0
    kv_gathered: int = 0


def qo_indptr(lengths) -> np.ndarray:
    return np.concatenate([[0], np.cumsum(np.asarray(lengths, dtype=np.int64))]).astype(np.int64)


def _order_blocks(blocks: list, bucketing: str) -> list:
    key = lambda b: (b.row, b.pos0)  # noqa: E731
    if bucketing == "exact":
        by_T: dict = {}
        for b in blocks:
            by_T.setdefault(b.T, []).append(b)
        return [sorted(by_T[T], key=key) for T in sorted(by_T)]
    if bucketing == "pad":
        return [sorted(blocks, key=key)] if blocks else []
    raise ValueError(bucketing)


def build_packed(model, blocks: list, bucketing: str = "exact") -> OPacked:
    groups = _order_blocks(blocks, bucketing)
    ordered = [b for g in groups for b in g]
    offsets = qo_indptr([b.T for b in ordered])
    N = int(offsets[-1])
    pos = torch.zeros(N, dtype=torch.long)
    rows = torch.zeros(N, dtype=torch.long)
    for i, b in enumerate(ordered):
        pos[offsets[i]:offsets[i + 1]] = torch.arange(b.pos0, b.pos0 + b.T)
        rows[offsets[i]:offsets[i + 1]] = b.row
    cos = model.rope_cos[pos].to(model.dtype).unsqueeze(1)
    sin = model.rope_sin[pos].to(model.dtype).unsqueeze(1)
    pb = OPacked(ordered, offsets, pos, rows, cos, sin, n_tokens=N)
    G, max_seq = model.group, model.cache.max_seq
    first = 0
    for g in groups:
        nb = len(g)
        start, end = int(offsets[first]), int(offsets[first + nb])
        Tm = max(b.T for b in g)
        L = min((max(b.pos0 + b.T - 1 for b in g) + 1 + 63) // 64 * 64, max_seq)
        row_list = [b.row for b in g]
        contiguous = row_list == list(range(row_list[0], row_list[0] + nb))
        qpos = torch.zeros(nb, Tm, dtype=torch.long)
        pad = None
        if bucketing == "pad" and any(b.T != Tm for b in g):
            pad = torch.full((nb, Tm), -1, dtype=torch.long)
        for j, b in enumerate(g):
            qpos[j, :b.T] = torch.arange(b.pos0, b.pos0 + b.T)
            qpos[j, b.T:] = b.pos0 + b.T - 1
            if pad is not None:
                pad[j, :b.T] = torch.arange(int(offsets[first + j]), int(offsets[first + j + 1]))
        allowed = torch.arange(L).view(1, 1, L) <= qpos.unsqueeze(-1)
        mask = allowed.unsqueeze(1).unsqueeze(1).expand(nb, 1, G, Tm, L).reshape(nb, 1, G * Tm, L)
        pb.buckets.append(OBucket(start, end, nb, Tm, L, None if contiguous else torch.tensor(row_list),
                                  row_list[0], mask, pad))
        pb.kv_read += sum(b.pos0 + b.T for b in g)
        pb.kv_read_padded += nb * L
        if not contiguous:
            pb.kv_gathered += nb * L
        first += nb
    return pb


def attend(model, i: int, q: torch.Tensor, pb: OPacked) -> torch.Tensor:
    """Per-bucket masked SDPA over the cache rows of layer i; q [N, Hq, D] -> [N, Hq*D]."""
    if getattr(model, "ordered", False):
        o = O.attend(O.t2n(q), O.t2n(model.cache.k[i]), O.t2n(model.cache.v[i]), pb.rows, pb.pos, model.group)
        return O.n2t(o.reshape(q.shape[0], model.q_size))
    if getattr(model, "attention", "sdpa") == "blocked":
        o = O.attend_bf16_blocked(O.t2n(q), O.t2n(model.cache.k[i]), O.t2n(model.cache.v[i]), pb.rows, pb.pos,
                                  model.group, model.attn_split)
        return O.n2t(o.reshape(q.shape[0], model.q_size)).to(q.dtype)
    G, Hkv, D = model.group, model.cfg.n_kv_heads, model.cfg.head_dim
    ck, cv = model.cache.k[i], model.cache.v[i]
    out = torch.empty(q.shape[0], model.q_size, dtype=q.dtype)
    for bk in pb.buckets:
        sel = slice(bk.b0, bk.b0 + bk.b) if bk.rows is None else bk.rows
        K, V = ck[sel, :, :bk.L], cv[sel, :, :bk.L]
        if bk.pad_index is None:
            qb = q[bk.start:bk.end].view(bk.b, bk.T, Hkv, G, D)
        else:
            qb = q[bk.pad_index.clamp(min=0).view(-1)].view(bk.b, bk.T, Hkv, G, D)
        qg = qb.permute(0, 2, 3, 1, 4).reshape(bk.b, Hkv, G * bk.T, D)
        o = F.scaled_dot_product_attention(qg, K, V, attn_mask=bk.mask)
        o = o.view(bk.b, Hkv, G, bk.T, D).permute(0, 3, 1, 2, 4).reshape(bk.b * bk.T, model.q_size)
        if bk.pad_index is None:
            out[bk.start:bk.end] = o
        else:
            keep = bk.pad_index.view(-1) >= 0
            out[bk.pad_index.view(-1)[keep]] = o[keep]
    return out


def _ordered_ops(model):
    """(norm, linear, act) of the layer: oracle/ordered.py's fixed-order fp32 forms, or torch's."""
    if not getattr(model, "ordered", False):
        return (lambda x, w: rms_norm(x, w, model.cfg.norm_eps)), F.linear, F.silu
    return (lambda x, w: O.n2t(O.rms_norm(O.t2n(x), O.t2n(w), model.cfg.norm_eps)),
            lambda x, w: O.n2t(O.linear(O.t2n(x), O.t2n(w))),
            lambda x: O.n2t(O.silu_f32(O.t2n(x))))


def packed_layer(model, i: int, x: torch.Tensor, pb: OPacked) -> torch.Tensor:
    cfg, lw = model.cfg, model.layers[i]
    N = x.shape[0]
    norm, linear, act = _ordered_ops(model)
    qkv = linear(norm(x, lw.attn_norm), lw.wqkv)
    q = qkv[:, :model.q_size].reshape(N, cfg.n_heads, cfg.head_dim)
    k = qkv[:, model.q_size:model.q_size + model.kv_size].reshape(N, cfg.n_kv_heads, cfg.head_dim)
    v = qkv[:, model.q_size + model.kv_size:].reshape(N, cfg.n_kv_heads, cfg.head_dim)
    q = rope(q, pb.cos, pb.sin)
    k = rope(k, pb.cos, pb.sin)
    model.cache.k[i][pb.rows, :, pb.pos] = k
    model.cache.v[i][pb.rows, :, pb.pos] = v
    x = x + linear(attend(model, i, q, pb), lw.wo)
    g, u = linear(norm(x, lw.ffn_norm), lw.w13).chunk(2, dim=-1)
    return x + linear(act(g) * u, lw.w2)


def packed_layers(model, x, pb, start: int, end: int, capture: Optional[dict] = None, capture_layers: tuple = ()):
    for i in range(start, end):
        x = packed_layer(model, i, x, pb)
        if capture is not None and (i + 1) in capture_layers:
            capture[i + 1] = x
    return x


# ----------------------------------------------------------------------------- brute force

def brute_attention(q: torch.Tensor, kc: torch.Tensor, vc: torch.Tensor, rows, pos, group: int) -> torch.Tensor:
    """fp64 per-token loop: token t (row r, position p), head h attends cache[r, h // G, 0..p]."""
    N, Hq, D = q.shape
    out = torch.zeros(N, Hq, D, dtype=torch.float64)
    scale = 1.0 / math.sqrt(D)
    for t in range(N):
        r, p = int(rows[t]), int(pos[t])
        for h in range(Hq):
            K = kc[r, h // group, :p + 1].double()
            V = vc[r, h // group, :p + 1].double()
            w = torch.softmax((K @ q[t, h].double()) * scale, dim=0)
            out[t, h] = w @ V
    return out.reshape(N, Hq * D)
