"""LayerSkip-Llama on MI355X: weights, static KV cache and RoPE tables in HBM, every op in liblsk.

Same object surface as the reference model (common/model.py:218-403): `cfg`, `device`, `dtype`,
`group`, `q_size`, `kv_size`, `layers[i].{wqkv,wo,w13,w2,attn_norm,ffn_norm}`, `cache.k[i]` /
`cache.v[i]` ([max_batch, Hkv, max_seq, D] views), `cache.max_seq`, `rope_cos` / `rope_sin`,
`embed()`, `head()`, `allocate_cache()`, `free_cache()`, `make_ctx()`, `forward_layers()`,
`prefill()`, `n_layers`.  The padded per-call path (`make_ctx` / `forward_layers`) runs on the same
ragged kernels as the packed path: a [b, T] call is b blocks of T tokens.

HBM layout: one (request, KV head) of a layer is a contiguous max_seq x D stripe that the attention kernel
streams once.  Inside a stripe the bf16 K cache keeps 32-position blocks in MFMA-fragment order and the V
cache keeps 32-position blocks transposed (`KVCache`); `cache.k[i]` / `cache.v[i]` return the reference
[max_batch, Hkv, max_seq, D] layout.  Weights keep the reference's fusion (wqkv = [q; k; v],
w13 = [gate; up], [out, in]); bf16 projection and LM-head weights are stored in the GEMMs' fragment-major
form (`_lsk.PackedWeight`, every 16 x 32 MFMA fragment 1 KiB contiguous), whose `unpack()` gives the
[out, in] tensor back bit for bit; fp32 weights stay row-major.  The RoPE tables are built on the CPU with
the reference's op sequence (common/model.py:113-140) and copied, so they are bitwise the CPU tables.
"""

from __future__ import annotations

import json
import math
from dataclasses import dataclass, field
from pathlib import Path
from typing import Optional

import numpy as np
import torch
from torch import Tensor

from .. import _lsk


# ----------------------------------------------------------------------------- config

@dataclass
class ModelConfig:
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
    bos_token_id: Optional[int] = None
    eos_token_ids: tuple = field(default_factory=tuple)

    @classmethod
    def from_hf_dir(cls, path) -> "ModelConfig":
        """HF config.json (+ generation_config.json eos ids); old and new RoPE formats
        (common/model.py:56-91)."""
        path = Path(path)
        c = json.loads((path / "config.json").read_text())
        eos = c.get("eos_token_id")
        eos_ids = tuple(eos) if isinstance(eos, list) else ((eos,) if eos is not None else ())
        gp = path / "generation_config.json"
        if gp.exists():
            ge = json.loads(gp.read_text()).get("eos_token_id")
            ge = ge if isinstance(ge, list) else ([ge] if ge is not None else [])
            eos_ids = tuple(dict.fromkeys(list(eos_ids) + ge))
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
                   tie_word_embeddings=c.get("tie_word_embeddings", False), rope_scaling=scaling,
                   bos_token_id=c.get("bos_token_id"), eos_token_ids=eos_ids)

    @property
    def kv_bytes_per_token(self) -> int:
        return self.n_layers * 2 * self.n_kv_heads * self.head_dim * 2

    @property
    def layer_param_count(self) -> int:
        attn = self.dim * (self.n_heads + 2 * self.n_kv_heads) * self.head_dim + self.n_heads * self.head_dim * self.dim
        return attn + 3 * self.dim * self.intermediate_size + 2 * self.dim

    @property
    def param_count(self) -> int:
        emb = self.vocab_size * self.dim
        return emb + (0 if self.tie_word_embeddings else emb) + self.n_layers * self.layer_param_count + self.dim


LLAMA3_ROPE_SCALING = {"rope_type": "llama3", "factor": 32.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
                       "original_max_position_embeddings": 8192}

PRESETS = {
    # Llama3-8B shape: 32 layers, hidden 4096, 32 q / 8 kv heads, head_dim 128, FFN 14336, vocab 128256
    "llama3-8b": ModelConfig(128256, 4096, 32, 32, 8, 128, 14336, 1e-5, 500000.0, 8192),
    # Llama3.2-1B shape: 16 layers, hidden 2048, 32 q / 8 kv heads, head_dim 64, FFN 8192, vocab 128256
    "llama3.2-1b": ModelConfig(128256, 2048, 16, 32, 8, 64, 8192, 1e-5, 500000.0, 131072,
                               rope_scaling=dict(LLAMA3_ROPE_SCALING)),
    # Llama2-7B shape: 32 layers, hidden 4096, 32 MHA heads, head_dim 128, FFN 11008, vocab 32000
    "llama2-7b": ModelConfig(32000, 4096, 32, 32, 32, 128, 11008, 1e-5, 10000.0, 4096),
}


# ----------------------------------------------------------------------------- rope

def _llama3_inv_freq(inv_freq: Tensor, scaling: dict) -> Tensor:
    factor, lo, hi = scaling["factor"], scaling["low_freq_factor"], scaling["high_freq_factor"]
    old = scaling["original_max_position_embeddings"]
    wavelen = 2 * math.pi / inv_freq
    base = torch.where(wavelen > old / lo, inv_freq / factor, inv_freq)
    smooth = (old / wavelen - lo) / (hi - lo)
    mixed = (1 - smooth) * base / factor + smooth * base
    medium = ~(wavelen < old / hi) & ~(wavelen > old / lo)
    return torch.where(medium, mixed, base)


def build_rope_cache(cfg: ModelConfig, max_seq: int, device) -> tuple[Tensor, Tensor]:
    """fp32 [max_seq, D] cos/sin, computed on the CPU (common/model.py:129-140) and copied to the device."""
    inv = 1.0 / (cfg.rope_theta ** (torch.arange(0, cfg.head_dim, 2, dtype=torch.int64).float() / cfg.head_dim))
    sc = cfg.rope_scaling or {}
    kind = sc.get("rope_type", sc.get("type"))
    if kind == "llama3":
        inv = _llama3_inv_freq(inv, sc)
    elif kind not in (None, "default"):
        raise NotImplementedError(f"rope_scaling type {kind!r} is not supported")
    ang = torch.outer(torch.arange(max_seq, dtype=torch.float32), inv)
    ang = torch.cat([ang, ang], dim=-1)
    return ang.cos().contiguous().to(device), ang.sin().contiguous().to(device)


# ----------------------------------------------------------------------------- weights / cache

@dataclass
class LayerWeights:
    """One layer's weights (common/model.py:161-168).  The four projections are GEMM weights: a
    `_lsk.PackedWeight` for bf16 (`.unpack()` -> [out, in]; wqkv packed for the fused qkv + RoPE GEMM when the
    head shape is given), the row-major tensor for fp32."""
    wqkv: object
    wo: object
    w13: object
    w2: object
    attn_norm: Tensor
    ffn_norm: Tensor

    @classmethod
    def from_dense(cls, wqkv: Tensor, wo: Tensor, w13: Tensor, w2: Tensor, attn_norm: Tensor,
                   ffn_norm: Tensor, qkv_heads: tuple | None = None) -> "LayerWeights":
        """qkv_heads = (n_heads, n_kv_heads, head_dim): a bf16 wqkv is stored for the fused qkv + RoPE GEMM."""
        g = _lsk.as_gemm_weight
        if qkv_heads is not None and wqkv.dtype == torch.bfloat16:
            pq = _lsk.PackedWeight(wqkv, qkv_heads=qkv_heads)
        else:
            pq = g(wqkv)
        return cls(pq, g(wo), g(w13), g(w2), attn_norm, ffn_norm)


_INPLACE_DUNDERS = {"__setitem__", "__iadd__", "__isub__", "__imul__", "__itruediv__", "__ifloordiv__",
                    "__imod__", "__ipow__", "__iand__", "__ior__", "__ixor__", "__ilshift__", "__irshift__"}


class DecodedCacheView(Tensor):
    """A decoded copy of one layer's K or V cache in the reference's [max_batch, Hkv, max_seq, D] layout.  The
    kernels keep their own storage (fragment-major K, blocked V^T), so a write into this copy would never reach
    the cache: every in-place operation on it or on a view of it (`view[rows, :, pos] = k`, `index_put_`,
    `copy_`, `out=` ...) raises instead of being lost.  Out-of-place results (clone, .cpu(), arithmetic) are
    ordinary tensors."""

    @classmethod
    def __torch_function__(cls, func, types, args=(), kwargs=None):
        kwargs = kwargs or {}
        name = getattr(func, "__name__", "")
        inplace = name in _INPLACE_DUNDERS or (name.endswith("_") and not name.startswith("_"))
        target = args[0] if args else None
        if (inplace and isinstance(target, DecodedCacheView)) or any(
                isinstance(o, DecodedCacheView) for o in _as_list(kwargs.get("out"))):
            raise _lsk.LskError(
                f"{name} on a decoded KV-cache view: cache.k[i] / cache.v[i] are copies of the kernels' storage "
                "(fragment-major K, blocked V^T), so the write would be lost; append with "
                "thesis_amd._lsk.kv_append (lsk_kv_append) or write cache.kstore[i] / cache.vb[i] through "
                "_lsk.k_to_frag / _lsk.v_to_blocked")
        with torch._C.DisableTorchFunctionSubclass():
            out = func(*args, **kwargs)
        src = target if isinstance(target, Tensor) else None
        if (isinstance(out, Tensor) and src is not None and out.device == src.device and out.numel()
                and out.untyped_storage().data_ptr() == src.untyped_storage().data_ptr()):
            return out.as_subclass(DecodedCacheView)            # a view of the copy stays guarded
        return out


def _as_list(o):
    if o is None:
        return []
    return list(o) if isinstance(o, (list, tuple)) else [o]


class _Decoded:
    """cache.k[i] / cache.v[i] of a layout the kernels store differently: layer i in the reference's
    [max_batch, Hkv, max_seq, D] layout, as a copy for inspection whose in-place writes raise
    (DecodedCacheView); the kernels write the storage."""

    def __init__(self, store: Tensor, decode):
        self.store, self.decode = store, decode

    def __getitem__(self, i):
        return self.decode(self.store[i]).as_subclass(DecodedCacheView)

    def __len__(self):
        return self.store.shape[0]


class KVCache:
    """Static contiguous KV cache, per layer, zero-initialised.
    K (bf16): kf_all [L, max_batch, Hkv, max_seq/32, D/16, 64, 8], fragment-major 32-position blocks (every
      16-position x 32-d MFMA fragment 1 KiB contiguous in lane order, `_lsk.k_to_frag`); K (fp32): k_all
      [L, max_batch, Hkv, max_seq, D] row-major.
    V: vb_all [L, max_batch, Hkv, max_seq/32, D, 32], 32-position blocks each transposed, so every V^T MFMA
      fragment is 1 KiB contiguous as well.
    `kstore[i]` / `vb[i]` are the per-layer storage tensors the kernels use; k[i] / v[i] and k_all / v_all
    present the reference's [max_batch, Hkv, max_seq, D] layout (views for fp32 K, copies otherwise)."""

    def __init__(self, cfg: ModelConfig, max_batch: int, max_seq: int, dtype, device):
        if max_seq % 64:
            raise ValueError("max_seq must be a multiple of 64")
        self.max_batch, self.max_seq = max_batch, max_seq
        L, Hkv, D = cfg.n_layers, cfg.n_kv_heads, cfg.head_dim
        self.frag_k = dtype == torch.bfloat16
        if self.frag_k:
            if D % 32:
                raise ValueError("bf16 caches need head_dim % 32 == 0")
            self.kf_all = torch.zeros((L, max_batch, Hkv, max_seq // 32, D // 16, 64, 8), dtype=dtype, device=device)
            self.kstore = [self.kf_all[i] for i in range(L)]
            self.k = _Decoded(self.kf_all, _lsk.k_from_frag)
        else:
            self._k_rows = torch.zeros((L, max_batch, Hkv, max_seq, D), dtype=dtype, device=device)
            self.kstore = [self._k_rows[i] for i in range(L)]
            self.k = self.kstore
        self.vb_all = torch.zeros((L, max_batch, Hkv, max_seq // 32, D, 32), dtype=dtype, device=device)
        self.vb = [self.vb_all[i] for i in range(L)]
        self.v = _Decoded(self.vb_all, _lsk.v_from_blocked)
        # KV positions per flash-decoding split of the attention kernel, fixed for the cache's lifetime so that
        # a query's result never depends on the batch it is packed in.  Measured on MI355X: 256 requests x 8 KV
        # heads with median-1500 contexts (up to 8192) stream best unsplit up to 8192 positions (2048-position
        # splits 7 % and 4096-position splits 3 % slower: more work items, split partials and the combine
        # launch); a B = 32 decode batch runs unsplit up to 2048 positions, its launches using the deep-prefetch
        # kernel.  The fp32 path does not split.
        if dtype == torch.bfloat16:
            self.attn_split = _lsk.ATTN_SPLIT if max_batch * cfg.n_kv_heads >= 1024 else 2048
        else:
            self.attn_split = 1 << 30

    @property
    def k_all(self) -> Tensor:
        return _lsk.k_from_frag(self.kf_all).as_subclass(DecodedCacheView) if self.frag_k else self._k_rows

    @property
    def v_all(self) -> Tensor:
        return _lsk.v_from_blocked(self.vb_all).as_subclass(DecodedCacheView)

    @staticmethod
    def bytes_needed(cfg: ModelConfig, max_batch: int, max_seq: int, dtype_bytes: int = 2) -> int:
        return cfg.n_layers * 2 * max_batch * cfg.n_kv_heads * max_seq * cfg.head_dim * dtype_bytes


@dataclass
class AttnCtx:
    """Per-call metadata of the padded path (common/model.py:186-211): b blocks of T tokens."""
    pos: Tensor
    b0: int
    L: int
    bidx: Tensor
    causal_prefill: bool
    rows: Optional[Tensor]
    pb: object  # PackedBatch over the call's blocks, in call order

    @property
    def batch(self) -> int:
        return self.pos.shape[0]

    @property
    def tokens(self) -> int:
        return self.pos.shape[0] * self.pos.shape[1]

    @property
    def kv_read(self) -> int:
        return self.pos.shape[0] * self.L


def _round_up(x: int, m: int) -> int:
    return (x + m - 1) // m * m


class LayerSkipLlama:
    """Inference-only LayerSkip-Llama whose forward runs in liblsk (no torch compute ops)."""

    def __init__(self, cfg: ModelConfig, embed: Tensor, layers: list, norm: Tensor, lm_head: Tensor, device, dtype,
                 max_seq: int):
        self.device = torch.device(device)
        if self.device.type == "cuda" and self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        if self.device.type != "cuda":
            raise _lsk.LskError("LayerSkipLlama runs on the GPU only (liblsk kernels); the CPU oracle lives in "
                                "oracle/ for tests")
        _lsk.load()
        self.cfg, self.dtype = cfg, dtype
        _lsk.dtype_code(dtype)
        self.embed_w, self.layers, self.norm_w, self.lm_head_w = embed, layers, norm, lm_head
        self.group = cfg.n_heads // cfg.n_kv_heads
        self.q_size = cfg.n_heads * cfg.head_dim
        self.kv_size = cfg.n_kv_heads * cfg.head_dim
        self.rope_cos, self.rope_sin = build_rope_cache(cfg, max_seq, self.device)
        self.cache: Optional[KVCache] = None
        self.native: Optional[_lsk.NativeModel] = None
        self._ws: Optional[Tensor] = None
        self._bufs: dict = {}
        # bumped whenever a reusable device buffer, the cache or the native handle is (re)allocated: captured
        # step graphs hold their addresses and are dropped when it changes
        self.buf_epoch = 0

    # ---------------------------------------------------------------- construction
    @classmethod
    def from_weights(cls, cfg: ModelConfig, weights: dict, device="cuda", dtype=torch.bfloat16,
                     max_seq: Optional[int] = None) -> "LayerSkipLlama":
        """HF-named tensors (any device / dtype) -> fused device layout (common/model.py:259-276)."""

        def take(k):
            return weights[k].to(device=device, dtype=dtype).contiguous()

        layers = []
        for i in range(cfg.n_layers):
            p = f"model.layers.{i}."
            wqkv = torch.cat([weights[p + "self_attn.q_proj.weight"], weights[p + "self_attn.k_proj.weight"],
                              weights[p + "self_attn.v_proj.weight"]], dim=0).to(device=device, dtype=dtype)
            w13 = torch.cat([weights[p + "mlp.gate_proj.weight"], weights[p + "mlp.up_proj.weight"]],
                            dim=0).to(device=device, dtype=dtype)
            layers.append(LayerWeights.from_dense(wqkv.contiguous(), take(p + "self_attn.o_proj.weight"),
                                                  w13.contiguous(), take(p + "mlp.down_proj.weight"),
                                                  take(p + "input_layernorm.weight"),
                                                  take(p + "post_attention_layernorm.weight"),
                                                  (cfg.n_heads, cfg.n_kv_heads, cfg.head_dim)))
            del wqkv, w13
        embed = take("model.embed_tokens.weight")
        norm = take("model.norm.weight")
        lm_head = _lsk.as_gemm_weight(take("lm_head.weight") if "lm_head.weight" in weights else embed)
        return cls(cfg, embed, layers, norm, lm_head, device, dtype, max_seq or cfg.max_position_embeddings)

    @classmethod
    def from_pretrained(cls, path, device="cuda", dtype=torch.bfloat16, max_seq: Optional[int] = None):
        from safetensors import safe_open

        path = Path(path)
        cfg = ModelConfig.from_hf_dir(path)
        idx = path / "model.safetensors.index.json"
        files = sorted(set(json.loads(idx.read_text())["weight_map"].values())) if idx.exists() else \
            ["model.safetensors"]
        raw = {}
        for f in files:
            with safe_open(str(path / f), framework="pt", device="cpu") as fh:
                for k in fh.keys():
                    raw[k] = fh.get_tensor(k)
        return cls.from_weights(cfg, raw, device, dtype, max_seq)

    @classmethod
    def random(cls, cfg: ModelConfig, seed: int = 0, device="cuda", dtype=torch.bfloat16, std: float = 0.02,
               max_seq: Optional[int] = None) -> "LayerSkipLlama":
        """Seeded random init generated on the device (N(0, std) matrices, unit norms): the synthetic
        weights of the benchmark configurations (no checkpoint download)."""
        g = torch.Generator(device=device).manual_seed(seed)
        qd, kvd = cfg.n_heads * cfg.head_dim, cfg.n_kv_heads * cfg.head_dim

        def mat(r, c):
            t = torch.empty(r, c, dtype=dtype, device=device)
            return t.normal_(0.0, std, generator=g)

        def ones(n):
            return torch.ones(n, dtype=dtype, device=device)

        layers = [LayerWeights.from_dense(mat(qd + 2 * kvd, cfg.dim), mat(cfg.dim, qd),
                                          mat(2 * cfg.intermediate_size, cfg.dim), mat(cfg.dim, cfg.intermediate_size),
                                          ones(cfg.dim), ones(cfg.dim), (cfg.n_heads, cfg.n_kv_heads, cfg.head_dim))
                  for _ in range(cfg.n_layers)]
        embed = mat(cfg.vocab_size, cfg.dim)
        lm_head = _lsk.as_gemm_weight(embed if cfg.tie_word_embeddings else mat(cfg.vocab_size, cfg.dim))
        return cls(cfg, embed, layers, ones(cfg.dim), lm_head, device, dtype, max_seq or cfg.max_position_embeddings)

    @property
    def n_layers(self) -> int:
        return self.cfg.n_layers

    # ---------------------------------------------------------------- cache
    def allocate_cache(self, max_batch: int, max_seq: int) -> KVCache:
        max_seq = _round_up(max_seq, 64)
        if max_seq > self.rope_cos.shape[0]:
            self.rope_cos, self.rope_sin = build_rope_cache(self.cfg, max_seq, self.device)
        self.cache = None
        self.native = None
        self.buf_epoch += 1
        self.cache = KVCache(self.cfg, max_batch, max_seq, self.dtype, self.device)
        c = self.cfg
        self.native = _lsk.NativeModel(self.dtype, c.n_layers, c.dim, c.n_heads, c.n_kv_heads, c.head_dim,
                                       c.intermediate_size, c.vocab_size, c.norm_eps, self.layers, self.cache.kstore,
                                       self.cache.vb, self.rope_cos, self.rope_sin)
        return self.cache

    def free_cache(self) -> None:
        self.cache = None
        self.native = None
        self.buf_epoch += 1
        torch.cuda.empty_cache()

    # ---------------------------------------------------------------- scratch
    def workspace(self, nbytes: int) -> Tensor:
        if self._ws is None or self._ws.numel() < nbytes:
            self._ws = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=self.device)
            self.buf_epoch += 1
        return self._ws

    def buffer(self, name: str, shape: tuple, dtype) -> Tensor:
        """Named reusable device buffer (grown on demand; stream-ordered reuse)."""
        n = int(np.prod(shape)) if shape else 1
        b = self._bufs.get((name, dtype))
        if b is None or b.numel() < n:
            b = torch.empty(max(n, 1), dtype=dtype, device=self.device)
            self._bufs[(name, dtype)] = b
            self.buf_epoch += 1
        return b[:n].view(shape)

    # ---------------------------------------------------------------- building blocks
    def embed(self, tokens: Tensor) -> Tensor:
        ids = tokens.reshape(-1).to(device=self.device, dtype=torch.long)
        out = torch.empty(ids.numel(), self.cfg.dim, dtype=self.dtype, device=self.device)
        _lsk.embed(self.embed_w, ids, out)
        return out.view(*tokens.shape, self.cfg.dim)

    def head(self, h: Tensor) -> Tensor:
        """Final norm + shared LM head (common/model.py:328-330) -> logits [.., V] in the model dtype."""
        shp = h.shape
        x = h.reshape(-1, shp[-1]).contiguous()
        xn = _lsk.rmsnorm(x, self.norm_w, self.cfg.norm_eps)
        return _lsk.gemm(xn, self.lm_head_w).view(*shp[:-1], self.cfg.vocab_size)

    def head_argmax(self, h: Tensor, out: Optional[Tensor] = None, dst_idx: Optional[Tensor] = None) -> Tensor:
        """argmax(head(h)) per row (first index on ties, over dtype-rounded logits); int64.
        With dst_idx the ids are scattered to out[dst_idx[m]] (e.g. into the engine's seq_buf)."""
        x = h.reshape(-1, h.shape[-1]).contiguous()
        n = x.shape[0]
        if out is None:
            out = torch.empty(n, dtype=torch.long, device=self.device)
        if n == 0:
            return out
        es, dim, V = self.dtype.itemsize, self.cfg.dim, self.cfg.vocab_size
        P = _lsk.Profiler
        if self.dtype == torch.bfloat16:
            # final norm + LM head with a per-tile argmax + the pick over tiles, one native call (no logits
            # materialised; up to 64 rows the normalised rows stay in the GEMM's fragment order)
            ws = self.buffer("head_ws", (int(_lsk.load().lsk_head_norm_workspace_bytes(n, V, dim)),), torch.uint8)
            P.start(7, es * (float(V) * dim + 3.0 * n * dim + dim), 2.0 * n * dim * V)
            _lsk.head_norm_argmax(x, self.norm_w, self.cfg.norm_eps, self.lm_head_w, out, dst_idx, workspace=ws)
            P.stop()
            return out
        xn = self.buffer("head_xn", (n, dim), self.dtype)
        P.start(0, es * (2.0 * n * dim + dim), 4.0 * n * dim)
        _lsk.rmsnorm(x, self.norm_w, self.cfg.norm_eps, out=xn)
        P.stop()
        logits = self.buffer("head_logits", (n, V), self.dtype)
        P.start(7, es * (float(V) * dim + n * dim + n * V), 2.0 * n * dim * V)
        _lsk.gemm(xn, self.lm_head_w, out=logits)
        P.stop()
        P.start(8, es * float(n) * V, float(n) * V)
        _lsk.argmax(logits, out, dst_idx)
        P.stop()
        return out

    # ---------------------------------------------------------------- padded path (DecodeEngine)
    def make_ctx(self, pos: Tensor, b0: int = 0, max_pos: Optional[int] = None, causal_prefill: bool = False,
                 rows: Optional[Tensor] = None) -> AttnCtx:
        """pos [b, T] (consecutive positions per row).  Every call is b ragged blocks of T tokens; the
        causal-prefill branch of common/model.py:346-351 is the same rule (query p reads 0..p)."""
        from ..solutions.packed import Block, pack_blocks

        pos_h = pos.detach().to("cpu").numpy().astype(np.int64)
        b, T = pos_h.shape
        if T > 1 and not (np.diff(pos_h, axis=1) == 1).all():
            raise ValueError("make_ctx: positions of a row must be consecutive")
        rows_h = rows.detach().to("cpu").numpy().astype(np.int64) if rows is not None else np.arange(b) + b0
        if max_pos is None:
            max_pos = int(pos_h.max())
        L = min(_round_up(max_pos + 1, 64), self.cache.max_seq)
        blocks = [Block(int(rows_h[i]), int(pos_h[i, 0]), T) for i in range(b)]
        pb = pack_blocks(self, blocks)
        bidx = torch.as_tensor(rows_h).view(b, 1).expand(b, T)
        return AttnCtx(pos, b0, L, bidx, causal_prefill, rows, pb)

    def forward_layers(self, h: Tensor, start: int, end: int, ctx: AttnCtx, capture: Optional[list] = None,
                       layer_hook=None) -> Tensor:
        """Layers [start, end) on h [b, T, dim].  capture (list) receives every layer's output;
        layer_hook(i, "pre"/"post") forces a per-layer call (used for per-layer timing)."""
        from ..solutions.packed import packed_layers

        b, T, dim = h.shape
        x = h.reshape(b * T, dim).contiguous()
        if layer_hook is None:
            if capture is None:
                return packed_layers(self, x, ctx.pb, start, end).view(b, T, dim)
            cap = {}
            out = packed_layers(self, x, ctx.pb, start, end, cap, tuple(range(start + 1, end + 1)))
            capture.extend(cap[j].view(b, T, dim) for j in range(start + 1, end + 1))
            return out.view(b, T, dim)
        for i in range(start, end):
            if layer_hook is not None:
                layer_hook(i, "pre")
            x = packed_layers(self, x, ctx.pb, i, i + 1)
            if layer_hook is not None:
                layer_hook(i, "post")
            if capture is not None:
                capture.append(x.view(b, T, dim))
        return x.view(b, T, dim)

    @torch.inference_mode()
    def prefill(self, tokens: list, slot: int, capture_exits: bool = False):
        """Prefill one request into cache row `slot` (common/model.py:392-403).  Returns (last-position
        logits [V], hidden states after every layer at the last position if capture_exits)."""
        from ..solutions.packed import Block, pack_blocks, packed_layers

        n = len(tokens)
        pb = pack_blocks(self, [Block(slot, 0, n)])
        x = self.embed(torch.tensor(tokens, dtype=torch.long))
        if capture_exits:
            cap = {}
            h = packed_layers(self, x, pb, 0, self.n_layers, cap, tuple(range(1, self.n_layers + 1)))
            hidden = [cap[k][-1] for k in range(1, self.n_layers + 1)]
        else:
            h = packed_layers(self, x, pb, 0, self.n_layers)
            hidden = None
        logits = self.head(h[-1:])[0]
        return logits, hidden
