"""Per-layer cost model consumed by the schedulers (solutions/cost_model.py surface; host-only NumPy).

    t_layer(n, C) = max(W / BW, 2 P n / F) + KV(C) / BW + n_op * t_op                 (roofline)

W / P = bytes / parameters of one decoder layer, n = tokens through the layer, C = cached positions
read by attention, BW / F = bandwidth and bf16 GEMM throughput, t_op x n_op = launch overhead
(solutions/cost_model.py:1-31).  `LinearCostModel` is the ASPIRE-style a + b n + c C variant.
`mi355x_cost_model` fills the GPU parameters from MI355X's published peaks scaled by the fractions
the package's kernels reach (measured by bench.py); `synthetic_cost_model` keeps the reference's
made-up constants for CPU tests (solutions/cost_model.py:220-227).
"""

from __future__ import annotations

import json
from dataclasses import asdict, dataclass, field
from pathlib import Path
from typing import Optional

import numpy as np


@dataclass
class ModelDims:
    n_layers: int
    dim: int
    vocab: int
    layer_params: int
    head_params: int
    kv_bytes_per_pos: int
    dtype_bytes: int = 2

    @property
    def layer_bytes(self) -> int:
        return self.layer_params * self.dtype_bytes

    @property
    def head_bytes(self) -> int:
        return self.head_params * self.dtype_bytes

    @classmethod
    def from_config(cls, cfg, dtype_bytes: int = 2) -> "ModelDims":
        return cls(cfg.n_layers, cfg.dim, cfg.vocab_size, cfg.layer_param_count, cfg.vocab_size * cfg.dim + cfg.dim,
                   2 * cfg.n_kv_heads * cfg.head_dim * dtype_bytes, dtype_bytes)


@dataclass
class GPUParams:
    bw: float                  # bytes / ms
    flops: float               # flop / ms
    t_op: float                # ms per launch
    n_op_layer: float
    n_op_bucket: float
    n_op_head: float
    n_op_segment: float
    meta: dict = field(default_factory=dict)
    flops_eff: Optional[float] = None
    knee_measured: Optional[float] = None


class _Base:
    dims: ModelDims

    def t_segment(self, n_layers: int, n, C, buckets: int = 1):
        n = np.asarray(n)
        if not n_layers:
            return np.zeros_like(n, dtype=np.float64)
        t = n_layers * (self.layer_gemm_ms(n) + self.kv_ms(C) + self.layer_ops_ms(buckets)) + self.segment_ops_ms()
        if n.ndim == 0:
            return t if n > 0 else 0.0
        return t if n.min() > 0 else np.where(n > 0, t, 0.0)

    def t_sh(self, B, k: int, C):
        return self.t_segment(k, B, C) + self.head_ms(B)

    def t_deep(self, n, k: int, C, n_req, buckets: int = 1, C_deep=None):
        Cd = C if C_deep is None else C_deep
        return self.t_segment(k, n_req, C) + self.t_segment(self.dims.n_layers - k, n, Cd, buckets) + self.head_ms(n)

    def t_prefill(self, n, C):
        return self.t_segment(self.dims.n_layers, n, C) + self.head_ms(1)

    def t_ar(self, B, C):
        return self.t_segment(self.dims.n_layers, B, C) + self.head_ms(B)

    def best_rate(self, alpha: float, B: int, k: int, C: float, d_max: int = 16) -> float:
        a = min(max(alpha, 0.0), 1 - 1e-6)
        s = np.arange(d_max + 1)
        tok = B * (1 - a ** (s + 1)) / (1 - a)
        return float(np.max(tok / (s * self.t_sh(B, k, C) + self.t_deep(B * (s + 1), k, C, B))))


class RooflineCostModel(_Base):
    kind = "roofline"

    def __init__(self, gpu: GPUParams, dims: ModelDims, n_max: int = 16384, variant: str = "measured"):
        self.gpu, self.dims, self.variant = gpu, dims, variant
        self.F = float(gpu.flops_eff) if (variant == "measured" and gpu.flops_eff) else float(gpu.flops)
        n = np.arange(n_max + 1, dtype=np.float64)
        self._layer = np.maximum(dims.layer_bytes / gpu.bw, 2.0 * dims.layer_params * n / self.F)
        self._head = np.maximum(dims.head_bytes / gpu.bw, 2.0 * dims.head_params * n / self.F)
        self._n_max = n_max

    def _look(self, tab, n, w, p):
        n = np.asarray(n)
        if n.dtype.kind in "iu":                     # the common cases: table entries (same values)
            if n.ndim == 0:
                v = int(n)
                return tab[max(v, 0)] if v <= self._n_max else max(w / self.gpu.bw, 2.0 * p * v / self.F)
            if n.size and n.min() >= 0 and n.max() <= self._n_max:
                return tab[n]
        exact = np.maximum(w / self.gpu.bw, 2.0 * p * n / self.F)
        return np.where(n <= self._n_max, tab[np.clip(n, 0, self._n_max).astype(np.int64)], exact)

    def layer_gemm_ms(self, n):
        return self._look(self._layer, n, self.dims.layer_bytes, self.dims.layer_params)

    def head_ms(self, n):
        n = np.asarray(n)
        t = self._look(self._head, n, self.dims.head_bytes, self.dims.head_params) + self.gpu.n_op_head * self.gpu.t_op
        if n.ndim == 0:
            return t if n > 0 else 0.0
        return t if n.size and n.min() > 0 else np.where(n > 0, t, 0.0)

    def kv_ms(self, C):
        if isinstance(C, (int, float, np.integer, np.floating)):
            return float(C) * self.dims.kv_bytes_per_pos / self.gpu.bw
        return np.asarray(C, dtype=np.float64) * self.dims.kv_bytes_per_pos / self.gpu.bw

    def layer_ops_ms(self, buckets: int = 1):
        return (self.gpu.n_op_layer + self.gpu.n_op_bucket * max(buckets - 1, 0)) * self.gpu.t_op

    def segment_ops_ms(self):
        return self.gpu.n_op_segment * self.gpu.t_op

    def knee(self, k: Optional[int] = None) -> float:
        if self.variant == "measured" and self.gpu.knee_measured:
            return float(self.gpu.knee_measured)
        return self.F * self.dims.layer_bytes / (2.0 * self.dims.layer_params * self.gpu.bw)


class LinearCostModel(_Base):
    kind = "linear"

    def __init__(self, a, b, c, head_a, head_b, dims: ModelDims, seg_ms: float = 0.0):
        self.a, self.b, self.c, self.head_a, self.head_b, self.dims, self.seg = a, b, c, head_a, head_b, dims, seg_ms

    def layer_gemm_ms(self, n):
        return self.a + self.b * np.asarray(n, dtype=np.float64)

    def head_ms(self, n):
        n = np.asarray(n, dtype=np.float64)
        return np.where(n > 0, self.head_a + self.head_b * n, 0.0)

    def kv_ms(self, C):
        return self.c * np.asarray(C, dtype=np.float64)

    def layer_ops_ms(self, buckets: int = 1):
        return 0.0

    def segment_ops_ms(self):
        return self.seg

    def knee(self, k: Optional[int] = None) -> float:
        return float("inf")


def synthetic_cost_model(cfg, kind: str = "roofline"):
    """The reference's deterministic made-up GPU (tests and dry runs only)."""
    dims = ModelDims.from_config(cfg)
    gpu = GPUParams(bw=1.0e9, flops=1.6e11, t_op=0.003, n_op_layer=52, n_op_bucket=12, n_op_head=11, n_op_segment=20,
                    meta={"source": "synthetic (tests only)"}, flops_eff=1.0e11, knee_measured=100.0)
    if kind in ("roofline", "roofline-peak"):
        return RooflineCostModel(gpu, dims, variant="measured" if kind == "roofline" else "peak")
    return LinearCostModel(0.6, 0.002, 4e-6, 1.2, 0.007, dims)


def mi355x_cost_model(cfg, bw_frac: float = 0.7, flops_frac: float = 0.5, t_op_ms: float = 0.004):
    """MI355X: HBM3E 8 TB/s, dense bf16 MFMA 2.5 PFLOP/s, scaled by the fractions the kernels reach.
    Launch terms follow the package's bf16 layer runner: 8 launches per layer (norm, QKV with RoPE + KV append,
    attention, combine, O, norm, W13, W2), 3 per head (norm, GEMM, argmax), ~4 per segment."""
    dims = ModelDims.from_config(cfg)
    gpu = GPUParams(bw=8.0e9 * bw_frac, flops=2.5166e12, t_op=t_op_ms, n_op_layer=8, n_op_bucket=0, n_op_head=3,
                    n_op_segment=4, meta={"source": "MI355X peaks x achieved fractions", "bw_frac": bw_frac,
                                          "flops_frac": flops_frac},
                    flops_eff=2.5166e12 * flops_frac)
    return RooflineCostModel(gpu, dims)


CALIBRATION_DIR = Path(__file__).resolve().parent / "calibration"


def calibration_path(model_name: str) -> Path:
    """Where the MI355X calibration of a preset model shape is kept (written by thesis_amd.solutions.calibrate)."""
    return CALIBRATION_DIR / f"{model_name}_mi355x.json"


def default_cost_model(cfg, kind: str = "roofline"):
    """(model, source): the MI355X calibration of the preset whose shape equals cfg when one is kept in the
    package (as the reference's drivers load <calibration dir>/<model>.json, solutions/run_ablation.py:183-195),
    else `mi355x_cost_model`."""
    from ..common.model import PRESETS

    for name, pc in PRESETS.items():
        p = calibration_path(name)
        if pc == cfg and p.exists():
            return load_cost_model(p, cfg, kind), f"{kind}, calibrated on MI355X ({name})"
    return mi355x_cost_model(cfg), "roofline, MI355X published peaks x achieved fractions"


def load_cost_model(path, cfg, kind: str = "roofline"):
    d = json.loads(Path(path).read_text())
    dims = ModelDims.from_config(cfg)
    if kind in ("roofline", "roofline-peak"):
        return RooflineCostModel(GPUParams(**d["gpu"]), dims, variant="measured" if kind == "roofline" else "peak")
    if kind == "linear":
        lin = d.get("linear")
        if lin is None:
            raise ValueError(f"{path} has no linear fit")
        return LinearCostModel(lin["a"], lin["b"], lin["c"], lin["head_a"], lin["head_b"], dims, lin.get("seg_ms", 0.0))
    raise ValueError(kind)


def save_json(path, obj: dict) -> None:
    Path(path).parent.mkdir(parents=True, exist_ok=True)
    Path(path).write_text(json.dumps(obj, indent=2, default=lambda o: asdict(o) if hasattr(o, "__dataclass_fields__")
                                     else str(o)))
