"""ctypes binding of liblsk.so, the C ABI of the gfx950 kernels (include/lsk.h).

Only device pointers, sizes and the current HIP stream cross the boundary.  Tensors stay owned by
PyTorch (device memory + streams are plumbing; every FLOP of the packed forward runs in liblsk).
There is no fallback: a missing or stale library raises at the first call.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np
import torch

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "liblsk.so"

DTYPE_F32 = 0
DTYPE_BF16 = 1
EPI_NONE, EPI_RESIDUAL, EPI_SILU_MUL = 0, 1, 2
EPI_PARTIAL, EPI_ARGMAX, EPI_QKV_ROPE = 3, 4, 5   # launch kinds known to lsk_gemm_wide_config
ATTN_SPLIT = 8192         # LSK_ATTN_SPLIT
ATTN_ROWS = 48            # query rows per attention work item (csrc/lsk_attention.hip ATTN_ROWS)
ABI_VERSION = 11

# name -> (restype, argtypes)
_P, _I, _L, _F, _Z = ctypes.c_void_p, ctypes.c_int, ctypes.c_long, ctypes.c_float, ctypes.c_size_t
_SIGS = {
    "lsk_last_error": (ctypes.c_char_p, []),
    "lsk_abi_version": (_I, []),
    "lsk_rmsnorm": (_I, [_I, _P, _P, _P, _I, _I, _F, _L, _L, _P]),
    "lsk_rope_append": (_I, [_I, _P, _P, _P, _P, _P, _P, _I, _P, _P, _I, _I, _I, _I, _I, _I, _P]),
    "lsk_kv_append": (_I, [_I, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P]),
    "lsk_attn_plan": (_I, [_P, _I, _I, _I, _I, _P, _I, _P, _I, _P, _P, _P]),
    "lsk_attn_rows_cap": (_I, [_P, _I, _I, _I, _I, _I, _I]),
    "lsk_attn_schedule": (_I, [_P, _I, _I, _I, _P, _I, _P]),
    "lsk_pack_segment": (_I, [_P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _P, _L, _P]),
    "lsk_attn_workspace_bytes": (_Z, [_I, _I, _I]),
    "lsk_ragged_attn": (_I, [_I, _P, _P, _P, _P, _P, _I, _P, _I, _I, _P, _I, _I, _I, _P, _I, _I, _I, _I, _F, _P,
                             _Z, _P]),
    "lsk_ragged_attn_static_scratch_bytes": (_Z, []),
    "lsk_ragged_attn_static": (_I, [_I, _P, _P, _P, _P, _P, _I, _P, _I, _I, _P, _I, _I, _I, _P, _I, _I, _I, _I, _F,
                                    _P]),
    "lsk_pack_weight": (_I, [_P, _L, _P, _I, _I, _P]),
    "lsk_unpack_weight": (_I, [_P, _P, _L, _I, _I, _P]),
    "lsk_pack_weight_qkv": (_I, [_P, _L, _P, _I, _I, _I, _I, _P]),
    "lsk_unpack_weight_qkv": (_I, [_P, _P, _L, _I, _I, _I, _I, _P]),
    "lsk_gemm_qkv_rope": (_I, [_P, _P, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _I, _P, _P, _I, _I, _P]),
    "lsk_gemm": (_I, [_I, _P, _L, _P, _L, _P, _L, _P, _L, _I, _I, _I, _I, _I, _P]),
    "lsk_gemm_plan": (_I, [_I, _I, _P, _P]),
    "lsk_gemm_wide_config": (_I, [_I, _I, _I, _I, _I, _I, _P]),
    "lsk_gemm_partial": (_I, [_P, _L, _P, _L, _P, _I, _I, _I, _I, _P]),
    "lsk_head_workspace_bytes": (_Z, [_I, _I]),
    "lsk_head_argmax": (_I, [_I, _P, _L, _P, _L, _I, _I, _I, _P, _L, _P, _P, _P, _Z, _P]),
    "lsk_head_norm_workspace_bytes": (_Z, [_I, _I, _I]),
    "lsk_head_norm_argmax": (_I, [_I, _P, _L, _P, _F, _P, _L, _I, _I, _I, _P, _L, _P, _P, _P, _Z, _P]),
    "lsk_add_rmsnorm": (_I, [_I, _P, _L, _P, _I, _P, _F, _P, _L, _P, _L, _I, _I, _P]),
    "lsk_rope_append_partial": (_I, [_I, _P, _I, _P, _P, _P, _P, _P, _I, _P, _P, _I, _I, _I, _I, _I, _I, _P]),
    "lsk_embed": (_I, [_P, _L, _L, _P, _L, _P, _P, _P, _I, _P]),
    "lsk_copy_rows": (_I, [_P, _P, _L, _P, _P, _L, _L, _I, _P]),
    "lsk_argmax": (_I, [_I, _P, _L, _I, _I, _P, _P, _P]),
    "lsk_greedy_accept": (_I, [_P, _P, _I, _P, _P, _P, _P, _I, _P, _P, _P, _P]),
    "lsk_kv_rollback": (_I, [_P, _P, _P, _I, _P]),
    "lsk_shift_segment_positions": (_I, [_P, _I, _I, _I, _I, _I, _I, _P, _P, _P, _I, _P]),
    "lsk_probe_matches": (_I, [_P, _P, _P, _P, _P, _I, _I, _P, _P]),
    "lsk_model_create": (_L, [_I, _I, _I, _I, _I, _I, _I, _I, _F] + [_P] * 8 + [_I, _I, _P, _P, _I]),
    "lsk_model_destroy": (_I, [_L]),
    "lsk_segment_workspace_bytes": (_Z, [_L, _I, _I]),
    "lsk_gemm_partial_frag": (_I, [_P, _P, _P, _I, _I, _I, _I, _P]),
    "lsk_gemm_silu_frag": (_I, [_P, _P, _P, _I, _I, _I, _I, _P]),
    "lsk_forward_layers": (_I, [_L, _P, _P, _I, _I, _I, _P, _I, _I, _I, _I, _I, _I, _I, _P, _Z, _P,
                                ctypes.c_double, ctypes.c_double, _P]),
    "lsk_prof_enable": (_I, [_I]),
    "lsk_prof_start": (_I, [_I, ctypes.c_double, ctypes.c_double, _P]),
    "lsk_prof_stop": (_I, [_P]),
    "lsk_prof_collect": (_I, [_I, _P, _P, _P, _P]),
}
PROF_CLASSES = ("rmsnorm", "gemm_qkv", "rope_append", "attention", "gemm_o", "gemm_w13", "gemm_w2", "gemm_lm_head",
                "argmax", "glue")
EXPORTS = tuple(_SIGS)

_lib = None


class LskError(RuntimeError):
    pass


def load(path: str | os.PathLike | None = None):
    """Load liblsk.so (once).  Raises if it is missing: there is no CPU fallback."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path is not None else LIB_PATH
    if not p.exists():
        raise LskError(f"{p} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'`")
    lib = ctypes.CDLL(str(p))
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.lsk_abi_version() != ABI_VERSION:
        raise LskError(f"liblsk ABI {lib.lsk_abi_version()} != {ABI_VERSION}; rebuild")
    if path is None:
        _lib = lib
    return lib


def _check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().lsk_last_error().decode(errors="replace")
        raise LskError(f"{what} failed ({rc}): {msg}")


def _ptr(t) -> int | None:
    if t is None:
        return None
    return t.data_ptr()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream() -> int:
    """The current HIP stream of the current device (raw handle; the cheap query when torch has it)."""
    if _raw_stream is not None:
        return _raw_stream(torch._C._cuda_getDevice())
    return torch.cuda.current_stream().cuda_stream


def k_to_frag(k: torch.Tensor) -> torch.Tensor:
    """[..., S, D] -> the bf16 K cache storage [..., S/32, D/16, 64, 8]: per 32-position block, 2 D/32 MFMA
    fragments (a, j) of 1 KiB; lane 16 lg + 4 q + r of fragment (a, j) holds position 8 q + 4 a + r of the
    block and d = 32 j + 8 lg .. +7."""
    *lead, S, D = k.shape
    n = len(lead)
    x = k.reshape(*lead, S // 32, 4, 2, 4, D // 32, 4, 8)          # blk, q, a, r, j, lg, e
    perm = list(range(n)) + [n + i for i in (0, 2, 4, 5, 1, 3, 6)]  # blk, a, j, lg, q, r, e
    return x.permute(*perm).reshape(*lead, S // 32, D // 16, 64, 8).contiguous()


def k_from_frag(kf: torch.Tensor) -> torch.Tensor:
    """bf16 K cache storage [..., S/32, D/16, 64, 8] -> [..., S, D] (a copy)."""
    *lead, nb, nf, _, _ = kf.shape
    n = len(lead)
    D = nf * 16
    x = kf.reshape(*lead, nb, 2, D // 32, 4, 4, 4, 8)               # blk, a, j, lg, q, r, e
    perm = list(range(n)) + [n + i for i in (0, 4, 1, 5, 2, 3, 6)]  # blk, q, a, r, j, lg, e
    return x.permute(*perm).reshape(*lead, nb * 32, D)


def k_dims(kcache: torch.Tensor) -> tuple:
    """(B, Hkv, S, D) of a K cache: fragment-major bf16 storage [B, Hkv, S/32, D/16, 64, 8] or row-major
    [B, Hkv, S, D] (fp32)."""
    if kcache.dim() == 6:
        B, Hkv, nb, nf = kcache.shape[:4]
        return B, Hkv, nb * 32, nf * 16
    return tuple(kcache.shape)


def _check_kcache(dtype: torch.dtype, kcache: torch.Tensor) -> None:
    if dtype == torch.bfloat16 and kcache.dim() != 6:
        raise LskError("bf16 K caches use the fragment-major storage [B, Hkv, S/32, D/16, 64, 8] (k_to_frag)")
    if dtype != torch.bfloat16 and kcache.dim() != 4:
        raise LskError("fp32 K caches are row-major [B, Hkv, S, D]")


def v_to_blocked(v: torch.Tensor) -> torch.Tensor:
    """[..., S, D] -> the V cache storage [..., S/32, D, 32] (32-position blocks, each transposed)."""
    *lead, S, D = v.shape
    return v.reshape(*lead, S // 32, 32, D).transpose(-1, -2).contiguous()


def v_from_blocked(vb: torch.Tensor) -> torch.Tensor:
    """V cache storage [..., S/32, D, 32] -> [..., S, D] (a copy)."""
    *lead, nb, D, b = vb.shape
    return vb.transpose(-1, -2).reshape(*lead, nb * b, D)


def dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.bfloat16:
        return DTYPE_BF16
    if dtype == torch.float32:
        return DTYPE_F32
    raise LskError(f"unsupported dtype {dtype} (bf16 and fp32 only)")


def _dev(*ts):
    for t in ts:
        if t is not None and t.device.type != "cuda":
            raise LskError(f"liblsk kernels need CUDA (HIP) tensors, got {t.device}")


# ----------------------------------------------------------------------------- weights

class PackedWeight:
    """A bf16 weight matrix [N, K] (F.linear's [out, in]) in the GEMM kernels' fragment-major storage
    (lsk_pack_weight): every 16-row x 32-column MFMA fragment is 1 KiB contiguous in lane order, so each
    wave's weight load is one contiguous 1 KiB stream.  `unpack()` returns the [N, K] tensor (a copy).
    qkv_heads=(n_heads, n_kv_heads, head_dim): a fused [q; k; v] weight stored for the fused qkv + RoPE GEMM
    (lsk_pack_weight_qkv, q and k row groups RoPE-paired); only `gemm_qkv_rope` reads it."""

    def __init__(self, w: torch.Tensor, qkv_heads: tuple | None = None):
        _dev(w)
        if w.dtype != torch.bfloat16 or w.dim() != 2 or w.stride(1) != 1:
            raise LskError("PackedWeight: a 2-D bf16 tensor with unit column stride is needed")
        N, K = w.shape
        self.shape = (N, K)
        self.dtype = w.dtype
        self.device = w.device
        self.qkv_heads = tuple(qkv_heads) if qkv_heads is not None else None
        self.data = torch.empty(N * K, dtype=w.dtype, device=w.device)
        if self.qkv_heads is None:
            _check(load().lsk_pack_weight(_ptr(w), w.stride(0), _ptr(self.data), N, K, _stream()), "lsk_pack_weight")
        else:
            hq, hkv, d = self.qkv_heads
            if N != (hq + 2 * hkv) * d:
                raise LskError(f"PackedWeight: {N} rows do not match qkv heads {self.qkv_heads}")
            _check(load().lsk_pack_weight_qkv(_ptr(w), w.stride(0), _ptr(self.data), hq, hkv, d, K, _stream()),
                   "lsk_pack_weight_qkv")

    def data_ptr(self) -> int:
        return self.data.data_ptr()

    def stride(self, dim: int) -> int:
        return self.shape[1] if dim == 0 else 1

    def dim(self) -> int:
        return 2

    def numel(self) -> int:
        return self.shape[0] * self.shape[1]

    def element_size(self) -> int:
        return 2

    def unpack(self) -> torch.Tensor:
        N, K = self.shape
        out = torch.empty(N, K, dtype=self.dtype, device=self.device)
        if getattr(self, "qkv_heads", None) is None:
            _check(load().lsk_unpack_weight(_ptr(self.data), _ptr(out), K, N, K, _stream()), "lsk_unpack_weight")
        else:
            hq, hkv, d = self.qkv_heads
            _check(load().lsk_unpack_weight_qkv(_ptr(self.data), _ptr(out), K, hq, hkv, d, K, _stream()),
                   "lsk_unpack_weight_qkv")
        return out

    def __repr__(self) -> str:
        return f"PackedWeight(shape={self.shape}, dtype={self.dtype}, device={self.device})"


GEMM_TOKEN_TILE = 64       # tokens per GEMM token tile: launches of up to this many rows read each weight once


def as_gemm_weight(w: torch.Tensor):
    """The storage the GEMMs read for a weight of this dtype: PackedWeight for bf16, the tensor for fp32."""
    return PackedWeight(w) if w.dtype == torch.bfloat16 else w.contiguous()


def _check_weight(a: torch.Tensor, w) -> None:
    if a.dtype == torch.bfloat16 and not isinstance(w, PackedWeight):
        raise LskError("bf16 GEMMs read packed weights: wrap the [out, in] tensor in PackedWeight")
    if a.dtype != torch.bfloat16 and isinstance(w, PackedWeight):
        raise LskError("packed weights are bf16 only")
    if isinstance(w, PackedWeight) and getattr(w, "qkv_heads", None) is not None:
        raise LskError("a qkv weight packed for the fused qkv + RoPE GEMM is read by gemm_qkv_rope only (its rows are "
                       "RoPE-paired); PackedWeight(w.unpack()) gives the plain storage")


# ----------------------------------------------------------------------------- ops

def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float, out: torch.Tensor | None = None) -> torch.Tensor:
    _dev(x, w)
    assert x.dim() == 2 and x.stride(1) == 1 and w.is_contiguous() and w.numel() == x.shape[1]
    if out is None:
        out = torch.empty_like(x)
    _check(load().lsk_rmsnorm(dtype_code(x.dtype), _ptr(x), _ptr(w), _ptr(out), x.shape[0], x.shape[1], float(eps),
                              x.stride(0), out.stride(0), _stream()), "lsk_rmsnorm")
    return out


def rope_append(qkv, q_out, kcache, vcache, cos_tab, sin_tab, rows_i32, pos_i32, n_heads, n_kv_heads, head_dim):
    """kcache: K cache storage (k_dims); vcache: the blocked-transposed V storage [B, Hkv, S/32, D, 32]."""
    _dev(qkv, q_out, kcache, vcache, cos_tab, sin_tab, rows_i32, pos_i32)
    _check_kcache(q_out.dtype, kcache)
    N = qkv.shape[0]
    B, Hkv, S, D = k_dims(kcache)
    assert qkv.is_contiguous() and q_out.is_contiguous() and kcache.is_contiguous() and vcache.is_contiguous()
    assert cos_tab.dtype == torch.float32 and cos_tab.is_contiguous() and cos_tab.shape[1] == head_dim
    _check(load().lsk_rope_append(dtype_code(qkv.dtype), _ptr(qkv), _ptr(q_out), _ptr(kcache), _ptr(vcache),
                                  _ptr(cos_tab), _ptr(sin_tab), cos_tab.shape[0], _ptr(rows_i32), _ptr(pos_i32), N,
                                  n_heads, n_kv_heads, head_dim, B, S, _stream()), "lsk_rope_append")


def kv_append(k, v, kcache, vcache, rows_i32, pos_i32):
    """kcache: K cache storage (k_dims); vcache: the blocked-transposed V storage [B, Hkv, S/32, D, 32]."""
    _dev(k, v, kcache, vcache, rows_i32, pos_i32)
    _check_kcache(k.dtype, kcache)
    B, Hkv, S, D = k_dims(kcache)
    assert k.is_contiguous() and v.is_contiguous() and k.shape[1:] == (Hkv, D)
    _check(load().lsk_kv_append(dtype_code(k.dtype), _ptr(k), _ptr(v), _ptr(kcache), _ptr(vcache), _ptr(rows_i32),
                                _ptr(pos_i32), k.shape[0], Hkv, D, B, S, _stream()), "lsk_kv_append")


def attn_plan(blocks: np.ndarray, group: int, split: int, rows_cap: int = ATTN_ROWS):
    """blocks int32 [nb, 4] = (q_start, pos0, T, row) -> (works [n,8], groups [n,8], n_parts); work items of at
    most rows_cap (16, 32 or 48) query rows."""
    blocks = np.ascontiguousarray(blocks, dtype=np.int32)
    nb = blocks.shape[0]
    rows = int(((blocks[:, 2].astype(np.int64) * group + rows_cap - 1) // max(rows_cap, 1)).sum()) if nb else 0
    max_ctx = int((blocks[:, 1].astype(np.int64) + blocks[:, 2]).max()) if nb else 0
    max_works = 8 * max(1, rows * max(1, (max_ctx + split - 1) // split)) + 64   # XCD-order padding
    max_groups = max(1, rows)
    works = np.zeros((max_works, 8), dtype=np.int32)
    groups = np.zeros((max_groups, 8), dtype=np.int32)
    nw, ng, npart = ctypes.c_int(0), ctypes.c_int(0), ctypes.c_int(0)
    _check(load().lsk_attn_plan(blocks.ctypes.data, nb, group, split, rows_cap, works.ctypes.data, max_works,
                                groups.ctypes.data, max_groups, ctypes.byref(nw), ctypes.byref(ng),
                                ctypes.byref(npart)), "lsk_attn_plan")
    return works[:nw.value], groups[:ng.value], npart.value


def attn_rows_cap(blocks: np.ndarray, group: int, split: int, n_kv_heads: int, head_dim: int, n_slots: int) -> int:
    """Rows per attention work item (16, 32 or 48) for a launch of these blocks over n_slots workgroups."""
    blocks = np.ascontiguousarray(blocks, dtype=np.int32)
    rc = load().lsk_attn_rows_cap(blocks.ctypes.data if len(blocks) else None, len(blocks), group, split,
                                  n_kv_heads, head_dim, n_slots)
    if rc < 0:
        _check(rc, "lsk_attn_rows_cap")
    return rc


_CU_COUNT: dict = {}


def cu_count(device) -> int:
    """Compute units of the device (the persistent attention kernel runs one workgroup per CU); 256 (MI355X)
    for a non-CUDA device, where plans are only built, never run."""
    device = torch.device(device)
    if device.type != "cuda":
        return 256
    idx = device.index if device.index is not None else torch.cuda.current_device()
    n = _CU_COUNT.get(idx)
    if n is None:
        n = _CU_COUNT[idx] = int(torch.cuda.get_device_properties(idx).multi_processor_count)
    return n


def attn_schedule(works: np.ndarray, n_kv_heads: int, n_slots: int):
    """Static longest-first schedule of (work, KV head) items over n_slots persistent workgroups
    -> (recs int32 [n_slots * n_rounds * 8], n_rounds): slot s's records are recs[s * n_rounds * 8 ...]."""
    works = np.ascontiguousarray(works, dtype=np.int32)
    lib = load()
    wp = works.ctypes.data if len(works) else None
    R = ctypes.c_int(0)
    _check(lib.lsk_attn_schedule(wp, len(works), n_kv_heads, n_slots, None, 0, ctypes.byref(R)), "lsk_attn_schedule")
    recs = np.zeros(max(n_slots * R.value * 8, 8), dtype=np.int32)
    _check(lib.lsk_attn_schedule(wp, len(works), n_kv_heads, n_slots, recs.ctypes.data, n_slots * R.value,
                                 ctypes.byref(R)), "lsk_attn_schedule")
    return recs[:n_slots * R.value * 8], R.value


_PACK_BUF = [np.zeros(1 << 16, dtype=np.int32)]
_PACK_COUNTS = np.zeros(11, dtype=np.int64)


def pack_segment(rows: np.ndarray, pos0: np.ndarray, T: np.ndarray, group: int, split: int, n_kv_heads: int,
                 head_dim: int, n_slots: int, bucketing: int, max_batch: int, max_seq: int, rope_len: int):
    """lsk_pack_segment over int64 block arrays in packed order -> (meta int32 [meta_len] (a fresh array),
    counts (N, n_works, n_groups, n_parts, n_rounds, meta_len, kv_read, kv_read_padded, kv_gathered, pairs,
    rows_cap)).
    Out-of-range blocks raise ValueError (the reference's build_packed behaviour)."""
    lib = load()
    nb = len(T)
    r = rows if rows.dtype == np.int64 and rows.flags.c_contiguous else np.ascontiguousarray(rows, dtype=np.int64)
    p = pos0 if pos0.dtype == np.int64 and pos0.flags.c_contiguous else np.ascontiguousarray(pos0, dtype=np.int64)
    t = T if T.dtype == np.int64 and T.flags.c_contiguous else np.ascontiguousarray(T, dtype=np.int64)
    cnt = _PACK_COUNTS
    for _ in range(2):
        buf = _PACK_BUF[0]
        rc = lib.lsk_pack_segment(r.ctypes.data, p.ctypes.data, t.ctypes.data, nb, group, split, n_kv_heads,
                                  head_dim, n_slots, bucketing, max_batch, max_seq, rope_len, buf.ctypes.data,
                                  buf.size, cnt.ctypes.data)
        if rc == -4:                                   # LSK_EWORKSPACE: grow to the reported length and retry
            _PACK_BUF[0] = np.zeros(int(cnt[5]) * 2, dtype=np.int32)
            continue
        if rc == -2:
            raise ValueError(lib.lsk_last_error().decode())
        _check(rc, "lsk_pack_segment")
        c = cnt.tolist()
        return buf[:c[5]].copy(), tuple(c)
    raise LskError("lsk_pack_segment: metadata buffer")


def attn_workspace_bytes(n_parts: int, n_kv_heads: int, head_dim: int) -> int:
    return int(load().lsk_attn_workspace_bytes(n_parts, n_kv_heads, head_dim))


def ragged_attn(q, kcache, vcache, blocks_dev, works_dev, n_works, groups_dev, n_groups, n_parts, out, n_heads,
                scale, workspace=None, recs_dev=None, n_rounds=0, n_slots=0, rows_cap=ATTN_ROWS):
    """kcache: K cache storage (k_dims); vcache: the blocked-transposed V storage [B, Hkv, S/32, D, 32];
    rows_cap: the cap the plan was made with."""
    _dev(q, kcache, vcache, blocks_dev, works_dev, out)
    _check_kcache(q.dtype, kcache)
    B_, H_, S_, D_ = k_dims(kcache)
    assert vcache.shape == (B_, H_, S_ // 32, D_, 32) and S_ % 64 == 0
    B, Hkv, S, D = k_dims(kcache)
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    _check(load().lsk_ragged_attn(dtype_code(q.dtype), _ptr(q), _ptr(kcache), _ptr(vcache), _ptr(blocks_dev),
                                  _ptr(works_dev), n_works, _ptr(groups_dev), n_groups, n_parts, _ptr(recs_dev),
                                  n_rounds, n_slots, rows_cap, _ptr(out), n_heads, Hkv, D, S, float(scale),
                                  _ptr(workspace), ws_bytes, _stream()), "lsk_ragged_attn")


def ragged_attn_static(q, kcache, vcache, blocks_dev, works_dev, n_works, groups_dev, n_groups, n_parts, out,
                       n_heads, scale, recs_dev=None, n_rounds=0, n_slots=0, rows_cap=ATTN_ROWS):
    """ragged_attn without a workspace: the split partials live in the library's static per-GPU scratch array
    (lsk_ragged_attn_static; plans needing more than lsk_ragged_attn_static_scratch_bytes() raise)."""
    _dev(q, kcache, vcache, blocks_dev, works_dev, out)
    _check_kcache(q.dtype, kcache)
    B, Hkv, S, D = k_dims(kcache)
    assert vcache.shape == (B, Hkv, S // 32, D, 32) and S % 64 == 0
    _check(load().lsk_ragged_attn_static(dtype_code(q.dtype), _ptr(q), _ptr(kcache), _ptr(vcache), _ptr(blocks_dev),
                                         _ptr(works_dev), n_works, _ptr(groups_dev), n_groups, n_parts,
                                         _ptr(recs_dev), n_rounds, n_slots, rows_cap, _ptr(out), n_heads, Hkv, D, S,
                                         float(scale), _stream()), "lsk_ragged_attn_static")


def gemm(a: torch.Tensor, w: torch.Tensor, out: torch.Tensor | None = None, residual: torch.Tensor | None = None,
         epilogue: int = EPI_NONE) -> torch.Tensor:
    _dev(a, w, out, residual)
    _check_weight(a, w)
    assert a.dim() == 2 and w.dim() == 2 and a.stride(1) == 1 and w.stride(1) == 1
    M, K = a.shape
    if epilogue == EPI_SILU_MUL:
        N = w.shape[0] // 2
        ffn = N
    else:
        N = w.shape[0]
        ffn = 0
    if out is None:
        out = torch.empty(M, N, dtype=a.dtype, device=a.device)
    ldr = residual.stride(0) if residual is not None else 0
    _check(load().lsk_gemm(dtype_code(a.dtype), _ptr(a), a.stride(0), _ptr(w), w.stride(0), _ptr(out), out.stride(0),
                           _ptr(residual), ldr, M, N, K, epilogue, ffn, _stream()), "lsk_gemm")
    return out


def embed(table: torch.Tensor, alt_ids: torch.Tensor, out: torch.Tensor, seq_buf: torch.Tensor | None = None,
          sel: torch.Tensor | None = None) -> torch.Tensor:
    _dev(table, alt_ids, out, seq_buf, sel)
    n = alt_ids.numel()
    row_bytes = table.shape[1] * table.element_size()
    _check(load().lsk_embed(_ptr(table), table.shape[0], row_bytes, _ptr(seq_buf),
                            seq_buf.numel() if seq_buf is not None else 0, _ptr(sel), _ptr(alt_ids), _ptr(out), n,
                            _stream()), "lsk_embed")
    return out


def copy_rows(dst: torch.Tensor, dst_idx, src: torch.Tensor, src_idx, n: int) -> None:
    _dev(dst, src, dst_idx, src_idx)
    row_bytes = dst[0].numel() * dst.element_size()
    assert src[0].numel() * src.element_size() == row_bytes
    _check(load().lsk_copy_rows(_ptr(dst), _ptr(dst_idx), dst.shape[0], _ptr(src), _ptr(src_idx), src.shape[0],
                                row_bytes, n, _stream()), "lsk_copy_rows")


def argmax(logits: torch.Tensor, out: torch.Tensor, dst_idx: torch.Tensor | None = None, n_rows: int | None = None):
    _dev(logits, out, dst_idx)
    n = logits.shape[0] if n_rows is None else n_rows
    _check(load().lsk_argmax(dtype_code(logits.dtype), _ptr(logits), logits.stride(0), n, logits.shape[1], _ptr(out),
                             _ptr(dst_idx), _stream()), "lsk_argmax")
    return out


def greedy_accept(Yv, seq_buf, Dm1, slots, starts, Ts, forced, nv, acc_out, y_out, kv_len=None):
    _dev(Yv, seq_buf, slots, starts, Ts, forced, acc_out, y_out, kv_len)
    _check(load().lsk_greedy_accept(_ptr(Yv), _ptr(seq_buf), Dm1, _ptr(slots), _ptr(starts), _ptr(Ts), _ptr(forced),
                                    nv, _ptr(acc_out), _ptr(y_out), _ptr(kv_len), _stream()), "lsk_greedy_accept")


def probe_matches(pred, Yv, acc, blk_i32, jl_i32, nc: int, nvt: int, out) -> None:
    _dev(pred, Yv, acc, blk_i32, jl_i32, out)
    _check(load().lsk_probe_matches(_ptr(pred), _ptr(Yv), _ptr(acc), _ptr(blk_i32), _ptr(jl_i32), nc, nvt, _ptr(out),
                                    _stream()), "lsk_probe_matches")


def kv_rollback(kv_len, slots, accepted, nv):
    _dev(kv_len, slots, accepted)
    _check(load().lsk_kv_rollback(_ptr(kv_len), _ptr(slots), _ptr(accepted), nv, _stream()), "lsk_kv_rollback")


def shift_segment_positions(meta, n_tokens: int, nb: int, n_works: int, n_groups: int, n_recs: int, group: int,
                            accepted, vslots, vdrafts, nv: int) -> None:
    """lsk_shift_segment_positions on a segment's device metadata `meta` (int32, pack_segment's layout; n_recs =
    n_slots * n_rounds of its plan): blocks in cache row vslots[j] planned vdrafts[j] - accepted[j] positions ahead
    move back to their actual positions (accepted: the device acc_out of greedy_accept)."""
    _dev(meta, accepted, vslots, vdrafts)
    _check(load().lsk_shift_segment_positions(_ptr(meta), n_tokens, nb, n_works, n_groups, n_recs, group,
                                              _ptr(accepted), _ptr(vslots), _ptr(vdrafts), nv, _stream()),
           "lsk_shift_segment_positions")


# ----------------------------------------------------------------------------- layer-range runner

def _ptr_array(ptrs):
    arr = (ctypes.c_void_p * len(ptrs))()
    for i, p in enumerate(ptrs):
        arr[i] = p
    return arr


class NativeModel:
    """Handle of the native layer-range runner for one (weights, KV cache, RoPE table) set."""

    def __init__(self, dtype, n_layers, dim, n_heads, n_kv_heads, head_dim, ffn, vocab, eps, layers, kcache, vcache,
                 cos_tab, sin_tab):
        if dtype == torch.bfloat16:
            # the bf16 runner's fused qkv + RoPE launch reads wqkv in the RoPE-paired packing
            for i, lw in enumerate(layers):
                if not (isinstance(lw.wqkv, PackedWeight) and lw.wqkv.qkv_heads == (n_heads, n_kv_heads, head_dim)):
                    raise LskError(f"layer {i}: bf16 wqkv must be a PackedWeight packed with qkv_heads="
                                   f"{(n_heads, n_kv_heads, head_dim)} (got "
                                   f"{getattr(lw.wqkv, 'qkv_heads', type(lw.wqkv).__name__)})")
        lib = load()
        _dev(cos_tab, sin_tab)
        _check_kcache(dtype, kcache[0])
        B, Hkv, S, D = k_dims(kcache[0])
        assert vcache[0].shape == (B, Hkv, S // 32, D, 32) and vcache[0].is_contiguous(), \
            "V cache must be the blocked-transposed [B, Hkv, S/32, D, 32] storage"
        self._keep = (layers, kcache, vcache, cos_tab, sin_tab)
        h = lib.lsk_model_create(
            dtype_code(dtype), n_layers, dim, n_heads, n_kv_heads, head_dim, ffn, vocab, float(eps),
            _ptr_array([lw.wqkv.data_ptr() for lw in layers]), _ptr_array([lw.wo.data_ptr() for lw in layers]),
            _ptr_array([lw.w13.data_ptr() for lw in layers]), _ptr_array([lw.w2.data_ptr() for lw in layers]),
            _ptr_array([lw.attn_norm.data_ptr() for lw in layers]),
            _ptr_array([lw.ffn_norm.data_ptr() for lw in layers]),
            _ptr_array([t.data_ptr() for t in kcache]), _ptr_array([t.data_ptr() for t in vcache]),
            B, S, cos_tab.data_ptr(), sin_tab.data_ptr(), cos_tab.shape[0])
        if h <= 0:
            _check(int(h), "lsk_model_create")
        self.handle = h
        self.n_layers = n_layers

    def workspace_bytes(self, n_tokens: int, n_parts: int) -> int:
        return int(load().lsk_segment_workspace_bytes(self.handle, n_tokens, n_parts))

    def forward_layers(self, x_in, x_out, n_tokens, start, end, meta_dev, nb, n_works, n_groups, n_parts, n_rounds,
                       n_slots, rows_cap, workspace, capture_ptrs=None, attn_bytes=0.0, attn_flops=0.0):
        _dev(x_in, x_out, meta_dev, workspace)
        cap = _ptr_array(capture_ptrs) if capture_ptrs is not None else None
        ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
        _check(load().lsk_forward_layers(self.handle, _ptr(x_in), _ptr(x_out), n_tokens, start, end, _ptr(meta_dev),
                                         nb, n_works, n_groups, n_parts, n_rounds, n_slots, rows_cap, _ptr(workspace),
                                         ws_bytes,
                                         cap,
                                         float(attn_bytes), float(attn_flops), _stream()),
               "lsk_forward_layers")

    def __del__(self):
        try:
            if getattr(self, "handle", 0) > 0 and _lib is not None:
                _lib.lsk_model_destroy(self.handle)
        except Exception:
            pass


# ----------------------------------------------------------------------------- profiling

class Profiler:
    """Per-class HIP-event timing of liblsk launches (algorithmic bytes / flops per launch)."""

    enabled = False

    @classmethod
    def enable(cls, on: bool = True) -> None:
        load().lsk_prof_enable(1 if on else 0)
        cls.enabled = on

    @staticmethod
    def start(cls_idx: int, nbytes: float, flops: float) -> None:
        if Profiler.enabled:
            load().lsk_prof_start(cls_idx, float(nbytes), float(flops), _stream())

    @staticmethod
    def stop() -> None:
        if Profiler.enabled:
            load().lsk_prof_stop(_stream())

    @staticmethod
    def collect() -> dict:
        n = len(PROF_CLASSES)
        ms, by, fl, ct = (np.zeros(n), np.zeros(n), np.zeros(n), np.zeros(n, dtype=np.int64))
        _check(load().lsk_prof_collect(n, ms.ctypes.data, by.ctypes.data, fl.ctypes.data, ct.ctypes.data),
               "lsk_prof_collect")
        return {PROF_CLASSES[i]: {"ms": float(ms[i]), "bytes": float(by[i]), "flops": float(fl[i]),
                                  "launches": int(ct[i])} for i in range(n) if ct[i]}


def gemm_plan(N: int, K: int) -> tuple:
    ns, ks = ctypes.c_int(0), ctypes.c_int(0)
    _check(load().lsk_gemm_plan(N, K, ctypes.byref(ns), ctypes.byref(ks)), "lsk_gemm_plan")
    return ns.value, ks.value


def gemm_wide_config(epilogue: int, M: int, N: int, K: int, ks: int = 1, af: bool = True) -> tuple:
    """(ns, blocks, groups per block, groups per wave) the wide-M tier picks; ns == 0: the tier does not apply."""
    cfg = (ctypes.c_int * 4)()
    _check(load().lsk_gemm_wide_config(epilogue, M, N, K, ks, int(af), cfg), "lsk_gemm_wide_config")
    return tuple(cfg)


def frag_rows(m: int) -> int:
    """Rows a fragment-major activation buffer of m tokens holds (whole 16-token groups)."""
    return (m + 15) // 16 * 16


def gemm_partial_frag(a_frag: torch.Tensor, m: int, w: torch.Tensor, ks: int,
                      out: torch.Tensor | None = None) -> torch.Tensor:
    """gemm_partial with A fragment-major (lsk_gemm_partial_frag): a_frag holds frag_rows(m) x K elements in
    lsk_pack_weight's layout; fp32 K-slice partials [ks, m, N]."""
    _dev(a_frag, w, out)
    _check_weight(a_frag, w)
    N, K = w.shape
    if a_frag.dtype != torch.bfloat16 or a_frag.numel() < frag_rows(m) * K or not a_frag.is_contiguous():
        raise LskError("gemm_partial_frag: a contiguous bf16 buffer of frag_rows(m) x K elements is needed")
    if out is None:
        out = torch.empty(ks, m, N, dtype=torch.float32, device=a_frag.device)
    _check(load().lsk_gemm_partial_frag(_ptr(a_frag), _ptr(w), _ptr(out), m, N, K, ks, _stream()),
           "lsk_gemm_partial_frag")
    return out


def gemm_silu_frag(a_frag: torch.Tensor, m: int, w: torch.Tensor, h: torch.Tensor, h_frag: bool) -> torch.Tensor:
    """w13 + silu-mul with A fragment-major (lsk_gemm_silu_frag); h row-major [m, ffn] or, with h_frag,
    fragment-major (frag_rows(m) x ffn elements)."""
    _dev(a_frag, w, h)
    _check_weight(a_frag, w)
    ffn, K = w.shape[0] // 2, w.shape[1]
    if a_frag.dtype != torch.bfloat16 or a_frag.numel() < frag_rows(m) * K or not a_frag.is_contiguous():
        raise LskError("gemm_silu_frag: a contiguous bf16 buffer of frag_rows(m) x K elements is needed")
    if h.numel() < (frag_rows(m) if h_frag else m) * ffn or not h.is_contiguous():
        raise LskError("gemm_silu_frag: output too small")
    _check(load().lsk_gemm_silu_frag(_ptr(a_frag), _ptr(w), _ptr(h), 1 if h_frag else 0, m, ffn, K, _stream()),
           "lsk_gemm_silu_frag")
    return h


def gemm_partial(a: torch.Tensor, w: torch.Tensor, ks: int, out: torch.Tensor | None = None) -> torch.Tensor:
    """fp32 K-slice partials [ks, M, N] of a @ w.T (bf16, w packed)."""
    _dev(a, w, out)
    _check_weight(a, w)
    M, K = a.shape
    N = w.shape[0]
    if out is None:
        out = torch.empty(ks, M, N, dtype=torch.float32, device=a.device)
    _check(load().lsk_gemm_partial(_ptr(a), a.stride(0), _ptr(w), w.stride(0), _ptr(out), M, N, K, ks, _stream()),
           "lsk_gemm_partial")
    return out


def head_argmax(a: torch.Tensor, w: torch.Tensor, out: torch.Tensor, dst_idx: torch.Tensor | None = None,
                logits: torch.Tensor | None = None, workspace: torch.Tensor | None = None) -> torch.Tensor:
    _dev(a, w, out, dst_idx, logits, workspace)
    _check_weight(a, w)
    M, K = a.shape
    N = w.shape[0]
    need = int(load().lsk_head_workspace_bytes(M, N))
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=a.device)
    _check(load().lsk_head_argmax(dtype_code(a.dtype), _ptr(a), a.stride(0), _ptr(w), w.stride(0), M, N, K,
                                  _ptr(logits), logits.stride(0) if logits is not None else 0, _ptr(out),
                                  _ptr(dst_idx), _ptr(workspace), workspace.numel() * workspace.element_size(),
                                  _stream()), "lsk_head_argmax")
    return out


def head_norm_argmax(h: torch.Tensor, norm_w: torch.Tensor, eps: float, w, out: torch.Tensor,
                     dst_idx: torch.Tensor | None = None, logits: torch.Tensor | None = None,
                     workspace: torch.Tensor | None = None) -> torch.Tensor:
    """argmax(lm_head(rmsnorm(h))) per row in one native call (bf16), bitwise equal to rmsnorm + head_argmax."""
    _dev(h, norm_w, out, dst_idx, logits, workspace)
    _check_weight(h, w)
    M, K = h.shape
    N = w.shape[0]
    need = int(load().lsk_head_norm_workspace_bytes(M, N, K))
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=h.device)
    _check(load().lsk_head_norm_argmax(dtype_code(h.dtype), _ptr(h), h.stride(0), _ptr(norm_w), float(eps), _ptr(w),
                                       w.stride(0), M, N, K, _ptr(logits), logits.stride(0) if logits is not None else 0,
                                       _ptr(out), _ptr(dst_idx), _ptr(workspace),
                                       workspace.numel() * workspace.element_size(), _stream()),
           "lsk_head_norm_argmax")
    return out


def add_rmsnorm(x: torch.Tensor, partials: torch.Tensor | None, w: torch.Tensor | None, eps: float,
                x_out: torch.Tensor | None = None, out: torch.Tensor | None = None) -> None:
    _dev(x, partials, w, x_out, out)
    n, dim = x.shape
    ks = partials.shape[0] if partials is not None else 0
    _check(load().lsk_add_rmsnorm(dtype_code(x.dtype), _ptr(x), x.stride(0), _ptr(partials), ks, _ptr(w), float(eps),
                                  _ptr(x_out), x_out.stride(0) if x_out is not None else 0, _ptr(out),
                                  out.stride(0) if out is not None else 0, n, dim, _stream()), "lsk_add_rmsnorm")


def gemm_qkv_rope(a_frag: torch.Tensor, w: "PackedWeight", M: int, q_out, kcache, vcache, cos_tab, sin_tab,
                  rows_i32, pos_i32) -> None:
    """Fused qkv projection + RoPE + KV append (lsk_gemm_qkv_rope): a_frag holds the normalised rows fragment-major
    (frag_rows(M) * K elements), w a PackedWeight packed with qkv_heads; writes q_out [M, Hq, D] and the caches."""
    _dev(a_frag, q_out, kcache, vcache, cos_tab, sin_tab, rows_i32, pos_i32)
    if not isinstance(w, PackedWeight) or w.qkv_heads is None:
        raise LskError("gemm_qkv_rope reads a PackedWeight packed with qkv_heads (lsk_pack_weight_qkv)")
    _check_kcache(q_out.dtype, kcache)
    hq, hkv, d = w.qkv_heads
    B, _, S, _ = k_dims(kcache)
    _check(load().lsk_gemm_qkv_rope(_ptr(a_frag), _ptr(w), M, hq, hkv, d, w.shape[1], _ptr(q_out), _ptr(kcache),
                                    _ptr(vcache), _ptr(cos_tab), _ptr(sin_tab), cos_tab.shape[0], _ptr(rows_i32),
                                    _ptr(pos_i32), B, S, _stream()), "lsk_gemm_qkv_rope")


def rope_append_partial(partials, q_out, kcache, vcache, cos_tab, sin_tab, rows_i32, pos_i32, n_heads, n_kv_heads,
                        head_dim):
    _dev(partials, q_out, kcache, vcache, cos_tab, sin_tab, rows_i32, pos_i32)
    _check_kcache(q_out.dtype, kcache)
    ks, N, _ = partials.shape
    B, Hkv, S, D = k_dims(kcache)
    _check(load().lsk_rope_append_partial(dtype_code(q_out.dtype), _ptr(partials), ks, _ptr(q_out), _ptr(kcache),
                                          _ptr(vcache), _ptr(cos_tab), _ptr(sin_tab), cos_tab.shape[0],
                                          _ptr(rows_i32), _ptr(pos_i32), N, n_heads, n_kv_heads, head_dim, B, S,
                                          _stream()), "lsk_rope_append_partial")
