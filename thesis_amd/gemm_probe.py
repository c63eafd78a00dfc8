"""A fixed sequence of projection-GEMM launches at the Llama3-8B layer shapes, for rocprofv3 counter runs.

    python -m thesis_amd.gemm_probe [--reps 10] [--tokens 16,32,64,288,512]

For every token count M and class -- qkv (6144 x 4096, fused with RoPE + KV append), o (4096 x 4096, partials), w13
([gate; up] 28672 x 4096, silu-mul), w2 (4096 x 14336, partials), LM head (128256 x 4096, fused argmax) -- it
issues `reps` launches on distinct random weights (two layers' worth, so repeated launches stream from HBM),
after one marker copy of 64 MiB per group (lsk_copy_rows, 16 KiB rows), and prints the sequence as JSON lines
({"class", "M", "launches"}) so per-dispatch counters can be attributed: dispatches between two markers belong
to the group printed in that position.  The launches and activations are the layer loop's: qkv is
lsk_gemm_qkv_rope (RoPE-paired weights, q and a scratch cache row written), fragment-major inputs for
qkv and o at every M and for w13 / w2 above 64 tokens (lsk_gemm_partial_frag, lsk_gemm_silu_frag), row-major
otherwise; the LM head is the engine's lsk_head_norm_argmax call (its final norm writes the head's input
fragment-major; only the GEMM kernels count in the summaries).
"""

from __future__ import annotations

import argparse
import json
import sys

import torch

from . import _lsk


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--reps", type=int, default=10)
    ap.add_argument("--tokens", default="16,32,64,288,512")
    ap.add_argument("--classes", default="qkv,o,w13,w2,head")
    args = ap.parse_args()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    g = torch.Generator(device=dev).manual_seed(0)
    dim, ffn, qkvd, V = 4096, 14336, 6144, 128256
    shapes = {"qkv": (qkvd, dim), "o": (dim, dim), "w13": (2 * ffn, dim), "w2": (dim, ffn), "head": (V, dim)}
    classes = args.classes.split(",")
    Ms = [int(t) for t in args.tokens.split(",")]
    heads = (32, 8, 128)                       # Llama3-8B q / kv heads, head_dim
    weights = {c: [_lsk.PackedWeight(torch.empty(*shapes[c], dtype=torch.bfloat16, device=dev).normal_(generator=g),
                                     qkv_heads=heads if c == "qkv" else None)
                   for _ in range(1 if c == "head" else 2)] for c in classes}
    m_max = max(Ms)
    s_kv = (m_max + 31) // 32 * 32             # one scratch cache row holding positions 0 .. M - 1
    q_out = torch.empty(m_max, heads[0], heads[2], dtype=torch.bfloat16, device=dev)
    kc = torch.zeros(1, heads[1], s_kv // 32, heads[2] // 16, 64, 8, dtype=torch.bfloat16, device=dev)
    vc = torch.zeros(1, heads[1], s_kv // 32, heads[2], 32, dtype=torch.bfloat16, device=dev)
    cos = torch.randn(s_kv, heads[2], device=dev)
    sin = torch.randn(s_kv, heads[2], device=dev)
    rows = torch.zeros(m_max, dtype=torch.int32, device=dev)
    pos = torch.arange(m_max, dtype=torch.int32, device=dev)
    a = torch.empty(max(Ms), ffn, dtype=torch.bfloat16, device=dev).normal_(generator=g)
    af = torch.empty(_lsk.frag_rows(max(Ms)) * ffn, dtype=torch.bfloat16, device=dev).normal_(generator=g)
    norm_w = torch.ones(dim, dtype=torch.bfloat16, device=dev)
    src = torch.empty(4096, 16384, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    af_max = 64                                # lsk_forward_layers' LSK_AF_MAX_TOKENS
    for M in Ms:
        x = {c: a[:M, :shapes[c][1]].contiguous() for c in classes}
        h = torch.empty(_lsk.frag_rows(M) * ffn, dtype=torch.bfloat16, device=dev)
        ids = torch.empty(M, dtype=torch.long, device=dev)
        ws = torch.empty(int(_lsk.load().lsk_head_norm_workspace_bytes(M, V, dim)), dtype=torch.uint8, device=dev)
        for c in classes:
            N, K = shapes[c]
            ks = _lsk.gemm_plan(N, K)[1]
            P = torch.empty(ks, M, N, dtype=torch.float32, device=dev) if c in ("o", "w2") else None
            torch.cuda.synchronize()
            _lsk.copy_rows(dst, None, src, None, src.shape[0])           # marker
            for r in range(args.reps):
                w = weights[c][r % len(weights[c])]
                if c == "w13":
                    if M > af_max:
                        _lsk.gemm_silu_frag(af, M, w, h, True)
                    else:
                        _lsk.gemm(x[c], w, h[:M * ffn].view(M, ffn), epilogue=_lsk.EPI_SILU_MUL)
                elif c == "head":
                    _lsk.head_norm_argmax(x[c], norm_w, 1e-5, w, ids, workspace=ws)
                elif c == "qkv":
                    _lsk.gemm_qkv_rope(af, w, M, q_out[:M], kc, vc, cos, sin, rows[:M], pos[:M])
                elif c == "o" or M > af_max:
                    _lsk.gemm_partial_frag(af, M, w, ks, out=P)
                else:
                    _lsk.gemm_partial(x[c], w, ks, out=P)
            torch.cuda.synchronize()
            print(json.dumps({"class": c, "M": M, "launches": args.reps}), flush=True)


if __name__ == "__main__":
    sys.exit(main())
