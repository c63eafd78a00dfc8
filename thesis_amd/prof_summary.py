"""Summaries of rocprofv3 CSV output for the decode benchmark (kernel durations, HBM traffic).

    python -m thesis_amd.prof_summary trace <prefix>_kernel_trace.csv [--bench bench.json] [--cmd "..."]
    python -m thesis_amd.prof_summary pmc <fetch>_counter_collection.csv <write>_counter_collection.csv
                                          --calib-mib 1024 [--bench bench.json] [--cmd "..."]
    python -m thesis_amd.prof_summary gemm <probe>_kernel_trace.csv <probe stdout> [<counter CSVs> ...] [--cmd "..."]

Both read the CSV files `rocprofv3 --output-format csv` writes.  Only dispatches after the calibration
copy are counted: bench.py's --copy-calib-mib issues one plain lsk_copy_rows copy of a known size
(16 KiB rows, a grid far larger than any copy the engine makes) right before its timed steps, so
start-up work (weight init, prefill) stays out of the per-kernel figures.

The pmc summary turns FETCH_SIZE / WRITE_SIZE (KiB per dispatch) into HBM bytes: each counter is
scaled by (known bytes of the calibration copy) / (what the counter read for that copy), and the
result is printed per kernel class with the algorithmic bytes per launch beside it.  The line
`traffic_bytes_per_launch <class> = <bytes>` is what bench.py reads for roofline.traffic.
"""

from __future__ import annotations

import argparse
import csv
import json
import re
import sys
from collections import defaultdict
from pathlib import Path

CALIB_ROW_BYTES = 16384
REQ_SIZE_WEIGHTS = {"TCC_EA0_RDREQ_32B_sum": 32.0, "TCC_EA0_RDREQ_64B_sum": 64.0, "TCC_EA0_RDREQ_128B_sum": 128.0}
MARKER_MIN_WGS = 4096           # calibration copy: >= 4096 rows of 16 KiB; engine copies have <= a few hundred

# kernel short name -> class of the decode step (names of the per-class HIP-event profiler in bench.py)
_EPI = {"0": "gemm", "1": "gemm_residual", "2": "gemm_w13", "3": "gemm_partial", "4": "gemm_lm_head", "5": "gemm_qkv"}


def short_name(name: str) -> str:
    """Kernel name without 'void ' and the argument list (template arguments kept)."""
    n = name[5:] if name.startswith("void ") else name
    depth = 0
    for i, ch in enumerate(n):
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0:
            return n[:i]
    return n


def classify(short: str, grid_x_threads=None) -> str:
    """Kernel class.  The bf16 qkv projection has its own epilogue (RoPE + KV append, 5); the split-K partial
    launches of o / w2 (and of qkv where it is launched as a plain partial GEMM) are told apart by their grid's x
    extent (weight row tiles), which the counter CSV does not carry (it reports the total grid)."""
    m = re.match(r"gemm_bf16_kernel<(\d+), (\d+), (\d+)(?:, (?:\d+|true|false))*>", short)
    if m:
        cls = _EPI.get(m.group(3), "gemm")
        if cls == "gemm_partial":
            if grid_x_threads is None:
                return "gemm_qkv_o_w2"
            ns = int(m.group(1))
            n_rows = grid_x_threads // 256 * 16 * ns
            cls = "gemm_qkv" if n_rows == 6144 else "gemm_o_w2"
        return cls
    m = re.match(r"gemm_wide_kernel<(\d+), (\d+), (\d+)(?:, (?:\d+|true|false))*>", short)
    if m:                                    # wide-M tier: same classes, qkv and o / w2 not told apart
        cls = _EPI.get(m.group(3), "gemm")
        return "gemm_qkv_o_w2" if cls == "gemm_partial" else cls
    for key, cls in (("attn_bf16_kernel", "attention"), ("attn_f32_kernel", "attention"),
                     ("attn_combine_kernel", "attention_combine"), ("add_rmsnorm_kernel", "rmsnorm"),
                     ("rope_append_kernel", "rope_append"), ("argmax_tiles_kernel", "head_pick"),
                     ("embed_kernel", "glue"), ("copy_rows_kernel", "glue"), ("greedy_accept_kernel", "glue"),
                     ("kv_rollback_kernel", "glue"), ("argmax_kernel", "glue"), ("kv_append_kernel", "kv_append")):
        if short.startswith(key):
            return cls
    return "other"


def _is_marker(short: str, grid_x_threads: int) -> bool:
    return short.startswith("copy_rows_kernel") and grid_x_threads // 256 >= MARKER_MIN_WGS


def _rows(path: str):
    with open(path, newline="") as f:
        yield from csv.DictReader(f)


def read_trace(path: str):
    """-> (marker duration ns, list of (short, class, duration ns)) of dispatches after the marker."""
    rows = sorted(_rows(path), key=lambda r: int(r["Dispatch_Id"]))
    out, marker, seen = [], None, False
    for r in rows:
        s = short_name(r["Kernel_Name"])
        gx = int(r["Grid_Size_X"])
        dur = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
        if not seen:
            if _is_marker(s, gx):
                seen, marker = True, dur
            continue
        out.append((s, classify(s, gx), dur))
    if not seen:
        raise SystemExit(f"{path}: no calibration copy found (run bench.py with --copy-calib-mib)")
    return marker, out


def read_counter(path: str, counter):
    """-> (marker value, {dispatch: (short, class, value)}) for dispatches after the marker.
    `counter` is a counter name, or a dict {name: weight} whose weighted sum is taken per dispatch."""
    weights = counter if isinstance(counter, dict) else {counter: 1.0}
    per = {}
    for r in _rows(path):
        if r["Counter_Name"] not in weights:
            continue
        d = int(r["Dispatch_Id"])
        s = short_name(r["Kernel_Name"])
        gx = int(r["Grid_Size"])
        v = weights[r["Counter_Name"]] * float(r["Counter_Value"])
        if d in per:
            per[d][3] += v
        else:
            per[d] = [s, gx, None, v]
    marker, out = None, {}
    for d in sorted(per):
        s, gx, _, v = per[d]
        if marker is None:
            if _is_marker(s, gx):
                marker = v
            continue
        out[d] = (s, classify(s), v)
    if marker is None:
        raise SystemExit(f"{path}: no calibration copy found (run bench.py with --copy-calib-mib)")
    return marker, out


def _bench(path):
    """Per-class figures of a bench.py JSON line: its `kernels` table, or, for an --attn-only run, the
    verify-attention launch (algorithmic bytes and the HIP-event average, which covers attention + combine)."""
    if not path:
        return {}
    line = json.loads(Path(path).read_text().strip().splitlines()[-1])
    out = dict(line.get("kernels") or {})
    va = line.get("verify_attn")
    if va and "attention" not in out:
        out["attention"] = {"bytes_per_launch": va["attn_bytes"], "avg_us": va["attn_us"]}
    return out


def cmd_trace(a):
    marker, disp = read_trace(a.csv)
    by_name = defaultdict(list)
    by_cls = defaultdict(list)
    for s, c, d in disp:
        by_name[s].append(d)
        by_cls[c].append(d)
    total = sum(d for _, _, d in disp)
    bench = _bench(a.bench)
    print("# Kernel durations (rocprofv3 --kernel-trace)\n")
    if a.cmd:
        print("Commands:\n")
        for c in a.cmd.split(" ;; "):
            print(f"    {c}")
        print()
    if a.title:
        print(a.title + "\n")
    print(f"Dispatches after the calibration copy: {len(disp)}; summed kernel time {total / 1e6:.3f} ms.\n")
    print("| class | launches | total ms | avg us | share | bench.py HIP-event avg us |")
    print("|---|---|---|---|---|---|")
    for c, ds in sorted(by_cls.items(), key=lambda kv: -sum(kv[1])):
        b = bench.get(c, {}).get("avg_us")
        print(f"| {c} | {len(ds)} | {sum(ds) / 1e6:.3f} | {sum(ds) / len(ds) / 1e3:.2f} | "
              f"{sum(ds) / total:.1%} | {'' if b is None else b} |")
    print("\n| kernel | launches | avg us | min us | max us |")
    print("|---|---|---|---|---|")
    for s, ds in sorted(by_name.items(), key=lambda kv: -sum(kv[1]))[:a.top]:
        print(f"| `{s}` | {len(ds)} | {sum(ds) / len(ds) / 1e3:.2f} | {min(ds) / 1e3:.2f} | {max(ds) / 1e3:.2f} |")


def cmd_pmc(a):
    known = a.calib_mib * 1024 * 1024
    fm, fetch = read_counter(a.fetch, "FETCH_SIZE")
    wm, write = read_counter(a.write, "WRITE_SIZE")
    f_scale = known / (fm * 1024)
    w_scale = known / (wm * 1024)
    bench = _bench(a.bench)
    fc, wc = defaultdict(list), defaultdict(list)
    for _, c, v in fetch.values():
        fc[c].append(v)
    for _, c, v in write.values():
        wc[c].append(v)
    print(f"# HBM traffic of {a.subject} (rocprofv3 --pmc FETCH_SIZE, then WRITE_SIZE)\n")
    if a.cmd:
        print("Commands:\n")
        for c in a.cmd.split(" ;; "):
            print(f"    {c}")
        print()
    if a.title:
        print(a.title + "\n")
    print(f"Calibration: a plain copy of {a.calib_mib} MiB read FETCH_SIZE = {fm:.0f} KiB and WRITE_SIZE = "
          f"{wm:.0f} KiB, so the scale factors are fetch x{f_scale:.3f} and write x{w_scale:.3f} "
          f"(counter KiB -> bytes moved).\n")
    print("| class | dispatches | fetch MB/launch | write MB/launch | traffic MB/launch | algorithmic MB/launch | traffic / algorithmic |")
    print("|---|---|---|---|---|---|---|")
    lines = []
    for c in sorted(fc, key=lambda c: -sum(fc[c])):
        f = sum(fc[c]) / len(fc[c]) * 1024 * f_scale
        w = (sum(wc[c]) / len(wc[c]) * 1024 * w_scale) if wc.get(c) else 0.0
        alg = bench.get(c, {}).get("bytes_per_launch")
        ratio = f"{(f + w) / alg:.3f}" if alg else ""
        algs = f"{alg / 1e6:.2f}" if alg else ""
        print(f"| {c} | {len(fc[c])} | {f / 1e6:.2f} | {w / 1e6:.2f} | {(f + w) / 1e6:.2f} | {algs} | {ratio} |")
        lines.append(f"traffic_bytes_per_launch {c} = {f + w:.0f}")
    if a.req_sizes:
        # exact read bytes from the request-size counters (FETCH_SIZE counts a 128-byte request as 64 bytes)
        rm, req = read_counter(a.req_sizes, REQ_SIZE_WEIGHTS)
        rc = defaultdict(list)
        for _, c, v in req.values():
            rc[c].append(v)
        print(f"\nRead bytes by request size (32 x TCC_EA0_RDREQ_32B + 64 x TCC_EA0_RDREQ_64B + 128 x "
              f"TCC_EA0_RDREQ_128B, summed over channels): the calibration copy reads {rm / known:.3f} x its "
              f"{a.calib_mib} MiB.\n")
        print("| class | read MB/launch (request sizes) | read MB/launch (scaled FETCH_SIZE) | algorithmic MB/launch |")
        print("|---|---|---|---|")
        for c in sorted(rc, key=lambda c: -sum(rc[c])):
            rb = sum(rc[c]) / len(rc[c])
            f = sum(fc[c]) / len(fc[c]) * 1024 * f_scale if fc.get(c) else 0.0
            alg = bench.get(c, {}).get("bytes_per_launch")
            print(f"| {c} | {rb / 1e6:.2f} | {f / 1e6:.2f} | {'' if not alg else f'{alg / 1e6:.2f}'} |")
            w = (sum(wc[c]) / len(wc[c]) * 1024 * w_scale) if wc.get(c) else 0.0
            lines.append(f"traffic_by_request_size {c} = {rb + w:.0f}")
    print("\n" + "\n".join(lines))


GEMM_SHAPES = {"qkv": (6144, 4096), "o": (4096, 4096), "w13": (28672, 4096), "w2": (4096, 14336),
               "head": (128256, 4096)}
HBM_PEAK = 8.0e12
BF16_PEAK = 2.5166e15


def _probe_groups(rows, seq):
    """Dispatch ids of the GEMM launches of each (class, M) group of a gemm_probe run: the dispatches after the
    i-th 64 MiB marker copy belong to seq[i] (the sequence the probe printed)."""
    out = defaultdict(list)
    gi = -1
    for d in sorted(rows):
        s, gx = rows[d]
        if s.startswith("copy_rows_kernel") and gx // 256 >= 4096:
            gi += 1
            continue
        if 0 <= gi < len(seq) and s.startswith("gemm_"):
            out[seq[gi]].append(d)
    return out


def cmd_gemm(a):
    """MFMA work, roofline fraction and cache behaviour of the projection GEMMs per class and token count."""
    seq = [(json.loads(l)["class"], json.loads(l)["M"]) for l in Path(a.sequence).read_text().splitlines()
           if l.startswith("{")]
    trace = {int(r["Dispatch_Id"]): r for r in _rows(a.trace)}
    names = {d: (short_name(r["Kernel_Name"]), int(r["Grid_Size_X"])) for d, r in trace.items()}
    groups = _probe_groups(names, seq)
    counters = defaultdict(lambda: defaultdict(float))
    cnames = {}
    for path in a.counters:
        for r in _rows(path):
            d = int(r["Dispatch_Id"])
            cnames.setdefault(path, {})[d] = (short_name(r["Kernel_Name"]), int(r["Grid_Size"]))
            counters[(path, d)][r["Counter_Name"]] += float(r["Counter_Value"])
    per = defaultdict(dict)
    for path in a.counters:
        for key, ds in _probe_groups(cnames[path], seq).items():
            for d in ds:
                for cn, v in counters[(path, d)].items():
                    per[key][cn] = per[key].get(cn, 0.0) + v / len(ds)
    print("# Projection GEMMs of the Llama3-8B layer shapes: MFMA work and roofline by token count\n")
    print("Commands:\n")
    for c in a.cmd.split(" ;; "):
        print(f"    {c}")
    print()
    print("Per (class, M): the probe's launches on distinct weights (one launch per GEMM call: the decode kernel up "
          "to 64 rows, the wide tier above).  t_roof = max(bytes / 8 TB/s, "
          "flops / 2.5166 PFLOP/s) with bytes = 2 (K N + M K + M N); frac = t_roof / measured.  MFMA flops = "
          "SQ_INSTS_VALU_MFMA_MOPS_BF16 x 512 (the counter's unit); MFMA util = MFMA flops / (time x 2.5166 PFLOP/s), "
          "the share of the dense bf16 peak the launch used.  L2 hit = TCC_HIT / (TCC_HIT + TCC_MISS).\n")
    print("| class | M | kernel(s) | us per call | t_roof us | bound | frac | MFMA flops / algorithmic | MFMA util | "
          "TFLOP/s | L2 hit |")
    print("|---|---|---|---|---|---|---|---|---|---|---|")
    for key in seq:
        ds = groups.get(key)
        if not ds:
            continue
        c, M = key
        N, K = GEMM_SHAPES[c]
        calls = a.reps
        us = sum((int(trace[d]["End_Timestamp"]) - int(trace[d]["Start_Timestamp"])) for d in ds) / 1e3 / calls
        flops = 2.0 * M * N * K
        t_hbm, t_mfma = 2.0 * (K * N + M * K + M * N) / HBM_PEAK, flops / BF16_PEAK
        t_roof = max(t_hbm, t_mfma) * 1e6
        cn = per.get(key, {})
        mops = cn.get("SQ_INSTS_VALU_MFMA_MOPS_BF16", 0.0) * 512 * len(ds) / calls
        hit, miss = cn.get("TCC_HIT_sum", 0.0), cn.get("TCC_MISS_sum", 0.0)
        kern = sorted({names[d][0] for d in ds})
        print(f"| {c} | {M} | {'; '.join('`' + k + '`' for k in kern)} | {us:.2f} | {t_roof:.2f} | "
              f"{'hbm' if t_hbm >= t_mfma else 'mfma'} | {t_roof / us:.3f} | {mops / flops:.3f} | "
              f"{mops / (us * 1e-6) / BF16_PEAK:.3f} | {flops / (us * 1e-6) / 1e12:.1f} | "
              f"{hit / max(hit + miss, 1):.2f} |")


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    sub = ap.add_subparsers(dest="mode", required=True)
    t = sub.add_parser("trace")
    t.add_argument("csv")
    t.add_argument("--bench")
    t.add_argument("--cmd")
    t.add_argument("--title")
    t.add_argument("--top", type=int, default=20)
    p = sub.add_parser("pmc")
    p.add_argument("fetch")
    p.add_argument("write")
    p.add_argument("--calib-mib", type=int, required=True)
    p.add_argument("--req-sizes", help="counter CSV of TCC_EA0_RDREQ_{32B,64B,128B}_sum")
    p.add_argument("--bench")
    p.add_argument("--cmd")
    p.add_argument("--title")
    p.add_argument("--subject", default="the decode steps")
    gm = sub.add_parser("gemm")
    gm.add_argument("trace")
    gm.add_argument("sequence", help="stdout of the thesis_amd.gemm_probe run (its JSON lines)")
    gm.add_argument("counters", nargs="*", help="counter_collection CSVs of the same probe sequence")
    gm.add_argument("--reps", type=int, default=10)
    gm.add_argument("--cmd", default="")
    gm.set_defaults(fn=cmd_gemm)
    a = ap.parse_args(argv)
    {"trace": cmd_trace, "pmc": cmd_pmc, "gemm": cmd_gemm}[a.mode](a)


def read_traffic(path: Path, cls: str):
    """Bytes per launch of kernel class `cls` from a committed pmc summary, or None."""
    try:
        for line in Path(path).read_text().splitlines():
            m = re.match(rf"traffic_bytes_per_launch {re.escape(cls)} = (\d+)", line.strip())
            if m:
                return float(m.group(1))
    except OSError:
        return None
    return None


if __name__ == "__main__":
    main(sys.argv[1:])
