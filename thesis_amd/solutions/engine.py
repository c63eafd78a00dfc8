"""EESD engine: batched early-exit self-speculation with packed shallow / deep steps on MI355X
(the reference's solutions/engine.py surface: EngineConfig, Request, EESDEngine.assign / step / run / run_poisson).

Step semantics are the reference's (solutions/engine.py:1-27, 269-489):
  shallow step  every decoding slot runs its current input token (last committed token if d = 0, else
                its newest draft) at position pos + d through layers [0, k) and the shared exit head
                -> one draft (seq_buf[i, d + 1]); its layer-k hidden state is kept in exit_h[i, d].
  deep step     the verifying slots (the policy's V) run their newest draft through [0, k) in the same
                shallow segment, then all d + 1 tokens (inputs exit_h[i, 0..d]) at pos..pos + d through
                [k, L) + head; greedy acceptance; the other slots draft in the same step.
  rollback      pointer only: pos += acc + 1, d = 0; rejected drafts' KV stays beyond pos, is never read
                (queries read positions <= their own) and is overwritten next round.
Device glue (id assembly + embedding, exit_h staging, draft head + argmax scatter into seq_buf, verify
gathers, greedy acceptance) runs in liblsk; the host reads the device once per deep step (accepted
counts + verified tokens) and never in a shallow step.

M2 (exit="m2", solutions/engine.py:284-288, 312-313, 458, 491-514): every probe_every-th deep step the
verifiers run all d + 1 tokens through the shallow layers, the hidden states entering every candidate exit are
captured in both segments, the shared head runs on all of them and lsk_probe_matches counts the agreement with Y on
the correct-prefix positions; ExitController may then move the exit layer (pending drafts are dropped).
M3 (prefill="m3", solutions/engine.py:289-305, 353-354, 424-426, 477-480): pieces of an admitted prompt ride on the
shallow segment (prompt ids through [0, k), layer-k states kept) and on the next deep segment (those states through
[k, L)); the last piece's head gives the request's first token.

Harness hook with no reference counterpart: `forced_accept_p` replaces each verifier's acceptance by
a seeded draw min(Geometric(p) - 1, d) and commits drafts[0..a-1] + Yv[a] (the tokens whose KV the deep
segment wrote), as the measured configurations prescribe.

Drivers: `run` (static pass / cyclic replay) and `run_poisson` (open loop) hand the slots to the shared
drivers of common/driver.py; `_report` turns the step log into the reference's metric names
(solutions/engine.py:694-753).
"""

from __future__ import annotations

import time
from dataclasses import asdict, dataclass, field
from typing import Callable, Optional

import numpy as np
import torch

from .. import _lsk
from ..common.driver import MeasureWindow, PoissonArrivals, run_arrivals, run_pool
from ..common.engine import commit_tokens
from ..common.timing import DeviceSpan
from .exit_select import ExitController
from .packed import Block, _attn_work, build_packed, build_packed_arrays, packed_layers, upload, upload_many
from .prefill import M3Planner
from .schedulers import make_scheduler
from .step_graph import ShallowGraphs

FREE, PREFILL, DECODE = 0, 1, 2


@dataclass
class EngineConfig:
    """Engine options (the reference's field names and defaults).

    mode / sched / gamma / k / d_max / min_draft / initial_draft / omega / alpha0 / sla_steps
        decoding mode ("spec" or "ar"), deep-step policy and its knobs (solutions/schedulers.py)
    exit / probe_every / k_cands / switch_margin / m2_force
        exit-layer policy: "fixed", or "m2" with probes every `probe_every` deep steps over `k_cands`
    prefill / prefill_chunk / max_wait / knee_safety / m3_chunk_cap
        "separate" prefill in `prefill_chunk` pieces, or "m3" piggybacking (solutions/prefill.py)
    bucketing
        build_packed's accounting mode ("exact" | "pad"); the native kernels serve both alike
    forced_accept_p / forced_seed
        harness hook: seeded geometric acceptance instead of the greedy comparison
    graphs
        replay fixed-shape shallow-only steps as captured HIP graphs
    """
    mode: str = "spec"
    sched: str = "fixed"
    gamma: int = 4
    k: int = 3
    exit: str = "fixed"
    prefill: str = "separate"
    d_max: int = 16
    sla_steps: int = 32
    initial_draft: int = 3
    min_draft: int = 1
    omega: float = 0.8
    alpha0: float = 0.9
    probe_every: int = 20
    k_cands: tuple = (2, 3, 4, 5, 6, 7, 8)
    switch_margin: float = 0.05
    max_wait: int = 3
    knee_safety: float = 0.9
    prefill_chunk: int = 512
    bucketing: str = "exact"
    m3_chunk_cap: Optional[int] = None
    m2_force: Optional[str] = None
    forced_accept_p: Optional[float] = None
    forced_seed: int = 0
    graphs: bool = True
    launch_ahead: bool = True          # launch the next shallow segment before a deep step's readback

    def check(self, n_layers: int) -> None:
        """ValueError for option combinations the engine cannot run."""
        if self.exit not in ("fixed", "m2"):
            raise ValueError(f"unknown exit policy {self.exit!r}")
        if self.prefill not in ("separate", "m3"):
            raise ValueError(f"unknown prefill policy {self.prefill!r}")
        if self.mode == "ar" and self.prefill != "separate":
            raise ValueError("AR mode supports --prefill separate only")
        if not 1 <= self.k < n_layers:
            raise ValueError("exit layer must be in [1, n_layers)")

    def label(self) -> str:
        if self.mode == "ar":
            return "ar"
        policy = self.sched + (f"-g{self.gamma}" if self.sched == "fixed" else "")
        exit_part = f"k{self.k}" if self.exit == "fixed" else "m2"
        return f"{policy}-{exit_part}-{self.prefill}"


@dataclass
class Request:
    """One request and its life in the engine: output tokens, finish reason, the step-log indices of its
    assignment / first token / last step (for TTFT and TPOT), wall times, and M3 progress."""
    pid: str
    prompt: list
    out: list = field(default_factory=list)
    finish: Optional[str] = None
    log_assign: int = 0
    log_first: int = -1
    log_finish: int = -1
    wall_arrival: float = 0.0
    wall_first: float = 0.0
    measured: bool = False
    pf_sh: int = 0                  # prompt tokens already through the shallow layers (M3)
    pf_dp: int = 0                  # prompt tokens already through every layer (M3)
    piggybacked: int = 0            # prompt tokens carried by decode steps (M3)
    key: int = -1                   # assignment counter: the forced-acceptance stream of the request


_RB_HOST: list = []


def _pinned_readback(n: int) -> torch.Tensor:
    """n int64 of a process-wide pinned buffer for step readbacks (grown, never freed: pinned memory released
    while a graph is being captured would record on the capturing stream).  Engines in one process read back
    one after another (each waits for its copy before the next step)."""
    if not _RB_HOST or _RB_HOST[0].numel() < n:
        _RB_HOST[:] = [torch.empty(max(n, 1024), dtype=torch.long, pin_memory=True)] + _RB_HOST
    return _RB_HOST[0][:n]


@dataclass
class StepEntry:
    """One engine call in the step log: its kind, device span, whether it counts, and its token mix."""
    kind: str                       # shallow | deep | probe | ar | prefill
    span: DeviceSpan
    measured: bool
    n_sh: int = 0
    n_dp: int = 0
    n_chunk: int = 0
    plan_ms: float = 0.0
    k: int = 0

    @property
    def ms(self) -> float:
        return self.span.ms


class ForcedAcceptance:
    """a = Geometric(p) - 1 per verification round, from default_rng([seed, key]) of the request."""

    def __init__(self, p: float, seed: int = 0):
        self.p, self.seed = p, seed
        self.streams: dict = {}

    def draw(self, key: int) -> int:
        rng = self.streams.get(key)
        if rng is None:
            rng = self.streams[key] = np.random.default_rng([self.seed, key])
        return int(rng.geometric(self.p)) - 1


_COUNTERS = ("steps", "deep_steps", "probe_steps", "deep_tokens", "verifiers", "drafted", "accepted", "committed",
             "plan_ms", "plan_calls", "prefill_tokens", "piggyback_tokens", "separate_prefills", "m3_fallbacks",
             "dropped_drafts", "kv_read_pos", "kv_gathered_pos")


class EESDEngine:
    def __init__(self, model, B: int, max_prompt: int, max_new: int, eos_ids, cfg: EngineConfig, cost_model,
                 stop_for: Optional[Callable] = None, ref: Optional[dict] = None):
        cfg.check(model.n_layers)
        self.m, self.dev, self.B, self.cfg, self.cm = model, model.device, B, cfg, cost_model
        self.max_new, self.eos = max_new, set(eos_ids)
        self.stop_for = stop_for or (lambda pid: None)
        self.k, self.L = cfg.k, model.n_layers
        self.Dm1 = cfg.d_max + 1
        self._allocate(max_prompt)
        self._policies(cost_model)
        self.records: list = []
        self.measuring = False
        self.stats = dict.fromkeys(_COUNTERS, 0)
        self.stats["plan_ms"] = 0.0
        self.fallback_reasons: dict = {}
        self.round_len = cfg.gamma          # steps per round last observed (M3's deep-size estimate)
        self.steps_since_deep = 0
        self.kv_bytes_per_pos = 2 * model.cfg.n_kv_heads * model.cfg.head_dim * model.dtype.itemsize
        self._keys = 0
        # set to [] to log every step's segment shapes: {"sh": shallow blocks, "n_draft", "dp": deep blocks (verify
        # blocks and M3 chunks), "committed", "m": measured, "pf": a separate prefill's chunks (entries of their own)}
        self.trace: Optional[list] = None
        self._dp_blocks: list = []

    def _allocate(self, max_prompt: int) -> None:
        """Cache rows for prompt + output + drafts + slack; device seq_buf / exit_h; host slot arrays."""
        m, B = self.m, self.B
        m.allocate_cache(B, max_prompt + self.max_new + self.cfg.d_max + 40)
        self.seq_buf = torch.zeros(B, self.Dm1, dtype=torch.long, device=self.dev)
        self.exit_h = torch.zeros(B, self.Dm1, m.cfg.dim, dtype=m.dtype, device=self.dev)
        self._flat_views = (self.seq_buf.view(-1), self.exit_h.view(-1, m.cfg.dim))
        self.state = np.zeros(B, dtype=np.int64)        # FREE / PREFILL / DECODE
        self.pos = np.zeros(B, dtype=np.int64)          # committed length = position of the current input token
        self.d = np.zeros(B, dtype=np.int64)            # drafts held
        self.gen = np.zeros(B, dtype=np.int64)          # tokens generated
        self.req: list = [None] * B
        self.pending: list = [[] for _ in range(B)]     # M3: (pos0, c, layer-k states) awaiting the deep segment

    def _policies(self, cm) -> None:
        cfg = self.cfg
        spec = cfg.mode == "spec"
        self.sched = make_scheduler(cfg.sched, self.B, cm, self.k, gamma=cfg.gamma, d_max=cfg.d_max,
                                    sla_steps=cfg.sla_steps, initial_draft=cfg.initial_draft, omega=cfg.omega,
                                    alpha0=cfg.alpha0, min_draft=cfg.min_draft) if spec else None
        cands = [c for c in cfg.k_cands if 1 <= c < self.L]
        self.exitc = ExitController(cm, self.k, cands, cfg.probe_every, cfg.switch_margin, cfg.omega, cfg.d_max,
                                    cfg.m2_force) if cfg.exit == "m2" else None
        self.m3 = M3Planner(cm, cfg.max_wait, cfg.m3_chunk_cap, cfg.prefill_chunk,
                            cfg.knee_safety) if cfg.prefill == "m3" else None
        self.forced = ForcedAcceptance(cfg.forced_accept_p, cfg.forced_seed) if cfg.forced_accept_p else None
        self.graphs = ShallowGraphs(self.dev) if cfg.graphs and spec else None
        self.launch_ahead = cfg.launch_ahead and spec
        self._ahead = None                 # the shallow segment _launch_ahead started for the next step
        self.ahead_used = 0                # steps that ran the shallow segment launched ahead of the readback

    # ------------------------------------------------------------------ bookkeeping
    def _log(self, kind, span, **kw) -> StepEntry:
        e = StepEntry(kind, span, self.measuring, k=self.k, **kw)
        self.records.append(e)
        return e

    def _commit(self, slot: int, toks) -> int:
        r = self.req[slot]
        if r.finish is not None:
            return 0
        n, r.finish = commit_tokens(r.out, toks, eos=self.eos, max_new=self.max_new,
                                    stop_checker=self.stop_for(r.pid))
        self.gen[slot] = len(r.out)
        return n

    def _start_decoding(self, slot: int, first: int) -> int:
        """The prompt is in the cache: the slot decodes from its first token (a fresh acceptance estimate)."""
        r = self.req[slot]
        r.log_first, r.wall_first = len(self.records) - 1, time.perf_counter()
        self.state[slot], self.pos[slot], self.d[slot] = DECODE, len(r.prompt), 0
        if self.sched is not None:
            self.sched.reset(slot)
        return self._commit(slot, [first])

    def _flat(self):
        """(seq_buf flat, exit_h as rows): views made once with the buffers (a step's host path is latency)."""
        return self._flat_views

    # ------------------------------------------------------------------ assignment / prefill
    def _piggyback(self, req: Request) -> bool:
        """M3 admission of a prompt next to the decoding slots; a refusal is counted by reason."""
        live = self.state == DECODE
        if self.m3 is None or not live.any():
            return False
        n_live = int(live.sum())
        ok, why = self.m3.admission(len(req.prompt), n_live, n_live * (self.round_len + 1), self.k,
                                    float((self.pos + self.d)[live].sum()))
        if not ok:
            self.stats["m3_fallbacks"] += 1
            self.fallback_reasons[why] = self.fallback_reasons.get(why, 0) + 1
        return ok

    def assign(self, slot: int, req: Request) -> int:
        """Put `req` in a free slot: piggybacked (its pieces ride the next steps) or prefilled now.  Returns the
        tokens committed (the first token of a separate prefill)."""
        req.log_assign, req.measured = len(self.records), self.measuring
        if req.key < 0:
            req.key = self._keys
        self._keys += 1
        self.req[slot], self.pending[slot], self.d[slot] = req, [], 0
        if self._piggyback(req):
            self.state[slot] = PREFILL
            req.pf_sh = req.pf_dp = 0
            return 0
        return self._prefill_separate(slot)

    @torch.inference_mode()
    def _prefill_separate(self, slot: int) -> int:
        m, r = self.m, self.req[slot]
        n = len(r.prompt)
        if n < 1:
            raise ValueError("empty prompt")
        span = DeviceSpan(self.dev).open()
        h = None
        for s in range(0, n, self.cfg.prefill_chunk):
            c = min(self.cfg.prefill_chunk, n - s)
            pb = build_packed(m, [Block(slot, s, c)], self.cfg.bucketing)
            self._count_kv(pb, self.L)
            h = packed_layers(m, m.embed(upload(r.prompt[s:s + c], self.dev)), pb, 0, self.L)
        sb, _ = self._flat()
        y0 = m.head_argmax(h[-1:])
        _lsk.copy_rows(sb.view(-1, 1), upload([slot * self.Dm1], self.dev), y0.view(-1, 1), None, 1)
        span.close()
        self._log("prefill", span, n_chunk=n)
        if self.trace is not None:
            pc = self.cfg.prefill_chunk
            self.trace.append({"sh": [], "n_draft": 0, "dp": [], "committed": 1, "m": bool(self.measuring),
                               "pf": [(slot, s0, min(pc, n - s0)) for s0 in range(0, n, pc)]})
        self.stats["separate_prefills"] += 1
        if self.measuring:
            self.stats["prefill_tokens"] += n
        return self._start_decoding(slot, int(y0.item()))

    # ------------------------------------------------------------------ one step
    @torch.inference_mode()
    def step(self) -> tuple:
        """Run one step; returns (committed tokens, slots that finished)."""
        if self.cfg.mode == "ar":
            return self._ar_step()
        return self._spec_step()

    def _ar_step(self):
        m = self.m
        dec = np.flatnonzero(self.state == DECODE)
        if len(dec) == 0:
            return 0, []
        pb = build_packed(m, [Block(int(i), int(self.pos[i]), 1) for i in dec], self.cfg.bucketing)
        self._count_kv(pb, self.L)
        slots = np.array([b.row for b in pb.blocks], dtype=np.int64)
        idx = upload(slots * self.Dm1, self.dev)
        sb, _ = self._flat()
        span = DeviceSpan(self.dev).open()
        x = m.buffer("x_in", (len(slots), m.cfg.dim), m.dtype)
        _lsk.embed(m.embed_w, idx, x, sb, idx)
        h = packed_layers(m, x, pb, 0, self.L)
        y = m.head_argmax(h)
        _lsk.copy_rows(sb.view(-1, 1), idx, y.view(-1, 1), None, len(slots))
        span.close()
        self._log("ar", span, n_sh=len(slots), n_dp=len(slots))
        y_h = y.tolist()
        committed, done = 0, []
        for s, t in zip(slots.tolist(), y_h):
            self.pos[s] += 1
            committed += self._commit(s, [t])
            if self.req[s].finish:
                done.append(s)
        self._tally(committed, deep=True, n_deep=len(slots), verifiers=len(slots))
        return committed, done

    def _verify_set(self, d, ctx, dec) -> np.ndarray:
        V = self.sched.decide(d, ctx, dec, self.steps_since_deep) if dec.any() else np.zeros(self.B, dtype=bool)
        return (V | (dec & (d >= self.cfg.d_max))) & dec & (d >= 1)

    def _spec_step(self):
        m, cfg, k = self.m, self.cfg, self.k
        Dm1 = self.Dm1
        t0 = time.perf_counter()
        dec = self.state == DECODE
        d = self.d.copy()
        ctx = np.where(dec, self.pos + d, 0)
        ahead, self._ahead = self._ahead, None
        if self.m3 is None and self.exitc is None and dec.any():
            return self._spec_step_early(dec, d, ctx, t0, ahead)
        return self._spec_step_general(dec, d, ctx, t0)

    def _spec_step_general(self, dec, d, ctx, t0):
        m, cfg, k = self.m, self.cfg, self.k
        Dm1 = self.Dm1
        V = self._verify_set(d, ctx, dec)
        # M3 progress guarantee: with no decoding slot, pending prompts run both segments in this step
        flush = (not dec.any()) and bool((self.state == PREFILL).any())
        deep = bool(V.any()) or flush
        Dr = dec & ~V
        probe = deep and self.exitc is not None and self.exitc.probe_due() and bool(V.any())
        chunks = self._plan_chunks(dec, d, V, deep, probe, flush, ctx) if self.m3 is not None else []
        plan_ms = 1000 * (time.perf_counter() - t0)

        # ---- shallow segment: one block per decoding slot (T = 1 at pos + d, or all d + 1 tokens of a probed
        # verifier), plus the M3 chunks
        dslots = np.flatnonzero(dec)
        chunk_slices = []
        gentry = None
        if not probe and not chunks:
            # every block is one token at pos + d: token j <-> packed block j
            if len(dslots) == 0:
                return 0, []
            pb = build_packed_arrays(m, dslots, self.pos[dslots] + d[dslots], np.ones(len(dslots), dtype=np.int64),
                                     cfg.bucketing, upload_meta=False)
            kb = sb_slot = None
            N = pb.n_tokens
            sl = dslots[pb.order]
            sel = sl * Dm1 + d[sl]
            drf_src = np.flatnonzero(Dr[sl])
            drf_dst = sel[drf_src] + 1
            nd, nex = len(drf_src), N
            if not deep and self.graphs is not None and not _lsk.Profiler.enabled:
                # shallow-only step of a fixed shape: staged at fixed addresses, replayed as a graph below
                gkey = (N, pb.nb, pb.n_works, pb.n_groups, pb.n_parts, pb.n_rounds, pb.n_slots, pb.rows_cap, nd, k)
                (pb.meta, sel_t, drf_src_t, drf_dst_t), gentry = self.graphs.stage(
                    gkey, [pb.meta_host, sel, drf_src, drf_dst])
            else:
                pb.meta, sel_t, drf_src_t, drf_dst_t = upload_many([pb.meta_host, sel, drf_src, drf_dst], self.dev)
            alt_t, ex_dst_t, ex_src_t = sel_t, sel_t, None
        else:
            full = V[dslots] if probe else np.zeros(len(dslots), dtype=bool)
            rows = np.concatenate([dslots, np.array([c[0] for c in chunks], dtype=np.int64)])
            pos0 = np.concatenate([np.where(full, self.pos[dslots], self.pos[dslots] + d[dslots]),
                                   np.array([c[1] for c in chunks], dtype=np.int64)])
            T = np.concatenate([np.where(full, d[dslots] + 1, 1), np.array([c[2] for c in chunks], dtype=np.int64)])
            kind = np.concatenate([np.where(full, 1, 0), np.full(len(chunks), 2)]).astype(np.int64)  # sh/full/chunk
            pb = build_packed_arrays(m, rows, pos0, T, cfg.bucketing, upload_meta=False)
            N = pb.n_tokens
            kb, sb_slot = kind[pb.order], rows[pb.order]
            tb = np.repeat(np.arange(pb.nb), pb.blk_T)                   # block of every token
            j = np.arange(N) - pb.offsets[:-1][tb]                       # position within its block
            kt, st = kb[tb], sb_slot[tb]
            dst_d = np.where(kt == 1, j, d[st])                          # exit_h / seq_buf column of the token
            sel = np.where(kt == 2, -1, st * Dm1 + dst_d)
            alt = np.zeros(N, dtype=np.int64)
            for bi in np.flatnonzero(kb == 2):
                s0, i, p = int(pb.offsets[bi]), int(sb_slot[bi]), int(pb.blk_pos0[bi])
                c = int(pb.blk_T[bi])
                alt[s0:s0 + c] = self.req[i].prompt[p:p + c]
                chunk_slices.append((i, p, c, s0))
            ex_src = np.flatnonzero(kt != 2)
            ex_dst = st[ex_src] * Dm1 + dst_d[ex_src]
            drf_src = np.flatnonzero((kt == 0) & Dr[st])
            drf_dst = st[drf_src] * Dm1 + d[st[drf_src]] + 1
            nd, nex = len(drf_src), len(ex_src)
            pb.meta, sel_t, alt_t, ex_dst_t, ex_src_t, drf_src_t, drf_dst_t = upload_many(
                [pb.meta_host, sel.astype(np.int64), alt, ex_dst.astype(np.int64), ex_src.astype(np.int64),
                 drf_src.astype(np.int64), drf_dst.astype(np.int64)], self.dev)
        self._count_kv(pb, k)
        sb, exh = self._flat()
        span = DeviceSpan(self.dev).open()
        if gentry is not None:
            def shallow_gpu():
                xg = m.buffer("x_in", (N, m.cfg.dim), m.dtype)
                _lsk.embed(m.embed_w, sel_t, xg, sb, sel_t)
                hg = packed_layers(m, xg, pb, 0, k)
                _lsk.copy_rows(exh, sel_t, hg, None, N)
                if nd:
                    hx = m.buffer("x_draft", (nd, m.cfg.dim), m.dtype)
                    _lsk.copy_rows(hx, None, hg, drf_src_t, nd)
                    m.head_argmax(hx, out=sb, dst_idx=drf_dst_t)
            self.graphs.run(gentry, lambda: m.buf_epoch, shallow_gpu)
            span.close()
            self._log("shallow", span, n_sh=N, n_dp=0, n_chunk=0, plan_ms=plan_ms)
            self.d[Dr] += 1
            if self.trace is not None:
                self.trace.append({"sh": list(zip(pb.blk_rows.tolist(), pb.blk_pos0.tolist(), pb.blk_T.tolist())),
                                   "n_draft": nd, "dp": [], "committed": 0, "m": bool(self.measuring)})
            self.steps_since_deep += 1
            self._tally(0, deep=False, plan_ms=plan_ms)
            return 0, []
        x = m.buffer("x_in", (N, m.cfg.dim), m.dtype)
        _lsk.embed(m.embed_w, alt_t, x, sb, sel_t)                        # seq_buf ids, or prompt ids for chunks
        cap_sh = {} if probe else None
        h = packed_layers(m, x, pb, 0, k, cap_sh, tuple(c for c in self.exitc.cands if c < k) if probe else ())
        if nex:
            _lsk.copy_rows(exh, ex_dst_t, h, ex_src_t, nex)               # exit_h[i, d_i] (all j of a probe) = h
        for (i, p, c, s0) in chunk_slices:
            self.pending[i].append((p, c, h[s0:s0 + c]))                  # layer-k states wait for the deep segment
        return self._finish_step(V, d, deep, probe, chunks, h, nd, drf_src_t, drf_dst_t, span, plan_ms, pb, kb,
                                 sb_slot, cap_sh, N, Dr)

    def _spec_step_early(self, dec, d, ctx, t0, ahead=None):
        """Steps without M2 probes or M3 chunks: the shallow segment (one token at pos + d per decoding slot,
        whatever the verify set) is staged and launched first -- replayed as a graph when its shape repeats --
        and the draft policy's host time overlaps it on the device.  After a deep step it was launched before that
        step's readback (_launch_ahead), so the device never waits for the host between steps.  Then the draft
        head and the deep segment follow as in any step; every launch is the one the general path makes, in the
        same stream order."""
        dslots = np.flatnonzero(dec)
        sh = self._take_ahead(ahead, dslots, d)
        if sh is None:
            sh = self._shallow_early(dslots, self.pos[dslots] + d[dslots], d)
            plan_ms = 1000 * (time.perf_counter() - t0)
        else:
            plan_ms = sh["plan_ms"] + 1000 * (time.perf_counter() - t0)
        pb, sl, sel, h, N, span = sh["pb"], sh["sl"], sh["sel"], sh["h"], sh["N"], sh["span"]
        self._count_kv(pb, self.k)
        t1 = time.perf_counter()
        V = self._verify_set(d, ctx, dec)
        deep = bool(V.any())
        Dr = dec & ~V
        drf_src = np.flatnonzero(Dr[sl])
        drf_dst = sel[drf_src] + 1
        nd = len(drf_src)
        drf_src_t = drf_dst_t = None
        if nd:
            drf_src_t, drf_dst_t = upload_many([drf_src, drf_dst], self.dev)
        plan_ms += 1000 * (time.perf_counter() - t1)
        return self._finish_step(V, d, deep, False, [], h, nd, drf_src_t, drf_dst_t, span, plan_ms, pb, None, None,
                                 None, N, Dr)

    def _shallow_early(self, dslots, positions, dnext, shift=None) -> dict:
        """Plan, stage and launch the early path's shallow segment: one token per slot of dslots at `positions`,
        input seq_buf[i, dnext[i]], exit state to exit_h[i, dnext[i]].  shift = (accepted device tensor, vslots
        device int32, vdrafts device int32, nv): the plan's positions are upper bounds for those slots, corrected
        on the device (lsk_shift_segment_positions) before the segment runs."""
        m, k, Dm1 = self.m, self.k, self.Dm1
        pb = build_packed_arrays(m, dslots, positions, np.ones(len(dslots), dtype=np.int64), self.cfg.bucketing,
                                 upload_meta=False)
        N = pb.n_tokens
        sl = dslots[pb.order]
        sel = sl * Dm1 + dnext[sl]
        sb, exh = self._flat()
        span = DeviceSpan(self.dev).open()

        def shift_meta():
            if shift is not None:
                acc_t, vslots_t, vdrafts_t, nv = shift
                _lsk.shift_segment_positions(pb.meta, N, pb.nb, pb.n_works, pb.n_groups, pb.n_slots * pb.n_rounds,
                                             m.group, acc_t, vslots_t, vdrafts_t, nv)
        if self.graphs is not None and not _lsk.Profiler.enabled:
            gkey = ("early", N, pb.nb, pb.n_works, pb.n_groups, pb.n_parts, pb.n_rounds, pb.n_slots, pb.rows_cap, k)
            (pb.meta, sel_t), gentry = self.graphs.stage(gkey, [pb.meta_host, sel])
            shift_meta()

            def shallow_gpu():
                xg = m.buffer("x_in", (N, m.cfg.dim), m.dtype)
                _lsk.embed(m.embed_w, sel_t, xg, sb, sel_t)
                hg = packed_layers(m, xg, pb, 0, k)
                _lsk.copy_rows(exh, sel_t, hg, None, N)                  # exit_h[i, d_i] = h
                return hg
            self.graphs.run(gentry, lambda: m.buf_epoch, shallow_gpu)
            h = gentry.out
        else:
            pb.meta, sel_t = upload_many([pb.meta_host, sel], self.dev)
            shift_meta()
            x = m.buffer("x_in", (N, m.cfg.dim), m.dtype)
            _lsk.embed(m.embed_w, sel_t, x, sb, sel_t)
            h = packed_layers(m, x, pb, 0, k)
            _lsk.copy_rows(exh, sel_t, h, None, N)
        return {"pb": pb, "sl": sl, "sel": sel, "h": h, "N": N, "span": span}

    def _launch_ahead(self, V, d, vslots, acc_t) -> None:
        """At the end of a deep step, before its readback: launch the next step's shallow segment (the early
        path's), so the device runs it while the host reads the acceptance back and plans.  Every decoding slot
        gets one token; a verifier's next position depends on its accepted count, so the segment is planned at
        its upper bound (all d drafts accepted) and moved back on the device from greedy_accept's output.  Skipped
        when a verifier's possible positions straddle a KV split (the plan's shape would depend on the count) or
        the upper bound leaves the cache.  A slot whose request finishes at this readback computes one unused
        token; its cache row is free until a new request's prefill rewrites it."""
        if not self.launch_ahead or self.m3 is not None or self.exitc is not None or self.cfg.mode == "ar":
            return
        if self.dev.type != "cuda" or not vslots:
            return
        t0 = time.perf_counter()
        dec = self.state == DECODE
        dslots = np.flatnonzero(dec)
        if not len(dslots):
            return
        m = self.m
        vs = np.asarray(vslots, dtype=np.int64)
        dnext = self.d.copy()                                              # drafting slots: d + 1 already
        dnext[vs] = 0
        est = self.pos + d + 1                                             # every slot's next position (upper bound)
        split = m.cache.attn_split
        lo_end, hi_end = self.pos[vs] + 2, self.pos[vs] + d[vs] + 2        # a verifier's possible KV ends
        if ((lo_end + split - 1) // split != (hi_end + split - 1) // split).any():
            return
        if int(est[dslots].max()) + 1 > min(m.cache.max_seq, m.rope_cos.shape[0]):
            return
        vslots_t, vdrafts_t = upload_many([vs.astype(np.int32), d[vs].astype(np.int32)], self.dev)
        sh = self._shallow_early(dslots, est[dslots], dnext, (acc_t, vslots_t, vdrafts_t, len(vs)))
        sh.update(slots=dslots, reqs=[self.req[i] for i in dslots], est=est.copy(), vslots=vs, vdrafts=d[vs].copy(),
                  plan_ms=1000 * (time.perf_counter() - t0))
        self._ahead = sh

    def _take_ahead(self, sh, dslots, d):
        """The shallow segment _launch_ahead started for this step (sh), when it covers every decoding slot with
        the request it was planned for.  Otherwise (a slot started decoding since, or a freed slot took a new
        request) the step plans its own segment, which rewrites the same values for the slots both cover; the
        ahead segment's other writes lie at positions its row's next request writes before reading.  Its host
        copies of the positions are set to the actual ones."""
        if sh is None or "acc" not in sh:
            return None
        planned = dict(zip(sh["slots"].tolist(), sh["reqs"]))
        if any(planned.get(i, None) is not self.req[i] for i in dslots.tolist()):
            return None
        actual = self.pos + d
        want = sh["est"].copy()
        want[sh["vslots"]] -= sh["vdrafts"] - sh["acc"]
        if not np.array_equal(actual[dslots], want[dslots]):
            raise RuntimeError("launch-ahead shallow segment: planned positions disagree with the committed ones")
        pb = sh["pb"]
        pos = actual[sh["sl"]]
        meta, cnt = _lsk.pack_segment(pb.blk_rows, pos, pb.blk_T, self.m.group, self.m.cache.attn_split,
                                      self.m.cfg.n_kv_heads, self.m.cfg.head_dim, pb.n_slots,
                                      0 if self.cfg.bucketing == "exact" else 1, self.m.cache.max_batch,
                                      self.m.cache.max_seq, self.m.rope_cos.shape[0])
        pb.blk_pos0, pb.pos_h = pos, np.repeat(pos, pb.blk_T)              # T = 1: one position per block
        pb.kv_read, pb.kv_read_padded, pb.kv_gathered = cnt[6], cnt[7], cnt[8]
        _attn_work(pb, self.m, cnt[6], cnt[9])
        self.ahead_used += 1
        return sh

    def _finish_step(self, V, d, deep, probe, chunks, h, nd, drf_src_t, drf_dst_t, span, plan_ms, pb, kb, sb_slot,
                     cap_sh, N, Dr):
        """After the shallow segment: the draft head, the deep segment with the step's LM-head launch and
        greedy acceptance, the readback and the host bookkeeping."""
        m = self.m
        sb, _ = self._flat()
        n_verify = int((d[V] + 1).sum()) if deep else 0
        merge_heads = deep and not probe
        if nd and not merge_heads:
            hx = m.buffer("x_draft", (nd, m.cfg.dim), m.dtype)
            _lsk.copy_rows(hx, None, h, drf_src_t, nd)
            m.head_argmax(hx, out=sb, dst_idx=drf_dst_t)                  # seq_buf[i, d_i + 1] = draft
        readback, n_v_tok, vinfo, cfin = None, 0, ([], [], []), []
        if deep:
            # the drafts are first read next step, so their head shares the verify head's launch: one pass over
            # the LM head weights per step (above 64 rows the wide tier still reads them once: 65-128 rows cost
            # ~270 us on MI355X against ~340-370 us for two launches); the batch-invariant GEMM gives every row
            # the same result either way
            draft = (h, drf_src_t, drf_dst_t, nd) if merge_heads else (h, None, None, 0)
            probe_ctx = (pb, kb, sb_slot, cap_sh) if probe else None
            rb_dev, n_v_tok, vinfo, cfin = self._deep(V, d, draft, probe_ctx)
            readback = self._readback(rb_dev)
        span.close()
        n_chunk = sum(c[2] for c in chunks)
        self._log("probe" if probe else ("deep" if deep else "shallow"), span, n_sh=N, n_dp=n_v_tok, n_chunk=n_chunk,
                  plan_ms=plan_ms)
        self.d[Dr] += 1
        if self.measuring:
            self.stats["piggyback_tokens"] += n_chunk
        for (i, _, c) in chunks:
            self.req[i].piggybacked += c
        if self.trace is not None:
            self.trace.append({"sh": list(zip(pb.blk_rows.tolist(), pb.blk_pos0.tolist(), pb.blk_T.tolist())),
                               "n_draft": nd, "dp": self._dp_blocks if deep else [], "committed": 0,
                               "m": bool(self.measuring)})
        if not deep:
            self.steps_since_deep += 1
            self._tally(0, deep=False, plan_ms=plan_ms)
            return 0, []
        vslots, vstarts, vT = vinfo
        nv = len(vslots)
        self._launch_ahead(V, d, vslots, rb_dev[:nv])
        rb = readback()
        acc = np.array(rb[:nv], dtype=np.int64)
        if self._ahead is not None:
            self._ahead["acc"] = acc
        Y = rb[nv:nv + n_v_tok]
        accepted = np.zeros(self.B, dtype=np.int64)
        committed, done = 0, []
        for jv, i in enumerate(vslots):
            a = int(acc[jv])
            accepted[i] = a
            toks = Y[vstarts[jv]:vstarts[jv] + a + 1]
            self.pos[i] += a + 1
            self.d[i] = 0
            committed += self._commit(i, toks)
            if self.measuring and self.req[i].finish is None:
                self.stats["drafted"] += int(d[i])
                self.stats["accepted"] += a
            if self.req[i].finish:
                done.append(i)
        off = nv + n_v_tok
        for jf, i in enumerate(cfin):                                     # M3: prompts whose last chunk finished
            committed += self._start_decoding(i, int(rb[off + jf]))
            if self.req[i].finish:
                done.append(i)
        off += len(cfin)
        self.sched.observe(V, accepted, d)
        if self.trace is not None:
            self.trace[-1]["committed"] = committed
        self.round_len = self.steps_since_deep
        self.steps_since_deep = 0
        t2 = time.perf_counter()
        if self.exitc is not None:
            if probe:
                nc = len(self.exitc.cands)
                self.exitc.absorb_probe(rb[off:off + nc], int(rb[off + nc]))
            self.exitc.deep_step_done()
            dec_now = self.state == DECODE
            new = self.exitc.propose(int(dec_now.sum()), float((self.pos + self.d)[dec_now].sum()),
                                          allowed=not (self.state == PREFILL).any())
            if new is not None:
                self._switch_exit(new)
        plan_ms += 1000 * (time.perf_counter() - t2)
        self._tally(committed, deep=True, n_deep=n_v_tok, verifiers=nv, plan_ms=plan_ms, probe=probe)
        return committed, done

    def _plan_chunks(self, dec, d, V, deep, probe, flush, ctx) -> list:
        """M3 chunks riding on this step's shallow segment: [(slot, pos0, c)] (solutions/engine.py:289-305)."""
        pf = np.flatnonzero(self.state == PREFILL)
        if not len(pf):
            return []
        n_sh = int(dec.sum()) + (int((d[V] + 1).sum() - V.sum()) if probe else 0)
        n_dp_est = int((d[V] + 1).sum()) if deep else int(dec.sum()) * (max(self.round_len, 1) + 1)
        pend = sum(c for i in range(self.B) for (_, c, _) in self.pending[i])
        chunks = []
        for i in pf:
            r = self.req[i]
            rem = len(r.prompt) - r.pf_sh
            if rem <= 0:
                continue
            c = min(rem, self.m3.chunk_budget(0 if flush else n_sh, 0 if flush else n_dp_est, 0 if flush else pend))
            if flush and c <= 0:
                c = min(rem, self.cfg.prefill_chunk)
            if c <= 0:
                continue
            chunks.append((int(i), r.pf_sh, c))
            r.pf_sh += c
            n_sh += c
            pend += c
        return chunks

    def _deep(self, V, d, draft, probe_ctx):
        """Deep segment (inside the step's interval) and the step's LM-head launch.  Blocks: every verifier's
        d + 1 tokens (inputs exit_h[i, 0..d]) and the pending M3 chunks (inputs their layer-k states).  Head rows:
        [drafts (when merged) | verify tokens | last token of every finished prompt]; with a probe, one more head
        launch over every candidate exit's states of the verify tokens.  Returns the int64 readback
        [accepted per verifier | committed/verified tokens | first tokens | probe matches per candidate, total],
        the verify token count, verifier info and the slots whose prompt finished."""
        m, k, L, Dm1 = self.m, self.k, self.L, self.Dm1
        vs = np.flatnonzero(V)
        crow, cpos, cT, chid = [], [], [], []
        if self.m3 is not None:
            for i in range(self.B):
                for (p0, c, hk) in self.pending[i]:
                    crow.append(i)
                    cpos.append(p0)
                    cT.append(c)
                    chid.append(hk)
        nvb = len(vs)
        rows = np.concatenate([vs, np.array(crow, dtype=np.int64)])
        pos0 = np.concatenate([self.pos[vs], np.array(cpos, dtype=np.int64)])
        T = np.concatenate([d[vs] + 1, np.array(cT, dtype=np.int64)])
        pb = build_packed_arrays(m, rows, pos0, T, self.cfg.bucketing, upload_meta=False)
        self._count_kv(pb, L - k)
        if self.trace is not None:                                        # the deep segment's blocks, chunks included
            self._dp_blocks = list(zip(rows.tolist(), pos0.tolist(), T.tolist()))
        n = pb.n_tokens
        is_v = pb.order < nvb
        vb = np.flatnonzero(is_v)                                         # verify blocks in packed order
        slots_a = rows[pb.order[vb]]
        T_a = pb.blk_T[vb]
        nv = len(vb)
        vstarts_a = np.concatenate([[0], np.cumsum(T_a)[:-1]]).astype(np.int64)
        nvt = int(T_a.sum())
        blk_of = np.repeat(np.arange(nv), T_a)
        jl = np.arange(nvt) - vstarts_a[blk_of]                             # position within its verify block
        vtok = pb.offsets[vb][blk_of] + jl                                 # packed index of every verify token
        src = slots_a[blk_of] * Dm1 + jl                                   # exit_h row of every verify token
        cfin, cfin_row = [], []
        for b in np.flatnonzero(~is_v):
            ci = int(pb.order[b]) - nvb
            i = crow[ci]
            if cpos[ci] + cT[ci] >= len(self.req[i].prompt):
                cfin.append(i)
                cfin_row.append(int(pb.offsets[b]) + cT[ci] - 1)
        if self.forced is not None:
            forced = np.array([self.forced.draw(self.req[i].key) for i in slots_a.tolist()], dtype=np.int64)
        else:
            forced = np.full(nv, -1, dtype=np.int64)
        fast = len(crow) == 0
        pb.meta, src_t, vtok_t, cfin_t, cfin_dst_t, info = upload_many(
            [pb.meta_host, src.astype(np.int64), vtok.astype(np.int64), np.array(cfin_row, dtype=np.int64),
             np.array(cfin, dtype=np.int64) * Dm1,
             np.concatenate([slots_a, vstarts_a, T_a, forced, blk_of, jl]).astype(np.int32)], self.dev)
        slots_t, starts_t, T_t, forced_t = info[:nv], info[nv:2 * nv], info[2 * nv:3 * nv], info[3 * nv:4 * nv]
        blk_t, jl_t = info[4 * nv:4 * nv + nvt], info[4 * nv + nvt:4 * nv + 2 * nvt]
        sb, exh = self._flat()
        h_sh, drf_src_t, drf_dst_t, nd = draft
        x = m.buffer("x_deep", (n, m.cfg.dim), m.dtype)
        if fast:
            _lsk.copy_rows(x, None, exh, src_t, n)                        # x = exit_h[i, 0..d_i]
        else:
            if nvt:
                _lsk.copy_rows(x, vtok_t, exh, src_t, nvt)
            for b in np.flatnonzero(~is_v):
                s0, ci = int(pb.offsets[b]), int(pb.order[b]) - nvb
                _lsk.copy_rows(x[s0:s0 + cT[ci]], None, chid[ci], None, cT[ci])
        probe = probe_ctx is not None
        cands = self.exitc.cands if probe else ()
        cap_dp = {} if probe else None
        nh = nd + nvt + len(cfin)
        xh = m.buffer("x_head", (nh, m.cfg.dim), m.dtype)
        if nd:
            _lsk.copy_rows(xh, None, h_sh, drf_src_t, nd)                 # drafting slots' layer-k states
        if fast and not probe:
            packed_layers(m, x, pb, k, L, out=xh[nd:])
            hd = xh[nd:]
        else:
            hd = packed_layers(m, x, pb, k, L, cap_dp, tuple(c for c in cands if c > k))
            if nvt:
                _lsk.copy_rows(xh[nd:], None, hd, vtok_t, nvt)
            if cfin:
                _lsk.copy_rows(xh[nd + nvt:], None, hd, cfin_t, len(cfin))
        nc = len(cands)
        rb = torch.empty(nv + nvt + len(cfin) + (nc + 1 if probe else 0), dtype=torch.long, device=self.dev)
        if nh:
            ids = m.head_argmax(xh, out=m.buffer("head_ids", (nh,), torch.long))
            if nd:
                _lsk.copy_rows(sb.view(-1, 1), drf_dst_t, ids.view(-1, 1), None, nd)   # seq_buf[i, d_i + 1] = draft
            Yv = ids[nd:nd + nvt]
            if nv:
                _lsk.greedy_accept(Yv, sb, Dm1, slots_t, starts_t, T_t, forced_t, nv, rb[:nv], rb[nv:nv + nvt])
            if cfin:
                y0 = ids[nd + nvt:]
                _lsk.copy_rows(sb.view(-1, 1), cfin_dst_t, y0.view(-1, 1), None, len(cfin))  # seq_buf[i, 0] = y0
                _lsk.copy_rows(rb[nv + nvt:nv + nvt + len(cfin)].view(-1, 1), None, y0.view(-1, 1), None, len(cfin))
        if probe:
            self._probe_counts(probe_ctx, cands, slots_a, T_a, vtok_t, x, cap_dp, Yv, rb, nv, nvt, blk_t, jl_t,
                               rb[nv + nvt + len(cfin):])
        if crow:                                                          # pending chunks are consumed here
            for i in range(self.B):
                for (p0, c, _) in self.pending[i]:
                    self.req[i].pf_dp = p0 + c
                self.pending[i] = []
        return rb, nvt, (slots_a.tolist(), vstarts_a.tolist(), T_a.tolist()), cfin

    def _readback(self, rb: torch.Tensor) -> Callable[[], list]:
        """Start copying the step's device results to the host; the returned call waits for them (a list)."""
        if rb.device.type != "cuda":
            return rb.tolist
        n = rb.numel()
        host = _pinned_readback(n)
        host.copy_(rb, non_blocking=True)
        done = torch.cuda.Event()
        done.record()

        def wait() -> list:
            done.synchronize()
            return host.tolist()
        return wait

    def _probe_counts(self, probe_ctx, cands, slots_a, T_a, vtok_t, x_k, cap_dp, Yv, rb, nv, nvt, blk_t, jl_t, out):
        """Agreement of every candidate exit with Y on the correct-prefix positions (solutions/engine.py:491-514):
        the hidden state entering candidate c of each verify token (shallow capture for c < k, the deep segment's
        input for c = k, deep capture for c > k) goes through the shared head; lsk_probe_matches counts."""
        m, k = self.m, self.k
        pb_sh, kb_sh, slot_sh, cap_sh = probe_ctx
        full_start = {int(slot_sh[b]): int(pb_sh.offsets[b]) for b in np.flatnonzero(kb_sh == 1)}
        sh_idx = np.concatenate([full_start[int(i)] + np.arange(t) for i, t in zip(slots_a, T_a)])
        sh_t = upload(sh_idx, self.dev)
        nc = len(cands)
        xp = m.buffer("x_probe", (nc * nvt, m.cfg.dim), m.dtype)
        for ci, c in enumerate(cands):
            dst = xp[ci * nvt:(ci + 1) * nvt]
            if c < k:
                _lsk.copy_rows(dst, None, cap_sh[c], sh_t, nvt)
            elif c == k:
                _lsk.copy_rows(dst, None, x_k, vtok_t, nvt)
            else:
                _lsk.copy_rows(dst, None, cap_dp[c], vtok_t, nvt)
        pred = m.head_argmax(xp, out=m.buffer("probe_ids", (nc * nvt,), torch.long))
        _lsk.probe_matches(pred, Yv, rb[:nv], blk_t, jl_t, nc, nvt, out)

    def _switch_exit(self, new_k: int) -> None:
        """Move to exit layer new_k (solutions/engine.py:522-527): the drafts in flight were made with the old exit
        and are dropped (lossless); every slot drafts again from its last committed token."""
        live = self.state == DECODE
        self.stats["dropped_drafts"] += int(self.d[live].sum())
        self.d[:] = 0
        self.k = new_k
        self.sched.set_exit(new_k, self.exitc.alpha.get(new_k))

    def _count_kv(self, pb, n_layers: int) -> None:
        """KV positions attention reads in this segment (the reference's padded accounting) and the gathered
        share, over n_layers layers."""
        if self.measuring:
            self.stats["kv_read_pos"] += pb.kv_read_padded * n_layers
            self.stats["kv_gathered_pos"] += pb.kv_gathered * n_layers

    def _tally(self, committed, deep, n_deep=0, verifiers=0, plan_ms=0.0, probe=False):
        if not self.measuring:
            return
        add = {"steps": 1, "committed": committed, "plan_ms": plan_ms, "plan_calls": 1}
        if deep:
            add.update(deep_steps=1, deep_tokens=n_deep, verifiers=verifiers, probe_steps=int(probe))
        for key, v in add.items():
            self.stats[key] += v

    # ------------------------------------------------------------------ drivers
    def _busy(self) -> bool:
        return bool(((self.state == DECODE) | (self.state == PREFILL)).any())

    def _release(self, slot: int, out: list, keep: bool) -> None:
        r = self.req[slot]
        r.log_finish = len(self.records) - 1
        rec = {"pid": r.pid, "prompt_len": len(r.prompt), "generated": len(r.out), "finish_reason": r.finish,
               "measured": r.measured, "log_assign": r.log_assign, "log_first": r.log_first,
               "log_finish": r.log_finish, "piggybacked": r.piggybacked,
               "wall_ttft_s": (r.wall_first - r.wall_arrival) if r.wall_arrival else None}
        if keep:
            rec["tokens"] = list(r.out)
        out.append(rec)
        self.state[slot] = FREE
        self.req[slot] = None

    def _decode_rate(self, first: int, tokens: int) -> float:
        ms = sum(e.ms for e in self.records[first:] if e.kind != "prefill")
        return tokens / (ms / 1000) if ms > 0 else 0.0

    def _begin_measuring(self, mark: dict) -> None:
        self.measuring = True
        mark["first_entry"] = len(self.records)
        if self.dev.type == "cuda":
            torch.cuda.synchronize(self.dev)

    def run(self, prompts: list, mode: str = "cyclic", warmup_samples: int = 8, warmup_per_slot: float = 1.0,
            min_eval: int = 16, min_eval_per_slot: float = 2.0, max_eval: int = 256, converge_threshold: float = 0.01,
            converge_window: int = 4, keep_outputs: bool = False, max_steps: Optional[int] = None) -> dict:
        """A static pass over the prompts, or a cyclic replay measured after warm-up completions until the
        decode throughput converges (solutions/engine.py:544-623 rules)."""
        cyclic = mode != "static"
        warm = max(warmup_samples, int(np.ceil(warmup_per_slot * self.B))) if cyclic else 0
        least = max(min_eval, int(np.ceil(min_eval_per_slot * self.B)))
        mark = {"first_entry": 0, "tokens": 0}
        self.measuring = False
        window = MeasureWindow(warm, least, max(max_eval, least) if cyclic else None, converge_threshold,
                               converge_window, converge=cyclic, on_start=lambda: self._begin_measuring(mark))
        done: list = []
        eng = self

        class Slots:
            n_slots = self.B

            def admit(self, slot, index, prompt):
                eng.assign(slot, Request(prompt.pid, list(prompt.tokens)))
                return eng.req[slot].finish is not None

            def advance(self):
                committed, finished = eng.step()
                if eng.measuring:
                    mark["tokens"] += committed
                return finished

            def release(self, slot):
                eng._release(slot, done, keep_outputs)

            def busy(self):
                return eng._busy()

        stop = run_pool(Slots(), prompts, cyclic, window, lambda: self._decode_rate(mark["first_entry"],
                                                                                   mark["tokens"]), max_steps)
        if self.dev.type == "cuda":
            torch.cuda.synchronize(self.dev)
        wall = time.perf_counter() - window.t_start if window.t_start is not None else None
        return self._report(done, mark["first_entry"], mark["tokens"], stop, wall)

    def run_poisson(self, prompts: list, rate_per_s: float, n_requests: int, warm_requests: int = 8, seed: int = 0,
                    keep_outputs: bool = False) -> dict:
        """Open loop (solutions/engine.py:625-673 rules): Poisson arrivals at rate_per_s in wall-clock time, FIFO
        into free slots; the first warm_requests completions are warm-up, the run ends after n_requests more."""
        mark = {"first_entry": 0, "tokens": 0, "released": 0, "t_meas": time.perf_counter()}
        self.measuring = warm_requests == 0
        done: list = []
        eng = self

        class Slots:
            n_slots = self.B

            def advance(self):
                committed, finished = eng.step()
                if eng.measuring:
                    mark["tokens"] += committed
                return finished

            def release(self, slot):
                eng._release(slot, done, keep_outputs)

            def busy(self):
                return eng._busy()

        def after_release():
            mark["released"] += 1
            if not self.measuring and mark["released"] >= warm_requests:
                self._begin_measuring(mark)
                mark["t_meas"] = time.perf_counter()

        def admit(slot, req):
            self.assign(slot, req)
            return self.req[slot].finish is not None

        def make(i, t_arrival):
            p = prompts[i % len(prompts)]
            return Request(p.pid, list(p.tokens), wall_arrival=t_arrival)

        arrivals = PoissonArrivals(rate_per_s, seed, mark["t_meas"])
        left = run_arrivals(Slots(), lambda: [int(s) for s in np.flatnonzero(self.state == FREE)], make, admit,
                            arrivals, n_requests + warm_requests, after_release)
        if self.dev.type == "cuda":
            torch.cuda.synchronize(self.dev)
        res = self._report(done, mark["first_entry"], mark["tokens"], "n_requests", time.perf_counter() - mark["t_meas"])
        res["metrics"]["poisson_rate_per_s"] = rate_per_s
        res["metrics"]["queue_left"] = left
        return res

    # ------------------------------------------------------------------ results
    def _report(self, completions, first_entry, tokens, stop_reason, wall_s=None) -> dict:
        """The reference's metrics (solutions/engine.py:694-753) from the step log and the completions."""
        log = self.records
        ms = np.fromiter((e.ms for e in log), dtype=np.float64, count=len(log))
        counted = np.fromiter((e.measured for e in log), dtype=bool, count=len(log))
        is_prefill = np.fromiter((e.kind == "prefill" for e in log), dtype=bool, count=len(log))
        decode_ms = float(ms[counted & ~is_prefill].sum())
        prefill_ms = float(ms[counted & is_prefill].sum())
        gpu_ms = decode_ms + prefill_ms
        before = np.concatenate([[0.0], np.cumsum(ms)])        # before[i] = time of entries [0, i)
        decode_before = np.concatenate([[0.0], np.cumsum(np.where(is_prefill, 0.0, ms))])
        ttft, tpot = [], []
        for c in completions:
            if not c["measured"] or c["log_first"] < 0:
                continue
            ttft.append(before[c["log_first"] + 1] - before[c["log_assign"]])
            if c["generated"] > 1 and c["log_finish"] > c["log_first"]:
                tpot.append((decode_before[c["log_finish"] + 1] - decode_before[c["log_first"] + 1])
                            / (c["generated"] - 1))
        st = self.stats

        def ratio(a, b):
            return a / max(b, 1)

        def mean_p99(x):
            return (float(np.mean(x)), float(np.percentile(x, 99))) if x else (None, None)

        ttft_mean, ttft_p99 = mean_p99(ttft)
        tpot_mean, tpot_p99 = mean_p99(tpot)
        timing = {
            "measured_tokens": tokens, "decode_ms": decode_ms, "prefill_ms": prefill_ms,
            "throughput_tok_s": tokens / (decode_ms / 1000) if decode_ms else None,
            "e2e_throughput_tok_s": tokens / (gpu_ms / 1000) if gpu_ms else None,
            "wall_s": wall_s,
            "wall_throughput_tok_s": tokens / wall_s if wall_s else None,
            "host_overhead_share": (1 - gpu_ms / (1000 * wall_s)) if wall_s else None,
            "prefill_time_share": prefill_ms / gpu_ms if gpu_ms else None,
            "ttft_ms_mean": ttft_mean, "ttft_ms_p99": ttft_p99, "tpot_ms_mean": tpot_mean, "tpot_ms_p99": tpot_p99,
            "plan_ms_per_step": st["plan_ms"] / max(st["plan_calls"], 1),
        }
        prefill = {
            "prefill_tokens_separate": st["prefill_tokens"], "prefill_tokens_piggyback": st["piggyback_tokens"],
            "piggyback_share_of_prefill_tokens": ratio(st["piggyback_tokens"],
                                                       st["piggyback_tokens"] + st["prefill_tokens"]),
            "steps_with_piggyback_ms": float(sum(e.ms for e in log if e.measured and e.n_chunk and e.kind != "prefill")),
            "m3_fallbacks": st["m3_fallbacks"], "m3_fallback_reasons": dict(self.fallback_reasons),
            "separate_prefills": st["separate_prefills"],
        }
        speculation = {
            "deep_steps_per_token": ratio(st["deep_steps"], st["committed"]),
            "deep_exec_fraction": ratio(st["deep_steps"], st["steps"]),
            "tokens_per_deep_step": ratio(st["deep_tokens"], st["deep_steps"]),
            "verifiers_per_deep_step": ratio(st["verifiers"], st["deep_steps"]),
            "acceptance_rate": ratio(st["accepted"], st["drafted"]),
            "gamma_final": getattr(self.sched, "gamma", None) if self.sched is not None else None,
            "oracle_coverage": None,
        }
        exits = {
            "k_final": self.k,
            "k_timeline": list(self.exitc.timeline) if self.exitc is not None else [(0, self.k)],
            "k_alpha": dict(self.exitc.alpha) if self.exitc is not None else None,
            "probe_steps": st["probe_steps"], "dropped_drafts_at_switch": st["dropped_drafts"],
        }
        kv = {
            "kv_gather_share": ratio(st["kv_gathered_pos"], st["kv_read_pos"]),
            "kv_read_bytes": st["kv_read_pos"] * self.kv_bytes_per_pos,
            "kv_gathered_bytes": st["kv_gathered_pos"] * self.kv_bytes_per_pos,
        }
        metrics = {"config": self.cfg.label(), "B": self.B, "stop_reason": stop_reason, **timing, **prefill,
                   **speculation, **exits, **kv,
                   "evaluated_completions": sum(1 for c in completions if c["measured"]),
                   "steps": st["steps"], "deep_steps": st["deep_steps"]}
        return {"metrics": metrics, "engine_config": asdict(self.cfg), "completions": completions}
