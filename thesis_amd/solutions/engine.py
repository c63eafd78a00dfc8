"""EESD engine: batched early-exit self-speculation with packed shallow / deep steps on MI355X
(solutions/engine.py surface: EngineConfig, Request, Rec, EESDEngine.assign / step / run / run_poisson).

Step semantics are the reference's (solutions/engine.py:1-27, 269-489):
  shallow step  every decoding slot runs its current input token (last committed token if d = 0, else
                its newest draft) at position pos + d through layers [0, k) and the shared exit head
                -> one draft (seq_buf[i, d + 1]); its layer-k hidden state is kept in exit_h[i, d].
  deep step     the verifying slots (scheduler's V) run their newest draft through [0, k) in the same
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
the correct-prefix positions; ExitController may then switch the exit layer (pending drafts are dropped).
M3 (prefill="m3", solutions/engine.py:289-305, 353-354, 424-426, 477-480): chunks of an admitted prompt ride on the
shallow segment (prompt ids through [0, k), layer-k states kept) and on the next deep segment (those states through
[k, L)); the last chunk's head gives the request's first token.

Harness hook with no reference counterpart: `forced_accept_p` replaces each verifier's acceptance by
a seeded draw min(Geometric(p) - 1, d) and commits drafts[0..a-1] + Yv[a] (the tokens whose KV the deep
segment wrote), as the measured configurations prescribe.
"""

from __future__ import annotations

import math
import time
from dataclasses import asdict, dataclass, field
from typing import Callable, Optional

import numpy as np
import torch

from .. import _lsk
from ..common.timing import Interval
from .packed import Block, build_packed, build_packed_arrays, packed_layers, upload, upload_many
from .exit_select import ExitController
from .prefill import M3Planner
from .schedulers import make_scheduler
from .step_graph import ShallowGraphs

FREE, PREFILL, DECODE = 0, 1, 2


@dataclass
class EngineConfig:
    mode: str = "spec"              # spec | ar
    sched: str = "fixed"            # fixed | aspire | m1 | fsm-sync | aspire-fsm
    gamma: int = 4
    k: int = 3
    exit: str = "fixed"             # fixed | m2
    prefill: str = "separate"       # separate | m3
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
    graphs: bool = True             # replay fixed-shape shallow steps as captured HIP graphs

    def label(self) -> str:
        if self.mode == "ar":
            return "ar"
        s = f"{self.sched}" + (f"-g{self.gamma}" if self.sched == "fixed" else "")
        return f"{s}-{'k' + str(self.k) if self.exit == 'fixed' else 'm2'}-{self.prefill}"


@dataclass
class Request:
    pid: str
    prompt: list
    out: list = field(default_factory=list)
    finish: Optional[str] = None
    rec_assign: int = 0
    rec_first: int = -1
    rec_finish: int = -1
    wall_arrival: float = 0.0
    wall_first: float = 0.0
    measured: bool = False
    pf_sh: int = 0
    pf_dp: int = 0
    piggybacked: int = 0
    key: int = -1                   # assignment counter (forced-acceptance stream)


@dataclass
class Rec:
    kind: str
    iv: Interval
    measured: bool
    n_sh: int = 0
    n_dp: int = 0
    n_chunk: int = 0
    plan_ms: float = 0.0
    k: int = 0
    _ms: Optional[float] = None

    @property
    def ms(self) -> float:
        if self._ms is None:
            self._ms = self.iv.ms
        return self._ms


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


class EESDEngine:
    def __init__(self, model, B: int, max_prompt: int, max_new: int, eos_ids, cfg: EngineConfig, cost_model,
                 stop_for: Optional[Callable] = None, ref: Optional[dict] = None):
        if cfg.mode == "ar" and cfg.prefill != "separate":
            raise ValueError("AR mode supports --prefill separate only")
        if cfg.exit not in ("fixed", "m2"):
            raise ValueError(f"unknown exit policy {cfg.exit!r}")
        if cfg.prefill not in ("separate", "m3"):
            raise ValueError(f"unknown prefill policy {cfg.prefill!r}")
        self.m, self.dev, self.B, self.cfg, self.cm = model, model.device, B, cfg, cost_model
        self.max_new, self.eos = max_new, set(eos_ids)
        self.stop_for = stop_for or (lambda pid: None)
        self.k = cfg.k
        self.L = model.n_layers
        if not 1 <= self.k < self.L:
            raise ValueError("exit layer must be in [1, n_layers)")
        Dm = cfg.d_max
        self.Dm1 = Dm + 1
        model.allocate_cache(B, max_prompt + max_new + Dm + 40)
        self.seq_buf = torch.zeros(B, self.Dm1, dtype=torch.long, device=self.dev)
        self.exit_h = torch.zeros(B, self.Dm1, model.cfg.dim, dtype=model.dtype, device=self.dev)
        self.state = np.zeros(B, dtype=np.int64)
        self.pos = np.zeros(B, dtype=np.int64)
        self.d = np.zeros(B, dtype=np.int64)
        self.gen = np.zeros(B, dtype=np.int64)
        self.req: list = [None] * B
        self.pending: list = [[] for _ in range(B)]
        self.steps_since_deep = 0
        self.records: list = []
        self.sched = make_scheduler(cfg.sched, B, cost_model, self.k, gamma=cfg.gamma, d_max=Dm,
                                    sla_steps=cfg.sla_steps, initial_draft=cfg.initial_draft, omega=cfg.omega,
                                    alpha0=cfg.alpha0, min_draft=cfg.min_draft) if cfg.mode == "spec" else None
        self.exitc = ExitController(cost_model, self.k, [c for c in cfg.k_cands if 1 <= c < self.L], cfg.probe_every,
                                    cfg.switch_margin, cfg.omega, Dm, cfg.m2_force) if cfg.exit == "m2" else None
        self.m3 = M3Planner(cost_model, cfg.max_wait, cfg.m3_chunk_cap, cfg.prefill_chunk,
                            cfg.knee_safety) if cfg.prefill == "m3" else None
        self.forced = ForcedAcceptance(cfg.forced_accept_p, cfg.forced_seed) if cfg.forced_accept_p else None
        self.graphs = ShallowGraphs(self.dev) if cfg.graphs and cfg.mode == "spec" else None
        self._keys = 0
        self.measuring = False
        self.stats = {"steps": 0, "deep_steps": 0, "probe_steps": 0, "deep_tokens": 0, "verifiers": 0, "drafted": 0,
                      "accepted": 0, "committed": 0, "plan_ms": 0.0, "plan_calls": 0, "prefill_tokens": 0,
                      "piggyback_tokens": 0, "separate_prefills": 0, "m3_fallbacks": 0, "dropped_drafts": 0,
                      "kv_read_pos": 0, "kv_gathered_pos": 0}
        self.round_len = cfg.gamma
        self.kv_bytes_per_pos = 2 * model.cfg.n_kv_heads * model.cfg.head_dim * model.dtype.itemsize
        self.fallback_reasons: dict = {}
        self.trace: Optional[list] = None     # set to [] to log every step's segment shapes

    # ------------------------------------------------------------------ helpers
    def _rec(self, kind, iv, **kw) -> Rec:
        r = Rec(kind, iv, self.measuring, k=self.k, **kw)
        self.records.append(r)
        return r

    def _commit(self, slot: int, toks) -> int:
        r = self.req[slot]
        n = 0
        for t in toks:
            if r.finish is not None:
                break
            r.out.append(int(t))
            n += 1
            if int(t) in self.eos:
                r.finish = "eos"
            elif len(r.out) >= self.max_new:
                r.finish = "length"
        stop = self.stop_for(r.pid)
        if n and stop and r.finish is None:
            cut = stop(r.out, n)
            if cut is not None:
                n -= len(r.out) - cut
                del r.out[cut:]
                r.finish = "stop"
        self.gen[slot] = len(r.out)
        return n

    def _first_token(self, slot: int, y0: int) -> int:
        r = self.req[slot]
        r.rec_first = len(self.records) - 1
        r.wall_first = time.perf_counter()
        self.state[slot] = DECODE
        self.pos[slot] = len(r.prompt)
        self.d[slot] = 0
        if self.sched is not None:
            self.sched.reset(slot)
        return self._commit(slot, [y0])

    def _flat(self):
        return self.seq_buf.view(-1), self.exit_h.view(-1, self.exit_h.shape[-1])

    # ------------------------------------------------------------------ assignment / prefill
    def assign(self, slot: int, req: Request) -> int:
        req.rec_assign = len(self.records)
        req.measured = self.measuring
        if req.key < 0:
            req.key = self._keys
        self._keys += 1
        self.req[slot] = req
        self.pending[slot] = []
        self.d[slot] = 0
        if self.m3 is not None and (self.state == DECODE).any():
            dec = self.state == DECODE
            n_dec = int(dec.sum())
            ok, why = self.m3.admit(len(req.prompt), n_dec, n_dec * (self.round_len + 1), self.k,
                                    float((self.pos + self.d)[dec].sum()))
            if ok:
                self.state[slot] = PREFILL
                req.pf_sh = req.pf_dp = 0
                return 0
            self.stats["m3_fallbacks"] += 1
            self.fallback_reasons[why] = self.fallback_reasons.get(why, 0) + 1
        return self._prefill_separate(slot)

    @torch.inference_mode()
    def _prefill_separate(self, slot: int) -> int:
        m, r = self.m, self.req[slot]
        n = len(r.prompt)
        if n < 1:
            raise ValueError("empty prompt")
        iv = Interval(self.dev).start()
        h = None
        for s in range(0, n, self.cfg.prefill_chunk):
            c = min(self.cfg.prefill_chunk, n - s)
            pb = build_packed(m, [Block(slot, s, c)], self.cfg.bucketing)
            self._kv(pb, self.L)
            x = m.embed(upload(r.prompt[s:s + c], self.dev))
            h = packed_layers(m, x, pb, 0, self.L)
        sb, _ = self._flat()
        y0 = m.head_argmax(h[-1:])
        _lsk.copy_rows(sb.view(-1, 1), upload([slot * self.Dm1], self.dev), y0.view(-1, 1), None, 1)
        iv.stop()
        self._rec("prefill", iv, n_chunk=n)
        self.stats["separate_prefills"] += 1
        if self.measuring:
            self.stats["prefill_tokens"] += n
        return self._first_token(slot, int(y0.item()))

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
        self._kv(pb, self.L)
        slots = np.array([b.row for b in pb.blocks], dtype=np.int64)
        idx = upload(slots * self.Dm1, self.dev)
        sb, _ = self._flat()
        iv = Interval(self.dev).start()
        x = m.buffer("x_in", (len(slots), m.cfg.dim), m.dtype)
        _lsk.embed(m.embed_w, idx, x, sb, idx)
        h = packed_layers(m, x, pb, 0, self.L)
        y = m.head_argmax(h)
        _lsk.copy_rows(sb.view(-1, 1), idx, y.view(-1, 1), None, len(slots))
        iv.stop()
        self._rec("ar", iv, n_sh=len(slots), n_dp=len(slots))
        y_h = y.tolist()
        committed, done = 0, []
        for s, t in zip(slots.tolist(), y_h):
            self.pos[s] += 1
            committed += self._commit(s, [t])
            if self.req[s].finish:
                done.append(s)
        self._account(committed, deep=True, n_deep=len(slots), verifiers=len(slots))
        return committed, done

    def _spec_step(self):
        m, cfg, k = self.m, self.cfg, self.k
        Dm1 = self.Dm1
        t0 = time.perf_counter()
        dec = self.state == DECODE
        d = self.d.copy()
        ctx = np.where(dec, self.pos + d, 0)
        V = self.sched.decide(d, ctx, dec, self.steps_since_deep) if dec.any() else np.zeros(self.B, dtype=bool)
        V = (V | (dec & (d >= cfg.d_max))) & dec & (d >= 1)
        # M3 progress guarantee: with no decoding slot, pending prompts run both segments in this step
        flush = (not dec.any()) and bool((self.state == PREFILL).any())
        deep = bool(V.any()) or flush
        Dr = dec & ~V
        probe = deep and self.exitc is not None and self.exitc.want_probe() and bool(V.any())
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
        self._kv(pb, k)
        sb, exh = self._flat()
        iv = Interval(self.dev).start()
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
            iv.stop()
            self._rec("shallow", iv, n_sh=N, n_dp=0, n_chunk=0, plan_ms=plan_ms)
            self.d[Dr] += 1
            if self.trace is not None:
                self.trace.append({"sh": list(zip(pb.blk_rows.tolist(), pb.blk_pos0.tolist(), pb.blk_T.tolist())),
                                   "n_draft": nd, "dp": [], "committed": 0})
            self.steps_since_deep += 1
            self._account(0, deep=False, plan_ms=plan_ms)
            return 0, []
        x = m.buffer("x_in", (N, m.cfg.dim), m.dtype)
        _lsk.embed(m.embed_w, alt_t, x, sb, sel_t)                        # seq_buf ids, or prompt ids for chunks
        cap_sh = {} if probe else None
        h = packed_layers(m, x, pb, 0, k, cap_sh, tuple(c for c in self.exitc.cands if c < k) if probe else ())
        if nex:
            _lsk.copy_rows(exh, ex_dst_t, h, ex_src_t, nex)               # exit_h[i, d_i] (all j of a probe) = h
        for (i, p, c, s0) in chunk_slices:
            self.pending[i].append((p, c, h[s0:s0 + c]))                  # layer-k states wait for the deep segment
        n_verify = int((d[V] + 1).sum()) if deep else 0
        merge_heads = deep and not probe and nd + n_verify <= _lsk.GEMM_TOKEN_TILE
        if nd and not merge_heads:
            hx = m.buffer("x_draft", (nd, m.cfg.dim), m.dtype)
            _lsk.copy_rows(hx, None, h, drf_src_t, nd)
            m.head_argmax(hx, out=sb, dst_idx=drf_dst_t)                  # seq_buf[i, d_i + 1] = draft
        readback, n_v_tok, vinfo, cfin = None, 0, ([], [], []), []
        if deep:
            # the drafts are first read next step, so when the rows fit one GEMM token tile their head shares
            # the verify head's launch (one pass over the LM head weights per step); the batch-invariant GEMM
            # gives every row the same result either way
            draft = (h, drf_src_t, drf_dst_t, nd) if merge_heads else (h, None, None, 0)
            probe_ctx = (pb, kb, sb_slot, cap_sh) if probe else None
            readback, n_v_tok, vinfo, cfin = self._deep(V, d, draft, probe_ctx)
        iv.stop()
        n_chunk = sum(c[2] for c in chunks)
        self._rec("probe" if probe else ("deep" if deep else "shallow"), iv, n_sh=N, n_dp=n_v_tok, n_chunk=n_chunk,
                  plan_ms=plan_ms)
        self.d[Dr] += 1
        if self.measuring:
            self.stats["piggyback_tokens"] += n_chunk
        for (i, _, c) in chunks:
            self.req[i].piggybacked += c
        if self.trace is not None:
            vs = np.flatnonzero(V)
            self.trace.append({"sh": list(zip(pb.blk_rows.tolist(), pb.blk_pos0.tolist(), pb.blk_T.tolist())),
                               "n_draft": nd,
                               "dp": list(zip(vs.tolist(), self.pos[vs].tolist(), (d[vs] + 1).tolist())),
                               "committed": 0})
        if not deep:
            self.steps_since_deep += 1
            self._account(0, deep=False, plan_ms=plan_ms)
            return 0, []
        rb = readback.tolist()
        vslots, vstarts, vT = vinfo
        nv = len(vslots)
        acc = np.array(rb[:nv], dtype=np.int64)
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
            committed += self._first_token(i, int(rb[off + jf]))
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
                self.exitc.observe_probe(rb[off:off + nc], int(rb[off + nc]))
            self.exitc.after_deep_step()
            dec_now = self.state == DECODE
            new = self.exitc.maybe_switch(int(dec_now.sum()), float((self.pos + self.d)[dec_now].sum()),
                                          can_switch=not (self.state == PREFILL).any())
            if new is not None:
                self._switch_exit(new)
        plan_ms += 1000 * (time.perf_counter() - t2)
        self._account(committed, deep=True, n_deep=n_v_tok, verifiers=nv, plan_ms=plan_ms, probe=probe)
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
            c = min(rem, self.m3.budget(0 if flush else n_sh, 0 if flush else n_dp_est, 0 if flush else pend))
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
        self._kv(pb, L - k)
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
        return rb.cpu(), nvt, (slots_a.tolist(), vstarts_a.tolist(), T_a.tolist()), cfin

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
        """Exit switch (solutions/engine.py:522-527): drafts in flight are dropped (lossless), every slot restarts
        drafting from its last committed token with the new exit layer."""
        self.stats["dropped_drafts"] += int(self.d[self.state == DECODE].sum())
        self.d[:] = 0
        self.k = new_k
        self.sched.set_exit(new_k, self.exitc.alpha.get(new_k))

    def _kv(self, pb, n_layers: int) -> None:
        if self.measuring:
            self.stats["kv_read_pos"] += pb.kv_read_padded * n_layers
            self.stats["kv_gathered_pos"] += pb.kv_gathered * n_layers

    def _account(self, committed, deep, n_deep=0, verifiers=0, plan_ms=0.0, probe=False):
        if not self.measuring:
            return
        st = self.stats
        st["steps"] += 1
        st["committed"] += committed
        st["plan_ms"] += plan_ms
        st["plan_calls"] += 1
        if deep:
            st["deep_steps"] += 1
            st["deep_tokens"] += n_deep
            st["verifiers"] += verifiers
            st["probe_steps"] += int(probe)

    # ------------------------------------------------------------------ drivers
    def run(self, prompts: list, mode: str = "cyclic", warmup_samples: int = 8, warmup_per_slot: float = 1.0,
            min_eval: int = 16, min_eval_per_slot: float = 2.0, max_eval: int = 256, converge_threshold: float = 0.01,
            converge_window: int = 4, keep_outputs: bool = False, max_steps: Optional[int] = None) -> dict:
        """ASPIRE cyclic replay or a static pass over the prompts (solutions/engine.py:544-623)."""
        B, n_pool = self.B, len(prompts)
        warmup_n = 0 if mode == "static" else max(warmup_samples, math.ceil(warmup_per_slot * B))
        min_eval_n = max(min_eval, math.ceil(min_eval_per_slot * B))
        max_eval_n = max(max_eval, min_eval_n)
        self.measuring = warmup_n == 0
        t_wall0 = self._wall_now() if self.measuring else None
        cursor, total_done, evaluated, stable, anchor, stop_reason = 0, 0, 0, 0, None, None
        completions, rec_measure_start, tok_measured = [], 0, 0

        def make(p):
            return Request(p.pid, list(p.tokens))

        for slot in range(B):
            if mode == "static" and cursor >= n_pool:
                break
            self.assign(slot, make(prompts[cursor % n_pool]))
            cursor += 1
        pre_done = [i for i in range(B) if self.req[i] is not None and self.req[i].finish]
        steps = 0
        while True:
            if not pre_done and not ((self.state == DECODE) | (self.state == PREFILL)).any():
                stop_reason = "pool_exhausted"
                break
            if pre_done:
                committed, done = 0, pre_done
                pre_done = []
            else:
                committed, done = self.step()
                steps += 1
            if self.measuring:
                tok_measured += committed
            queue = list(done)
            while queue:
                slot = queue.pop(0)
                r = self.req[slot]
                if r is None:
                    continue
                r.rec_finish = len(self.records) - 1
                completions.append(self._completion(r, keep_outputs))
                total_done += 1
                self.state[slot] = FREE
                self.req[slot] = None
                if not self.measuring:
                    if total_done >= warmup_n:
                        self.measuring = True
                        rec_measure_start = len(self.records)
                        t_wall0 = self._wall_now()
                elif mode == "cyclic":
                    evaluated += 1
                    if evaluated >= min_eval_n:
                        thr = self._throughput(rec_measure_start, tok_measured)
                        if anchor is None:
                            anchor = thr
                        elif abs(thr - anchor) / max(anchor, 1e-9) < converge_threshold:
                            stable += 1
                        else:
                            stable, anchor = 0, thr
                        if stable >= converge_window:
                            stop_reason = "converged"
                    if stop_reason is None and evaluated >= max_eval_n:
                        stop_reason = "max_eval_samples"
                if stop_reason is None and (mode == "cyclic" or cursor < n_pool):
                    self.assign(slot, make(prompts[cursor % n_pool]))
                    cursor += 1
                    if self.req[slot].finish:
                        queue.append(slot)
            if stop_reason is not None:
                break
            if max_steps is not None and steps >= max_steps:
                stop_reason = "max_steps"
                break
        if self.dev.type == "cuda":
            torch.cuda.synchronize(self.dev)
        wall_s = time.perf_counter() - t_wall0 if t_wall0 is not None else None
        return self._result(completions, rec_measure_start, tok_measured, stop_reason, wall_s)

    def run_poisson(self, prompts: list, rate_per_s: float, n_requests: int, warm_requests: int = 8, seed: int = 0,
                    keep_outputs: bool = False) -> dict:
        """Open loop: Poisson arrivals in wall-clock time, FIFO into free slots (solutions/engine.py:625-673)."""
        rng = np.random.default_rng(seed)
        queue, completions, cursor = [], [], 0
        t0 = time.perf_counter()
        next_arr = t0 + rng.exponential(1 / rate_per_s)
        rec_measure_start, tok_measured = 0, 0
        self.measuring = warm_requests == 0
        total_done = 0
        t_meas = t0
        while total_done < n_requests + warm_requests:
            now = time.perf_counter()
            while next_arr <= now:
                p = prompts[cursor % len(prompts)]
                cursor += 1
                queue.append(Request(p.pid, list(p.tokens), wall_arrival=next_arr))
                next_arr += rng.exponential(1 / rate_per_s)
            instant = []
            for slot in np.flatnonzero(self.state == FREE):
                if not queue:
                    break
                self.assign(int(slot), queue.pop(0))
                if self.req[int(slot)].finish:
                    instant.append(int(slot))
            if not instant and not ((self.state == DECODE) | (self.state == PREFILL)).any():
                time.sleep(max(0.0, min(next_arr - time.perf_counter(), 0.01)))
                continue
            committed, done = (0, instant) if instant else self.step()
            if self.measuring:
                tok_measured += committed
            for slot in done:
                r = self.req[slot]
                r.rec_finish = len(self.records) - 1
                completions.append(self._completion(r, keep_outputs))
                total_done += 1
                self.state[slot] = FREE
                self.req[slot] = None
                if not self.measuring and total_done >= warm_requests:
                    self.measuring = True
                    rec_measure_start = len(self.records)
                    t_meas = self._wall_now()
        if self.dev.type == "cuda":
            torch.cuda.synchronize(self.dev)
        res = self._result(completions, rec_measure_start, tok_measured, "n_requests", time.perf_counter() - t_meas)
        res["metrics"]["poisson_rate_per_s"] = rate_per_s
        res["metrics"]["queue_left"] = len(queue)
        return res

    # ------------------------------------------------------------------ results
    def _throughput(self, start: int, tokens: int) -> float:
        ms = sum(r.ms for r in self.records[start:] if r.kind != "prefill")
        return tokens / (ms / 1000) if ms > 0 else 0.0

    def _completion(self, r: Request, keep: bool) -> dict:
        c = {"pid": r.pid, "prompt_len": len(r.prompt), "generated": len(r.out), "finish_reason": r.finish,
             "measured": r.measured, "rec_assign": r.rec_assign, "rec_first": r.rec_first, "rec_finish": r.rec_finish,
             "piggybacked": r.piggybacked, "wall_ttft_s": (r.wall_first - r.wall_arrival) if r.wall_arrival else None}
        if keep:
            c["tokens"] = list(r.out)
        return c

    def _wall_now(self) -> float:
        if self.dev.type == "cuda":
            torch.cuda.synchronize(self.dev)
        return time.perf_counter()

    def _result(self, completions, start, tokens, stop_reason, wall_s=None) -> dict:
        """Metrics with the reference's names and definitions (solutions/engine.py:694-753)."""
        recs = self.records
        ms = np.array([r.ms for r in recs]) if recs else np.zeros(0)
        cum = np.concatenate([[0.0], np.cumsum(ms)])
        meas = np.array([r.measured for r in recs], dtype=bool)
        kinds = np.array([r.kind for r in recs])
        decode_ms = float(ms[meas & (kinds != "prefill")].sum()) if len(ms) else 0.0
        prefill_ms = float(ms[meas & (kinds == "prefill")].sum()) if len(ms) else 0.0
        ttft, tpot = [], []
        for c in completions:
            if not c["measured"] or c["rec_first"] < 0:
                continue
            ttft.append(cum[c["rec_first"] + 1] - cum[c["rec_assign"]])
            if c["generated"] > 1 and c["rec_finish"] > c["rec_first"]:
                seg = slice(c["rec_first"] + 1, c["rec_finish"] + 1)
                tpot.append(ms[seg][kinds[seg] != "prefill"].sum() / (c["generated"] - 1))
        st = dict(self.stats)
        nsteps = max(st["steps"], 1)
        piggy_ms = float(sum(r.ms for r in recs if r.measured and r.n_chunk and r.kind != "prefill"))
        tot = decode_ms + prefill_ms
        metrics = {
            "config": self.cfg.label(), "B": self.B, "stop_reason": stop_reason,
            "measured_tokens": tokens, "decode_ms": decode_ms, "prefill_ms": prefill_ms,
            "throughput_tok_s": tokens / (decode_ms / 1000) if decode_ms else None,
            "e2e_throughput_tok_s": tokens / (tot / 1000) if tot else None,
            "wall_s": wall_s,
            "wall_throughput_tok_s": tokens / wall_s if wall_s else None,
            "host_overhead_share": (1 - tot / (1000 * wall_s)) if wall_s else None,
            "prefill_time_share": prefill_ms / tot if tot else None,
            "prefill_tokens_separate": st["prefill_tokens"], "prefill_tokens_piggyback": st["piggyback_tokens"],
            "piggyback_share_of_prefill_tokens": st["piggyback_tokens"] / max(st["piggyback_tokens"]
                                                                              + st["prefill_tokens"], 1),
            "steps_with_piggyback_ms": piggy_ms,
            "deep_steps_per_token": st["deep_steps"] / max(st["committed"], 1),
            "deep_exec_fraction": st["deep_steps"] / nsteps,
            "tokens_per_deep_step": st["deep_tokens"] / max(st["deep_steps"], 1),
            "verifiers_per_deep_step": st["verifiers"] / max(st["deep_steps"], 1),
            "acceptance_rate": st["accepted"] / max(st["drafted"], 1),
            "plan_ms_per_step": st["plan_ms"] / max(st["plan_calls"], 1),
            "ttft_ms_mean": float(np.mean(ttft)) if ttft else None,
            "ttft_ms_p99": float(np.percentile(ttft, 99)) if ttft else None,
            "tpot_ms_mean": float(np.mean(tpot)) if tpot else None,
            "tpot_ms_p99": float(np.percentile(tpot, 99)) if tpot else None,
            "k_final": self.k,
            "k_timeline": list(self.exitc.timeline) if self.exitc is not None else [(0, self.k)],
            "k_alpha": dict(self.exitc.alpha) if self.exitc is not None else None,
            "probe_steps": st["probe_steps"], "dropped_drafts_at_switch": st["dropped_drafts"],
            "m3_fallbacks": st["m3_fallbacks"], "m3_fallback_reasons": dict(self.fallback_reasons),
            "oracle_coverage": None,
            "gamma_final": getattr(self.sched, "gamma", None) if self.sched is not None else None,
            "kv_gather_share": st["kv_gathered_pos"] / max(st["kv_read_pos"], 1),
            "kv_read_bytes": st["kv_read_pos"] * self.kv_bytes_per_pos,
            "kv_gathered_bytes": st["kv_gathered_pos"] * self.kv_bytes_per_pos,
            "separate_prefills": st["separate_prefills"],
            "evaluated_completions": sum(1 for c in completions if c["measured"]),
            "steps": st["steps"], "deep_steps": st["deep_steps"],
        }
        return {"metrics": metrics, "engine_config": asdict(self.cfg), "completions": completions}
