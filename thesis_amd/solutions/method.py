"""The "eesd" method of the registry: EESDEngine behind the DecodeEngine contract.

EESDEngine.run returns its own metric names (solutions/engine.py:680-753); through this adapter the
shared driver (`DecodeEngine.run`) measures it the same way as the built-in methods: one driver
iteration is one EESD step (a packed shallow segment, plus a deep verify segment when the scheduler
verifies), and the `spec` metrics carry `acceptance_rate` and `tokens_per_verify`.
"""

from __future__ import annotations

import numpy as np
import torch

from ..common.engine import DecodeEngine, SlotState, StepRecord
from ..common.methods import MethodSpec, register
from .cost_model import default_cost_model, load_cost_model
from .engine import FREE, EESDEngine, EngineConfig, Request


class EESDDecodeEngine(DecodeEngine):
    name = "eesd"

    def __init__(self, model, batch_size: int, max_prompt_len: int, max_new_tokens: int, eos_ids,
                 cfg: EngineConfig, cost_model, *, ignore_eos: bool = False, **_):
        self.model = model
        self.device = model.device
        self.B = batch_size
        self.max_new = max_new_tokens
        self.ignore_eos = ignore_eos
        self.eos = set() if ignore_eos else set(eos_ids)
        self.temperature, self.top_k, self.top_p, self.gen = 0.0, 0, 1.0, None
        self.probe = None
        self.stop_checker = None
        self.eng = EESDEngine(model, batch_size, max_prompt_len, max_new_tokens, tuple(self.eos), cfg, cost_model,
                              stop_for=lambda pid: None if self.ignore_eos else self.stop_checker)
        self.max_seq = model.cache.max_seq
        self.slots = [SlotState() for _ in range(batch_size)]
        self.records: list = []

    def _sync_slot(self, slot: int) -> None:
        r, s = self.eng.req[slot], self.slots[slot]
        s.output = r.out
        s.finish_reason = r.finish
        s.pos = int(self.eng.pos[slot])

    def _assign(self, slot: int, prompt_idx: int, prompt) -> None:
        if self.eng.req[slot] is not None:
            self.eng.state[slot] = FREE
            self.eng.req[slot] = None
        s = self.slots[slot]
        s.prompt_idx, s.pid, s.prompt_len = prompt_idx, prompt.pid, len(prompt.tokens)
        s.idle, s.decode_ms = False, 0.0
        self.eng.assign(slot, Request(prompt.pid, list(prompt.tokens)))
        self._sync_slot(slot)
        if s.finish_reason is not None:          # finished by its first token: never stepped
            self.eng.state[slot] = FREE

    def _iteration(self, measured: bool) -> int:
        eng = self.eng
        eng.measuring = measured
        first = len(eng.records)
        committed, done = eng.step()
        for r in eng.records[first:]:
            kind = {"shallow": "draft", "deep": "verify"}.get(r.kind, r.kind)
            self.records.append(StepRecord(kind, r.ms, r.n_sh, r.n_sh, r.n_dp, 0, measured))
        for i in self._active():
            self._sync_slot(i)
        for i in done:
            eng.state[i] = FREE
        return committed

    def extra_metrics(self) -> dict:
        st = self.eng.stats
        nv = max(st["verifiers"], 1)
        return {"spec": {"exit_layer": self.eng.k, "acceptance_rate": st["accepted"] / max(st["drafted"], 1),
                         "tokens_per_verify": (st["accepted"] + st["verifiers"]) / nv,
                         "deep_steps": st["deep_steps"], "steps": st["steps"],
                         "tokens_per_deep_step": st["deep_tokens"] / max(st["deep_steps"], 1),
                         "verifiers_per_deep_step": st["verifiers"] / max(st["deep_steps"], 1)},
                "eesd": {"config": self.eng.cfg.label()}}


def _args(g) -> None:
    g.add_argument("--sched", default="aspire", choices=["fixed", "aspire", "m1", "fsm-sync", "aspire-fsm"])
    g.add_argument("--k", type=int, default=None, help="[eesd] exit layer (default: the --exit-layer value)")
    g.add_argument("--d-max", type=int, default=16)
    g.add_argument("--min-draft", type=int, default=1)
    g.add_argument("--eesd-gamma", type=int, default=4, help="[eesd] draft length of the fixed scheduler")
    g.add_argument("--cost-model", default=None, help="[eesd] JSON of a calibrated cost model")
    g.add_argument("--forced-accept-p", type=float, default=None)


def _config(args) -> EngineConfig:
    k = args.k if getattr(args, "k", None) is not None else getattr(args, "exit_layer", None)
    if k is None:
        raise SystemExit("eesd needs --k (or --exit-layer)")
    return EngineConfig(sched=args.sched, k=k, gamma=args.eesd_gamma, d_max=args.d_max, min_draft=args.min_draft,
                        forced_accept_p=args.forced_accept_p, forced_seed=getattr(args, "seed", 0))


def _build(model, args, batch_size, max_prompt_len, eos):
    cfg = _config(args)
    cm = load_cost_model(args.cost_model, model.cfg) if args.cost_model else default_cost_model(model.cfg)[0]
    return EESDDecodeEngine(model, batch_size, max_prompt_len, args.max_new_tokens, eos, cfg, cm,
                            ignore_eos=args.ignore_eos)


register(MethodSpec("eesd", "merged shallow/deep packed engine (KV pointer rollback, batch-level deep scheduling)",
                    _args, _build, tag=lambda a: f"-{_config(a).label()}", spec_slack=64,
                    step_tokens=lambda a: a.d_max + 1,
                    params=lambda a: {"sched": a.sched, "k": _config(a).k, "d_max": a.d_max}))
