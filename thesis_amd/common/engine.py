"""DecodeEngine contract (common/engine.py:102-436) over the native packed forward.

* `DecodeEngine`    slot bookkeeping + the cyclic-replay / static driver (`run`) and its metrics
                    (`throughput_tok_s`, `wall_throughput_tok_s`, `mean_tpot_ms`, `evaluated_completions`,
                    `stop_reason`, per-kind step stats; the `spec` dict of speculative engines).
* `ARBatchEngine`   one token per active request per step, layers [0, L) (common/engine.py:302-333).
* `SyncSpecEngine`  synchronous LayerSkip self-speculation: every active request drafts `gamma` tokens
                    through layers [0, k), then the batch verifies gamma + 1 tokens through [k, L) from the
                    cached exit-layer hidden states (common/engine.py:336-436).

Both step through the padded per-call path of the model (`make_ctx` / `forward_layers`, which packs
the call into ragged blocks for the native kernels) and only the requests that are active: idle slots
cost nothing.  Greedy picks use the fused LM-head argmax; sampling (temperature > 0) draws from the
logits with torch ops on the device (`sample_tokens`).  One host readback per step (AR) or per
round (sync spec), as in the reference.
"""

from __future__ import annotations

import math
import time
from dataclasses import asdict, dataclass, field
from typing import Optional

import numpy as np
import torch

from .timing import Interval


@dataclass
class StepRecord:
    kind: str               # "ar" | "draft" | "verify"
    forward_ms: float
    batch: int              # requests in the call
    shallow_tokens: int     # tokens through layers [0, k)
    deep_tokens: int        # tokens through layers [k, L)
    kv_read: int            # KV positions read per layer (padded, as the reference counts them)
    measured: bool


@dataclass
class SlotState:
    prompt_idx: int = -1
    pid: str = ""
    prompt_len: int = 0
    pos: int = 0            # position of `last_token` (its KV is not written yet)
    last_token: int = 0
    output: list = field(default_factory=list)
    finish_reason: Optional[str] = None
    idle: bool = True
    t_assigned: float = 0.0
    decode_ms: float = 0.0


@dataclass
class RunConfig:
    mode: str = "cyclic"             # cyclic | static
    warmup_samples: int = 8
    max_eval_samples: int = 256
    converge: bool = True
    converge_threshold: float = 0.01
    converge_window: int = 4
    converge_min_samples: int = 16
    max_steps: Optional[int] = None
    keep_outputs: bool = False
    warmup_per_slot: float = 1.0
    min_eval_per_slot: float = 2.0


def sample_tokens(logits: torch.Tensor, temperature: float, top_k: int, top_p: float,
                  generator: Optional[torch.Generator] = None) -> torch.Tensor:
    """logits [..., V] -> ids [...]; temperature <= 0 is greedy (first index on ties).  Otherwise
    temperature scaling, top-k, then nucleus (top-p) truncation, then one multinomial draw."""
    if temperature <= 0:
        return logits.argmax(dim=-1)
    shape = logits.shape[:-1]
    x = logits.reshape(-1, logits.shape[-1]).float() / temperature
    if top_k and top_k > 0:
        kth = torch.topk(x, min(top_k, x.shape[-1]), dim=-1).values[:, -1:]
        x = torch.where(x < kth, torch.full_like(x, float("-inf")), x)
    if top_p < 1.0:
        sx, order = torch.sort(x, dim=-1, descending=True)
        p = sx.softmax(-1)
        drop = (p.cumsum(-1) - p) > top_p          # keep the smallest prefix whose mass reaches top_p
        sx = sx.masked_fill(drop, float("-inf"))
        x = torch.empty_like(x).scatter_(-1, order, sx)
    return torch.multinomial(x.softmax(-1), 1, generator=generator).view(shape)


class DecodeEngine:
    name = "base"

    def __init__(self, model, batch_size: int, max_prompt_len: int, max_new_tokens: int, eos_ids, *,
                 ignore_eos: bool = False, spec_slack: int = 32, temperature: float = 0.0, top_k: int = 50,
                 top_p: float = 0.9, seed: int = 0):
        self.model = model
        self.device = model.device
        self.B = batch_size
        self.max_new = max_new_tokens
        self.eos = set(eos_ids)
        self.ignore_eos = ignore_eos
        self.temperature, self.top_k, self.top_p = temperature, top_k, top_p
        self.gen = torch.Generator(device=self.device).manual_seed(seed) if temperature > 0 else None
        self.max_seq = max_prompt_len + max_new_tokens + spec_slack + 2
        model.allocate_cache(batch_size, self.max_seq)
        self.slots = [SlotState() for _ in range(batch_size)]
        self.records: list = []
        self.probe = None          # optional observer: on_prefill / on_step / on_finish
        self.stop_checker = None   # optional (output, n_new) -> cut index or None

    # ---------------------------------------------------------------- slots
    def _pick(self, h: torch.Tensor) -> torch.Tensor:
        """Next-token ids for hidden states h [n, dim] (greedy: fused head + argmax, no logits)."""
        if self.temperature <= 0:
            return self.model.head_argmax(h)
        return sample_tokens(self.model.head(h), self.temperature, self.top_k, self.top_p, self.gen)

    def _assign(self, slot: int, prompt_idx: int, prompt) -> None:
        s = self.slots[slot]
        tokens = list(prompt.tokens)
        if len(tokens) + self.max_new + 2 > self.model.cache.max_seq:
            raise ValueError(f"prompt of {len(tokens)} tokens does not fit max_seq={self.model.cache.max_seq}")
        logits, hidden = self.model.prefill(tokens, slot, capture_exits=self.probe is not None)
        if self.temperature <= 0:
            first = int(logits.argmax())
        else:
            first = int(sample_tokens(logits.unsqueeze(0), self.temperature, self.top_k, self.top_p, self.gen)[0])
        s.prompt_idx, s.pid, s.prompt_len = prompt_idx, prompt.pid, len(tokens)
        s.pos, s.last_token = len(tokens), first
        s.output, s.finish_reason, s.idle = [], None, False
        s.t_assigned, s.decode_ms = time.perf_counter(), 0.0
        if self.probe is not None:
            self.probe.on_prefill(slot, s, hidden, logits, first)
        self._commit(slot, [first])

    def _commit(self, slot: int, tokens: list) -> int:
        """Append tokens, stop at EOS / max_new / a stop string; returns the tokens that count."""
        s = self.slots[slot]
        n = 0
        for t in tokens:
            if s.finish_reason is not None:
                break
            s.output.append(int(t))
            n += 1
            if not self.ignore_eos and int(t) in self.eos:
                s.finish_reason = "eos"
            elif len(s.output) >= self.max_new:
                s.finish_reason = "length"
        if n and self.stop_checker and not self.ignore_eos:
            cut = self.stop_checker(s.output, n)
            if cut is not None:
                n -= len(s.output) - cut
                del s.output[cut:]
                s.finish_reason = "stop"
        return n

    def _active(self) -> list:
        return [i for i, s in enumerate(self.slots) if not s.idle]

    def _iteration(self, measured: bool) -> int:
        raise NotImplementedError

    def extra_metrics(self) -> dict:
        return {}

    # ---------------------------------------------------------------- driver
    @torch.inference_mode()
    def run(self, prompts: list, cfg: RunConfig) -> dict:
        """Cyclic replay (finished slots refilled from the pool; the first completions are warm-up;
        stop on converged decode throughput or max_eval_samples) or one static pass."""
        self.records = []
        n_pool = len(prompts)
        warmup_n = max(cfg.warmup_samples, math.ceil(cfg.warmup_per_slot * self.B)) if cfg.warmup_samples else 0
        min_eval_n = max(cfg.converge_min_samples, math.ceil(cfg.min_eval_per_slot * self.B))
        max_eval_n = max(cfg.max_eval_samples, min_eval_n) if cfg.converge else cfg.max_eval_samples
        warm = cfg.mode == "static" or warmup_n == 0
        cursor, total_completed, evaluated = 0, 0, 0
        anchor, stable, stop_reason = None, 0, None
        measured_tokens, measured_ms = 0, 0.0
        completions: list = []
        wall_t0 = time.perf_counter() if warm else None

        for slot in range(self.B):
            if cfg.mode == "static" and cursor >= n_pool:
                break
            self._assign(slot, cursor % n_pool, prompts[cursor % n_pool])
            cursor += 1

        steps = 0
        while True:
            if not self._active():
                stop_reason = "pool_exhausted"
                break
            first_rec = len(self.records)
            committed = self._iteration(measured=warm)
            new = self.records[first_rec:]
            step_ms = sum(r.forward_ms for r in new)
            steps += len(new)
            for i in self._active():
                self.slots[i].decode_ms += step_ms
            if warm:
                measured_tokens += committed
                measured_ms += step_ms
            was_warm = warm
            for slot, s in enumerate(self.slots):
                if s.idle or s.finish_reason is None or stop_reason is not None:
                    continue
                comp = {"pid": s.pid, "prompt_idx": s.prompt_idx, "prompt_len": s.prompt_len,
                        "generated": len(s.output), "finish_reason": s.finish_reason, "decode_ms": s.decode_ms,
                        "measured": was_warm}
                if cfg.keep_outputs:
                    comp["tokens"] = list(s.output)
                if self.probe is not None:
                    self.probe.on_finish(slot, s)
                completions.append(comp)
                total_completed += 1
                s.idle = True
                if not was_warm:
                    if not warm and total_completed >= warmup_n:
                        warm = True
                        wall_t0 = time.perf_counter()
                elif cfg.mode == "cyclic":
                    evaluated += 1
                    if cfg.converge and evaluated >= min_eval_n and measured_ms > 0:
                        thr = measured_tokens / (measured_ms / 1000)
                        if anchor is None:
                            anchor = thr
                        elif abs(thr - anchor) / anchor < cfg.converge_threshold:
                            stable += 1
                        else:
                            stable, anchor = 0, thr
                        if stable >= cfg.converge_window:
                            stop_reason = "converged"
                    if stop_reason is None and evaluated >= max_eval_n:
                        stop_reason = "max_eval_samples"
                if cfg.mode == "cyclic" or cursor < n_pool:
                    self._assign(slot, cursor % n_pool, prompts[cursor % n_pool])
                    cursor += 1
            if stop_reason is not None:
                break
            if cfg.max_steps is not None and steps >= cfg.max_steps:
                stop_reason = "max_steps"
                break
        wall = time.perf_counter() - wall_t0 if wall_t0 is not None else 0.0

        rec = [r for r in self.records if r.measured]
        per_kind = {}
        for kind in sorted({r.kind for r in rec}):
            ms = [r.forward_ms for r in rec if r.kind == kind]
            per_kind[kind] = {"steps": len(ms), "mean_ms": float(np.mean(ms)), "p50_ms": float(np.median(ms))}
        meas = [c for c in completions if c["measured"]]
        tpot = [c["decode_ms"] / max(c["generated"] - 1, 1) for c in meas]
        metrics = {
            "stop_reason": stop_reason,
            "warmup_samples_effective": warmup_n,
            "min_eval_samples_effective": min_eval_n,
            "total_completions": total_completed,
            "evaluated_completions": evaluated if cfg.mode == "cyclic" else total_completed,
            "measured_tokens": measured_tokens,
            "measured_forward_s": measured_ms / 1000,
            "measured_wall_s": wall,
            "throughput_tok_s": measured_tokens / (measured_ms / 1000) if measured_ms else None,
            "wall_throughput_tok_s": measured_tokens / wall if wall else None,
            "mean_tpot_ms": float(np.mean(tpot)) if tpot else None,
            "steps": per_kind,
            **self.extra_metrics(),
        }
        return {"metrics": metrics, "completions": completions, "steps": [asdict(r) for r in self.records]}


class ARBatchEngine(DecodeEngine):
    name = "autoregressive"

    def _iteration(self, measured: bool) -> int:
        m, dev = self.model, self.device
        act = self._active()
        toks = torch.tensor([[self.slots[i].last_token] for i in act], dtype=torch.long)
        pos_h = [self.slots[i].pos for i in act]
        pos = torch.tensor(pos_h, dtype=torch.long).unsqueeze(1)
        rows = torch.tensor(act, dtype=torch.long)
        cap = [] if self.probe is not None else None
        t = Interval(dev).start()
        ctx = m.make_ctx(pos, 0, max(pos_h), rows=rows)
        h = m.forward_layers(m.embed(toks), 0, m.n_layers, ctx, capture=cap)
        if self.probe is not None:
            logits = m.head(h[:, -1])
            nxt = sample_tokens(logits, self.temperature, self.top_k, self.top_p, self.gen)
        else:
            logits = None
            nxt = self._pick(h[:, -1])
        t.stop()
        nxt_h = nxt.tolist()
        n = len(act)
        self.records.append(StepRecord("ar", t.ms, n, n, n, ctx.kv_read, measured))
        if self.probe is not None:
            self.probe.on_step(self, [c[:, -1] for c in cap], logits, nxt_h)
        committed = 0
        for j, i in enumerate(act):
            s = self.slots[i]
            s.pos += 1
            s.last_token = nxt_h[j]
            committed += self._commit(i, [nxt_h[j]])
        return committed


class SyncSpecEngine(DecodeEngine):
    """Every active request drafts `gamma` tokens through layers [0, k), then the batch verifies."""

    name = "sync_layerskip"

    def __init__(self, model, batch_size: int, max_prompt_len: int, max_new_tokens: int, eos_ids, *,
                 exit_layer: int, gamma: int, **kw):
        if kw.get("temperature", 0.0) > 0:
            raise NotImplementedError("SyncSpecEngine implements greedy verification only")
        if not 1 <= exit_layer < model.n_layers:
            raise ValueError(f"exit_layer must be in [1, {model.n_layers - 1}]")
        super().__init__(model, batch_size, max_prompt_len, max_new_tokens, eos_ids, spec_slack=gamma + 32, **kw)
        self.k, self.gamma = exit_layer, gamma
        self.exit_h = torch.zeros(batch_size, max(gamma, 1), model.cfg.dim, dtype=model.dtype, device=self.device)
        self.stats = {"rounds": 0, "request_rounds": 0, "drafted": 0, "accepted": 0, "rejected": 0,
                      "overdraft_steps": 0, "full_accept_rounds": 0}
        self.accept_hist = np.zeros(gamma + 1, dtype=np.int64)

    def _iteration(self, measured: bool) -> int:
        m, dev, k, g = self.model, self.device, self.k, self.gamma
        act = self._active()
        n = len(act)
        rows = torch.tensor(act, dtype=torch.long)
        P_h = [self.slots[i].pos for i in act]
        P = torch.tensor(P_h, dtype=torch.long).unsqueeze(1)
        maxP = max(P_h)
        inp = m.embed(torch.tensor([[self.slots[i].last_token] for i in act], dtype=torch.long))
        rows_d = rows.to(dev)
        drafts = torch.empty(n, g, dtype=torch.long, device=dev)
        timers = []
        for j in range(g):                                   # draft: layers [0, k), one token per request
            t = Interval(dev).start()
            ctx = m.make_ctx(P + j, 0, maxP + j, rows=rows)
            h = m.forward_layers(inp, 0, k, ctx)
            self.exit_h[rows_d, j] = h[:, 0]
            d = m.head_argmax(h[:, 0])
            t.stop()
            drafts[:, j] = d
            inp = m.embed(d.view(n, 1))
            timers.append(("draft", t, n, n, 0, ctx.kv_read))
        t = Interval(dev).start()                            # verify: last draft shallow, gamma + 1 deep
        ctx_s = m.make_ctx(P + g, 0, maxP + g, rows=rows)
        h_last = m.forward_layers(inp, 0, k, ctx_s)
        deep_in = torch.cat([self.exit_h[rows_d, :g], h_last], dim=1) if g > 0 else h_last
        pos_d = P + torch.arange(g + 1).unsqueeze(0)
        ctx_d = m.make_ctx(pos_d, 0, maxP + g, rows=rows)
        hd = m.forward_layers(deep_in.contiguous(), k, m.n_layers, ctx_d)
        Y = m.head_argmax(hd.reshape(n * (g + 1), -1)).view(n, g + 1)
        if g > 0:
            acc = (drafts == Y[:, :g]).int().cumprod(dim=1).sum(dim=1)
        else:
            acc = torch.zeros(n, dtype=torch.long, device=dev)
        t.stop()
        timers.append(("verify", t, n, n, n * (g + 1), ctx_d.kv_read))
        acc_h, Y_h, D_h = acc.tolist(), Y.tolist(), drafts.tolist()
        for kind, tm, b, st, dt, kv in timers:
            self.records.append(StepRecord(kind, tm.ms, b, st, dt, kv, measured))
        committed = 0
        self.stats["rounds"] += 1
        for j, i in enumerate(act):
            s = self.slots[i]
            a = acc_h[j]
            s.pos = P_h[j] + a + 1
            s.last_token = Y_h[j][a]
            committed += self._commit(i, D_h[j][:a] + [Y_h[j][a]])
            if measured and s.finish_reason is None:
                st = self.stats
                st["request_rounds"] += 1
                st["drafted"] += g
                st["accepted"] += a
                st["rejected"] += g - a
                st["overdraft_steps"] += max(g - a - 1, 0)
                st["full_accept_rounds"] += int(a == g)
                self.accept_hist[a] += 1
        return committed

    def extra_metrics(self) -> dict:
        st = dict(self.stats)
        rr = max(st["request_rounds"], 1)
        st.update(exit_layer=self.k, gamma=self.gamma,
                  acceptance_rate=st["accepted"] / max(st["drafted"], 1),
                  rejected_draft_ratio=st["rejected"] / max(st["drafted"], 1),
                  overdraft_step_ratio=st["overdraft_steps"] / max(st["drafted"], 1),
                  full_accept_round_ratio=st["full_accept_rounds"] / rr,
                  tokens_per_verify=(st["accepted"] + st["request_rounds"]) / rr,
                  accept_hist=self.accept_hist.tolist())
        return {"spec": st}


def add_run_args(parser) -> None:
    g = parser.add_argument_group("run (cyclic replay)")
    g.add_argument("--mode", default="cyclic", choices=["cyclic", "static"])
    g.add_argument("--warmup-samples", type=int, default=8)
    g.add_argument("--max-eval-samples", type=int, default=256)
    g.add_argument("--no-converge", action="store_true")
    g.add_argument("--converge-threshold", type=float, default=0.01)
    g.add_argument("--converge-window", type=int, default=4)
    g.add_argument("--converge-min-samples", type=int, default=16)
    g.add_argument("--max-steps", type=int, default=None)
    g.add_argument("--warmup-per-slot", type=float, default=1.0)
    g.add_argument("--min-eval-per-slot", type=float, default=2.0)
    g.add_argument("--max-new-tokens", type=int, default=512)
    g.add_argument("--ignore-eos", action="store_true")


def run_config_from_args(args, keep_outputs: bool = False) -> RunConfig:
    return RunConfig(mode=args.mode, warmup_samples=args.warmup_samples, max_eval_samples=args.max_eval_samples,
                     converge=not args.no_converge, converge_threshold=args.converge_threshold,
                     converge_window=args.converge_window, converge_min_samples=args.converge_min_samples,
                     max_steps=args.max_steps, keep_outputs=keep_outputs, warmup_per_slot=args.warmup_per_slot,
                     min_eval_per_slot=args.min_eval_per_slot)
