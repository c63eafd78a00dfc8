"""The DecodeEngine contract (reference common/engine.py:102-436) over the native packed forward.

* `DecodeEngine`    a table of request slots, the token-commit rule (EOS, length, stop strings) and `run`, which
                    hands the slots to the shared pool driver (common/driver.py) and reports the reference's metric
                    names (`throughput_tok_s`, `wall_throughput_tok_s`, `mean_tpot_ms`, `evaluated_completions`,
                    `stop_reason`, per-kind step statistics, plus `extra_metrics()` of subclasses).
* `ARBatchEngine`   one token per active request per step through layers [0, L).
* `SyncSpecEngine`  synchronous LayerSkip self-speculation: every active request drafts `gamma` tokens through
                    [0, k), then the batch verifies gamma + 1 tokens through [k, L) from the exit-layer states.

Both engines step only the active requests through the padded per-call path of the model (`make_ctx` /
`forward_layers`, which packs the call into ragged blocks for the native kernels), so idle slots cost nothing.
Greedy picks use the fused LM-head argmax; temperature > 0 samples from the logits with torch ops on the device.
The host reads the device once per step (AR) or once per round (sync spec).
"""

from __future__ import annotations

import time
from dataclasses import asdict, dataclass, field
from typing import Callable, Optional

import numpy as np
import torch

from .driver import MeasureWindow, run_pool, warmup_count
from .timing import DeviceSpan


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
    max_steps: Optional[int] = None  # engine steps (a draft and a verify call count one each)
    keep_outputs: bool = False
    warmup_per_slot: float = 1.0     # warm-up completions >= this x slots (every slot turns over once)
    min_eval_per_slot: float = 2.0   # measured completions before convergence >= this x slots


def commit_tokens(output: list, tokens, *, eos: set, max_new: int, stop_checker: Optional[Callable] = None,
                  check_finished: bool = False) -> tuple:
    """Append `tokens` to `output` until the request ends; returns (tokens that count, finish reason or None).
    Ends at an EOS id (which is kept), at `max_new` tokens, or where `stop_checker(output, n_new)` returns a
    cut index (the output is truncated there and the cut tokens do not count).  The stop checker runs on
    outputs still open, or on every commit with check_finished (the DecodeEngine rule)."""
    reason, n = None, 0
    for t in tokens:
        t = int(t)
        output.append(t)
        n += 1
        if t in eos:
            reason = "eos"
        elif len(output) >= max_new:
            reason = "length"
        if reason:
            break
    if n and (reason is None or check_finished) and stop_checker is not None:
        cut = stop_checker(output, n)
        if cut is not None:
            n -= len(output) - cut
            del output[cut:]
            reason = "stop"
    return n, reason


def sample_tokens(logits: torch.Tensor, temperature: float, top_k: int, top_p: float,
                  generator: Optional[torch.Generator] = None) -> torch.Tensor:
    """logits [..., V] -> ids [...].  temperature <= 0: greedy (first index on ties).  Otherwise the logits are
    divided by the temperature; top_k > 0 keeps the values >= the k-th largest (ties kept); top_p < 1 keeps,
    in descending order, every token whose preceding probability mass is <= top_p; one multinomial draw."""
    if temperature <= 0:
        return logits.argmax(dim=-1)
    lead = logits.shape[:-1]
    vals, order = (logits.reshape(-1, logits.shape[-1]).float() / temperature).sort(dim=-1, descending=True)
    if top_k and top_k > 0:
        kth = vals[:, min(top_k, vals.shape[-1]) - 1:min(top_k, vals.shape[-1])]
        vals = vals.masked_fill(vals < kth, float("-inf"))
    if top_p < 1.0:
        p = vals.softmax(-1)
        vals = vals.masked_fill(p.cumsum(-1) - p > top_p, float("-inf"))
    pick = torch.multinomial(vals.softmax(-1), 1, generator=generator)
    return order.gather(-1, pick).view(lead)


class _EngineSlots:
    """The DecodeEngine's slots behind the pool driver's SlotOps calls."""

    def __init__(self, eng: "DecodeEngine", keep_outputs: bool):
        self.eng, self.keep = eng, keep_outputs
        self.n_slots = eng.B
        self.window: Optional[MeasureWindow] = None
        self.completions: list = []
        self.tokens = 0
        self.ms = 0.0

    def admit(self, slot: int, index: int, prompt) -> bool:
        self.eng._assign(slot, index, prompt)
        return self.eng.slots[slot].finish_reason is not None

    def busy(self) -> bool:
        return bool(self.eng._active())

    def advance(self) -> list:
        eng = self.eng
        measured = self.window.measuring
        n0 = len(eng.records)
        committed = eng._iteration(measured=measured)
        step_ms = sum(r.forward_ms for r in eng.records[n0:])
        for s in eng.slots:
            if not s.idle:
                s.decode_ms += step_ms
        if measured:
            self.tokens += committed
            self.ms += step_ms
        return [i for i, s in enumerate(eng.slots) if not s.idle and s.finish_reason is not None]

    def release(self, slot: int) -> None:
        s = self.eng.slots[slot]
        rec = {"pid": s.pid, "prompt_idx": s.prompt_idx, "prompt_len": s.prompt_len, "generated": len(s.output),
               "finish_reason": s.finish_reason, "decode_ms": s.decode_ms,
               "measured": bool(self.window.step_measured)}
        if self.keep:
            rec["tokens"] = list(s.output)
        if self.eng.probe is not None:
            self.eng.probe.on_finish(slot, s)
        self.completions.append(rec)
        s.idle = True

    def throughput(self) -> Optional[float]:
        return self.tokens / (self.ms / 1000) if self.ms > 0 else None


class DecodeEngine:
    name = "base"

    def __init__(self, model, batch_size: int, max_prompt_len: int, max_new_tokens: int, eos_ids, *,
                 ignore_eos: bool = False, spec_slack: int = 32, temperature: float = 0.0, top_k: int = 50,
                 top_p: float = 0.9, seed: int = 0):
        self.model, self.device, self.B = model, model.device, batch_size
        self.max_new, self.eos, self.ignore_eos = max_new_tokens, set(eos_ids), ignore_eos
        self.temperature, self.top_k, self.top_p = temperature, top_k, top_p
        self.gen = torch.Generator(device=self.device).manual_seed(seed) if temperature > 0 else None
        self.max_seq = max_prompt_len + max_new_tokens + spec_slack + 2
        model.allocate_cache(batch_size, self.max_seq)
        self.slots = [SlotState() for _ in range(batch_size)]
        self.records: list = []
        self.probe = None          # optional observer: on_prefill / on_step / on_finish
        self.stop_checker = None   # optional (output, n_new) -> cut index or None

    # ---------------------------------------------------------------- slots
    def _choose(self, h: torch.Tensor, logits: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Next-token ids of hidden states h [n, dim]: greedy through the fused head + argmax (no logits), or a
        sample from the logits."""
        if self.temperature <= 0 and logits is None:
            return self.model.head_argmax(h)
        if logits is None:
            logits = self.model.head(h)
        return sample_tokens(logits, self.temperature, self.top_k, self.top_p, self.gen)

    def _assign(self, slot: int, prompt_idx: int, prompt) -> None:
        tokens = list(prompt.tokens)
        if len(tokens) + self.max_new + 2 > self.model.cache.max_seq:
            raise ValueError(f"prompt of {len(tokens)} tokens does not fit max_seq={self.model.cache.max_seq}")
        logits, hidden = self.model.prefill(tokens, slot, capture_exits=self.probe is not None)
        first = int(self._choose(None, logits.unsqueeze(0))[0]) if self.temperature > 0 else int(logits.argmax())
        self.slots[slot] = s = SlotState(prompt_idx=prompt_idx, pid=prompt.pid, prompt_len=len(tokens),
                                         pos=len(tokens), last_token=first, idle=False)
        if self.probe is not None:
            self.probe.on_prefill(slot, s, hidden, logits, first)
        self._commit(slot, [first])

    def _commit(self, slot: int, tokens: list) -> int:
        """Append tokens to the slot's output under the stop rules; returns the tokens that count."""
        s = self.slots[slot]
        if s.finish_reason is not None:
            return 0
        n, s.finish_reason = commit_tokens(s.output, tokens, eos=set() if self.ignore_eos else self.eos,
                                           max_new=self.max_new,
                                           stop_checker=None if self.ignore_eos else self.stop_checker,
                                           check_finished=True)
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
        """One static pass over the prompts, or a cyclic replay whose first completions are warm-up and which
        stops on converged decode throughput or after max_eval_samples measured completions."""
        self.records = []
        cyclic = cfg.mode == "cyclic"
        warm = warmup_count(cfg.warmup_samples, cfg.warmup_per_slot, self.B) if cyclic else 0
        min_eval = max(cfg.converge_min_samples, int(np.ceil(cfg.min_eval_per_slot * self.B)))
        max_eval = (max(cfg.max_eval_samples, min_eval) if cfg.converge else cfg.max_eval_samples) if cyclic else None
        ops = _EngineSlots(self, cfg.keep_outputs)
        ops.window = window = MeasureWindow(warm, min_eval, max_eval, cfg.converge_threshold, cfg.converge_window,
                                            converge=cyclic and cfg.converge, per_step=True)
        stop = run_pool(ops, prompts, cyclic, window, ops.throughput, cfg.max_steps, drain_after_stop=False)
        wall = (_now() - window.t_start) if window.t_start is not None else 0.0
        measured = [r for r in self.records if r.measured]
        by_kind = {}
        for kind in sorted({r.kind for r in measured}):
            ms = np.array([r.forward_ms for r in measured if r.kind == kind])
            by_kind[kind] = {"steps": int(ms.size), "mean_ms": float(ms.mean()), "p50_ms": float(np.median(ms))}
        done = [c for c in ops.completions if c["measured"]]
        tpot = [c["decode_ms"] / max(c["generated"] - 1, 1) for c in done]
        metrics = {
            "stop_reason": stop,
            "warmup_samples_effective": warm,
            "min_eval_samples_effective": min_eval,
            "total_completions": len(ops.completions),
            "evaluated_completions": window.evaluated if cyclic else len(ops.completions),
            "measured_tokens": ops.tokens,
            "measured_forward_s": ops.ms / 1000,
            "measured_wall_s": wall,
            "throughput_tok_s": ops.tokens / (ops.ms / 1000) if ops.ms else None,
            "wall_throughput_tok_s": ops.tokens / wall if wall else None,
            "mean_tpot_ms": float(np.mean(tpot)) if tpot else None,
            "steps": by_kind,
            **self.extra_metrics(),
        }
        return {"metrics": metrics, "completions": ops.completions, "steps": [asdict(r) for r in self.records]}


def _now() -> float:
    return time.perf_counter()


class ARBatchEngine(DecodeEngine):
    name = "autoregressive"

    def _iteration(self, measured: bool) -> int:
        m = self.model
        live = self._active()
        pos = [self.slots[i].pos for i in live]
        ids = torch.tensor([[self.slots[i].last_token] for i in live], dtype=torch.long)
        capture = [] if self.probe is not None else None
        span = DeviceSpan(self.device).open()
        ctx = m.make_ctx(torch.tensor(pos, dtype=torch.long)[:, None], 0, max(pos), rows=torch.tensor(live))
        h = m.forward_layers(m.embed(ids), 0, m.n_layers, ctx, capture=capture)[:, -1]
        logits = m.head(h) if self.probe is not None else None
        nxt = self._choose(h, logits).tolist()
        span.close()
        self.records.append(StepRecord("ar", span.ms, len(live), len(live), len(live), ctx.kv_read, measured))
        if self.probe is not None:
            self.probe.on_step(self, [c[:, -1] for c in capture], logits, nxt)
        committed = 0
        for i, t in zip(live, nxt):
            s = self.slots[i]
            s.pos, s.last_token = s.pos + 1, t
            committed += self._commit(i, [t])
        return committed


@dataclass
class _RoundStats:
    """Acceptance bookkeeping of synchronous rounds (rounds that end a request are left out: EOS / length
    truncate them)."""
    gamma: int
    rounds: int = 0
    request_rounds: int = 0
    drafted: int = 0
    accepted: int = 0
    rejected: int = 0
    overdraft_steps: int = 0
    full_accept_rounds: int = 0
    hist: np.ndarray = None

    def __post_init__(self):
        self.hist = np.zeros(self.gamma + 1, dtype=np.int64)

    def add(self, a: int) -> None:
        g = self.gamma
        self.request_rounds += 1
        self.drafted += g
        self.accepted += a
        self.rejected += g - a
        self.overdraft_steps += max(g - a - 1, 0)
        self.full_accept_rounds += int(a == g)
        self.hist[a] += 1

    def summary(self, exit_layer: int) -> dict:
        rr, dr = max(self.request_rounds, 1), max(self.drafted, 1)
        out = {k: getattr(self, k) for k in ("rounds", "request_rounds", "drafted", "accepted", "rejected",
                                             "overdraft_steps", "full_accept_rounds")}
        out.update(exit_layer=exit_layer, gamma=self.gamma, acceptance_rate=self.accepted / dr,
                   rejected_draft_ratio=self.rejected / dr, overdraft_step_ratio=self.overdraft_steps / dr,
                   full_accept_round_ratio=self.full_accept_rounds / rr,
                   tokens_per_verify=(self.accepted + self.request_rounds) / rr, accept_hist=self.hist.tolist())
        return out


class SyncSpecEngine(DecodeEngine):
    """Every active request drafts `gamma` tokens through layers [0, k), then the batch verifies them."""

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
        self.round_stats = _RoundStats(gamma)

    @property
    def stats(self) -> dict:
        return self.round_stats.summary(self.k)

    def _draft(self, rows, rows_d, pos, top, ids, spans) -> tuple:
        """gamma shallow steps from the last committed tokens; keeps each step's exit-layer state.  Returns the
        drafts [n, gamma] and the embedded newest draft (the verify step's shallow input)."""
        m, n, g = self.model, len(ids), self.gamma
        drafts = torch.empty(n, g, dtype=torch.long, device=self.device)
        x = m.embed(ids)
        for j in range(g):
            span = DeviceSpan(self.device).open()
            ctx = m.make_ctx(pos + j, 0, top + j, rows=rows)
            h = m.forward_layers(x, 0, self.k, ctx)[:, 0]
            self.exit_h[rows_d, j] = h
            d = m.head_argmax(h)
            span.close()
            drafts[:, j] = d
            x = m.embed(d.view(n, 1))
            spans.append(("draft", span, n, n, 0, ctx.kv_read))
        return drafts, x

    def _iteration(self, measured: bool) -> int:
        m, g = self.model, self.gamma
        live = self._active()
        n = len(live)
        rows = torch.tensor(live, dtype=torch.long)
        rows_d = rows.to(self.device)
        base = [self.slots[i].pos for i in live]
        pos = torch.tensor(base, dtype=torch.long)[:, None]
        top = max(base)
        spans: list = []
        drafts, x_last = self._draft(rows, rows_d, pos, top,
                                     torch.tensor([[self.slots[i].last_token] for i in live]), spans)
        span = DeviceSpan(self.device).open()
        h_last = m.forward_layers(x_last, 0, self.k, m.make_ctx(pos + g, 0, top + g, rows=rows))
        deep_in = torch.cat([self.exit_h[rows_d, :g], h_last], dim=1) if g else h_last
        ctx = m.make_ctx(pos + torch.arange(g + 1)[None, :], 0, top + g, rows=rows)
        Y = m.head_argmax(m.forward_layers(deep_in.contiguous(), self.k, m.n_layers, ctx).reshape(n * (g + 1), -1))
        Y = Y.view(n, g + 1)
        # accepted = length of the leading run of drafts equal to the full model's tokens
        acc = (drafts == Y[:, :g]).int().cumprod(dim=1).sum(dim=1) if g else torch.zeros(n, dtype=torch.long)
        span.close()
        spans.append(("verify", span, n, n, n * (g + 1), ctx.kv_read))
        acc_h, Y_h, D_h = acc.tolist(), Y.tolist(), drafts.tolist()
        for kind, sp, b, sh, dp, kv in spans:
            self.records.append(StepRecord(kind, sp.ms, b, sh, dp, kv, measured))
        self.round_stats.rounds += 1
        committed = 0
        for j, i in enumerate(live):
            s, a = self.slots[i], acc_h[j]
            s.pos, s.last_token = base[j] + a + 1, Y_h[j][a]
            committed += self._commit(i, D_h[j][:a] + [Y_h[j][a]])
            if measured and s.finish_reason is None:
                self.round_stats.add(a)
        return committed

    def extra_metrics(self) -> dict:
        return {"spec": self.stats}


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
