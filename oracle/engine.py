"""CPU oracle of the EESD step glue (TEST INFRASTRUCTURE ONLY; see oracle/__init__.py).

Restates, on the oracle model of oracle/model.py:
  _prefill_separate   solutions/engine.py:217-234   chunks of 512 through [0, L) + head, first token
  _ar_step            solutions/engine.py:244-267   T = 1 per decoding slot through [0, L)
  _spec_step / _deep  solutions/engine.py:269-489   (fixed scheduler, fixed exit layer, separate prefill)
                      shallow: T = 1 at pos + d through [0, k); exit_h[i, d] = h; drafters write
                      seq_buf[i, d + 1] = argmax head(h).  deep: verify blocks (i, pos, d + 1) with
                      inputs exit_h[i, 0..d] through [k, L); Yv = argmax head; acc = first mismatch
                      against the drafts; seq_buf[i, 0] = Yv[acc]; pos += acc + 1; d = 0 (pointer rollback)
  FixedScheduler      solutions/schedulers.py:77-89
Forced acceptance (the measured configs' harness hook; no reference counterpart): acc = min(draw, d)
and the committed tokens are drafts[0..acc-1] + Yv[acc], as common/engine.py:406 commits them.
"""

from __future__ import annotations

import numpy as np
import torch

from .model import OBlock, build_packed, packed_layers

FREE, DECODE = 0, 2


class ForcedAcceptance:
    """Seeded per-request acceptance draws: a = Geometric(p) - 1 (then clipped to d by the engine).
    Request j (its index in the prompt pool) draws from default_rng([seed, j]) in round order."""

    def __init__(self, p: float, seed: int = 0):
        self.p, self.seed = p, seed
        self.streams: dict = {}

    def draw(self, req_index: int) -> int:
        rng = self.streams.get(req_index)
        if rng is None:
            rng = self.streams[req_index] = np.random.default_rng([self.seed, req_index])
        return int(rng.geometric(self.p)) - 1


class OracleEngine:
    def __init__(self, model, B: int, max_prompt: int, max_new: int, *, mode: str = "spec", k: int = 2,
                 gamma: int = 3, d_max: int = 8, prefill_chunk: int = 512, forced: ForcedAcceptance | None = None,
                 eos=()):
        if mode not in ("spec", "ar"):
            raise ValueError(mode)
        if not 1 <= k < model.n_layers:
            raise ValueError("exit layer must be in [1, n_layers)")
        self.m, self.B, self.mode, self.k, self.gamma, self.d_max = model, B, mode, k, gamma, d_max
        self.max_new, self.chunk, self.forced, self.eos = max_new, prefill_chunk, forced, set(eos)
        model.allocate_cache(B, max_prompt + max_new + d_max + 40)
        self.Dm1 = d_max + 1
        self.seq_buf = torch.zeros(B, self.Dm1, dtype=torch.long)
        self.exit_h = torch.zeros(B, self.Dm1, model.cfg.dim, dtype=model.dtype)
        self.state = np.zeros(B, dtype=np.int64)
        self.pos = np.zeros(B, dtype=np.int64)
        self.d = np.zeros(B, dtype=np.int64)
        self.req = [None] * B
        self.steps_since_deep = 0
        self.n_steps = 0
        self.n_deep = 0

    # ---- requests: dict(pid, index, prompt, out, finish)
    def _commit(self, slot, toks) -> int:
        r = self.req[slot]
        n = 0
        for t in toks:
            if r["finish"] is not None:
                break
            r["out"].append(int(t))
            n += 1
            if int(t) in self.eos:
                r["finish"] = "eos"
            elif len(r["out"]) >= self.max_new:
                r["finish"] = "length"
        return n

    @torch.inference_mode()
    def assign(self, slot: int, pid, index: int, prompt: list) -> int:
        m = self.m
        self.req[slot] = {"pid": pid, "index": index, "prompt": list(prompt), "out": [], "finish": None}
        h = None
        n = len(prompt)
        for s in range(0, n, self.chunk):
            c = min(self.chunk, n - s)
            pb = build_packed(m, [OBlock(slot, s, c)])
            h = packed_layers(m, m.embed(torch.tensor(prompt[s:s + c])), pb, 0, m.n_layers)
        y0 = int(m.head(h[-1:]).argmax(-1)[0])
        self.seq_buf[slot, 0] = y0
        self.state[slot] = DECODE
        self.pos[slot] = n
        self.d[slot] = 0
        return self._commit(slot, [y0])

    @torch.inference_mode()
    def step(self):
        self.n_steps += 1
        return self._ar_step() if self.mode == "ar" else self._spec_step()

    def _ar_step(self):
        m = self.m
        dec = np.flatnonzero(self.state == DECODE)
        pb = build_packed(m, [OBlock(int(i), int(self.pos[i]), 1) for i in dec])
        slots = [b.row for b in pb.blocks]
        h = packed_layers(m, m.embed(self.seq_buf[slots, 0]), pb, 0, m.n_layers)
        y = m.head(h).argmax(-1)
        self.seq_buf[slots, 0] = y
        done = []
        for s, t in zip(slots, y.tolist()):
            self.pos[s] += 1
            self._commit(s, [t])
            if self.req[s]["finish"]:
                done.append(s)
        return done

    def _spec_step(self):
        m, k, L, Dm1 = self.m, self.k, self.m.n_layers, self.Dm1
        dec = self.state == DECODE
        d = self.d.copy()
        if self.steps_since_deep >= self.gamma:
            V = dec & (d >= 1)
        else:
            V = dec & (d >= self.d_max)
        V = (V | (dec & (d >= self.d_max))) & dec & (d >= 1)
        deep = bool(V.any())
        Dr = dec & ~V
        blocks = [OBlock(int(i), int(self.pos[i] + d[i]), 1, int(i)) for i in np.flatnonzero(dec)]
        pb = build_packed(m, blocks)
        slots = [b.tag for b in pb.blocks]
        ids = torch.tensor([int(self.seq_buf[i, d[i]]) for i in slots])
        h = packed_layers(m, m.embed(ids), pb, 0, k)
        for j, i in enumerate(slots):
            self.exit_h[i, d[i]] = h[j]
        drafters = [j for j, i in enumerate(slots) if Dr[i]]
        if drafters:
            y = m.head(h[drafters]).argmax(-1)
            for jj, j in enumerate(drafters):
                i = slots[j]
                self.seq_buf[i, d[i] + 1] = y[jj]
        self.d[Dr] += 1
        if not deep:
            self.steps_since_deep += 1
            return []
        self.n_deep += 1
        vblocks = [OBlock(int(i), int(self.pos[i]), int(d[i]) + 1, int(i)) for i in np.flatnonzero(V)]
        pbd = build_packed(m, vblocks)
        x = torch.cat([self.exit_h[b.tag, :b.T] for b in pbd.blocks])
        hd = packed_layers(m, x, pbd, k, L)
        Yv = m.head(hd).argmax(-1).tolist()
        done = []
        for bi, b in enumerate(pbd.blocks):
            i, s0 = b.tag, int(pbd.offsets[bi])
            drafts = [int(self.seq_buf[i, j + 1]) for j in range(b.T - 1)]
            acc = b.T - 1
            for j in range(b.T - 1):
                if Yv[s0 + j] != drafts[j]:
                    acc = j
                    break
            toks = Yv[s0:s0 + acc + 1]
            if self.forced is not None:
                acc = min(self.forced.draw(self.req[i]["index"]), b.T - 1)
                toks = drafts[:acc] + [Yv[s0 + acc]]
            self.seq_buf[i, 0] = toks[-1]
            self.pos[i] += acc + 1
            self.d[i] = 0
            self._commit(i, toks)
            if self.req[i]["finish"]:
                done.append(i)
        self.steps_since_deep = 0
        return done

    def run_static(self, prompts: list) -> dict:
        """Every prompt once (pid, tokens); freed slots take the next prompt.  Returns pid -> tokens."""
        out, cursor = {}, 0
        for slot in range(self.B):
            if cursor >= len(prompts):
                break
            pid, toks = prompts[cursor]
            self.assign(slot, pid, cursor, toks)
            cursor += 1
        while (self.state == DECODE).any():
            finished = [s for s in range(self.B) if self.state[s] == DECODE and self.req[s]["finish"]]
            if not finished:
                finished = self.step()
            for s in finished:
                r = self.req[s]
                out[r["pid"]] = list(r["out"])
                self.state[s] = FREE
                self.req[s] = None
                if cursor < len(prompts):
                    pid, toks = prompts[cursor]
                    self.assign(s, pid, cursor, toks)
                    cursor += 1
        return out
