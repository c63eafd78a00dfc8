"""Registry of decoding methods (common/methods.py:27-101): each method adds its CLI arguments and an
engine factory returning a `DecodeEngine`, so every method is driven and measured the same way.

    from thesis_amd.common.methods import MethodSpec, register
    register(MethodSpec("name", "description", add_args, build, tag=lambda a: "-k8"))

Built in: "autoregressive" and "sync_layerskip".  `load_plugins()` imports `thesis_amd.solutions`,
which registers "eesd" (the merged shallow/deep engine).
"""

from __future__ import annotations

import importlib
from dataclasses import dataclass, field
from typing import Callable, Optional

from .engine import ARBatchEngine, DecodeEngine, SyncSpecEngine


@dataclass
class MethodSpec:
    """One decoding method as the benchmark driver sees it.

    `add_args(group)` declares the method's command-line options on an argparse group; `build(model, args,
    batch_size, max_prompt_len, eos)` returns the ready `DecodeEngine`.  The remaining hooks have defaults:
    `tag(args)` is appended to result file names (for example "-k8-g4"); `supports_sampling` says whether
    temperature / top-k / top-p apply; `spec_slack` is how many cache positions a request may need past
    its `max_new` budget (drafts that are later rolled back); `step_tokens(args)` bounds the tokens one
    request adds in a single step, which sizes the per-step buffers; `params(args)` is the dictionary of
    method settings stored next to the measured metrics."""

    name: str
    description: str
    add_args: Callable
    build: Callable[..., DecodeEngine]
    tag: Callable = field(default=lambda args: "")
    supports_sampling: bool = False
    spec_slack: int = 0
    step_tokens: Callable = field(default=lambda args: 1)
    params: Callable = field(default=lambda args: {})


METHODS: dict = {}


def register(spec: MethodSpec) -> MethodSpec:
    if spec.name in METHODS:
        raise ValueError(f"method {spec.name!r} already registered")
    METHODS[spec.name] = spec
    return spec


def load_plugins(modules: Optional[list] = None) -> list:
    """Import thesis_amd.solutions (and any extra modules) so that they register their methods.
    A module that does not exist is skipped; a module whose own imports fail raises."""
    loaded = []
    for name in ["thesis_amd.solutions"] + list(modules or []):
        try:
            importlib.import_module(name)
            loaded.append(name)
        except ModuleNotFoundError as e:
            if e.name != name:
                raise
    return loaded


def _sampling_kw(args) -> dict:
    return dict(temperature=args.temperature, top_k=args.top_k, top_p=args.top_p, seed=args.seed)


def _ar_build(model, args, batch_size, max_prompt_len, eos):
    return ARBatchEngine(model, batch_size, max_prompt_len, args.max_new_tokens, eos, ignore_eos=args.ignore_eos,
                         **_sampling_kw(args))


register(MethodSpec("autoregressive", "all N layers per token (baseline)", lambda g: None, _ar_build,
                    supports_sampling=True))


def _sync_args(g) -> None:
    g.add_argument("--exit-layer", type=int, default=None, help="[sync_layerskip] exit layer k")
    g.add_argument("--gamma", type=int, default=4, help="[sync_layerskip] draft length")


def _sync_build(model, args, batch_size, max_prompt_len, eos):
    if args.exit_layer is None:
        raise SystemExit("--exit-layer is required for sync_layerskip")
    return SyncSpecEngine(model, batch_size, max_prompt_len, args.max_new_tokens, eos, ignore_eos=args.ignore_eos,
                          exit_layer=args.exit_layer, gamma=args.gamma)


register(MethodSpec("sync_layerskip", "synchronous batched LayerSkip (fixed k, gamma)", _sync_args, _sync_build,
                    tag=lambda a: f"-k{a.exit_layer}-g{a.gamma}", spec_slack=64,
                    step_tokens=lambda a: a.gamma + 1,
                    params=lambda a: {"exit_layer": a.exit_layer, "gamma": a.gamma}))
