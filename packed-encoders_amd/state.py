"""Per-model state that ``pack()`` attaches to the encoder (packed_encoders/state.py:21-61).

``pack()`` patches the encoder in place; the state hangs off the module under one attribute and
keeps the original forward, so ``unpack()`` restores it and validation can compare against it.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Callable

from .config import ModernBertParams
from .errors import PackedEncodersError

ATTR = "_packed_encoders"


@dataclass
class PatchState:
    params: ModernBertParams
    original_forward: Callable[..., Any]
    attention_backend: str = "hip"     # "hip" | "sdpa"
    graph_enabled: bool = False
    graph_skip_warned: bool = False
    packed_graph_runner: Any = None    # graph.PackedGraphRunner | None
    validation_report: Any = None
    pieces: Any = None                 # pieces.ModernBertPieces
    execution: Any = None              # the pieces' bound callables (pieces.ModernBertOps)


def find_state(target: object) -> PatchState | None:
    from .locate import walk_targets

    for module in walk_targets(target):
        state = module.__dict__.get(ATTR) if hasattr(module, "__dict__") else None
        if state is not None:
            return state
    return None


def get_state(target: object) -> PatchState:
    state = find_state(target)
    if state is None:
        raise PackedEncodersError("this model has not been packed with packed_encoders_amd.pack()")
    return state
