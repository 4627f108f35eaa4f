"""Basis-state replay for activation checkpointing (interface of stacr/adaptive_checkpointing.py:1-71).

When a checkpointed region is recomputed in backward, a STAC-R layer inside it must reproduce the
forward it is replacing: the same basis version and the same residual budget, not a freshly
refreshed basis.  Each checkpointed forward therefore writes a tape: one (layer, state) entry per
STAC-R layer call, in call order.  Its recomputation reads the tape back from the start, and a
layer met in a different order is an error.

Design: the active tape and the current phase ("record" or "replay") live in a context variable,
so nested regions and concurrent threads each see their own; the recorded entries hold the layer's
id and the state object the layer chose.  `checkpoint_contexts` is the `context_fn` that
`torch.utils.checkpoint.checkpoint(use_reentrant=False)` takes: it returns the recording context
for the forward and the replay context for the recomputation, sharing one new tape.
"""
from __future__ import annotations

import contextvars
from contextlib import contextmanager
from typing import Any


class _Tape:
    """Layer states one checkpointed forward recorded, read back in order by its recomputation."""

    __slots__ = ("entries", "cursor")

    def __init__(self, entries=None):
        self.entries: list = entries if entries is not None else []
        self.cursor = 0

    def write(self, layer, state) -> None:
        self.entries.append((id(layer), state))

    def read(self, layer):
        if self.cursor >= len(self.entries):
            raise RuntimeError("STAC-R layer order changed during checkpoint replay")
        ident, state = self.entries[self.cursor]
        if ident != id(layer):
            raise RuntimeError("STAC-R layer order changed during checkpoint replay")
        self.cursor += 1
        return state


# (phase, tape): phase None outside any region, "record" in a checkpointed forward, "replay" in
# its recomputation (tape None there means "recomputing without a recorded tape")
_PHASE: contextvars.ContextVar = contextvars.ContextVar("stacr_checkpoint_phase", default=(None, None))


@contextmanager
def _phase(phase: str, entries):
    # the tape (and its read cursor) is made on entry, so a region recomputed twice reads from
    # the start both times
    token = _PHASE.set((phase, None if entries is None else _Tape(entries)))
    try:
        yield
    finally:
        _PHASE.reset(token)


class RecomputationGuard:
    """The layers' view of the current checkpoint phase (names as the reference's guard)."""

    @property
    def is_recomputing(self) -> bool:
        return _PHASE.get()[0] == "replay"

    def forward_context(self, records: list):
        """Record layer states into `records` (a list) for the enclosed forward."""
        return _phase("record", records)

    def recomputation_context(self, records: list | None = None):
        """Replay `records` in order for the enclosed recomputation (None: recompute, no tape)."""
        return _phase("replay", records)

    def record_layer(self, layer, state: Any) -> None:
        phase, tape = _PHASE.get()
        if phase == "record":
            tape.write(layer, state)

    def replay_layer(self, layer):
        """The state `layer` recorded in the forward being recomputed, or None without a tape."""
        phase, tape = _PHASE.get()
        if phase != "replay" or tape is None:
            return None
        return tape.read(layer)


_GUARD = RecomputationGuard()


def get_global_recomputation_guard() -> RecomputationGuard:
    return _GUARD


def checkpoint_contexts():
    """context_fn for torch.utils.checkpoint.checkpoint(use_reentrant=False): one fresh tape shared
    by the forward's recording context and the recomputation's replay context."""
    entries: list = []
    return _GUARD.forward_context(entries), _GUARD.recomputation_context(entries)


def checkpoint(function, *args, **kwargs):
    """torch's non-reentrant checkpoint with STAC-R basis replay (reentrant mode is refused: it
    gives no context hook to replay through)."""
    from torch.utils.checkpoint import checkpoint as torch_checkpoint

    if kwargs.pop("use_reentrant", False):
        raise ValueError("Adaptive checkpointing requires use_reentrant=False")
    kwargs.setdefault("context_fn", checkpoint_contexts)
    return torch_checkpoint(function, *args, use_reentrant=False, **kwargs)


__all__ = ["RecomputationGuard", "get_global_recomputation_guard", "checkpoint_contexts", "checkpoint"]
