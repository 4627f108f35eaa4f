"""Record/replay of per-layer basis state across activation-checkpoint recomputation.

Same contract as stacr/adaptive_checkpointing.py:7-71: a forward records (layer, state) pairs,
the recomputation replays them in order so a replayed layer reuses the basis and budget of the
original forward instead of refreshing it.
"""
from __future__ import annotations

import threading
from contextlib import contextmanager


class RecomputationGuard:
    def __init__(self):
        self._tls = threading.local()

    @property
    def is_recomputing(self) -> bool:
        return bool(getattr(self._tls, "recomputing", False))

    @contextmanager
    def forward_context(self, records):
        saved = getattr(self._tls, "recording", None)
        self._tls.recording = records
        try:
            yield
        finally:
            self._tls.recording = saved

    def record_layer(self, layer, state) -> None:
        records = getattr(self._tls, "recording", None)
        if records is not None and not self.is_recomputing:
            records.append((id(layer), state))

    def replay_layer(self, layer):
        replay = getattr(self._tls, "replay", None)
        if replay is None:
            return None
        ident, state = next(replay)
        if ident != id(layer):
            raise RuntimeError("STAC-R layer order changed during checkpoint replay")
        return state

    @contextmanager
    def recomputation_context(self, records=None):
        saved_flag = self.is_recomputing
        saved_replay = getattr(self._tls, "replay", None)
        self._tls.recomputing = True
        self._tls.replay = None if records is None else iter(records)
        try:
            yield
        finally:
            self._tls.recomputing = saved_flag
            self._tls.replay = saved_replay


_GUARD = RecomputationGuard()


def get_global_recomputation_guard() -> RecomputationGuard:
    return _GUARD


def checkpoint_contexts():
    """context_fn for torch.utils.checkpoint.checkpoint(use_reentrant=False)."""
    records: list = []
    return _GUARD.forward_context(records), _GUARD.recomputation_context(records)


def checkpoint(function, *args, **kwargs):
    """Non-reentrant checkpoint that replays recorded basis state."""
    from torch.utils.checkpoint import checkpoint as torch_checkpoint

    if kwargs.pop("use_reentrant", False):
        raise ValueError("STAC-R checkpointing requires use_reentrant=False")
    kwargs.setdefault("context_fn", checkpoint_contexts)
    return torch_checkpoint(function, *args, use_reentrant=False, **kwargs)
