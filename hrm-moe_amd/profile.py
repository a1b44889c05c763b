"""Per-phase GPU timing of the MoE layer, switched on with HRM_MOE_PROFILE=1.

Public surface of the reference's models/moe_profile.py: the HRM_MOE_PROFILE
switch, ``record_moe_profile_phase(name)`` as a context manager around a
phase, ``pop_moe_profile()`` returning seconds per phase name summed over
calls (and clearing them), ``reset_moe_profile()``.

Mechanism: a phase does not wait for the GPU.  Entering it enqueues a timing
event on the current stream; leaving it enqueues a second one and files the
pair in a ledger.  ``pop_moe_profile()`` waits for each filed end event (the
first wait usually covers the rest), folds every pair's elapsed time into the
per-name totals, and hands the totals out.  So profiling adds two event
records per phase and no host synchronisation inside the layer; the times
are GPU times between the two records on the phase's stream.  Off by
default; then a phase is a shared no-op context manager, as it is while the
current stream is being captured into a HIP graph (events in a graph cannot
be timed).
"""
from __future__ import annotations

import os
from typing import Dict, List, Tuple

import torch


def _switch_from_env() -> bool:
    return os.environ.get("HRM_MOE_PROFILE", "0").strip().lower() in ("1", "true", "yes", "on")


class _Ledger:
    """Event pairs not yet resolved, and resolved seconds per phase name."""

    def __init__(self) -> None:
        self.on = _switch_from_env()
        self.open_pairs: List[Tuple[str, "torch.cuda.Event", "torch.cuda.Event"]] = []
        self.seconds: Dict[str, float] = {}

    def settle(self) -> None:
        pairs, self.open_pairs = self.open_pairs, []
        for name, first, last in pairs:
            last.synchronize()
            self.seconds[name] = self.seconds.get(name, 0.0) + first.elapsed_time(last) * 1e-3


_LEDGER = _Ledger()


class _NoPhase:
    def __enter__(self):
        return self

    def __exit__(self, *exc):
        return False


_NO_PHASE = _NoPhase()


class MoEProfilePhase:
    """Brackets one phase with two timing events on the current stream."""

    __slots__ = ("name", "_first")

    def __init__(self, name: str):
        self.name = name
        self._first = None

    def __enter__(self):
        self._first = torch.cuda.Event(enable_timing=True)
        self._first.record()
        return self

    def __exit__(self, *exc):
        last = torch.cuda.Event(enable_timing=True)
        last.record()
        _LEDGER.open_pairs.append((self.name, self._first, last))
        return False


def enabled() -> bool:
    return _LEDGER.on


def set_enabled(flag: bool) -> None:
    """Switch profiling on or off at run time (the environment switch sets the initial state)."""
    _LEDGER.on = bool(flag)


def record_moe_profile_phase(name: str):
    """Context manager timing the enclosed GPU work under ``name`` (a no-op while profiling is off)."""
    if not _LEDGER.on or not torch.cuda.is_available() or torch.cuda.is_current_stream_capturing():
        return _NO_PHASE
    return MoEProfilePhase(name)


def reset_moe_profile() -> None:
    """Drop unresolved phases and all totals."""
    _LEDGER.open_pairs.clear()
    _LEDGER.seconds.clear()


def pop_moe_profile() -> Dict[str, float]:
    """Seconds per phase name since the last pop or reset; waits for the GPU to finish the filed phases."""
    _LEDGER.settle()
    totals, _LEDGER.seconds = _LEDGER.seconds, {}
    return totals
