"""Per-phase timing of the MoE layer, switched on with HRM_MOE_PROFILE=1.

Same switch, phase names and accumulate/pop interface as the reference's
models/moe_profile.py:9-47.  Each phase records two HIP events on the current
stream and waits for the end event, so it adds a synchronisation per phase
(as the reference does).  Off by default; then a phase costs one dict lookup.
"""
from __future__ import annotations

import os
from typing import Dict, Optional

import torch

_ENABLED = os.environ.get("HRM_MOE_PROFILE", "0").lower() in ("1", "true", "yes")
_SECONDS: Dict[str, float] = {}


def enabled() -> bool:
    return _ENABLED


def set_enabled(flag: bool) -> None:
    global _ENABLED
    _ENABLED = bool(flag)


class MoEProfilePhase:
    def __init__(self, name: str):
        self.name = name
        self.start: Optional[torch.cuda.Event] = None
        self.end: Optional[torch.cuda.Event] = None

    def __enter__(self):
        if not _ENABLED or not torch.cuda.is_available():
            return self
        self.start = torch.cuda.Event(enable_timing=True)
        self.end = torch.cuda.Event(enable_timing=True)
        self.start.record()
        return self

    def __exit__(self, exc_type, exc, tb):
        if self.start is None or self.end is None:
            return False
        self.end.record()
        self.end.synchronize()
        _SECONDS[self.name] = _SECONDS.get(self.name, 0.0) + self.start.elapsed_time(self.end) / 1000.0
        return False


def record_moe_profile_phase(name: str) -> MoEProfilePhase:
    return MoEProfilePhase(name)


def reset_moe_profile() -> None:
    _SECONDS.clear()


def pop_moe_profile() -> Dict[str, float]:
    out = dict(_SECONDS)
    _SECONDS.clear()
    return out
