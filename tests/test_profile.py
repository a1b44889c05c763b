"""The per-phase profiling hook (hrm-moe_amd/profile.py) on the CPU, with a stand-in event class.

Checks the reference's interface semantics (models/moe_profile.py): seconds
per phase name, summed over calls; pop returns the totals and clears them;
reset drops everything; off means nothing is recorded.  Also checks this
build's mechanism: no host wait while phases run, one wait per filed phase at
pop time, and no phases while a graph is being captured.
"""
import importlib

import pytest
import torch

import hrm_moe_amd


class _Clock:
    now_ms = 0.0


class _FakeEvent:
    """Timing event whose record() reads a shared fake clock (milliseconds)."""

    created = 0
    waits = 0

    def __init__(self, enable_timing=False):
        assert enable_timing
        self.t = None
        _FakeEvent.created += 1

    def record(self, stream=None):
        self.t = _Clock.now_ms

    def synchronize(self):
        _FakeEvent.waits += 1

    def elapsed_time(self, other):
        return other.t - self.t


@pytest.fixture()
def prof(monkeypatch):
    mod = importlib.import_module("hrm_moe_amd.profile")
    monkeypatch.setattr(torch.cuda, "Event", _FakeEvent)
    monkeypatch.setattr(torch.cuda, "is_available", lambda: True)
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: False)
    _FakeEvent.created = _FakeEvent.waits = 0
    _Clock.now_ms = 0.0
    was = mod.enabled()
    mod.set_enabled(True)
    mod.reset_moe_profile()
    yield mod
    mod.reset_moe_profile()
    mod.set_enabled(was)


def _phase(mod, name, ms):
    with mod.record_moe_profile_phase(name):
        _Clock.now_ms += ms


def test_accumulates_per_name_and_pop_clears(prof):
    _phase(prof, "router", 2.0)
    _phase(prof, "gate_up_gemm", 5.0)
    _phase(prof, "router", 3.0)
    assert _FakeEvent.waits == 0, "a phase must not wait for the GPU"
    got = prof.pop_moe_profile()
    assert got == pytest.approx({"router": 0.005, "gate_up_gemm": 0.005})
    assert _FakeEvent.waits == 3
    assert prof.pop_moe_profile() == {}


def test_nested_phases_each_count(prof):
    with prof.record_moe_profile_phase("experts"):
        _Clock.now_ms += 1.0
        _phase(prof, "down_gemm", 4.0)
    assert prof.pop_moe_profile() == pytest.approx({"experts": 0.005, "down_gemm": 0.004})


def test_reset_drops_pending_and_totals(prof):
    _phase(prof, "combine", 1.0)
    prof.pop_moe_profile()
    _phase(prof, "combine", 1.0)
    prof.reset_moe_profile()
    assert prof.pop_moe_profile() == {}


def test_off_records_nothing(prof):
    prof.set_enabled(False)
    _phase(prof, "router", 1.0)
    assert _FakeEvent.created == 0
    assert prof.pop_moe_profile() == {}


def test_no_phase_during_graph_capture(prof, monkeypatch):
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)
    _phase(prof, "router", 1.0)
    assert _FakeEvent.created == 0


def test_public_names_exported():
    for n in ("record_moe_profile_phase", "reset_moe_profile", "pop_moe_profile"):
        assert callable(getattr(hrm_moe_amd, n))
