"""Tuning knobs on the CPU: the CU margin's validation and precedence, and the library's configuration reload.

The reference reads HRM_MOE_TRITON_SM_MARGIN (falling back to
XTUNER_SM_MARGIN) when its module is imported and raises ValueError for a
negative or non-integer value (models/moe_triton_grouped_gemm.py:24-52).  This
build honours both names and its own HRM_MOE_HIP_CU_MARGIN (first), in the
Python layer and in the kernel library.  No kernel is launched here.
"""
import os
import subprocess
import sys

import pytest

from hrm_moe_amd import _lib
from hrm_moe_amd.grouped_gemm import cu_margin_from_env
from conftest import ROOT, lib_env


@pytest.mark.parametrize("env,want", [
    ({}, 0),
    ({"HRM_MOE_TRITON_SM_MARGIN": "16"}, 16),
    ({"XTUNER_SM_MARGIN": "8"}, 8),
    ({"HRM_MOE_TRITON_SM_MARGIN": "16", "XTUNER_SM_MARGIN": "8"}, 16),
    ({"HRM_MOE_HIP_CU_MARGIN": "4", "HRM_MOE_TRITON_SM_MARGIN": "16"}, 4),
    ({"HRM_MOE_TRITON_SM_MARGIN": "", "XTUNER_SM_MARGIN": " 3 "}, 3),
    ({"HRM_MOE_HIP_CU_MARGIN": "0", "XTUNER_SM_MARGIN": "12"}, 0),
])
def test_margin_precedence(env, want):
    assert cu_margin_from_env(env) == want


@pytest.mark.parametrize("env", [
    {"HRM_MOE_TRITON_SM_MARGIN": "-1"},
    {"XTUNER_SM_MARGIN": "-4"},
    {"HRM_MOE_TRITON_SM_MARGIN": "16", "XTUNER_SM_MARGIN": "-4"},  # every set name is checked
    {"HRM_MOE_HIP_CU_MARGIN": "abc"},
    {"HRM_MOE_HIP_CU_MARGIN": "1.5"},
    {"HRM_MOE_HIP_CU_MARGIN": "0x10"},
])
def test_margin_rejects_bad_values(env):
    with pytest.raises(ValueError):
        cu_margin_from_env(env)


def test_import_raises_for_negative_margin():
    env = dict(os.environ, HRM_MOE_TRITON_SM_MARGIN="-2")
    env.pop("HRM_MOE_HIP_CU_MARGIN", None)
    r = subprocess.run([sys.executable, "-c", "import hrm_moe_amd"], cwd=ROOT, env=env, capture_output=True,
                       text=True, timeout=300)
    assert r.returncode != 0
    assert "ValueError" in r.stderr and "HRM_MOE_TRITON_SM_MARGIN" in r.stderr


def test_library_reads_margin_names():
    lib = _lib.load()
    clear = dict(HRM_MOE_HIP_CU_MARGIN=None, HRM_MOE_TRITON_SM_MARGIN=None, XTUNER_SM_MARGIN=None)
    with lib_env(**dict(clear, XTUNER_SM_MARGIN="24")):
        assert lib.hrm_moe_cu_margin() == 24
    with lib_env(**dict(clear, HRM_MOE_TRITON_SM_MARGIN="16", XTUNER_SM_MARGIN="24")):
        assert lib.hrm_moe_cu_margin() == 16
    with lib_env(**dict(clear, HRM_MOE_HIP_CU_MARGIN="2", HRM_MOE_TRITON_SM_MARGIN="16")):
        assert lib.hrm_moe_cu_margin() == 2
    with lib_env(**clear):
        assert lib.hrm_moe_cu_margin() == 0


def test_library_rejects_malformed_knobs():
    lib = _lib.load()
    for name, bad in (("HRM_MOE_HIP_CU_MARGIN", "-5"), ("HRM_MOE_HIP_CU_MARGIN", "7x"),
                      ("HRM_MOE_WGRAD_STAGES", "9"), ("HRM_MOE_GATE_SPLIT_ROWS", "-1"), ("HRM_MOE_GEMM_CFG", "big")):
        saved = os.environ.get(name)
        os.environ[name] = bad
        try:
            assert lib.hrm_moe_reload_config() == _lib.ERR_INVALID, name
            if name == "HRM_MOE_HIP_CU_MARGIN":
                assert lib.hrm_moe_cu_margin() == 0
        finally:
            if saved is None:
                os.environ.pop(name, None)
            else:
                os.environ[name] = saved
    assert lib.hrm_moe_reload_config() == _lib.OK
