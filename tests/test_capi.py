"""CPU checks of the C ABI library and the host layer (no kernel launches).

The library must load, export every function include/hrm_moe.h declares,
report its ABI version, and reject bad arguments with the documented status
before touching the GPU.  The Python layer must raise the reference's
exceptions for the same conditions and refuse CPU tensors.
"""
import ctypes
import os
import re

import pytest
import torch

import hrm_moe_amd
from hrm_moe_amd import _lib, ops

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "hrm_moe.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(hrm_moe_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_entry_points():
    names = declared_functions()
    for want in ("hrm_moe_router_topk", "hrm_moe_permute", "hrm_moe_grouped_gemm_nt", "hrm_moe_grouped_gemm_nn",
                 "hrm_moe_grouped_gemm_tn", "hrm_moe_gate_up_swiglu", "hrm_moe_combine"):
        assert want in names


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_functions():
        assert hasattr(lib, name), f"{name} declared in hrm_moe.h but not exported"
    assert set(declared_functions()) == set(_lib.PROTOTYPES), "ctypes prototypes out of sync with the header"


def test_abi_version_and_status_strings():
    lib = _lib.load()
    assert lib.hrm_moe_abi_version() == _lib.ABI_VERSION
    for code in (0, -1, -2, -3, -4):
        assert _lib.status_string(code)


NULL = ctypes.c_void_p(0)


def test_router_rejects_bad_arguments():
    lib = _lib.load()
    call = lambda t, e, k, ldt=0, wdt=0: lib.hrm_moe_router_topk(NULL, ldt, t, e, k, 1, NULL, NULL, NULL, wdt, NULL)
    assert call(4, 0, 1) == _lib.ERR_INVALID
    assert call(4, 8, 9) == _lib.ERR_INVALID
    assert call(4, 2000, 8) == _lib.ERR_UNSUPPORTED  # up to 1024 experts
    assert call(4, 200, 8) == _lib.ERR_INVALID  # supported; null tensors
    assert call(4, 64, 33) == _lib.ERR_UNSUPPORTED
    assert call(4, 64, 8, ldt=7) == _lib.ERR_DTYPE
    assert call(0, 64, 8) == _lib.OK  # nothing to do
    assert call(4, 64, 8) == _lib.ERR_INVALID  # null tensors


def test_down_combine_decode_rejects_bad_arguments():
    lib = _lib.load()
    f = lib.hrm_moe_down_combine_decode
    buf = ctypes.c_void_p(1 << 20)  # never dereferenced: every call below returns before launching
    assert f(buf, buf, buf, buf, buf, buf, 3, 8, 1536, 512, 64, _lib.BF16, buf, NULL) == _lib.ERR_UNSUPPORTED
    assert f(buf, buf, buf, buf, buf, buf, 1, 9, 1536, 512, 64, _lib.BF16, buf, NULL) == _lib.ERR_UNSUPPORTED
    assert f(buf, buf, buf, buf, buf, buf, 1, 8, 1536, 1024, 64, _lib.BF16, buf, NULL) == _lib.ERR_UNSUPPORTED
    assert f(buf, buf, buf, buf, buf, buf, 1, 8, 1536, 496, 64, _lib.BF16, buf, NULL) == _lib.ERR_UNSUPPORTED
    assert f(buf, buf, buf, buf, buf, buf, 1, 8, 1535, 512, 64, _lib.BF16, buf, NULL) == _lib.ERR_UNSUPPORTED
    assert f(buf, buf, buf, buf, buf, buf, 1, 8, 1536, 512, 64, _lib.F32, buf, NULL) == _lib.ERR_DTYPE
    assert f(buf, NULL, buf, buf, buf, buf, 1, 8, 1536, 512, 64, _lib.BF16, buf, NULL) == _lib.ERR_INVALID
    assert f(buf, buf, buf, buf, buf, buf, 0, 8, 1536, 512, 64, _lib.BF16, buf, NULL) == _lib.OK


def test_router_gate_up_decode_limits_and_bad_arguments():
    lib = _lib.load()
    ok = lib.hrm_moe_router_gate_up_decode_supported
    assert ok(1, 1536, 512, 64, 8) == 1 and ok(2, 1536, 512, 64, 8) == 1
    assert ok(3, 1536, 512, 64, 8) == 0          # more than two tokens
    assert ok(1, 1536, 512, 64, 6) == 0          # k outside {2, 4, 8}
    assert ok(2, 1536, 512, 32, 8) == 0          # 4 T k > E: the grouped GEMM would not only stream weights
    assert ok(1, 1536, 512, 128, 8) == 0         # one wave routes a token: E <= 64
    assert ok(1, 1504, 512, 64, 8) == 0          # H not a multiple of 64
    assert ok(1, 4096, 512, 64, 8) == 0          # H above 2048
    assert ok(1, 1536, 504, 64, 8) == 0          # I not a multiple of 16
    f = lib.hrm_moe_router_gate_up_decode
    buf = ctypes.c_void_p(1 << 20)  # never dereferenced: every call below returns before launching
    args = lambda t=1, h=1536, i=512, e=64, k=8, dt=_lib.BF16, ldt=_lib.BF16, act=buf: (
        buf, ldt, buf, buf, t, h, i, e, k, 1, dt, NULL, buf, buf, buf, buf, buf, NULL, buf, act, NULL)
    assert f(*args(t=3)) == _lib.ERR_UNSUPPORTED
    assert f(*args(k=6)) == _lib.ERR_UNSUPPORTED
    assert f(*args(k=65)) == _lib.ERR_INVALID
    assert f(*args(dt=_lib.F32)) == _lib.ERR_DTYPE
    assert f(*args(ldt=7)) == _lib.ERR_DTYPE
    assert f(*args(act=NULL)) == _lib.ERR_INVALID
    assert f(*args(t=0)) == _lib.OK


def test_permute_rejects_bad_arguments():
    lib = _lib.load()
    assert lib.hrm_moe_permute_workspace_size(16, 2048, 2) == 0
    assert lib.hrm_moe_permute_workspace_size(16, 64, 8) > 0
    st = lib.hrm_moe_permute(NULL, 16, 2048, 2, NULL, NULL, NULL, NULL, NULL, NULL, 0, NULL)
    assert st == _lib.ERR_UNSUPPORTED
    st = lib.hrm_moe_permute(NULL, 16, 64, 8, NULL, NULL, NULL, NULL, NULL, NULL, 0, NULL)
    assert st == _lib.ERR_INVALID


def test_grouped_gemm_rejects_bad_arguments():
    lib = _lib.load()
    ws = lib.hrm_moe_grouped_gemm_workspace_size(1024, 64)
    assert ws > 0
    buf = ctypes.c_void_p(1 << 20)  # never dereferenced: every call below returns before launching
    f = lib.hrm_moe_grouped_gemm_nt
    assert f(buf, buf, buf, 1024, 128, 64, 64, _lib.F32, buf, buf, ws, NULL) == _lib.ERR_DTYPE
    assert f(buf, buf, buf, 1024, 128, 64, 64, _lib.BF16, buf, buf, ws - 1, NULL) == _lib.ERR_WORKSPACE
    assert f(buf, buf, buf, 1024, 100, 64, 64, _lib.BF16, buf, buf, ws, NULL) == _lib.ERR_UNSUPPORTED
    assert f(buf, buf, buf, 1024, 128, 60, 64, _lib.BF16, buf, buf, ws, NULL) == _lib.ERR_UNSUPPORTED
    assert f(buf, buf, buf, 1024, 128, 64, 2000, _lib.BF16, buf, buf, ws, NULL) == _lib.ERR_UNSUPPORTED
    assert f(buf, buf, buf, 0, 128, 64, 64, _lib.BF16, buf, buf, ws, NULL) == _lib.OK
    g = lib.hrm_moe_gate_up_swiglu
    assert g(buf, buf, buf, buf, 16, 128, 256, 100, 64, _lib.BF16, buf, buf, ws, NULL) == _lib.ERR_UNSUPPORTED
    c = lib.hrm_moe_combine
    assert c(buf, buf, buf, buf, 16, 40, 256, 64, _lib.BF16, buf, NULL) == _lib.ERR_UNSUPPORTED
    assert c(buf, buf, buf, buf, 16, 8, 256, 64, 9, buf, NULL) == _lib.ERR_DTYPE


def test_training_entry_points_reject_bad_arguments():
    lib = _lib.load()
    ws = lib.hrm_moe_grouped_gemm_workspace_size(1024, 64)
    buf = ctypes.c_void_p(1 << 20)  # never dereferenced: every call below returns before launching
    s = lib.hrm_moe_gate_up_swiglu_save
    assert s(buf, buf, buf, buf, 16, 128, 256, 64, 64, _lib.BF16, buf, buf, NULL, 0, NULL) == _lib.ERR_WORKSPACE
    assert s(buf, buf, buf, buf, 16, 128, 96, 64, 64, _lib.BF16, buf, buf, buf, ws, NULL) == _lib.ERR_UNSUPPORTED
    assert s(buf, buf, buf, buf, 16, 128, 256, 64, 64, _lib.F32, buf, buf, buf, ws, NULL) == _lib.ERR_DTYPE
    assert s(buf, buf, buf, buf, 16, 128, 256, 64, 64, _lib.BF16, buf, NULL, buf, ws, NULL) == _lib.ERR_INVALID
    assert s(buf, buf, buf, buf, 16, 0, 256, 64, 64, _lib.BF16, buf, buf, buf, ws, NULL) == _lib.OK
    d = lib.hrm_moe_down_dgrad_swiglu
    assert d(buf, buf, buf, buf, 128, 64, 200, 64, _lib.BF16, buf, buf, ws, NULL) == _lib.ERR_UNSUPPORTED
    assert d(buf, buf, buf, buf, 128, 60, 256, 64, _lib.BF16, buf, buf, ws, NULL) == _lib.ERR_UNSUPPORTED
    assert d(buf, buf, buf, NULL, 128, 64, 256, 64, _lib.BF16, buf, buf, ws, NULL) == _lib.ERR_INVALID
    assert d(buf, buf, buf, buf, 0, 64, 256, 64, _lib.BF16, buf, buf, ws, NULL) == _lib.OK
    gws = lib.hrm_moe_gate_wgrad_workspace_size(16384, 64, 1280)
    assert gws >= 16 * 64 * 1280 * 4  # fp32 partials of 16 splits of 1024 rows
    gw = lib.hrm_moe_gate_wgrad
    assert gw(buf, buf, 16384, 64, 1280, _lib.BF16, buf, buf, gws - 1, NULL) == _lib.ERR_WORKSPACE
    assert gw(buf, buf, 16384, 60, 1280, _lib.BF16, buf, buf, gws, NULL) == _lib.ERR_UNSUPPORTED
    assert gw(buf, buf, 16384, 64, 1280, _lib.F32, buf, buf, gws, NULL) == _lib.ERR_DTYPE
    assert gw(NULL, buf, 16384, 64, 1280, _lib.BF16, buf, buf, gws, NULL) == _lib.ERR_INVALID
    assert lib.hrm_moe_router_dispatch_workspace_size(16, 200, 8) == 0
    rd = lib.hrm_moe_router_topk_dispatch
    rws = lib.hrm_moe_router_dispatch_workspace_size(16, 64, 8)
    assert rd(buf, _lib.BF16, 16, 64, 16, 1, buf, buf, buf, _lib.BF16, buf, buf, buf, NULL, buf, buf, rws,
              NULL) == _lib.ERR_UNSUPPORTED
    assert rd(buf, _lib.BF16, 16, 64, 8, 1, buf, buf, buf, _lib.BF16, buf, buf, buf, NULL, buf, buf, rws - 1,
              NULL) == _lib.ERR_WORKSPACE
    assert rd(buf, _lib.BF16, 16, 64, 8, 1, buf, NULL, buf, _lib.BF16, buf, buf, buf, NULL, buf, buf, rws,
              NULL) == _lib.ERR_INVALID
    assert rd(buf, 7, 16, 64, 8, 1, buf, buf, buf, _lib.BF16, buf, buf, buf, NULL, buf, buf, rws,
              NULL) == _lib.ERR_DTYPE
    rb = lib.hrm_moe_router_topk_backward
    assert rb(buf, buf, buf, _lib.BF16, NULL, 0, 16, 2000, 8, 1, buf, _lib.BF16, NULL) == _lib.ERR_UNSUPPORTED
    assert rb(buf, buf, buf, 9, NULL, 0, 16, 64, 8, 1, buf, _lib.BF16, NULL) == _lib.ERR_DTYPE
    assert rb(buf, buf, buf, _lib.BF16, NULL, 0, 16, 64, 65, 1, buf, _lib.BF16, NULL) == _lib.ERR_INVALID
    assert rb(buf, NULL, buf, _lib.BF16, NULL, 0, 16, 64, 8, 1, buf, _lib.BF16, NULL) == _lib.ERR_INVALID
    assert rb(buf, buf, buf, _lib.BF16, buf, 32, 16, 64, 8, 1, buf, _lib.BF16, NULL) == _lib.ERR_INVALID  # stride < E
    assert rb(buf, buf, buf, _lib.BF16, NULL, 0, 0, 64, 8, 1, buf, _lib.BF16, NULL) == _lib.OK
    aw = lib.hrm_moe_aux_loss_workspace_size(16384, 64)
    assert aw >= 64 * 4 and lib.hrm_moe_aux_loss_workspace_size(0, 64) == 0
    al = lib.hrm_moe_aux_loss
    assert al(buf, 16384, 64, buf, buf, buf, buf, buf, aw - 1, NULL) == _lib.ERR_WORKSPACE
    assert al(buf, 16384, 2000, buf, buf, buf, buf, buf, aw, NULL) == _lib.ERR_UNSUPPORTED
    assert al(buf, 0, 64, buf, buf, buf, buf, buf, aw, NULL) == _lib.ERR_INVALID
    assert al(buf, 16384, 64, NULL, buf, buf, buf, buf, aw, NULL) == _lib.ERR_INVALID
    ab = lib.hrm_moe_aux_loss_backward
    assert ab(NULL, buf, 16384, 64, buf, NULL) == _lib.ERR_INVALID
    assert ab(buf, buf, 0, 64, buf, NULL) == _lib.ERR_INVALID
    tg = lib.hrm_moe_grouped_gemm_tn_gather
    assert tg(buf, buf, buf, 100, buf, 1024, 256, 252, 64, _lib.BF16, buf, buf, ws, NULL) == _lib.ERR_UNSUPPORTED
    assert tg(buf, buf, NULL, 100, buf, 1024, 256, 256, 64, _lib.BF16, buf, buf, ws, NULL) == _lib.ERR_INVALID
    assert tg(buf, buf, buf, -1, buf, 1024, 256, 256, 64, _lib.BF16, buf, buf, ws, NULL) == _lib.ERR_INVALID
    assert tg(buf, buf, buf, 100, buf, 1024, 256, 256, 64, _lib.F32, buf, buf, ws, NULL) == _lib.ERR_DTYPE
    b = lib.hrm_moe_combine_backward
    assert b(buf, buf, buf, buf, buf, 16, 33, 256, 64, _lib.BF16, buf, buf, NULL) == _lib.ERR_UNSUPPORTED
    assert b(buf, buf, buf, buf, buf, 16, 8, 252, 64, _lib.BF16, buf, buf, NULL) == _lib.ERR_UNSUPPORTED
    assert b(buf, buf, buf, buf, buf, 16, 8, 256, 64, 9, buf, buf, NULL) == _lib.ERR_DTYPE
    assert b(buf, buf, buf, buf, buf, 16, 8, 256, 64, _lib.BF16, buf, NULL, NULL) == _lib.ERR_INVALID
    assert b(buf, buf, buf, buf, buf, 0, 8, 256, 64, _lib.BF16, buf, buf, NULL) == _lib.OK


def test_check_maps_status_to_reference_exceptions():
    with pytest.raises(TypeError):
        _lib.check(_lib.ERR_DTYPE, "x")
    with pytest.raises(ValueError):
        _lib.check(_lib.ERR_INVALID, "x")
    with pytest.raises(RuntimeError):
        _lib.check(700, "x")


# -------------------------------------------------------------- host layer --

def test_ops_refuse_cpu_tensors():
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ops.router_topk(torch.zeros(4, 8), 2, True, torch.float32)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        ops.permute(torch.zeros(4, 2, dtype=torch.int64), 8)


def test_grouped_linear_contract_on_host():
    w = torch.zeros(4, 16, 32, dtype=torch.bfloat16)
    # M == 0 follows the reference: input @ weight[0].T
    out = hrm_moe_amd.hip_grouped_linear(torch.zeros(0, 32, dtype=torch.bfloat16), w, torch.zeros(4))
    assert out.shape == (0, 16)
    with pytest.raises(RuntimeError, match="no CPU path"):
        hrm_moe_amd.hip_grouped_linear(torch.zeros(3, 32, dtype=torch.bfloat16), w, torch.tensor([3, 0, 0, 0]))
    assert hrm_moe_amd.triton_grouped_linear is hrm_moe_amd.hip_grouped_linear


def test_module_surface_matches_reference():
    m = hrm_moe_amd.SparseMoESwiGLU(hidden_size=32, intermediate_size=16, num_experts=8, top_k=2,
                                    norm_topk_prob=True, implementation="grouped_triton")
    shapes = {n: tuple(p.shape) for n, p in m.named_parameters()}
    assert shapes == {"gate.weight": (8, 32), "experts.gate_up_weight": (8, 32, 32),
                      "experts.down_weight": (8, 32, 16)}
    with pytest.raises(ValueError):
        hrm_moe_amd.SparseMoESwiGLU(32, 16, 8, 9, True)
    with pytest.raises(ValueError):
        hrm_moe_amd.SparseMoESwiGLU(32, 16, 8, 2, True, expert_in_one_shard=3)
    with pytest.raises(ValueError, match="not provided"):
        hrm_moe_amd.SparseMoESwiGLU(32, 16, 8, 2, True, implementation="origin")


def test_init_statistics_match_reference_formula():
    torch.manual_seed(0)
    m = hrm_moe_amd.SparseMoESwiGLU(256, 128, 16, 2, True)
    for p, std in ((m.gate.weight, 256 ** -0.5), (m.experts.gate_up_weight, 256 ** -0.5),
                   (m.experts.down_weight, 128 ** -0.5)):
        assert abs(float(p.std()) / std - 1.0) < 0.05
        assert float(p.abs().max()) < 3.0 * 1.0148 * std + 1e-6


def test_aux_loss_closed_form():
    probs = torch.softmax(torch.randn(10, 4), -1)
    idx = torch.tensor([[0, 1]] * 5 + [[2, 3]] * 5)
    want = 4 * sum((5 / 10) * probs[:, e].mean() for e in range(4))
    assert torch.allclose(hrm_moe_amd.load_balancing_loss_func(probs, idx, 4), want)
