"""Every built tile variant of the DMA grouped GEMMs gives the same bits.

The wgrad kernels (8-wave 256 x 256 and the 4-wave 128 x 128 ones with 2 or 3
stages, HRM_MOE_WGRAD_STAGES) are checked the same way.

The variants differ in tile shape (128 x 128 with 4 waves, 256 x 256 with 8
waves, 32 x 256 and 32 x 128 with 4 waves along N for decode sizes), pipeline depth and K
step (64 or 32), and the gate/up kernel's
256 x 256 variant runs its last N tile as a half tile when the width is an odd
multiple of 64.  All of them accumulate each output over K in the same order
(16-wide MFMA steps, ascending), so outputs must be bit-identical to the
default choice, which the oracle checks elsewhere (test_gpu_gemm.py,
test_gpu_layer.py).  HRM_MOE_GEMM_CFG selects the variant per call.
"""
import numpy as np
import pytest
import torch

from hrm_moe_amd import ops
from oracle import synth
from conftest import lib_env

pytestmark = pytest.mark.gpu

VARIANTS = ["128x128x2x4x64", "128x128x3x4x64", "128x128x4x4x32", "128x128x5x4x32",
            "256x128x2x4x32", "256x128x3x4x32", "256x256x2x8x64", "256x256x4x8x32", "32x256x4x4x64",
            "32x128x4x4x64", "32x128x5x4x64", "64x128x3x4x64", "64x128x5x4x64"]


def _ragged(seed, m, e):
    rng = np.random.default_rng(seed)
    w = rng.random(e) + 0.2
    w[rng.integers(0, e)] = 0.0  # one empty expert
    tpe = np.floor(w / w.sum() * m).astype(np.int64)
    tpe[np.argmax(w)] += m - tpe.sum()
    return tpe


def _run_all(fn):
    out = {}
    for v in [""] + VARIANTS:
        with lib_env(HRM_MOE_GEMM_CFG=v):
            out[v or "default"] = fn()
            torch.cuda.synchronize()
    return out


def _assert_same(outs, what):
    ref = outs["default"]
    for name, o in outs.items():
        assert torch.equal(o, ref), f"{what}: variant {name} differs from the default"


@pytest.mark.parametrize("t,h,e,i", [(2048, 1280, 8, 448), (1024, 1536, 8, 512)])
def test_gate_up_swiglu_variants_identical(cuda, t, h, e, i):
    k = 2
    r = t * k
    x = torch.from_numpy(synth.normal(71, (t, h))).to(cuda, torch.bfloat16)
    wgu = torch.from_numpy(synth.normal(72, (e, 2 * i, h), std=0.03)).to(cuda, torch.bfloat16)
    idx = torch.from_numpy(np.random.default_rng(73).integers(0, e, size=(t, k))).to(cuda)
    idx[:, 1] = (idx[:, 0] + 1 + idx[:, 1] % (e - 1)) % e  # distinct experts per token
    d = ops.permute(idx, e)
    assert int(d.tokens_per_expert.sum()) == r
    outs = _run_all(lambda: ops.gate_up_swiglu(x, d, wgu))
    _assert_same(outs, f"gate_up t{t} i{i}")


@pytest.mark.parametrize("m,n,kk,e", [(6000, 1280, 448, 8), (5000, 1024, 1536, 4)])
def test_nt_nn_variants_identical(cuda, m, n, kk, e):
    tpe = torch.from_numpy(_ragged(m, m, e)).to(cuda)
    a = torch.from_numpy(synth.normal(81, (m, kk))).to(cuda, torch.bfloat16)
    w = torch.from_numpy(synth.normal(82, (e, n, kk), std=0.05)).to(cuda, torch.bfloat16)
    _assert_same(_run_all(lambda: ops.grouped_gemm_nt(a, w, tpe)), f"nt {m}x{n}x{kk}")
    g = torch.from_numpy(synth.normal(83, (m, n))).to(cuda, torch.bfloat16)
    _assert_same(_run_all(lambda: ops.grouped_gemm_nn(g, w, tpe)), f"nn {m}x{kk}x{n}")


def _run_wgrad(fn):
    out = {}
    for v in ["", "2", "3"]:
        with lib_env(HRM_MOE_WGRAD_STAGES=v):
            out[v or "default"] = fn()
            torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("m,na,nb,e", [(4096, 512, 768, 8), (3000, 1024, 256, 4)])
def test_wgrad_variants_identical(cuda, m, na, nb, e):
    tpe = torch.from_numpy(_ragged(m + 7, m, e)).to(cuda)
    g = torch.from_numpy(synth.normal(91, (m, na))).to(cuda, torch.bfloat16)
    a = torch.from_numpy(synth.normal(92, (m, nb))).to(cuda, torch.bfloat16)
    outs = _run_wgrad(lambda: ops.grouped_gemm_tn(g, a, tpe))
    _assert_same(outs, f"tn {m}x{na}x{nb}")
