"""The skinny (decode-size) grouped GEMM against the oracle and the tiled path.

Chosen by default at no more than one row per four experts; HRM_MOE_SKINNY=1
forces it up to 16 rows per expert, which these tests do so that ragged,
empty and multi-pass experts (one expert far above the rows of one pass) are
all covered at the L and XL shapes.  Bar as for the other grouped GEMMs:
max|d| <= 1e-2 max|ref|, mean|d| <= 2e-3 mean|ref|.  HRM_MOE_SKINNY=0 forces
the tiled kernels for the same call, which must agree to the same bar.
"""
import numpy as np
import pytest
import torch

from hrm_moe_amd import ops
from oracle import moe_oracle as mo
from oracle import synth
from conftest import lib_env

pytestmark = pytest.mark.gpu


def close(got, ref, what):
    got, ref = got.float().cpu(), ref.float().cpu()
    d = (got - ref).abs()
    scale = ref.abs().max().item() or 1.0
    mean_ref = ref.abs().mean().item() or 1.0
    print(f"{what}: max|d|/max|ref| {d.max().item() / scale:.2e}, mean|d| {d.mean().item():.2e}")
    assert d.max().item() <= 1e-2 * scale, what
    assert d.mean().item() <= 2e-3 * mean_ref, what


def skewed_tpe(seed, m, e):
    rng = np.random.default_rng(seed)
    tpe = rng.multinomial(m // 2, np.ones(e) / e).astype(np.int64)
    tpe[rng.integers(0, e)] += m - tpe.sum()  # one expert holds about half the rows
    tpe[rng.integers(0, e, size=3)] = 0
    tpe[np.argmax(tpe)] += m - tpe.sum()
    return tpe


def _with_skinny(flag, fn):
    with lib_env(HRM_MOE_SKINNY=flag):
        return fn()


def _tiled(fn):
    return _with_skinny("0", fn)


@pytest.mark.parametrize("m,n,k,e", [(8, 1536, 512, 64), (700, 1280, 448, 64), (1000, 1536, 512, 64), (30, 256, 128, 4)])
def test_skinny_nt(cuda, m, n, k, e):
    tpe_np = skewed_tpe(m, m, e)
    assert tpe_np.sum() == m and m <= 16 * e
    tpe = torch.from_numpy(tpe_np).to(cuda)
    a = torch.from_numpy(synth.normal(m + 5, (m, k))).to(torch.bfloat16)
    w = torch.from_numpy(synth.normal(n + 5, (e, n, k), std=0.05)).to(torch.bfloat16)
    got = _with_skinny("1", lambda: ops.grouped_gemm_nt(a.to(cuda), w.to(cuda), tpe))
    close(got, mo.grouped_linear(a, w, tpe_np), f"skinny nt {m}x{n}x{k}")
    tiled = _tiled(lambda: ops.grouped_gemm_nt(a.to(cuda), w.to(cuda), tpe))
    close(got, tiled, "skinny vs tiled")


@pytest.mark.parametrize("t,h,e,i,k", [(1, 1536, 64, 512, 8), (64, 1536, 64, 512, 8), (100, 1280, 64, 448, 8)])
def test_skinny_gate_up_swiglu(cuda, t, h, e, i, k):
    x_, wg, wgu, _ = synth.moe_inputs(200 + t, t, h, e, i)
    x = torch.from_numpy(x_).to(torch.bfloat16)
    wgu_t = torch.from_numpy(wgu).to(torch.bfloat16)
    logits = torch.nn.functional.linear(x.to(cuda), torch.from_numpy(wg).to(cuda, torch.bfloat16))
    _, _, idx = ops.router_topk(logits, k, True, torch.bfloat16)
    d = ops.permute(idx, e)
    act = _with_skinny("1", lambda: ops.gate_up_swiglu(x.to(cuda), d, wgu_t.to(cuda)))
    rows = x[d.sorted_token_idx.long().cpu()]
    tpe = d.tokens_per_expert.cpu().numpy()
    ref = mo.swiglu(mo.grouped_linear(rows, wgu_t, tpe))
    close(act, ref, f"skinny gate_up t{t}")
    tiled = _tiled(lambda: ops.gate_up_swiglu(x.to(cuda), d, wgu_t.to(cuda)))
    close(act, tiled, "skinny vs tiled gate_up")
