"""Grouped GEMM kernels on the GPU against the oracle (fp32 accumulation, one rounding).

Forward (NT), dgrad (NN) and wgrad (TN) replace the reference's Triton
kernels (models/moe_triton_grouped_gemm.py:113-347).  Each kernel accumulates
in fp32 and rounds once, as the oracle does.  Only the summation order
differs, so outputs agree to about one 16-bit ulp.  The bar: max |diff| <=
1e-2 * max |ref| and mean |diff| <= 2e-3 * mean |ref|.  Cases cover ragged
and empty experts, one expert holding every row, sizes that are not tile
multiples, fp16, the L / XL expert shapes and decode sizes (at most 16 rows
per expert on average, where the kernels take 32-row tiles).
"""
import numpy as np
import pytest
import torch

import hrm_moe_amd
from hrm_moe_amd import ops
from oracle import moe_oracle as mo
from oracle import synth
from conftest import lib_env

pytestmark = pytest.mark.gpu


def ragged_tpe(seed, m, e, empty_frac=0.25):
    rng = np.random.default_rng(seed)
    w = rng.random(e) * (rng.random(e) > empty_frac)
    if w.sum() == 0:
        w[0] = 1.0
    tpe = np.floor(w / w.sum() * m).astype(np.int64)
    tpe[np.argmax(w)] += m - tpe.sum()
    return tpe


def close(got, ref, what):
    got = got.float().cpu()
    ref = ref.float()
    d = (got - ref).abs()
    scale = ref.abs().max().item() or 1.0
    mean_ref = ref.abs().mean().item() or 1.0
    print(f"{what}: max|d|/max|ref| {d.max().item() / scale:.2e}, mean|d| {d.mean().item():.2e}")
    assert d.max().item() <= 1e-2 * scale, what
    assert d.mean().item() <= 2e-3 * mean_ref, what


NT_CASES = [
    # m, n, k, e, dtype, pattern
    (1000, 256, 512, 8, torch.bfloat16, "ragged"),
    (777, 96, 72, 5, torch.bfloat16, "ragged"),
    (300, 200, 136, 4, torch.float16, "ragged"),
    (513, 128, 64, 6, torch.bfloat16, "one"),
    (20000, 1280, 448, 64, torch.bfloat16, "ragged"),
    (8192, 1024, 1536, 64, torch.bfloat16, "ragged"),
    (64, 896, 1280, 64, torch.bfloat16, "ragged"),
    # decode sizes (32-row tiles): every row in one expert, and a ragged spread
    (512, 1024, 1536, 64, torch.bfloat16, "one"),
    (700, 320, 512, 64, torch.float16, "ragged"),
    # decode sizes with K below the 32-row tiles' ring depth (they take the 2-stage 128 x 128 tile)
    (700, 320, 64, 64, torch.bfloat16, "ragged"),
    (900, 256, 128, 64, torch.bfloat16, "ragged"),
    (1000, 512, 192, 64, torch.bfloat16, "one"),
    # 16 to 48 rows per expert (64-row tiles), and the same with K below their ring depth
    (2000, 640, 512, 64, torch.bfloat16, "ragged"),
    (2000, 256, 64, 64, torch.bfloat16, "ragged"),
]


def make_tpe(pattern, seed, m, e):
    if pattern == "one":
        tpe = np.zeros(e, np.int64)
        tpe[e // 2] = m
        return tpe
    return ragged_tpe(seed, m, e)


@pytest.mark.parametrize("m,n,k,e,dtype,pattern", NT_CASES)
def test_grouped_gemm_nt(cuda, m, n, k, e, dtype, pattern):
    tpe = make_tpe(pattern, m + n, m, e)
    a = torch.from_numpy(synth.normal(m, (m, k))).to(dtype)
    w = torch.from_numpy(synth.normal(n, (e, n, k), std=0.05)).to(dtype)
    got = ops.grouped_gemm_nt(a.to(cuda), w.to(cuda), torch.from_numpy(tpe).to(cuda))
    close(got, mo.grouped_linear(a, w, tpe), f"nt {m}x{n}x{k} e{e}")


NN_CASES = [
    (1000, 512, 256, 8, torch.bfloat16, "ragged"),
    (777, 72, 96, 5, torch.bfloat16, "ragged"),
    (300, 136, 200, 4, torch.float16, "ragged"),
    (513, 64, 128, 6, torch.bfloat16, "one"),
    (20000, 448, 1280, 64, torch.bfloat16, "ragged"),
]


@pytest.mark.parametrize("m,n,k,e,dtype,pattern", NN_CASES)
def test_grouped_gemm_nn(cuda, m, n, k, e, dtype, pattern):
    # dgrad shape: grad_out [m, k] times W[e] [k, n]
    tpe = make_tpe(pattern, m + k, m, e)
    g = torch.from_numpy(synth.normal(m + 1, (m, k))).to(dtype)
    w = torch.from_numpy(synth.normal(k + 1, (e, k, n), std=0.05)).to(dtype)
    got = ops.grouped_gemm_nn(g.to(cuda), w.to(cuda), torch.from_numpy(tpe).to(cuda))
    close(got, mo.grouped_linear_dgrad(g, w, tpe), f"nn {m}x{n}x{k} e{e}")


TN_CASES = [
    (1000, 256, 512, 8, torch.bfloat16, "ragged"),
    (777, 96, 72, 5, torch.bfloat16, "ragged"),
    (300, 136, 200, 4, torch.float16, "ragged"),
    (513, 128, 64, 6, torch.bfloat16, "one"),
    (16384, 1024, 1536, 64, torch.bfloat16, "ragged"),
]


@pytest.mark.parametrize("m,na,nb,e,dtype,pattern", TN_CASES)
def test_grouped_gemm_tn(cuda, m, na, nb, e, dtype, pattern):
    tpe = make_tpe(pattern, m + na, m, e)
    g = torch.from_numpy(synth.normal(m + 2, (m, na))).to(dtype)
    a = torch.from_numpy(synth.normal(m + 3, (m, nb))).to(dtype)
    got = ops.grouped_gemm_tn(g.to(cuda), a.to(cuda), torch.from_numpy(tpe).to(cuda))
    ref = mo.grouped_linear_wgrad(g, a, tpe, num_experts=e)
    close(got, ref, f"tn {m}x{na}x{nb} e{e}")
    empty = np.where(tpe == 0)[0]
    if empty.size:
        assert torch.count_nonzero(got[torch.from_numpy(empty).to(cuda)]) == 0


GATHER_TN_CASES = [
    # m, na, nb, e, b_rows, dtype, kernel (HRM_MOE_WGRAD_STAGES: "" picks 256 x 256 where it fits)
    (1000, 256, 512, 8, 300, torch.bfloat16, ""),
    (777, 136, 200, 5, 777, torch.float16, ""),
    (16384, 896, 1280, 64, 2048, torch.bfloat16, ""),
    (16384, 896, 1280, 64, 2048, torch.bfloat16, "2"),
    (4096, 512, 768, 4, 100, torch.bfloat16, ""),
]


@pytest.mark.parametrize("m,na,nb,e,b_rows,dtype,kernel", GATHER_TN_CASES)
def test_grouped_gemm_tn_gather(cuda, m, na, nb, e, b_rows, dtype, kernel):
    """Gathered B rows give exactly the wgrad over the materialised rows (same accumulation order)."""
    tpe = make_tpe("ragged", m + nb, m, e)
    g = torch.from_numpy(synth.normal(m + 5, (m, na))).to(dtype).to(cuda)
    b = torch.from_numpy(synth.normal(m + 6, (b_rows, nb))).to(dtype).to(cuda)
    idx = torch.from_numpy(np.random.default_rng(m).integers(0, b_rows, size=m)).to(torch.int32).to(cuda)
    tpe_d = torch.from_numpy(tpe).to(cuda)
    with lib_env(HRM_MOE_WGRAD_STAGES=kernel):
        got = ops.grouped_gemm_tn_gather(g, b, idx, tpe_d)
        want = ops.grouped_gemm_tn(g, b.index_select(0, idx.long()), tpe_d)
    assert torch.equal(got, want)
    ref = mo.grouped_linear_wgrad(g.cpu(), b.cpu().index_select(0, idx.cpu().long()), tpe, num_experts=e)
    close(got, ref, f"tn_gather {m}x{na}x{nb} e{e}")


def test_grouped_linear_autograd_matches_oracle(cuda):
    m, n, k, e = 3000, 512, 384, 16
    tpe = ragged_tpe(77, m, e)
    a = torch.from_numpy(synth.normal(31, (m, k))).to(torch.bfloat16)
    w = torch.from_numpy(synth.normal(32, (e, n, k), std=0.05)).to(torch.bfloat16)
    g = torch.from_numpy(synth.normal(33, (m, n))).to(torch.bfloat16)
    ag = a.to(cuda).requires_grad_(True)
    wg = w.to(cuda).requires_grad_(True)
    y = hrm_moe_amd.hip_grouped_linear(ag, wg, torch.from_numpy(tpe).to(cuda))
    y.backward(g.to(cuda))
    close(y.detach(), mo.grouped_linear(a, w, tpe), "fwd")
    close(ag.grad, mo.grouped_linear_dgrad(g, w, tpe), "dgrad")
    close(wg.grad, mo.grouped_linear_wgrad(g, a, tpe), "wgrad")
    assert wg.grad.dtype == torch.bfloat16


def test_grouped_gemm_deterministic(cuda):
    m, n, k, e = 4096, 512, 512, 32
    tpe = torch.from_numpy(ragged_tpe(5, m, e)).to(cuda)
    a = torch.from_numpy(synth.normal(41, (m, k))).to(cuda, torch.bfloat16)
    w = torch.from_numpy(synth.normal(42, (e, n, k), std=0.05)).to(cuda, torch.bfloat16)
    y1 = ops.grouped_gemm_nt(a, w, tpe)
    y2 = ops.grouped_gemm_nt(a, w, tpe)
    d1 = ops.grouped_gemm_tn(y1, a, tpe)
    d2 = ops.grouped_gemm_tn(y2, a, tpe)
    assert torch.equal(y1, y2) and torch.equal(d1, d2)


# Row counts on both sides of every 32-row block edge of 128- and 256-row
# tiles, plus empty experts: the last M tile of an expert runs only the row
# blocks that hold rows (down and dgrad kernels).
EDGE_TPE = np.array([1, 31, 32, 33, 0, 63, 64, 65, 95, 96, 97, 127, 128, 129, 0, 159, 191, 223, 255, 256, 257,
                     288, 289, 383, 385, 511, 513], np.int64)


@pytest.mark.parametrize("cfg", ["", "128x128x2x4x64", "256x256x2x8x64"])
def test_grouped_gemm_row_block_edges(cuda, cfg):
    e, m = EDGE_TPE.size, int(EDGE_TPE.sum())
    n, k = 512, 448
    tpe = torch.from_numpy(EDGE_TPE).to(cuda)
    a = torch.from_numpy(synth.normal(11, (m, k))).to(torch.bfloat16)
    w = torch.from_numpy(synth.normal(12, (e, n, k), std=0.05)).to(torch.bfloat16)
    g = torch.from_numpy(synth.normal(13, (m, n))).to(torch.bfloat16)
    with lib_env(HRM_MOE_GEMM_CFG=cfg):
        got = ops.grouped_gemm_nt(a.to(cuda), w.to(cuda), tpe)
        dg = ops.grouped_gemm_nn(g.to(cuda), w.to(cuda), tpe)
    close(got, mo.grouped_linear(a, w, EDGE_TPE), f"nt edges {cfg}")
    close(dg, mo.grouped_linear_dgrad(g, w, EDGE_TPE), f"nn edges {cfg}")
    # the tile shapes accumulate K in the same order: identical bits
    with lib_env(HRM_MOE_GEMM_CFG="128x128x2x4x64"):
        assert torch.equal(got, ops.grouped_gemm_nt(a.to(cuda), w.to(cuda), tpe))
        assert torch.equal(dg, ops.grouped_gemm_nn(g.to(cuda), w.to(cuda), tpe))
