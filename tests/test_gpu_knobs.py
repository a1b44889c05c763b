"""The CU margin on the GPU: a margin set before the library loads shrinks the persistent grids and leaves the
results bit-identical.

A child process starts with HRM_MOE_TRITON_SM_MARGIN (the reference's name,
models/moe_triton_grouped_gemm.py:44-47) set, runs the fused gather + gate_up
GEMM, the down GEMM, dgrad and wgrad, then clears the margin, reloads the
library's configuration and runs them again.  Each workgroup computes whole
tiles with a fixed K order, so the grid size cannot change any bit.
"""
import os
import subprocess
import sys

import pytest

from conftest import ROOT

pytestmark = pytest.mark.gpu

CHILD = r"""
import os, sys, torch
sys.path.insert(0, os.environ["HRM_TEST_ROOT"])
import hrm_moe_amd
from hrm_moe_amd import _lib, ops
lib = _lib.load()
assert lib.hrm_moe_cu_margin() == 200, lib.hrm_moe_cu_margin()
dev = torch.device("cuda:0")
g = torch.Generator(device=dev).manual_seed(5)
t, h, e, i, k = 2048, 1280, 64, 448, 8
x = torch.randn(t, h, device=dev, generator=g).to(torch.bfloat16)
wgu = (torch.randn(e, 2 * i, h, device=dev, generator=g) * 0.02).to(torch.bfloat16)
wdn = (torch.randn(e, h, i, device=dev, generator=g) * 0.02).to(torch.bfloat16)
logits = torch.randn(t, e, device=dev, generator=g).to(torch.bfloat16)
_, w, idx, d = ops.router_topk_dispatch(logits, k, True, torch.bfloat16, want_probs=False)
dy = torch.randn(t * k, h, device=dev, generator=g).to(torch.bfloat16)
def run():
    act = ops.gate_up_swiglu(x, d, wgu)
    y = ops.grouped_gemm_nt(act, wdn, d.tokens_per_expert)
    da = ops.grouped_gemm_nn(dy, wdn, d.tokens_per_expert)
    dw = ops.grouped_gemm_tn(dy, act, d.tokens_per_expert)
    torch.cuda.synchronize()
    return [act, y, da, dw]
with_margin = run()
os.environ["HRM_MOE_TRITON_SM_MARGIN"] = ""
_lib.reload_config()
assert lib.hrm_moe_cu_margin() == 0
without = run()
for name, a, b in zip(("act", "down", "dgrad", "wgrad"), with_margin, without):
    assert torch.equal(a, b), name
print("margin ok", flush=True)
"""


def test_cu_margin_keeps_results(cuda):
    env = dict(os.environ, HRM_MOE_TRITON_SM_MARGIN="200", HRM_TEST_ROOT=ROOT)
    env.pop("HRM_MOE_HIP_CU_MARGIN", None)
    env.pop("XTUNER_SM_MARGIN", None)
    print("child: HRM_MOE_TRITON_SM_MARGIN=200, L-shape GEMMs at 2048 tokens", flush=True)
    r = subprocess.run([sys.executable, "-u", "-c", CHILD], cwd=ROOT, env=env, capture_output=True, text=True,
                       timeout=240)
    print(r.stdout[-2000:], r.stderr[-2000:])
    assert r.returncode == 0 and "margin ok" in r.stdout
