"""Router kernel parity on the GPU.

The reference's router (models/layers.py:605-610) runs torch's softmax and
topk on the device that holds the activations.  The kernel must reproduce
both bit for bit from the same logits: probabilities, top-k indices (tie
order included) and the normalised, cast weights.  The oracle's top-k
(oracle/moe_oracle.py:topk_rocm) must agree as well.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from hrm_moe_amd import ops
from oracle import moe_oracle as mo
from oracle import synth

pytestmark = pytest.mark.gpu


def torch_router(logits, k, norm, dtype):
    probs = F.softmax(logits, dim=-1, dtype=torch.float32)
    w, idx = torch.topk(probs, k, dim=-1)
    if norm:
        w = w / w.sum(dim=-1, keepdim=True).clamp_min(1e-12)
    return probs, w.to(dtype), idx


def make_logits(seed, t, e, dtype, dev, scale=1.0, levels=0):
    if levels:
        rng = np.random.default_rng(seed)
        z = rng.integers(0, levels, size=(t, e)).astype(np.float32) * 0.25
    else:
        z = synth.normal(seed, (t, e), std=scale)
    return torch.from_numpy(z).to(dev).to(dtype)


CASES = [
    # t, e, k, logits dtype, weight dtype, norm, scale, levels
    (4096, 64, 8, torch.bfloat16, torch.bfloat16, True, 0.8, 0),
    (4096, 128, 8, torch.bfloat16, torch.bfloat16, True, 0.8, 0),
    (2048, 8, 2, torch.bfloat16, torch.bfloat16, True, 0.8, 0),
    (1000, 64, 4, torch.float32, torch.float32, True, 1.0, 0),
    (513, 64, 8, torch.float16, torch.float16, True, 1.0, 0),
    (300, 16, 3, torch.bfloat16, torch.bfloat16, True, 1.0, 0),
    (200, 128, 16, torch.bfloat16, torch.bfloat16, True, 1.0, 0),
    (64, 64, 32, torch.bfloat16, torch.bfloat16, True, 1.0, 0),
    (777, 64, 8, torch.bfloat16, torch.bfloat16, False, 1.0, 0),
    # exact ties everywhere
    (2048, 64, 8, torch.bfloat16, torch.bfloat16, True, 0, 4),
    (1024, 128, 8, torch.bfloat16, torch.bfloat16, True, 0, 6),
    (1024, 8, 2, torch.bfloat16, torch.bfloat16, True, 0, 3),
    (512, 64, 6, torch.bfloat16, torch.bfloat16, True, 0, 5),
    # more than 128 experts: one wave per token, torch's warp-softmax layout
    (1024, 256, 8, torch.bfloat16, torch.bfloat16, True, 0.8, 0),
    (500, 200, 8, torch.bfloat16, torch.bfloat16, True, 1.0, 0),
    (300, 512, 8, torch.float32, torch.float32, True, 1.0, 0),
    (257, 1024, 8, torch.bfloat16, torch.bfloat16, True, 1.0, 0),
    (200, 640, 3, torch.float16, torch.float16, False, 1.0, 0),
    (128, 384, 16, torch.bfloat16, torch.bfloat16, True, 1.0, 0),
    (64, 1000, 32, torch.bfloat16, torch.bfloat16, True, 1.0, 0),
    (512, 256, 8, torch.bfloat16, torch.bfloat16, True, 0, 5),
    (256, 1024, 8, torch.bfloat16, torch.bfloat16, True, 0, 7),
    (256, 300, 2, torch.bfloat16, torch.bfloat16, True, 0, 3),
]


@pytest.mark.parametrize("t,e,k,ldt,wdt,norm,scale,levels", CASES)
def test_router_bit_exact_vs_torch_on_device(cuda, t, e, k, ldt, wdt, norm, scale, levels):
    logits = make_logits(t * 131 + e, t, e, ldt, cuda, scale, levels)
    probs, w, idx = ops.router_topk(logits, k, norm, wdt)
    rp, rw, ridx = torch_router(logits, k, norm, wdt)
    torch.cuda.synchronize()
    assert torch.equal(probs.view(torch.int32), rp.view(torch.int32)), "probabilities differ from torch's softmax"
    assert torch.equal(idx, ridx), f"indices differ in {(idx != ridx).any(-1).sum().item()} rows"
    wb = w.view(torch.int16) if w.dtype != torch.float32 else w.view(torch.int32)
    rb = rw.view(torch.int16) if rw.dtype != torch.float32 else rw.view(torch.int32)
    assert torch.equal(wb, rb), f"weights differ in {(wb != rb).sum().item()} entries"
    # the oracle's tie rule agrees
    _, oidx = mo.topk_rocm(probs.cpu().numpy(), k)
    assert np.array_equal(oidx, idx.cpu().numpy())


def test_router_l_scale_from_gate_gemm(cuda):
    """L config router: 16384 tokens, H=1280, E=64, top-8, bf16 logits from the gate GEMM."""
    x = torch.from_numpy(synth.normal(21, (16384, 1280))).to(cuda, torch.bfloat16)
    wg = torch.from_numpy(synth.normal(22, (64, 1280), std=0.02)).to(cuda, torch.bfloat16)
    logits = F.linear(x, wg)
    probs, w, idx = ops.router_topk(logits, 8, True, torch.bfloat16)
    rp, rw, ridx = torch_router(logits, 8, True, torch.bfloat16)
    torch.cuda.synchronize()
    top = torch.sort(logits.float(), -1, descending=True).values[:, :9]
    ties = (top[:, 1:] == top[:, :-1]).any(-1).float().mean().item()
    print(f"tokens with a tie inside the top-9: {ties:.3f}")
    assert torch.equal(idx, ridx)
    assert torch.equal(probs, rp)
    assert torch.equal(w.view(torch.int16), rw.view(torch.int16))


def test_router_without_probs_output(cuda):
    logits = make_logits(5, 100, 64, torch.bfloat16, cuda)
    probs, w, idx = ops.router_topk(logits, 8, True, torch.bfloat16, want_probs=False)
    _, rw, ridx = torch_router(logits, 8, True, torch.bfloat16)
    assert probs is None
    assert torch.equal(idx, ridx) and torch.equal(w, rw)


def test_router_zero_tokens(cuda):
    probs, w, idx = ops.router_topk(torch.empty(0, 64, device=cuda, dtype=torch.bfloat16), 8, True, torch.bfloat16)
    assert idx.shape == (0, 8) and w.shape == (0, 8)


@pytest.mark.parametrize("t,e,k,norm,with_gp", [
    (300, 8, 2, True, True), (1000, 64, 8, True, True), (513, 128, 8, True, False),
    (257, 64, 4, False, True), (64, 16, 16, True, True),
    (300, 256, 8, True, True), (129, 1024, 8, True, True), (200, 600, 4, False, False),
])
def test_router_backward_matches_oracle(cuda, t, e, k, norm, with_gp):
    """d logits of the router kernel vs CPU autograd of softmax -> gather -> renormalise (oracle.router_vjp)."""
    from oracle import moe_oracle as mo
    from oracle import synth
    logits = torch.from_numpy(synth.normal(t + e, (t, e))).to(torch.bfloat16)
    probs, _, idx = ops.router_topk(logits.to(cuda), k, norm, torch.bfloat16)
    gw = torch.from_numpy(synth.normal(t + 1, (t, k))).to(torch.bfloat16)
    gp = torch.from_numpy(synth.normal(t + 2, (t, e), std=0.1)) if with_gp else None
    got = ops.router_topk_backward(probs, idx, gw.to(cuda), gp.to(cuda) if gp is not None else None, norm,
                                   torch.bfloat16)
    ref = mo.router_vjp(logits, norm, idx.cpu().numpy(), gw, gp)
    assert got.dtype == torch.bfloat16 and got.shape == (t, e)
    d = (got.float().cpu() - ref.float()).abs()
    rel = d.max().item() / ref.float().abs().max().item()
    print(f"router backward E={e} k={k}: max rel err {rel:.3e}, mean abs err {d.mean().item():.3e}")
    assert rel <= 1e-2
    again = ops.router_topk_backward(probs, idx, gw.to(cuda), gp.to(cuda) if gp is not None else None, norm,
                                     torch.bfloat16)
    assert torch.equal(got, again)


@pytest.mark.parametrize("t,e,k", [(1000, 64, 8), (300, 128, 4)])
def test_router_backward_broadcast_prob_grad(cuda, t, e, k):
    """A probability gradient that is one row for every token (stride 0, as the auxiliary loss's)
    gives the bits of the same gradient materialised as a [T,E] tensor."""
    from oracle import synth
    logits = torch.from_numpy(synth.normal(t + 5, (t, e))).to(torch.bfloat16).to(cuda)
    probs, _, idx = ops.router_topk(logits, k, True, torch.bfloat16)
    gw = torch.from_numpy(synth.normal(t + 6, (t, k))).to(torch.bfloat16).to(cuda)
    row = torch.from_numpy(synth.normal(t + 7, (e,), std=0.01)).to(cuda)
    bcast = row.unsqueeze(0).expand(t, e)
    assert bcast.stride() == (0, 1)
    got = ops.router_topk_backward(probs, idx, gw, bcast, True, torch.bfloat16)
    want = ops.router_topk_backward(probs, idx, gw, bcast.contiguous(), True, torch.bfloat16)
    assert torch.equal(got, want)


@pytest.mark.parametrize("t,e,h", [(16384, 64, 1280), (512, 8, 256), (1000, 128, 1536), (100, 16, 264),
                                   (40000, 64, 1536)])
def test_gate_wgrad_matches_fp32_product(cuda, t, e, h):
    """Split-K router gate weight gradient vs one fp32 product rounded once (the F.linear weight grad)."""
    from oracle import synth
    dz = torch.from_numpy(synth.normal(t + e, (t, e), std=0.1)).to(torch.bfloat16)
    x = torch.from_numpy(synth.normal(t + h, (t, h))).to(torch.bfloat16)
    got = ops.gate_wgrad(dz.to(cuda), x.to(cuda))
    ref = (dz.float().T @ x.float())
    d = (got.float().cpu() - ref).abs()
    rel = d.max().item() / ref.abs().max().item()
    print(f"gate wgrad T={t} E={e} H={h}: max rel err {rel:.3e}")
    assert got.shape == (e, h) and rel <= 1e-2
    assert torch.equal(got, ops.gate_wgrad(dz.to(cuda), x.to(cuda))), "not deterministic"
