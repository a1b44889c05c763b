"""The fused auxiliary load-balancing loss against torch's form of it.

load_balancing_loss_func (models/layers.py:163-170) in torch fp32 on the same
device is the reference: the HIP version sums in a different but fixed order,
so the loss agrees to fp32 rounding (relative 1e-6) and repeats bit for bit.
The counts are the dispatch counts as fp32, exactly.  The gradient is checked
against torch autograd of the same function, and it must arrive as a stride-0
row (one row for every token) rather than a [T,E] tensor.
"""
import numpy as np
import pytest
import torch

from hrm_moe_amd import ops
from hrm_moe_amd.layers import _AuxLoss, load_balancing_loss_func
from oracle import synth

pytestmark = pytest.mark.gpu


def _inputs(cuda, t, e, k, seed):
    logits = torch.from_numpy(synth.normal(seed, (t, e))).to(cuda)
    probs = torch.softmax(logits, dim=-1)
    idx = torch.from_numpy(np.argsort(np.random.default_rng(seed).random((t, e)), axis=1)[:, :k]).to(cuda)
    tpe = torch.bincount(idx.reshape(-1), minlength=e)
    return probs, idx, tpe


@pytest.mark.parametrize("t,e,k", [(16384, 64, 8), (1000, 128, 8), (300, 8, 2), (5, 1000, 3), (1, 64, 8)])
def test_aux_loss_matches_torch(cuda, t, e, k):
    probs, idx, tpe = _inputs(cuda, t, e, k, t + e)
    aux, counts, frac = ops.aux_loss(probs, tpe)
    want = load_balancing_loss_func(probs, idx, e, tokens_per_expert=tpe)
    assert aux.dtype == torch.float32 and aux.dim() == 0
    assert abs(aux.item() - want.item()) <= 1e-6 * abs(want.item()) + 1e-7, (aux.item(), want.item())
    assert torch.equal(counts, tpe.to(torch.float32))
    assert torch.equal(frac, tpe.to(torch.float32) / t)  # torch: times the reciprocal of t
    aux2, _, _ = ops.aux_loss(probs, tpe)
    assert torch.equal(aux, aux2)


@pytest.mark.parametrize("t,e,k", [(4096, 64, 8), (333, 128, 4)])
def test_aux_loss_gradient(cuda, t, e, k):
    probs, idx, tpe = _inputs(cuda, t, e, k, 3 * t + e)
    p1 = probs.clone().requires_grad_(True)
    aux, counts = _AuxLoss.apply(p1, tpe)
    g = torch.autograd.grad(aux * 1.7, p1)[0]
    assert g.shape == (t, e) and g.stride() == (0, 1), "the gradient row is not broadcast"
    p2 = probs.clone().requires_grad_(True)
    want = torch.autograd.grad(load_balancing_loss_func(p2, idx, e, tokens_per_expert=tpe) * 1.7, p2)[0]
    assert torch.equal(g.contiguous(), want)  # same expression, same order as torch's backward
    assert not counts.requires_grad
