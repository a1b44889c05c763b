"""Dispatch kernel parity on the GPU: bit-exact against the oracle and torch's stable sort.

Replaces models/layers.py:312-322.  Checked: tokens_per_expert (bincount),
expert offsets, the stable permutation (torch.sort(stable=True) indices),
sorted token ids and the inverse permutation; empty experts, one expert
taking every slot, a single token, E up to 1024, ids outside [0, E).
"""
import numpy as np
import pytest
import torch

from hrm_moe_amd import ops
from oracle import moe_oracle as mo
from conftest import lib_env

pytestmark = pytest.mark.gpu


def random_routing(seed, t, e, k, skew=0.0):
    rng = np.random.default_rng(seed)
    if skew > 0:
        p = np.exp(rng.normal(0, skew, size=e))
        p /= p.sum()
    else:
        p = None
    return np.stack([rng.choice(e, size=k, replace=False, p=p) for _ in range(t)]).astype(np.int64)


def check(idx_np, e, cuda):
    idx = torch.from_numpy(idx_np).to(cuda)
    d = ops.permute(idx, e, want_sort_idx=True)
    ref = mo.permute(idx_np, e)
    assert np.array_equal(d.tokens_per_expert.cpu().numpy(), ref["tokens_per_expert"])
    assert np.array_equal(d.expert_offsets.cpu().numpy(), ref["expert_offsets"])
    assert np.array_equal(d.sort_idx.cpu().numpy(), ref["sort_idx"])
    assert np.array_equal(d.sorted_token_idx.cpu().numpy(), ref["sorted_token_idx"])
    assert np.array_equal(d.slot_to_row.cpu().numpy(), ref["slot_to_row"])
    # torch's own stable sort and bincount on the device agree
    se, si = torch.sort(idx.reshape(-1), stable=True)
    assert torch.equal(si, d.sort_idx)
    assert torch.equal(torch.bincount(idx.reshape(-1), minlength=e), d.tokens_per_expert)


@pytest.mark.parametrize("t,e,k,skew", [(4096, 64, 8, 0.0), (16384, 64, 8, 0.0), (4096, 64, 8, 1.5),
                                        (32768, 128, 8, 1.5), (512, 8, 2, 0.0), (1, 64, 8, 0.0),
                                        (100, 1024, 4, 0.0), (3000, 256, 8, 2.5), (7, 3, 3, 0.0)])
def test_permute_matches_oracle(cuda, t, e, k, skew):
    check(random_routing(t * 7 + e, t, e, k, skew), e, cuda)


def test_permute_all_to_one_expert(cuda):
    idx = np.zeros((5000, 1), np.int64)
    idx[:, 0] = 13
    check(idx, 64, cuda)


def test_permute_zero_tokens(cuda):
    d = ops.permute(torch.zeros((0, 8), dtype=torch.int64, device=cuda), 64)
    assert d.tokens_per_expert.cpu().tolist() == [0] * 64
    assert d.expert_offsets.cpu().tolist() == [0] * 65


def test_permute_out_of_range_ids_go_last(cuda):
    rng = np.random.default_rng(3)
    idx = random_routing(4, 1000, 16, 4)
    bad = rng.random(idx.shape) < 0.05
    idx[bad] = np.where(rng.random(bad.sum()) < 0.5, -1, 16)
    d = ops.permute(torch.from_numpy(idx).to(cuda), 16, want_sort_idx=True)
    flat = idx.reshape(-1)
    bucket = np.where((flat >= 0) & (flat < 16), flat, 16)
    order = np.argsort(bucket, kind="stable")
    assert np.array_equal(d.sort_idx.cpu().numpy(), order)
    valid = int((bucket < 16).sum())
    assert d.expert_offsets.cpu().numpy()[-1] == valid
    assert d.tokens_per_expert.sum().item() == valid


@pytest.mark.parametrize("t,e,k,skew", [(1, 64, 8, 0.0), (8, 64, 8, 0.0), (100, 8, 2, 0.0), (4096, 64, 8, 1.5),
                                         (16384, 64, 8, 0.0), (333, 128, 8, 0.0), (1000, 16, 1, 0.0),
                                         (777, 32, 3, 2.0), (2048, 64, 4, 0.0)])
def test_router_dispatch_matches_router_then_permute(cuda, t, e, k, skew):
    """The two-launch router + dispatch gives the bits of router_topk followed by permute."""
    from oracle import synth
    rng = np.random.default_rng(t + e + k)
    logits = torch.from_numpy(rng.standard_normal((t, e)).astype(np.float32) +
                              (rng.standard_normal(e).astype(np.float32) * skew)[None, :]).to(torch.bfloat16)
    lg = logits.to(cuda)
    probs, w, idx, d = ops.router_topk_dispatch(lg, k, True, torch.bfloat16, want_probs=True, want_sort_idx=True)
    probs2, w2, idx2 = ops.router_topk(lg, k, True, torch.bfloat16)
    d2 = ops.permute(idx2, e, want_sort_idx=True)
    assert torch.equal(idx, idx2) and torch.equal(w, w2) and torch.equal(probs, probs2)
    for name in ("tokens_per_expert", "expert_offsets", "sorted_token_idx", "slot_to_row", "sort_idx"):
        assert torch.equal(getattr(d, name), getattr(d2, name)), name
    ref = mo.permute(idx.cpu().numpy(), e)
    assert np.array_equal(d.sort_idx.cpu().numpy(), ref["sort_idx"])


def test_router_dispatch_zero_tokens(cuda):
    lg = torch.zeros((0, 64), dtype=torch.bfloat16, device=cuda)
    _, w, idx, d = ops.router_topk_dispatch(lg, 8, True, torch.bfloat16, want_probs=False)
    assert idx.shape == (0, 8) and int(d.tokens_per_expert.abs().sum()) == 0
    assert int(d.expert_offsets.abs().sum()) == 0


@pytest.mark.parametrize("wave", ["1", "0"])
@pytest.mark.parametrize("t,e,k,ldt,wdt,norm,levels", [
    (1, 64, 8, torch.bfloat16, torch.bfloat16, True, 0), (8, 64, 8, torch.bfloat16, torch.bfloat16, True, 0),
    (16, 64, 8, torch.bfloat16, torch.bfloat16, True, 0), (5, 48, 6, torch.bfloat16, torch.bfloat16, True, 0),
    (3, 8, 2, torch.float32, torch.float32, True, 0), (16, 16, 1, torch.float16, torch.float16, False, 0),
    (7, 64, 4, torch.float32, torch.bfloat16, False, 0), (11, 33, 3, torch.bfloat16, torch.float32, True, 0),
    # exact ties inside and at the edge of the top k
    (16, 64, 8, torch.bfloat16, torch.bfloat16, True, 3), (16, 64, 8, torch.bfloat16, torch.bfloat16, True, 6),
    (9, 64, 5, torch.bfloat16, torch.bfloat16, True, 2), (16, 8, 8, torch.bfloat16, torch.bfloat16, True, 2),
    (12, 64, 2, torch.bfloat16, torch.bfloat16, False, 4), (1, 64, 8, torch.bfloat16, torch.bfloat16, True, 1),
    # 17..64 tokens: the single-block quad kernel; 65..256: the wave kernel in blocks of 16 tokens with the
    # rank step, then scan + scatter (with HRM_MOE_WAVE_ROUTER=0 the quad kernel's blocks of 64)
    (17, 64, 8, torch.bfloat16, torch.bfloat16, True, 0), (64, 64, 8, torch.bfloat16, torch.bfloat16, True, 0),
    (50, 40, 5, torch.float32, torch.float16, True, 0), (64, 64, 8, torch.bfloat16, torch.bfloat16, True, 3),
    (33, 8, 2, torch.bfloat16, torch.bfloat16, False, 2), (63, 64, 7, torch.bfloat16, torch.float32, True, 5),
    (100, 64, 8, torch.bfloat16, torch.bfloat16, True, 0), (256, 64, 8, torch.bfloat16, torch.bfloat16, True, 4),
    (255, 48, 3, torch.float16, torch.bfloat16, True, 0), (200, 64, 8, torch.bfloat16, torch.bfloat16, False, 2),
    (257, 64, 8, torch.bfloat16, torch.bfloat16, True, 0)])
def test_router_dispatch_decode_sizes(cuda, wave, t, e, k, ldt, wdt, norm, levels):
    """Decode and mid token counts (the wave-per-token kernel up to 16 tokens and from 65 to 256, the quad kernel
    otherwise and with the knob off) give the bits of router_topk followed by permute, ties included; the indices
    and weights also equal torch's on the device."""
    rng = np.random.default_rng(1000 * t + 10 * e + k + levels)
    if levels:
        z = rng.integers(0, levels, size=(t, e)).astype(np.float32) * 0.25
    else:
        z = rng.standard_normal((t, e)).astype(np.float32)
    lg = torch.from_numpy(z).to(ldt).to(cuda)
    with lib_env(HRM_MOE_WAVE_ROUTER=wave):
        probs, w, idx, d = ops.router_topk_dispatch(lg, k, norm, wdt, want_probs=True, want_sort_idx=True)
    probs2, w2, idx2 = ops.router_topk(lg, k, norm, wdt)
    d2 = ops.permute(idx2, e, want_sort_idx=True)
    assert torch.equal(idx, idx2) and torch.equal(w.view(-1).float(), w2.view(-1).float())
    assert torch.equal(probs.view(torch.int32), probs2.view(torch.int32))
    for name in ("tokens_per_expert", "expert_offsets", "sorted_token_idx", "slot_to_row", "sort_idx"):
        assert torch.equal(getattr(d, name), getattr(d2, name)), name
    rp = torch.softmax(lg, dim=-1, dtype=torch.float32)
    rw, ri = torch.topk(rp, k, dim=-1)
    if norm:
        rw = rw / rw.sum(dim=-1, keepdim=True).clamp_min(1e-12)
    assert torch.equal(idx, ri), "top-k indices differ from torch.topk on the device"
    assert torch.equal(w.float(), rw.to(wdt).float()), "weights differ from torch on the device"
    assert torch.equal(probs.view(torch.int32), rp.view(torch.int32))
