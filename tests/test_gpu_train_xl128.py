"""Backward of the XL 128x8 shape (H=1536, E=128, I=512, top-8) on the GPU: dgrad and per-expert wgrad.

The reference's backward is _TritonGroupedLinear.backward
(models/moe_triton_grouped_gemm.py:466-475): dgrad by the N-grouped kernel
(:187-260) and wgrad by the K-grouped kernel (:277-347), whose expert loop is
empty for an expert without rows (:341), giving zeros.

Two token counts, 4096 and the full 32768 (262144 routed rows), with the
router's real dispatch of skewed logits: one expert never chosen, one chosen
by most tokens, the rest near-uniform.  Checked:
  * the grouped linear op (hip_grouped_linear forward + autograd backward);
  * each kernel of the fused expert-block backward on its own inputs: down
    wgrad, down dgrad with the SwiGLU backward, gate_up dgrad, gate_up wgrad
    over gathered hidden rows, and the un-permute;
  * the fused block's own gradients equal those kernels' outputs bit for bit.
References: the oracle (fp32 accumulation, one rounding) on a bounded subset
of experts (the heaviest, the empty one, three ordinary ones), and a torch
fp32 per-expert product on the GPU for every expert.  Bar for a GEMM:
max|d| <= 1e-2 max|ref|, mean|d| <= 2e-3 mean|ref|; for the SwiGLU backward
(a rounded chain after the rounded dgrad), max|d| <= 2e-2 max|ref|.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import hrm_moe_amd
from hrm_moe_amd import ops
from hrm_moe_amd.layers import _GroupedExpertsFn
from oracle import moe_oracle as mo

pytestmark = pytest.mark.gpu
BF = torch.bfloat16
H, E, I, K = 1536, 128, 512, 8
EMPTY, HEAVY = 5, 77


def close(got, ref, what, max_tol=1e-2, mean_tol=2e-3):
    got, ref = got.float(), ref.float()
    d = (got - ref).abs()
    scale = ref.abs().max().item() or 1.0
    mean_ref = ref.abs().mean().item() or 1.0
    print(f"{what}: max|d|/max|ref| {d.max().item() / scale:.2e}, mean|d| {d.mean().item():.2e}", flush=True)
    assert d.max().item() <= max_tol * scale, what
    if mean_tol is not None:
        assert d.mean().item() <= mean_tol * mean_ref, what


def _routed(cuda, t, seed):
    g = torch.Generator(device=cuda).manual_seed(seed)
    x = torch.randn(t, H, device=cuda, generator=g).to(BF)
    wg = (torch.randn(E, H, device=cuda, generator=g) * 0.02).to(BF)
    wgu = (torch.randn(E, 2 * I, H, device=cuda, generator=g) * 0.02).to(BF)
    wdn = (torch.randn(E, H, I, device=cuda, generator=g) * 0.02).to(BF)
    logits = F.linear(x, wg)
    logits[:, EMPTY] = -100.0
    logits[:, HEAVY] += 1.5
    _, w, idx, d = ops.router_topk_dispatch(logits, K, True, BF, want_probs=False)
    grad = torch.randn(t, H, device=cuda, generator=g).to(BF)
    return x, w, idx, d, wgu, wdn, grad


def _subset(tpe):
    """(experts, their row ranges): the heaviest, the empty one and three ordinary ones."""
    order = np.argsort(tpe)
    pick = [int(order[-1]), EMPTY, int(order[len(order) // 4]), int(order[len(order) // 2]),
            int(order[3 * len(order) // 4])]
    starts = np.concatenate([[0], np.cumsum(tpe)])
    return sorted(set(pick)), starts


def _sub_rows(t_gpu, experts, starts):
    """Rows of the chosen experts (on the CPU), with their counts, in expert order."""
    parts = [t_gpu[int(starts[e]):int(starts[e + 1])].cpu() for e in experts]
    return torch.cat(parts, 0), np.array([p.shape[0] for p in parts], np.int64)


def _per_expert_fp32(fn, tpe, *tensors):
    """fn(e, rows...) for every expert on the GPU in fp32; results stacked (dgrad rows) or per expert."""
    starts = np.concatenate([[0], np.cumsum(tpe)])
    return [fn(e, *(t[int(starts[e]):int(starts[e + 1])].float() for t in tensors)) for e in range(len(tpe))]


@pytest.mark.parametrize("t", [4096, 32768])
def test_grouped_linear_backward_xl128(cuda, t):
    """hip_grouped_linear (gate_up shape) forward, dgrad and wgrad at the XL 128x8 shape."""
    print(f"case: hip_grouped_linear XL128 T={t} rows={t * K}", flush=True)
    x, w, idx, d, wgu, wdn, _ = _routed(cuda, t, 31)
    tpe = d.tokens_per_expert.cpu().numpy()
    assert tpe[EMPTY] == 0 and tpe.sum() == t * K
    a = x.index_select(0, d.sorted_token_idx.long()).requires_grad_(True)
    wq = wgu.clone().requires_grad_(True)
    y = hrm_moe_amd.hip_grouped_linear(a, wq, d.tokens_per_expert)
    g = torch.randn(y.shape, device=cuda, generator=torch.Generator(device=cuda).manual_seed(32)).to(BF)
    y.backward(g)
    torch.cuda.synchronize()
    experts, starts = _subset(tpe)
    a_s, cnt = _sub_rows(a.detach(), experts, starts)
    g_s, _ = _sub_rows(g, experts, starts)
    w_s = wgu[experts].cpu()
    close(_sub_rows(y.detach(), experts, starts)[0], mo.grouped_linear(a_s, w_s, cnt), f"forward T={t}")
    close(_sub_rows(a.grad, experts, starts)[0], mo.grouped_linear_dgrad(g_s, w_s, cnt), f"dgrad T={t}")
    close(wq.grad[experts].cpu(), mo.grouped_linear_wgrad(g_s, a_s, cnt), f"wgrad T={t} experts {experts}")
    assert torch.count_nonzero(wq.grad[EMPTY]) == 0, "an expert without rows has a zero weight gradient"
    # every expert against a torch fp32 product on the device
    ref_dw = torch.stack(_per_expert_fp32(lambda e, gg, aa: gg.T @ aa, tpe, g, a.detach()))
    close(wq.grad, ref_dw, f"wgrad T={t}, all experts (fp32 on the device)")
    ref_da = torch.cat(_per_expert_fp32(lambda e, gg: gg @ wgu[e].float(), tpe, g), 0)
    close(a.grad, ref_da, f"dgrad T={t}, all rows (fp32 on the device)")


@pytest.mark.parametrize("t", [4096, 32768])
def test_expert_block_backward_xl128(cuda, t):
    """The fused expert-block backward at the XL 128x8 shape, kernel by kernel, then as one autograd function."""
    print(f"case: expert block XL128 T={t} rows={t * K}", flush=True)
    x, w, idx, d, wgu, wdn, grad = _routed(cuda, t, 41)
    tpe_d = d.tokens_per_expert
    tpe = tpe_d.cpu().numpy()
    assert tpe[EMPTY] == 0
    tok = d.sorted_token_idx.long()

    # the kernels the backward runs, one at a time
    act, gate_up = ops.gate_up_swiglu_save(x, d, wgu)
    y = ops.grouped_gemm_nt(act, wdn, tpe_d)
    d_rows, d_w = ops.combine_backward(grad, y, d, w)
    d_dn = ops.grouped_gemm_tn(d_rows, act, tpe_d)
    d_gate_up = ops.down_dgrad_swiglu(d_rows, wdn, tpe_d, gate_up)
    d_h_rows = ops.grouped_gemm_nn(d_gate_up, wgu, tpe_d)
    d_h = ops.combine(d_h_rows, d, None, top_k=K)
    d_gu_w = ops.grouped_gemm_tn_gather(d_gate_up, x, d.sorted_token_idx, tpe_d)
    torch.cuda.synchronize()

    # oracle on a subset of experts, each kernel fed the GPU's own inputs
    experts, starts = _subset(tpe)
    act_s, cnt = _sub_rows(act, experts, starts)
    rows_s, _ = _sub_rows(d_rows, experts, starts)
    gu_s, _ = _sub_rows(gate_up, experts, starts)
    dgu_s, _ = _sub_rows(d_gate_up, experts, starts)
    h_s = _sub_rows(x.index_select(0, tok), experts, starts)[0]
    close(d_dn[experts].cpu(), mo.grouped_linear_wgrad(rows_s, act_s, cnt), f"down wgrad T={t} experts {experts}")
    dact = mo.grouped_linear_dgrad(rows_s, wdn[experts].cpu(), cnt)
    gu_leaf = gu_s.clone().requires_grad_(True)
    mo.swiglu(gu_leaf).backward(dact)
    close(dgu_s, gu_leaf.grad, f"down dgrad + SwiGLU backward T={t}", max_tol=2e-2, mean_tol=None)
    close(_sub_rows(d_h_rows, experts, starts)[0], mo.grouped_linear_dgrad(dgu_s, wgu[experts].cpu(), cnt),
          f"gate_up dgrad T={t}")
    close(d_gu_w[experts].cpu(), mo.grouped_linear_wgrad(dgu_s, h_s, cnt), f"gate_up wgrad T={t}")
    assert torch.count_nonzero(d_dn[EMPTY]) == 0 and torch.count_nonzero(d_gu_w[EMPTY]) == 0

    # every expert against torch fp32 products on the device
    close(d_dn, torch.stack(_per_expert_fp32(lambda e, r, a_: r.T @ a_, tpe, d_rows, act)),
          f"down wgrad T={t}, all experts (fp32 on the device)")
    close(d_gu_w, torch.stack(_per_expert_fp32(lambda e, g_, h_: g_.T @ h_, tpe, d_gate_up, x.index_select(0, tok))),
          f"gate_up wgrad T={t}, all experts (fp32 on the device)")
    close(d_h_rows, torch.cat(_per_expert_fp32(lambda e, g_: g_ @ wgu[e].float(), tpe, d_gate_up), 0),
          f"gate_up dgrad T={t}, all rows (fp32 on the device)")
    # un-permute: each token's k rows summed in fp32, once rounded
    ref_dh = torch.zeros(t, H, device=cuda).index_add_(0, tok, d_h_rows.float())
    close(d_h, ref_dh, f"un-permute T={t}", max_tol=1e-2, mean_tol=None)

    # the fused autograd function returns exactly those kernels' results
    leaves = [a.clone().requires_grad_(True) for a in (x, w, wgu, wdn)]
    out = _GroupedExpertsFn.apply(*leaves, d)
    out.backward(grad)
    torch.cuda.synchronize()
    for name, got, want in (("d_hidden", leaves[0].grad, d_h), ("d_weights", leaves[1].grad, d_w),
                            ("d_gate_up_weight", leaves[2].grad, d_gu_w), ("d_down_weight", leaves[3].grad, d_dn)):
        assert torch.equal(got, want), name
    assert torch.equal(out, ops.combine(y, d, w))
