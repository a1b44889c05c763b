"""CPU restatement of HRM-MoE's routed SwiGLU MoE FFN (grouped_triton path).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, to check results or as the timed CPU baseline.
The product path never calls it.

Every function names the reference lines it follows (paths relative to the
reference repository).  Floating-point arithmetic uses torch on the CPU with
the reference's own ops; the integer work (top-k tie order, stable sort,
histogram) is numpy.

Pinning (what checks each function; tests/test_oracle.py):
  router_topk     top-k order vs torch.topk on ROCm over tie-heavy rows
                  (tests/golden/topk_ties_rocm.npz); softmax vs float64 closed
                  form; C1 golden from the reference module.
  permute         brute-force stable sort and bincount; C1 golden.
  grouped_linear  per-row dot products in float64 (tiny), empty groups,
                  one expert holding every row, M == 0.
  dgrad / wgrad   float64 per-expert products and finite differences of
                  grouped_linear (autograd identity <dC, A W^T> = <dA, ...>).
  swiglu, combine closed forms on tiny inputs; C1 golden.
  moe_forward     C1 golden (fp32, reference imported on CPU), bf16 golden at a
                  small shape, and the per-expert "origin" formulation
                  (models/layers.py:481-515) computed independently.
  experts_vjp     float64 gradients equal those of the independent per-expert
                  formulation and a central finite difference along a random
                  direction; with router_vjp and the aux loss it reproduces the
                  C1 golden's gate-weight and hidden-state gradients.
  router_vjp      the same C1 golden chain; float64 finite differences.
  aux_loss        closed form vs C1 golden.
"""
from __future__ import annotations

from typing import Optional

import numpy as np
import torch
import torch.nn.functional as F

TORCH_TOPK_SORT_SLOTS = 32  # torch sorts top-k results in a 32-slot bitonic network when k <= 32


# ---------------------------------------------------------------------------
# Router: models/layers.py:604-610
# ---------------------------------------------------------------------------

def softmax_fp32(logits: torch.Tensor) -> torch.Tensor:
    """``F.softmax(router_logits, dim=-1, dtype=torch.float32)`` (models/layers.py:606)."""
    return F.softmax(logits, dim=-1, dtype=torch.float32)


def _bitonic_sort_slots(keys: np.ndarray, idx: np.ndarray, valid: np.ndarray):
    """Descending in-place bitonic sort of 32 slots per row, as torch's small sort does it.

    Restates the network torch 2.10 uses to order top-k results on CUDA/ROCm
    (aten/src/ATen/native/cuda/SortUtils.cuh bitonicSortKVInPlace with
    GTOp, called from TensorTopK's sortKeyValueInplace for sort sizes <= 32):
    sizes 2..16 build bitonic runs with direction flag (t & size/2) != 0, then
    a final merge with direction false.  A compare-exchange on slots (a, b)
    computes swap = (a > b and valid[a]) or not valid[b] and exchanges when
    swap == direction, so equal keys are exchanged whenever direction is false.
    That exchange is what makes the order of tied experts differ from a
    stable sort.
    """
    keys, idx, valid = keys.copy(), idx.copy(), valid.copy()
    slots = keys.shape[1]

    def step(stride: int, direction_of):
        for t in range(slots // 2):
            a = 2 * t - (t & (stride - 1))
            b = a + stride
            swap = ((keys[:, a] > keys[:, b]) & valid[:, a]) | ~valid[:, b]
            do = swap == direction_of(t)
            for arr in (keys, idx, valid):
                va, vb = arr[:, a].copy(), arr[:, b].copy()
                arr[:, a] = np.where(do, vb, va)
                arr[:, b] = np.where(do, va, vb)

    size = 2
    while size < slots:
        stride = size // 2
        while stride > 0:
            step(stride, lambda t, s=size: (t & (s // 2)) != 0)
            stride //= 2
        size *= 2
    stride = slots // 2
    while stride > 0:
        step(stride, lambda t: False)
        stride //= 2
    return keys, idx, valid


def topk_rocm(values: np.ndarray, k: int):
    """``torch.topk(values, k, dim=-1)`` (sorted=True) as torch 2.10 computes it on ROCm.

    The reference calls torch.topk on the routing probabilities
    (models/layers.py:607).  Its result for tied values is implementation
    defined; on the device it is (TensorTopK.cu gatherTopK + sort):
      1. the k-th largest value v_k is found;
      2. values > v_k are gathered in ascending index order, then values == v_k
         in ascending index order until k are taken (lowest index wins ties at
         the k boundary);
      3. the k gathered (value, index) pairs are ordered by the 32-slot bitonic
         network of ``_bitonic_sort_slots``.
    Pinned against torch.topk on an MI355X (tests/golden/topk_ties_rocm.npz).
    Returns (values float32 [T,k], indices int64 [T,k]).
    """
    values = np.asarray(values, dtype=np.float32)
    if values.ndim != 2:
        raise ValueError("topk_rocm expects [T, E]")
    t, e = values.shape
    if not 1 <= k <= min(e, TORCH_TOPK_SORT_SLOTS):
        raise NotImplementedError(f"top_k={k} outside 1..min(E, 32)")
    if t == 0:
        return np.zeros((0, k), np.float32), np.zeros((0, k), np.int64)
    cols = np.broadcast_to(np.arange(e), (t, e))
    order = np.lexsort((cols, -values), axis=-1)  # value desc, index asc
    kth = np.take_along_axis(values, order[:, k - 1:k], axis=1)
    selected = np.zeros((t, e), dtype=bool)
    np.put_along_axis(selected, order[:, :k], True, axis=1)
    group = np.where(selected & (values > kth), 0, np.where(selected, 1, 2))
    gathered = np.argsort(group * e + cols, axis=1, kind="stable")[:, :k]
    slots = TORCH_TOPK_SORT_SLOTS
    keys = np.zeros((t, slots), np.float32)
    idx = np.zeros((t, slots), np.int64)
    valid = np.zeros((t, slots), bool)
    keys[:, :k] = np.take_along_axis(values, gathered, 1)
    idx[:, :k] = gathered
    valid[:, :k] = True
    keys, idx, valid = _bitonic_sort_slots(keys, idx, valid)
    assert valid[:, :k].all()
    return keys[:, :k].copy(), idx[:, :k].copy()


def router_topk(logits: torch.Tensor, top_k: int, norm_topk_prob: bool, out_dtype: torch.dtype):
    """Router after the gate GEMM (models/layers.py:606-610).

    probs = softmax(logits) in fp32; (w, idx) = topk(probs, k);
    if norm: w = w / clamp_min(sum_k w, 1e-12) (fp32); w = w.to(out_dtype).
    Returns (probs fp32 [T,E], weights out_dtype [T,k], idx int64 [T,k]).
    """
    probs = softmax_fp32(logits)
    vals, idx = topk_rocm(probs.numpy(), top_k)
    w = torch.from_numpy(vals)
    if norm_topk_prob:
        w = w / w.sum(dim=-1, keepdim=True).clamp_min(1e-12)
    return probs, w.to(out_dtype), torch.from_numpy(idx)


# ---------------------------------------------------------------------------
# Dispatch: models/layers.py:311-322
# ---------------------------------------------------------------------------

def permute(idx, num_experts: int):
    """Stable dispatch of routed slots to expert-contiguous rows (models/layers.py:312-322).

    flat_experts = idx.reshape(-1) (token-major slots t*k + j);
    sort_idx = stable argsort(flat_experts); sorted_token_idx = sort_idx // k;
    tokens_per_expert = bincount(flat_experts, minlength=E).
    Also returns slot_to_row, the inverse permutation (row of slot t*k + j).
    """
    idx = np.asarray(idx, dtype=np.int64)
    t, k = idx.shape
    flat = idx.reshape(-1)
    if flat.size and (flat.min() < 0 or flat.max() >= num_experts):
        raise ValueError("expert index out of range")
    sort_idx = np.argsort(flat, kind="stable").astype(np.int64)
    sorted_experts = flat[sort_idx]
    sorted_token_idx = sort_idx // k
    tpe = np.bincount(flat, minlength=num_experts).astype(np.int64)
    slot_to_row = np.empty_like(sort_idx)
    slot_to_row[sort_idx] = np.arange(sort_idx.size, dtype=np.int64)
    offsets = np.concatenate([[0], np.cumsum(tpe)]).astype(np.int64)
    return dict(sort_idx=sort_idx, sorted_experts=sorted_experts, sorted_token_idx=sorted_token_idx,
                tokens_per_expert=tpe, expert_offsets=offsets, slot_to_row=slot_to_row)


# ---------------------------------------------------------------------------
# Grouped linear: models/moe_triton_grouped_gemm.py:55-65 (CPU), :358-485 (device semantics)
# ---------------------------------------------------------------------------

def _groups(tpe):
    start = 0
    for e, n in enumerate(np.asarray(tpe, dtype=np.int64).tolist()):
        yield e, start, start + int(n)
        start += int(n)


def grouped_linear(inp: torch.Tensor, weight: torch.Tensor, tpe) -> torch.Tensor:
    """out[rows_e] = inp[rows_e] @ weight[e].T, fp32 accumulation, one rounding to inp.dtype.

    Follows ``_torch_grouped_linear`` (moe_triton_grouped_gemm.py:55-65) with the
    device kernel's arithmetic (fp32 accumulator, cast once at the store,
    :175-184).  M == 0 gives ``inp @ weight[0].T`` (:479-480).
    """
    m, k = inp.shape
    e, n, wk = weight.shape
    if wk != k:
        raise ValueError(f"grouped GEMM K mismatch: input K={k}, weight K={wk}")
    acc = torch.promote_types(inp.dtype, torch.float32)  # fp32, or float64 for float64 checks
    out = torch.zeros((m, n), dtype=acc)
    a32 = inp.to(acc)
    w32 = weight.to(acc)
    for g, s, t in _groups(tpe):
        if t > s:
            out[s:t] = a32[s:t] @ w32[g].T
    return out.to(inp.dtype)


def grouped_linear_dgrad(grad_out: torch.Tensor, weight: torch.Tensor, tpe) -> torch.Tensor:
    """grad_input[rows_e] = grad_out[rows_e] @ weight[e] (moe_triton_grouped_gemm.py:472, :187-260)."""
    m, n = grad_out.shape
    e, wn, k = weight.shape
    if wn != n:
        raise ValueError("dgrad N mismatch")
    out = torch.zeros((m, k), dtype=torch.float32)
    g32 = grad_out.float()
    w32 = weight.float()
    for g, s, t in _groups(tpe):
        if t > s:
            out[s:t] = g32[s:t] @ w32[g]
    return out.to(grad_out.dtype)


def grouped_linear_wgrad(grad_out: torch.Tensor, inp: torch.Tensor, tpe, num_experts: Optional[int] = None,
                         out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """grad_weight[e] = grad_out[rows_e].T @ inp[rows_e]; empty expert -> zeros (:420-456, :277-347).

    Returned in fp32 unless ``out_dtype`` is given (the reference stores the
    input dtype, :430).
    """
    tpe = np.asarray(tpe, dtype=np.int64)
    e = num_experts if num_experts is not None else tpe.shape[0]
    n = grad_out.shape[1]
    k = inp.shape[1]
    out = torch.zeros((e, n, k), dtype=torch.float32)
    g32 = grad_out.float()
    a32 = inp.float()
    for g, s, t in _groups(tpe):
        if t > s:
            out[g] = g32[s:t].T @ a32[s:t]
    return out if out_dtype is None else out.to(out_dtype)


# ---------------------------------------------------------------------------
# Expert activation and combine: models/layers.py:327-334
# ---------------------------------------------------------------------------

def swiglu(gate_up: torch.Tensor) -> torch.Tensor:
    """``gate, up = gate_up.chunk(2, -1); F.silu(gate) * up`` in gate_up's dtype (models/layers.py:328-329)."""
    gate, up = gate_up.chunk(2, dim=-1)
    return F.silu(gate) * up


def combine(expert_out: torch.Tensor, sorted_weights: torch.Tensor, sorted_token_idx, num_tokens: int) -> torch.Tensor:
    """``(expert_out * w[:, None])`` then ``zeros.index_add_(0, token, ...)`` (models/layers.py:333-334).

    On the CPU, index_add_ on bf16 accumulates each output row in fp32 in
    ascending source-row order and rounds once.
    """
    weighted = expert_out * sorted_weights[:, None]
    out = torch.zeros((num_tokens, expert_out.shape[1]), dtype=expert_out.dtype)
    out.index_add_(0, torch.as_tensor(np.asarray(sorted_token_idx), dtype=torch.int64), weighted.to(expert_out.dtype))
    return out


# ---------------------------------------------------------------------------
# Whole layer: models/layers.py:596-634 (grouped branch :285-335)
# ---------------------------------------------------------------------------

def moe_forward(x: torch.Tensor, gate_weight: torch.Tensor, gate_up_weight: torch.Tensor, down_weight: torch.Tensor,
                top_k: int, norm_topk_prob: bool = True, intermediates: bool = False,
                logits: Optional[torch.Tensor] = None):
    """SparseMoESwiGLU.forward with the grouped_triton experts, on the CPU.

    Op order (models/layers.py): reshape :602; gate F.linear :605; router
    :606-610; dispatch :312-322; gate_up :326; SwiGLU :328-329; down :331;
    combine :333-334; reshape :634.  All tensors share x's dtype except the
    fp32 probabilities.  ``logits`` replaces the gate GEMM's output when given
    (the GEMM that produced them on a device is the same call the reference
    makes there, so checks start from the device's own logits).
    """
    shape = x.shape
    h = x.reshape(-1, x.shape[-1])
    t = h.shape[0]
    num_experts = gate_weight.shape[0]
    if logits is None:
        logits = F.linear(h, gate_weight)
    probs, w, idx = router_topk(logits, top_k, norm_topk_prob, h.dtype)
    p = permute(idx.numpy(), num_experts)
    flat_w = w.reshape(-1)
    sorted_w = flat_w[torch.from_numpy(p["sort_idx"])]
    sorted_h = h[torch.from_numpy(p["sorted_token_idx"])]
    gu = grouped_linear(sorted_h, gate_up_weight.to(h.dtype), p["tokens_per_expert"])
    act = swiglu(gu)
    y = grouped_linear(act, down_weight.to(h.dtype), p["tokens_per_expert"])
    out = combine(y, sorted_w, p["sorted_token_idx"], t).reshape(shape)
    if not intermediates:
        return out
    return out, dict(logits=logits, probs=probs, weights=w, idx=idx, sorted_weights=sorted_w, gate_up=gu,
                     act=act, expert_out=y, **p)


def moe_forward_origin(x: torch.Tensor, gate_weight: torch.Tensor, gate_up_weight: torch.Tensor,
                       down_weight: torch.Tensor, top_k: int, norm_topk_prob: bool = True) -> torch.Tensor:
    """Per-expert loop formulation (SparseMoEExpertCollection, models/layers.py:497-506, SwiGLU :173-183).

    Independent of ``permute``: for each expert it finds its (token, slot)
    pairs with torch.where, runs the expert on those rows and index_adds the
    weighted result.  Uses the same router as ``moe_forward``.
    """
    shape = x.shape
    h = x.reshape(-1, x.shape[-1])
    logits = F.linear(h, gate_weight)
    _, w, idx = router_topk(logits, top_k, norm_topk_prob, h.dtype)
    out = torch.zeros_like(h)
    for e in range(gate_weight.shape[0]):
        tok, slot = torch.where(idx == e)
        if tok.numel() == 0:
            continue
        gu = (h[tok].float() @ gate_up_weight[e].float().T).to(h.dtype)
        gate, up = gu.chunk(2, dim=-1)
        y = ((F.silu(gate) * up).float() @ down_weight[e].float().T).to(h.dtype)
        out.index_add_(0, tok, (y * w[tok, slot, None]).to(h.dtype))
    return out.reshape(shape)


def router_vjp(logits: torch.Tensor, norm_topk_prob: bool, idx, g_weights: torch.Tensor,
               g_probs: Optional[torch.Tensor] = None) -> torch.Tensor:
    """d logits of softmax(fp32) -> top-k gather -> renormalise (models/layers.py:606-609) by CPU autograd.

    torch.topk's backward scatters the value grads to the selected experts,
    which is what gathering the probabilities at ``idx`` differentiates to.
    ``g_probs`` is the gradient reaching the probabilities directly (the aux
    loss, :619-627).  Returned in the logits' dtype, as softmax(dtype=float32)
    hands its gradient back.
    """
    z = logits.detach().clone().requires_grad_(True)
    p = F.softmax(z, dim=-1, dtype=torch.float32)
    v = p.gather(1, torch.as_tensor(np.asarray(idx), dtype=torch.int64))
    w = v / v.sum(dim=-1, keepdim=True).clamp_min(1e-12) if norm_topk_prob else v
    outs, grads = [w], [g_weights.float()]
    if g_probs is not None:
        outs.append(p)
        grads.append(g_probs.float())
    torch.autograd.backward(outs, grads)
    return z.grad


def experts_vjp(h: torch.Tensor, w: torch.Tensor, gate_up_weight: torch.Tensor, down_weight: torch.Tensor,
                idx, grad_out: torch.Tensor) -> dict:
    """Gradients of the grouped expert block by torch autograd on the CPU (models/layers.py:311-334).

    The forward is the reference's composition in the tensors' dtype: stable
    dispatch (:312-322), index_select of the hidden rows (:320), gate_up
    grouped linear (:326), silu(gate) * up (:328-329), down grouped linear
    (:331), weighting and index_add_ (:333-334); the grouped linears follow
    the device op (fp32 accumulation, one rounding, moe_triton_grouped_gemm.py:
    466-475 for the backward).  Returns d_hidden [T,H], d_weights [T,k],
    d_gate_up_weight, d_down_weight and the forward intermediates.
    """
    h = h.detach().clone().requires_grad_(True)
    w = w.detach().clone().requires_grad_(True)
    wgu = gate_up_weight.detach().clone().requires_grad_(True)
    wdn = down_weight.detach().clone().requires_grad_(True)
    t = h.shape[0]
    p = permute(np.asarray(idx), wgu.shape[0])
    sorted_w = w.reshape(-1)[torch.from_numpy(p["sort_idx"])]
    sorted_h = h.index_select(0, torch.from_numpy(p["sorted_token_idx"]))
    gu = grouped_linear(sorted_h, wgu, p["tokens_per_expert"])
    gu.retain_grad()
    act = swiglu(gu)
    y = grouped_linear(act, wdn, p["tokens_per_expert"])
    y.retain_grad()
    out = combine(y, sorted_w, p["sorted_token_idx"], t)
    out.backward(grad_out.to(out.dtype))
    return dict(out=out.detach(), d_hidden=h.grad, d_weights=w.grad, d_gate_up_weight=wgu.grad,
                d_down_weight=wdn.grad, gate_up=gu.detach(), act=act.detach(), expert_out=y.detach(),
                d_gate_up=gu.grad, d_expert_out=y.grad, **p)


def load_balancing_loss(probs: torch.Tensor, idx: torch.Tensor, num_experts: int) -> torch.Tensor:
    """E * sum_e (count_e / T) * mean_t probs[t, e] (models/layers.py:163-170); divides by T, not T*k."""
    counts = torch.bincount(idx.reshape(-1), minlength=num_experts).to(torch.float32) / idx.shape[0]
    return torch.sum(counts * probs.mean(dim=0)) * num_experts


def expert_counts(idx: torch.Tensor, num_experts: int) -> torch.Tensor:
    """bincount of selected experts as fp32 (models/layers.py:631)."""
    return torch.bincount(idx.reshape(-1), minlength=num_experts).to(torch.float32)


def moe_forward_eager(x: torch.Tensor, gate_weight: torch.Tensor, gate_up_weight: torch.Tensor,
                      down_weight: torch.Tensor, top_k: int, norm_topk_prob: bool = True) -> torch.Tensor:
    """The reference's eager PyTorch CPU path, op for op, for timing as the CPU baseline.

    SparseMoESwiGLU.forward (models/layers.py:596-634) with the grouped_triton
    experts on CPU tensors: torch.topk on the CPU, stable sort + index_select
    dispatch (:311-322), the per-expert F.linear loop of _torch_grouped_linear
    (moe_triton_grouped_gemm.py:55-65) for both projections, then the
    weighted index_add_ (:333-334).  Numerically this is the reference on the
    CPU (its top-k tie order is the CPU one); it is timed, not used to check results.
    """
    shape = x.shape
    h = x.reshape(-1, x.shape[-1])
    t = h.shape[0]
    e = gate_weight.shape[0]
    probs = F.softmax(F.linear(h, gate_weight), dim=-1, dtype=torch.float32)
    w, idx = torch.topk(probs, top_k, dim=-1)
    if norm_topk_prob:
        w = w / w.sum(dim=-1, keepdim=True).clamp_min(1e-12)
    w = w.to(h.dtype)
    flat_e = idx.reshape(-1)
    flat_t = torch.arange(t).repeat_interleave(top_k)
    sorted_e, order = torch.sort(flat_e, stable=True)
    tok = flat_t.index_select(0, order)
    sw = w.reshape(-1).index_select(0, order)
    sh = h.index_select(0, tok)
    tpe = torch.bincount(sorted_e, minlength=e)

    def per_expert_linear(inp, weight):
        outs, start = [], 0
        for ex, n in enumerate(tpe.tolist()):
            if n:
                outs.append(F.linear(inp[start:start + n], weight[ex]))
            start += n
        return torch.cat(outs, dim=0) if outs else inp @ weight[0].T

    gu = per_expert_linear(sh, gate_up_weight)
    gate, up = gu.chunk(2, dim=-1)
    y = per_expert_linear(F.silu(gate) * up, down_weight)
    out = torch.zeros_like(h).index_add_(0, tok, (y * sw[:, None]).to(h.dtype))
    return out.reshape(shape)
