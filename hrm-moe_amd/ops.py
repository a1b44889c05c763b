"""Device ops: torch tensors in, torch tensors out, one C ABI call each.

Each op checks devices, dtypes and shapes on the host, makes its inputs
contiguous, allocates outputs and scratch with torch's caching allocator,
and enqueues the kernel on torch's current stream.  Nothing here reads device
memory on the host, so no op synchronises.  Every op needs its tensors on a
ROCm GPU and raises otherwise: there is no CPU path.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib


def _require_cuda(*tensors: torch.Tensor) -> torch.device:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError("hrm_moe_amd kernels need tensors on a ROCm GPU (got a CPU tensor); there is no CPU path")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} and {t.device}")
    return dev


def _workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=device)


# ---------------------------------------------------------------------------
# Router (models/layers.py:606-610)
# ---------------------------------------------------------------------------

def router_topk(logits: torch.Tensor, top_k: int, norm_topk_prob: bool, weight_dtype: torch.dtype,
                want_probs: bool = True):
    """(probs fp32 [T,E] or None, weights [T,k] weight_dtype, idx int64 [T,k]) from router logits [T,E]."""
    dev = _require_cuda(logits)
    if logits.dim() != 2:
        raise ValueError(f"router logits must be [tokens, experts], got {tuple(logits.shape)}")
    logits = logits.contiguous()
    t, e = logits.shape
    probs = torch.empty((t, e), dtype=torch.float32, device=dev) if want_probs else None
    idx = torch.empty((t, top_k), dtype=torch.int64, device=dev)
    w = torch.empty((t, top_k), dtype=weight_dtype, device=dev)
    with _lib.device_guard(dev):
        st = _lib.lib().hrm_moe_router_topk(
            _lib.ptr(logits), _lib.dtype_code(logits.dtype), t, e, top_k, int(bool(norm_topk_prob)), _lib.ptr(probs),
            _lib.ptr(idx), _lib.ptr(w), _lib.dtype_code(weight_dtype), _lib.stream_of(dev))
    _lib.check(st, "router_topk")
    return probs, w, idx


def gate_wgrad(grad_logits: torch.Tensor, hidden: torch.Tensor) -> torch.Tensor:
    """grad of the gate weight [E,H] = grad_logits[T,E]^T @ hidden[T,H] (split-K, fp32 partials, one rounding)."""
    dev = _require_cuda(grad_logits, hidden)
    t, e = grad_logits.shape
    th, h = hidden.shape
    if th != t:
        raise ValueError(f"gate wgrad: {t} logit rows for {th} hidden rows")
    if grad_logits.dtype != hidden.dtype:
        raise TypeError(f"gate wgrad dtype mismatch: {grad_logits.dtype} vs {hidden.dtype}")
    dt = _gemm_dtype(hidden)
    grad_logits, hidden = grad_logits.contiguous(), hidden.contiguous()
    out = hidden.new_empty((e, h))
    lib = _lib.lib()
    ws = _workspace(lib.hrm_moe_gate_wgrad_workspace_size(t, e, h), dev)
    with _lib.device_guard(dev):
        st = lib.hrm_moe_gate_wgrad(_lib.ptr(grad_logits), _lib.ptr(hidden), t, e, h, dt, _lib.ptr(out),
                                    _lib.ptr(ws), ws.numel(), _lib.stream_of(dev))
    _lib.check(st, "gate_wgrad")
    return out


def router_topk_backward(probs: torch.Tensor, topk_idx: torch.Tensor, grad_weight: torch.Tensor,
                         grad_probs: Optional[torch.Tensor], norm_topk_prob: bool,
                         logits_dtype: torch.dtype) -> torch.Tensor:
    """d logits [T,E] of router_topk, from the grads of its weights [T,k] and (optionally) probs [T,E]."""
    dev = _require_cuda(probs, topk_idx, grad_weight, grad_probs)
    t, e = probs.shape
    k = topk_idx.shape[1]
    if probs.dtype != torch.float32 or (grad_probs is not None and grad_probs.dtype != torch.float32):
        raise TypeError("router backward needs fp32 probabilities and probability grads")
    probs = probs.contiguous()
    topk_idx = topk_idx.to(torch.int64).contiguous()
    grad_weight = grad_weight.contiguous()
    gp_stride = e
    if grad_probs is not None:
        if grad_probs.shape != (t, e):
            raise ValueError(f"grad_probs has shape {tuple(grad_probs.shape)}, expected {(t, e)}")
        if grad_probs.stride() == (0, 1):
            gp_stride = 0  # one row broadcast over the tokens (e.g. the auxiliary loss's gradient): not copied
        else:
            grad_probs = grad_probs.contiguous()
    out = torch.empty((t, e), dtype=logits_dtype, device=dev)
    with _lib.device_guard(dev):
        st = _lib.lib().hrm_moe_router_topk_backward(
            _lib.ptr(probs), _lib.ptr(topk_idx), _lib.ptr(grad_weight), _lib.dtype_code(grad_weight.dtype),
            _lib.ptr(grad_probs), gp_stride, t, e, k, int(bool(norm_topk_prob)), _lib.ptr(out),
            _lib.dtype_code(logits_dtype), _lib.stream_of(dev))
    _lib.check(st, "router_topk_backward")
    return out


def aux_loss(probs: torch.Tensor, tokens_per_expert: torch.Tensor):
    """(aux [] fp32, expert_counts [E] fp32, expert_fraction [E] fp32) of the load-balancing loss.

    aux = (sum_e (tpe[e] / T) * mean_t probs[t, e]) * E (models/layers.py:163-170), in two
    launches with a fixed summation order.
    """
    dev = _require_cuda(probs, tokens_per_expert)
    if probs.dim() != 2 or probs.dtype != torch.float32:
        raise TypeError("aux_loss needs fp32 probabilities [tokens, experts]")
    t, e = probs.shape
    if t < 1:
        raise ValueError("aux_loss needs at least one token")
    probs = probs.contiguous()
    tpe = _tpe64(tokens_per_expert, dev)
    if tpe.numel() != e:
        raise ValueError(f"tokens_per_expert has {tpe.numel()} entries for {e} experts")
    aux = torch.empty((), dtype=torch.float32, device=dev)
    counts = torch.empty(e, dtype=torch.float32, device=dev)
    frac = torch.empty(e, dtype=torch.float32, device=dev)
    lib = _lib.lib()
    ws = _workspace(lib.hrm_moe_aux_loss_workspace_size(t, e), dev)
    with _lib.device_guard(dev):
        st = lib.hrm_moe_aux_loss(_lib.ptr(probs), t, e, _lib.ptr(tpe), _lib.ptr(aux), _lib.ptr(counts),
                                  _lib.ptr(frac), _lib.ptr(ws), ws.numel(), _lib.stream_of(dev))
    _lib.check(st, "aux_loss")
    return aux, counts, frac


def aux_loss_backward(grad_aux: torch.Tensor, expert_fraction: torch.Tensor, num_tokens: int) -> torch.Tensor:
    """d aux / d probs[t, e] for every token: the row ((g * E) * f[e]) * (1 / T), [E] fp32."""
    dev = _require_cuda(grad_aux, expert_fraction)
    grad_aux = grad_aux.to(torch.float32).contiguous()
    e = expert_fraction.numel()
    row = torch.empty(e, dtype=torch.float32, device=dev)
    with _lib.device_guard(dev):
        st = _lib.lib().hrm_moe_aux_loss_backward(_lib.ptr(grad_aux), _lib.ptr(expert_fraction), int(num_tokens), e,
                                                  _lib.ptr(row), _lib.stream_of(dev))
    _lib.check(st, "aux_loss_backward")
    return row


# ---------------------------------------------------------------------------
# Dispatch (models/layers.py:312-322)
# ---------------------------------------------------------------------------

@dataclass
class Dispatch:
    tokens_per_expert: torch.Tensor  # [E] int64
    expert_offsets: torch.Tensor     # [E+1] int32
    sorted_token_idx: torch.Tensor   # [T*k] int32
    slot_to_row: torch.Tensor        # [T*k] int32
    sort_idx: Optional[torch.Tensor]  # [T*k] int64 or None


def permute(topk_idx: torch.Tensor, num_experts: int, want_sort_idx: bool = False) -> Dispatch:
    """Stable expert-major order of the routed slots of ``topk_idx`` [T,k] (int64)."""
    dev = _require_cuda(topk_idx)
    if topk_idx.dim() != 2:
        raise ValueError(f"topk_idx must be [tokens, top_k], got {tuple(topk_idx.shape)}")
    topk_idx = topk_idx.to(torch.int64).contiguous()
    t, k = topk_idx.shape
    r = t * k
    lib = _lib.lib()
    tpe = torch.empty(num_experts, dtype=torch.int64, device=dev)
    offs = torch.empty(num_experts + 1, dtype=torch.int32, device=dev)
    sti = torch.empty(r, dtype=torch.int32, device=dev)
    s2r = torch.empty(r, dtype=torch.int32, device=dev)
    sidx = torch.empty(r, dtype=torch.int64, device=dev) if want_sort_idx else None
    ws_bytes = lib.hrm_moe_permute_workspace_size(t, num_experts, k)
    if ws_bytes == 0:
        _lib.check(_lib.ERR_UNSUPPORTED if num_experts > 1024 else _lib.ERR_INVALID, "permute")
    ws = _workspace(ws_bytes, dev)
    with _lib.device_guard(dev):
        st = lib.hrm_moe_permute(_lib.ptr(topk_idx), t, num_experts, k, _lib.ptr(tpe), _lib.ptr(offs), _lib.ptr(sti),
                                 _lib.ptr(sidx), _lib.ptr(s2r), _lib.ptr(ws), ws.numel(), _lib.stream_of(dev))
    _lib.check(st, "permute")
    return Dispatch(tpe, offs, sti, s2r, sidx)


# ---------------------------------------------------------------------------
# Grouped GEMMs (models/moe_triton_grouped_gemm.py:358-456)
# ---------------------------------------------------------------------------

def _gemm_dtype(t: torch.Tensor) -> int:
    if t.dtype not in (torch.bfloat16, torch.float16):
        raise TypeError(f"HIP grouped GEMM only supports bf16/fp16, got {t.dtype}")
    return _lib.dtype_code(t.dtype)


def _tpe64(tokens_per_expert: torch.Tensor, device: torch.device) -> torch.Tensor:
    return tokens_per_expert.to(device=device, dtype=torch.int64).contiguous()


def grouped_gemm_nt(a: torch.Tensor, w: torch.Tensor, tokens_per_expert: torch.Tensor) -> torch.Tensor:
    """C[M,N] = A[M,K] @ W[e][N,K]^T per expert row group."""
    dev = _require_cuda(a, w)
    m, k = a.shape
    e, n, wk = w.shape
    if wk != k:
        raise ValueError(f"grouped GEMM K mismatch: input K={k}, weight K={wk}")
    if w.dtype != a.dtype:
        raise TypeError(f"grouped GEMM dtype mismatch: input {a.dtype}, weight {w.dtype}")
    dt = _gemm_dtype(a)
    a, w = a.contiguous(), w.contiguous()
    tpe = _tpe64(tokens_per_expert, dev)
    if tpe.numel() != e:
        raise ValueError(f"tokens_per_expert has {tpe.numel()} entries for {e} experts")
    c = a.new_empty((m, n))
    lib = _lib.lib()
    ws = _workspace(lib.hrm_moe_grouped_gemm_workspace_size(m, e), dev)
    with _lib.device_guard(dev):
        st = lib.hrm_moe_grouped_gemm_nt(_lib.ptr(a), _lib.ptr(w), _lib.ptr(tpe), m, n, k, e, dt, _lib.ptr(c),
                                         _lib.ptr(ws), ws.numel(), _lib.stream_of(dev))
    _lib.check(st, "grouped_gemm_nt")
    return c


def grouped_gemm_nn(a: torch.Tensor, w: torch.Tensor, tokens_per_expert: torch.Tensor) -> torch.Tensor:
    """C[M,N] = A[M,K] @ W[e][K,N] per expert row group (dgrad of grouped_gemm_nt)."""
    dev = _require_cuda(a, w)
    m, k = a.shape
    e, wk, n = w.shape
    if wk != k:
        raise ValueError(f"grouped GEMM K mismatch: input K={k}, weight K={wk}")
    if w.dtype != a.dtype:
        raise TypeError(f"grouped GEMM dtype mismatch: input {a.dtype}, weight {w.dtype}")
    dt = _gemm_dtype(a)
    a, w = a.contiguous(), w.contiguous()
    tpe = _tpe64(tokens_per_expert, dev)
    if tpe.numel() != e:
        raise ValueError(f"tokens_per_expert has {tpe.numel()} entries for {e} experts")
    c = a.new_empty((m, n))
    lib = _lib.lib()
    ws = _workspace(lib.hrm_moe_grouped_gemm_workspace_size(m, e), dev)
    with _lib.device_guard(dev):
        st = lib.hrm_moe_grouped_gemm_nn(_lib.ptr(a), _lib.ptr(w), _lib.ptr(tpe), m, n, k, e, dt, _lib.ptr(c),
                                         _lib.ptr(ws), ws.numel(), _lib.stream_of(dev))
    _lib.check(st, "grouped_gemm_nn")
    return c


def grouped_gemm_tn(a: torch.Tensor, b: torch.Tensor, tokens_per_expert: torch.Tensor) -> torch.Tensor:
    """C[e][Na,Nb] = A[rows_e]^T @ B[rows_e] (wgrad); experts without rows get zeros.

    The workspace leaves room for the fp32 partial sums of experts split into
    row chunks (loads above twice the mean), which keeps skewed loads balanced.
    """
    dev = _require_cuda(a, b)
    m, na = a.shape
    mb, nb = b.shape
    if m != mb:
        raise ValueError(f"grouped wgrad K mismatch: A K={m}, B K={mb}")
    if b.dtype != a.dtype:
        raise TypeError(f"grouped wgrad dtype mismatch: {a.dtype} vs {b.dtype}")
    dt = _gemm_dtype(a)
    a, b = a.contiguous(), b.contiguous()
    tpe = _tpe64(tokens_per_expert, dev)
    e = tpe.numel()
    c = a.new_empty((e, na, nb))
    lib = _lib.lib()
    ws = _workspace(lib.hrm_moe_grouped_wgrad_workspace_size(m, na, nb, e), dev)
    with _lib.device_guard(dev):
        st = lib.hrm_moe_grouped_gemm_tn(_lib.ptr(a), _lib.ptr(b), _lib.ptr(tpe), m, na, nb, e, dt, _lib.ptr(c),
                                         _lib.ptr(ws), ws.numel(), _lib.stream_of(dev))
    _lib.check(st, "grouped_gemm_tn")
    return c


def router_topk_dispatch(logits: torch.Tensor, top_k: int, norm_topk_prob: bool, weight_dtype: torch.dtype,
                         want_probs: bool = True, want_sort_idx: bool = False):
    """router_topk then permute, in two launches: (probs or None, weights [T,k], idx [T,k], Dispatch).

    Needs E <= 128 and k <= 8 (the fused rank step); callers fall back to the two ops otherwise.
    """
    dev = _require_cuda(logits)
    if logits.dim() != 2:
        raise ValueError(f"router logits must be [tokens, experts], got {tuple(logits.shape)}")
    logits = logits.contiguous()
    t, e = logits.shape
    r = t * top_k
    probs = torch.empty((t, e), dtype=torch.float32, device=dev) if want_probs else None
    idx = torch.empty((t, top_k), dtype=torch.int64, device=dev)
    w = torch.empty((t, top_k), dtype=weight_dtype, device=dev)
    tpe = torch.empty(e, dtype=torch.int64, device=dev)
    offsets = torch.empty(e + 1, dtype=torch.int32, device=dev)
    sorted_token_idx = torch.empty(r, dtype=torch.int32, device=dev)
    slot_to_row = torch.empty(r, dtype=torch.int32, device=dev)
    sort_idx = torch.empty(r, dtype=torch.int64, device=dev) if want_sort_idx else None
    lib = _lib.lib()
    ws = _workspace(lib.hrm_moe_router_dispatch_workspace_size(t, e, top_k), dev)
    with _lib.device_guard(dev):
        st = lib.hrm_moe_router_topk_dispatch(
            _lib.ptr(logits), _lib.dtype_code(logits.dtype), t, e, top_k, int(bool(norm_topk_prob)), _lib.ptr(probs),
            _lib.ptr(idx), _lib.ptr(w), _lib.dtype_code(weight_dtype), _lib.ptr(tpe), _lib.ptr(offsets),
            _lib.ptr(sorted_token_idx), _lib.ptr(sort_idx), _lib.ptr(slot_to_row), _lib.ptr(ws), ws.numel(),
            _lib.stream_of(dev))
    _lib.check(st, "router_topk_dispatch")
    return probs, w, idx, Dispatch(tpe, offsets, sorted_token_idx, slot_to_row, sort_idx)


def grouped_gemm_tn_gather(a: torch.Tensor, b: torch.Tensor, b_row_index: torch.Tensor,
                           tokens_per_expert: torch.Tensor) -> torch.Tensor:
    """C[e][Na,Nb] = A[rows_e]^T @ B[b_row_index[rows_e]]: wgrad over gathered B rows (B [b_rows, Nb])."""
    dev = _require_cuda(a, b, b_row_index)
    m, na = a.shape
    b_rows, nb = b.shape
    if b_row_index.shape != (m,):
        raise ValueError(f"b_row_index has shape {tuple(b_row_index.shape)}, expected ({m},)")
    if b.dtype != a.dtype:
        raise TypeError(f"grouped wgrad dtype mismatch: {a.dtype} vs {b.dtype}")
    dt = _gemm_dtype(a)
    a, b = a.contiguous(), b.contiguous()
    idx = b_row_index.to(torch.int32).contiguous()
    tpe = _tpe64(tokens_per_expert, dev)
    e = tpe.numel()
    c = a.new_empty((e, na, nb))
    lib = _lib.lib()
    ws = _workspace(lib.hrm_moe_grouped_wgrad_workspace_size(m, na, nb, e), dev)
    with _lib.device_guard(dev):
        st = lib.hrm_moe_grouped_gemm_tn_gather(_lib.ptr(a), _lib.ptr(b), _lib.ptr(idx), b_rows, _lib.ptr(tpe), m, na,
                                                nb, e, dt, _lib.ptr(c), _lib.ptr(ws), ws.numel(), _lib.stream_of(dev))
    _lib.check(st, "grouped_gemm_tn_gather")
    return c


# ---------------------------------------------------------------------------
# Fused expert projections (models/layers.py:318-334)
# ---------------------------------------------------------------------------

def gate_up_swiglu(hidden: torch.Tensor, dispatch: Dispatch, gate_up_weight: torch.Tensor) -> torch.Tensor:
    """act[R,I] = silu(h[tok] @ Wg^T) * (h[tok] @ Wu^T) with the row gather fused into the GEMM."""
    dev = _require_cuda(hidden, gate_up_weight)
    t, h = hidden.shape
    e, two_i, wk = gate_up_weight.shape
    if wk != h or two_i % 2:
        raise ValueError(f"gate_up_weight {tuple(gate_up_weight.shape)} does not match hidden size {h}")
    if gate_up_weight.dtype != hidden.dtype:
        raise TypeError(f"dtype mismatch: hidden {hidden.dtype}, weight {gate_up_weight.dtype}")
    dt = _gemm_dtype(hidden)
    inter = two_i // 2
    hidden, gate_up_weight = hidden.contiguous(), gate_up_weight.contiguous()
    r = dispatch.sorted_token_idx.numel()
    act = hidden.new_empty((r, inter))
    lib = _lib.lib()
    ws = _workspace(lib.hrm_moe_grouped_gemm_workspace_size(r, e), dev)
    with _lib.device_guard(dev):
        st = lib.hrm_moe_gate_up_swiglu(_lib.ptr(hidden), _lib.ptr(dispatch.sorted_token_idx),
                                        _lib.ptr(dispatch.tokens_per_expert), _lib.ptr(gate_up_weight), t, r, h, inter,
                                        e, dt, _lib.ptr(act), _lib.ptr(ws), ws.numel(), _lib.stream_of(dev))
    _lib.check(st, "gate_up_swiglu")
    return act


def combine(expert_out: torch.Tensor, dispatch: Dispatch, topk_weight: Optional[torch.Tensor],
            top_k: Optional[int] = None) -> torch.Tensor:
    """out[t] = sum_j round(expert_out[row(t,j)] * w[t,j]) in fp32, rounded once; [T,H].

    ``topk_weight=None`` (then ``top_k`` is required) means unit weights: the
    plain sum of each token's rows, as the layer's backward un-permutes d(hidden).
    """
    if topk_weight is None:
        if top_k is None:
            raise ValueError("combine without weights needs top_k")
        dev = _require_cuda(expert_out)
        k = int(top_k)
        r, h = expert_out.shape
        if k < 1 or r % k:
            raise ValueError(f"expert_out has {r} rows, not a multiple of top-{k}")
        t = r // k
    else:
        dev = _require_cuda(expert_out, topk_weight)
        t, k = topk_weight.shape
        r, h = expert_out.shape
        if r != t * k:
            raise ValueError(f"expert_out has {r} rows for {t} tokens x top-{k}")
        if topk_weight.dtype != expert_out.dtype:
            raise TypeError(f"dtype mismatch: expert_out {expert_out.dtype}, weights {topk_weight.dtype}")
        topk_weight = topk_weight.contiguous()
    expert_out = expert_out.contiguous()
    e = dispatch.tokens_per_expert.numel()
    out = expert_out.new_empty((t, h))
    with _lib.device_guard(dev):
        st = _lib.lib().hrm_moe_combine(_lib.ptr(expert_out), _lib.ptr(dispatch.slot_to_row), _lib.ptr(topk_weight),
                                         _lib.ptr(dispatch.expert_offsets), t, k, h, e,
                                         _lib.dtype_code(expert_out.dtype), _lib.ptr(out), _lib.stream_of(dev))
    _lib.check(st, "combine")
    return out


def down_combine_decode_ok(act: torch.Tensor, down_weight: torch.Tensor, topk_weight: torch.Tensor) -> bool:
    """Whether down_combine_decode covers this call (its limits in include/hrm_moe.h)."""
    _, h, i = down_weight.shape
    t, k = topk_weight.shape
    return (0 < t <= 2 and k <= 8 and h % 2 == 0 and i % 32 == 0 and i <= 512
            and act.dtype in (torch.bfloat16, torch.float16) and down_weight.dtype == act.dtype
            and topk_weight.dtype == act.dtype)


def down_combine_decode(act: torch.Tensor, down_weight: torch.Tensor, dispatch: Dispatch, topk_idx: torch.Tensor,
                        topk_weight: torch.Tensor) -> torch.Tensor:
    """combine(grouped_gemm_nt(act, down_weight), dispatch, topk_weight) in one launch, for one or two tokens.

    The down projection's dot products are this kernel's own fp32 order (not the GEMM kernels'), then the
    combine's roundings: [T,H].
    """
    dev = _require_cuda(act, down_weight, topk_weight)
    t, k = topk_weight.shape
    e, h, i = down_weight.shape
    if act.shape != (t * k, i):
        raise ValueError(f"act {tuple(act.shape)} for {t} tokens x top-{k} and expert width {i}")
    if not (act.dtype == down_weight.dtype == topk_weight.dtype):
        raise TypeError("down_combine_decode needs one dtype for act, weights and routing weights")
    act, down_weight, topk_weight = act.contiguous(), down_weight.contiguous(), topk_weight.contiguous()
    topk_idx = topk_idx.to(torch.int64).contiguous()
    out = act.new_empty((t, h))
    with _lib.device_guard(dev):
        st = _lib.lib().hrm_moe_down_combine_decode(
            _lib.ptr(act), _lib.ptr(down_weight), _lib.ptr(dispatch.slot_to_row), _lib.ptr(topk_idx),
            _lib.ptr(topk_weight), _lib.ptr(dispatch.expert_offsets), t, k, h, i, e, _lib.dtype_code(act.dtype),
            _lib.ptr(out), _lib.stream_of(dev))
    _lib.check(st, "down_combine_decode")
    return out


def router_gate_up_decode_ok(logits: torch.Tensor, hidden: torch.Tensor, gate_up_weight: torch.Tensor,
                             top_k: int) -> bool:
    """Whether router_gate_up_decode covers this call (its limits in include/hrm_moe.h)."""
    if hidden.dim() != 2 or logits.dim() != 2 or gate_up_weight.dim() != 3:
        return False
    t, h = hidden.shape
    e, i2, h2 = gate_up_weight.shape
    return (hidden.dtype in (torch.bfloat16, torch.float16) and gate_up_weight.dtype == hidden.dtype
            and logits.dtype in _lib.DTYPE_CODE and h2 == h and i2 % 2 == 0 and tuple(logits.shape) == (t, e)
            and bool(_lib.lib().hrm_moe_router_gate_up_decode_supported(t, h, i2 // 2, e, top_k)))


def router_gate_up_decode(logits: torch.Tensor, hidden: torch.Tensor, gate_up_weight: torch.Tensor, top_k: int,
                          norm_topk_prob: bool, want_probs: bool = False, want_sort_idx: bool = False):
    """router_topk_dispatch then gate_up_swiglu, in one launch, for one or two tokens.

    Returns (probs or None, weights [T,k], idx [T,k], Dispatch, act [T*k, I]), the same bits as the two ops;
    down_combine_decode finishes the layer.
    """
    dev = _require_cuda(logits, hidden, gate_up_weight)
    if not router_gate_up_decode_ok(logits, hidden, gate_up_weight, top_k):
        raise ValueError("router_gate_up_decode does not cover this call (see router_gate_up_decode_ok)")
    logits, hidden, gate_up_weight = logits.contiguous(), hidden.contiguous(), gate_up_weight.contiguous()
    t, h = hidden.shape
    e, i2, _ = gate_up_weight.shape
    i = i2 // 2
    r = t * top_k
    probs = torch.empty((t, e), dtype=torch.float32, device=dev) if want_probs else None
    idx = torch.empty((t, top_k), dtype=torch.int64, device=dev)
    w = torch.empty((t, top_k), dtype=hidden.dtype, device=dev)
    tpe = torch.empty(e, dtype=torch.int64, device=dev)
    offsets = torch.empty(e + 1, dtype=torch.int32, device=dev)
    sorted_token_idx = torch.empty(r, dtype=torch.int32, device=dev)
    slot_to_row = torch.empty(r, dtype=torch.int32, device=dev)
    sort_idx = torch.empty(r, dtype=torch.int64, device=dev) if want_sort_idx else None
    act = hidden.new_empty((r, i))
    with _lib.device_guard(dev):
        st = _lib.lib().hrm_moe_router_gate_up_decode(
            _lib.ptr(logits), _lib.dtype_code(logits.dtype), _lib.ptr(hidden), _lib.ptr(gate_up_weight), t, h, i, e,
            top_k, int(bool(norm_topk_prob)), _lib.dtype_code(hidden.dtype), _lib.ptr(probs), _lib.ptr(idx),
            _lib.ptr(w), _lib.ptr(tpe), _lib.ptr(offsets), _lib.ptr(sorted_token_idx), _lib.ptr(sort_idx),
            _lib.ptr(slot_to_row), _lib.ptr(act), _lib.stream_of(dev))
    _lib.check(st, "router_gate_up_decode")
    return probs, w, idx, Dispatch(tpe, offsets, sorted_token_idx, slot_to_row, sort_idx), act


# ---------------------------------------------------------------------------
# Training path: saved gate/up, fused SwiGLU backward, combine backward
# (the quantities torch autograd computes for models/layers.py:317-334)
# ---------------------------------------------------------------------------

def gate_up_swiglu_save(hidden: torch.Tensor, dispatch: Dispatch, gate_up_weight: torch.Tensor):
    """(act [R,I], gate_up [R,2I]): gate_up_swiglu that also returns the rounded gate/up values."""
    dev = _require_cuda(hidden, gate_up_weight)
    t, h = hidden.shape
    e, two_i, wk = gate_up_weight.shape
    if wk != h or two_i % 2:
        raise ValueError(f"gate_up_weight {tuple(gate_up_weight.shape)} does not match hidden size {h}")
    if gate_up_weight.dtype != hidden.dtype:
        raise TypeError(f"dtype mismatch: hidden {hidden.dtype}, weight {gate_up_weight.dtype}")
    dt = _gemm_dtype(hidden)
    inter = two_i // 2
    hidden, gate_up_weight = hidden.contiguous(), gate_up_weight.contiguous()
    r = dispatch.sorted_token_idx.numel()
    act = hidden.new_empty((r, inter))
    gate_up = hidden.new_empty((r, two_i))
    lib = _lib.lib()
    ws = _workspace(lib.hrm_moe_grouped_gemm_workspace_size(r, e), dev)
    with _lib.device_guard(dev):
        st = lib.hrm_moe_gate_up_swiglu_save(_lib.ptr(hidden), _lib.ptr(dispatch.sorted_token_idx),
                                             _lib.ptr(dispatch.tokens_per_expert), _lib.ptr(gate_up_weight), t, r, h,
                                             inter, e, dt, _lib.ptr(act), _lib.ptr(gate_up), _lib.ptr(ws), ws.numel(),
                                             _lib.stream_of(dev))
    _lib.check(st, "gate_up_swiglu_save")
    return act, gate_up


def down_dgrad_swiglu(grad_expert_out: torch.Tensor, down_weight: torch.Tensor, tokens_per_expert: torch.Tensor,
                      gate_up: torch.Tensor) -> torch.Tensor:
    """d(gate_up) [R,2I]: dact = grad @ W_dn[e], then the backward of silu(gate) * up."""
    dev = _require_cuda(grad_expert_out, down_weight, gate_up)
    r, h = grad_expert_out.shape
    e, wh, inter = down_weight.shape
    if wh != h:
        raise ValueError(f"down_weight {tuple(down_weight.shape)} does not match grad width {h}")
    if gate_up.shape != (r, 2 * inter):
        raise ValueError(f"gate_up {tuple(gate_up.shape)} is not [{r}, {2 * inter}]")
    if down_weight.dtype != grad_expert_out.dtype or gate_up.dtype != grad_expert_out.dtype:
        raise TypeError("dtype mismatch between grad, down_weight and gate_up")
    dt = _gemm_dtype(grad_expert_out)
    grad_expert_out, down_weight, gate_up = grad_expert_out.contiguous(), down_weight.contiguous(), gate_up.contiguous()
    tpe = _tpe64(tokens_per_expert, dev)
    if tpe.numel() != e:
        raise ValueError(f"tokens_per_expert has {tpe.numel()} entries for {e} experts")
    out = grad_expert_out.new_empty((r, 2 * inter))
    lib = _lib.lib()
    ws = _workspace(lib.hrm_moe_grouped_gemm_workspace_size(r, e), dev)
    with _lib.device_guard(dev):
        st = lib.hrm_moe_down_dgrad_swiglu(_lib.ptr(grad_expert_out), _lib.ptr(down_weight), _lib.ptr(tpe),
                                           _lib.ptr(gate_up), r, inter, h, e, dt, _lib.ptr(out), _lib.ptr(ws),
                                           ws.numel(), _lib.stream_of(dev))
    _lib.check(st, "down_dgrad_swiglu")
    return out


def combine_backward(grad_out: torch.Tensor, expert_out: torch.Tensor, dispatch: Dispatch,
                     topk_weight: torch.Tensor):
    """(grad_expert_out [R,H], grad_weight [T,k]) of combine(expert_out, dispatch, topk_weight)."""
    dev = _require_cuda(grad_out, expert_out, topk_weight)
    t, k = topk_weight.shape
    r, h = expert_out.shape
    if r != t * k or grad_out.shape != (t, h):
        raise ValueError(f"shapes: grad_out {tuple(grad_out.shape)}, expert_out {tuple(expert_out.shape)}, "
                         f"weights {tuple(topk_weight.shape)}")
    if not (grad_out.dtype == expert_out.dtype == topk_weight.dtype):
        raise TypeError("combine_backward needs one dtype for grad_out, expert_out and weights")
    grad_out, expert_out, topk_weight = grad_out.contiguous(), expert_out.contiguous(), topk_weight.contiguous()
    e = dispatch.tokens_per_expert.numel()
    grad_rows = expert_out.new_empty((r, h))
    grad_w = topk_weight.new_empty((t, k))
    with _lib.device_guard(dev):
        st = _lib.lib().hrm_moe_combine_backward(_lib.ptr(grad_out), _lib.ptr(expert_out),
                                                  _lib.ptr(dispatch.slot_to_row), _lib.ptr(topk_weight),
                                                  _lib.ptr(dispatch.expert_offsets), t, k, h, e,
                                                  _lib.dtype_code(expert_out.dtype), _lib.ptr(grad_rows),
                                                  _lib.ptr(grad_w), _lib.stream_of(dev))
    _lib.check(st, "combine_backward")
    return grad_rows, grad_w
