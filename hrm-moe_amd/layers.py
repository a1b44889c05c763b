"""Drop-in MoE FFN module for HRM-MoE's ``grouped_triton`` path on gfx950.

``SparseMoESwiGLU`` keeps the constructor, parameter names and shapes, forward
signature and ``moe_context`` side effects of the reference module
(models/layers.py:518-634), so configs and checkpoints written for
``implementation: grouped_triton`` load unchanged.

Forward paths (same arithmetic, same routing bits):
  * no autograd needed (inference, ``torch.no_grad()``, or nothing requires
    grad): router kernel -> dispatch kernel -> fused gather + gate_up GEMM +
    SwiGLU -> down GEMM -> deterministic combine.  Five HIP launches plus the
    gate GEMM; no host synchronisation.  Any hidden size that is a multiple
    of 8.  A decode step of one or two tokens (within the limits of
    ops.router_gate_up_decode_ok and ops.down_combine_decode_ok) runs the
    router, dispatch and gate_up in one launch and the down GEMM and combine
    in a second, with the same bits.
  * autograd needed: the same forward kernels (the gate/up kernel also saving
    the rounded gate/up values) inside one autograd function whose backward
    is HIP too: combine backward, down dgrad with the SwiGLU backward fused,
    both wgrads, gate_up dgrad and a deterministic un-permute; the router's
    softmax/top-k backward and the aux loss are HIP kernels as well.  The
    fused training kernels stream hidden rows 64 values at a time, so this
    path needs a hidden size that is a multiple of 64 and raises
    NotImplementedError otherwise.
"""
from __future__ import annotations

import math
from typing import Any, Optional, Sequence

import torch
import torch.nn.functional as F
from torch import Tensor, nn

from . import ops
from .profile import record_moe_profile_phase


def trunc_normal_init_(tensor: Tensor, std: float = 1.0) -> Tensor:
    """The reference's approximate truncated normal (models/common.py:10-13): N(0,1) folded into (-3, 3)
    by fmod, rescaled so the standard deviation is ``std``."""
    return tensor.normal_().fmod_(3.0).mul_(1.014762601732121 * std)


def unwrap_tensor(value):
    """Tensor or a wrapper with ``.value`` (models/common.py:26-32)."""
    return getattr(value, "value", value)


class LinearInit(nn.Module):
    """Bias-free linear with truncated LeCun-normal init (models/layers.py:65-90)."""

    def __init__(self, in_features: int, out_features: int, bias: bool, batch_out_features: Sequence[int] = (),
                 init_std: Optional[float] = None, **kwargs):
        super().__init__()
        self.in_features = in_features
        if init_std is None:
            init_std = 1.0 / (in_features ** 0.5)
        self.weight = nn.Parameter(trunc_normal_init_(
            torch.empty((math.prod(batch_out_features) * out_features, in_features), **kwargs), std=init_std))
        self.bias = None
        if bias:
            self.bias = nn.Parameter(torch.zeros((math.prod(batch_out_features) * out_features,), **kwargs))

    def forward(self, input: Tensor) -> Tensor:
        return F.linear(input, self.weight, self.bias)


def load_balancing_loss_func(routing_weights: Tensor, selected_experts: Tensor, num_experts: int,
                             tokens_per_expert: Optional[Tensor] = None) -> Tensor:
    """Qwen-style auxiliary load-balancing loss (models/layers.py:163-170).

    ``tokens_per_expert`` may pass in the dispatch kernel's counts, which equal
    ``bincount(selected_experts, minlength=num_experts)``; bincount on the
    device would first synchronise with the host to size its output.
    """
    if tokens_per_expert is None:
        tokens_per_expert = torch.bincount(selected_experts.reshape(-1), minlength=num_experts)
    tokens_per_expert = tokens_per_expert.to(torch.float32) / selected_experts.shape[0]
    router_prob_per_expert = routing_weights.mean(dim=0)
    return torch.sum(tokens_per_expert * router_prob_per_expert) * num_experts


_ONE_GROUP: dict = {}


def _one_group_counts(rows: int, device: torch.device) -> Tensor:
    """tokens_per_expert = [rows] on the device, cached so the backward launches no copy for it."""
    key = (rows, device)
    t = _ONE_GROUP.get(key)
    if t is None:
        if len(_ONE_GROUP) > 64:
            _ONE_GROUP.clear()
        t = _ONE_GROUP[key] = torch.tensor([rows], dtype=torch.int64, device=device)
    return t


class _GateLinear(torch.autograd.Function):
    """The router gate ``F.linear(h, W)`` (models/layers.py:605, :89-90) with a HIP weight gradient.

    Forward is the same F.linear call, so the logits are the same bits.  The
    backward's input grad is ``dlogits @ W`` (a one-group HIP grouped GEMM); the weight grad ``dlogits^T @ h``
    (one long reduction over the tokens into a small [E,H] output) runs as a
    split-K HIP kernel with fp32 partials.
    """

    @staticmethod
    def forward(ctx, hidden: Tensor, weight: Tensor):
        ctx.save_for_backward(hidden, weight)
        return F.linear(hidden, weight)

    @staticmethod
    def backward(ctx, grad_logits: Tensor):
        hidden, weight = ctx.saved_tensors
        grad_logits = grad_logits.to(hidden.dtype).contiguous()
        d_hidden = None
        if ctx.needs_input_grad[0]:
            # dlogits [T,E] . W [E,H] as a one-group NN grouped GEMM (K = E): at T = 16384,
            # E = 64, H = 1280 it takes 15 us against 26 us for the hipBLASLt matmul
            t = grad_logits.shape[0]
            d_hidden = ops.grouped_gemm_nn(grad_logits, weight.unsqueeze(0), _one_group_counts(t, hidden.device))
        d_weight = None
        if ctx.needs_input_grad[1]:
            d_weight = ops.gate_wgrad(grad_logits, hidden).to(weight.dtype)
        return d_hidden, d_weight


class _RouterTopK(torch.autograd.Function):
    """Router kernel with the gradient of softmax -> top-k gather -> renormalise -> cast.

    Forward and backward are one HIP launch each (models/layers.py:606-610):
      dv  = dw / c - <dw, v> / c^2 * [s >= 1e-12],  c = max(s, 1e-12), s = sum(v)
      dp  = dprobs + scatter(idx, dv)
      dz  = p * (dp - <p, dp>)
    """

    @staticmethod
    def forward(ctx, logits: Tensor, top_k: int, norm_topk_prob: bool, out_dtype: torch.dtype):
        """(probs, weights, idx, tokens_per_expert, expert_offsets, sorted_token_idx, slot_to_row).

        The dispatch tensors come from the router's fused dispatch when E <= 128
        and k <= 8, else from the permute kernel.
        """
        if logits.shape[1] <= 128 and top_k <= 8:
            probs, w, idx, d = ops.router_topk_dispatch(logits, top_k, norm_topk_prob, out_dtype, want_probs=True)
        else:
            probs, w, idx = ops.router_topk(logits, top_k, norm_topk_prob, out_dtype, want_probs=True)
            d = ops.permute(idx, logits.shape[1])
        ctx.save_for_backward(probs, idx)
        ctx.norm = norm_topk_prob
        ctx.logits_dtype = logits.dtype
        extra = (d.tokens_per_expert, d.expert_offsets, d.sorted_token_idx, d.slot_to_row)
        ctx.mark_non_differentiable(idx, *extra)
        # outputs without a gradient arrive as None, not as zero tensors that
        # autograd would fill (five fill launches for the integer outputs)
        ctx.set_materialize_grads(False)
        return (probs, w, idx) + extra

    @staticmethod
    def backward(ctx, g_probs, g_w, _g_idx, *_g_dispatch):
        probs, idx = ctx.saved_tensors
        if g_w is None:
            g_w = torch.zeros(idx.shape, dtype=torch.float32, device=probs.device)
        g_probs = None if g_probs is None else g_probs.float()
        dz = ops.router_topk_backward(probs, idx, g_w, g_probs, ctx.norm, ctx.logits_dtype)
        return dz, None, None, None


class _AuxLoss(torch.autograd.Function):
    """load_balancing_loss_func and the expert counts as two HIP launches (models/layers.py:163-170, :619-632).

    The loss's gradient is the same row for every token, ((g * E) * f[e]) * (1 / T);
    it is returned as a stride-0 view, which the router backward reads as one
    row instead of a [T,E] tensor.
    """

    @staticmethod
    def forward(ctx, probs: Tensor, tokens_per_expert: Tensor):
        aux, counts, frac = ops.aux_loss(probs, tokens_per_expert)
        ctx.save_for_backward(frac)
        ctx.num_tokens = probs.shape[0]
        ctx.mark_non_differentiable(counts)
        ctx.set_materialize_grads(False)
        return aux, counts

    @staticmethod
    def backward(ctx, g_aux, _g_counts):
        if g_aux is None:
            return None, None
        (frac,) = ctx.saved_tensors
        row = ops.aux_loss_backward(g_aux, frac, ctx.num_tokens)
        return row.unsqueeze(0).expand(ctx.num_tokens, row.numel()), None


class _GroupedExpertsFn(torch.autograd.Function):
    """Grouped expert block (models/layers.py:317-334) with a HIP backward.

    Forward: gather + gate_up GEMM + SwiGLU (saving the rounded gate/up values),
    down GEMM, combine.  Backward, with the reference's rounding points:
      combine backward   -> d_rows = round(dout[tok] * w), d_w = sum_h round(dout * rows)
      down dgrad + SwiGLU backward (one kernel) -> d(gate_up)
      down wgrad         -> dW_dn[e] = d_rows_e^T . act_e
      gate_up dgrad      -> d_h_rows = d(gate_up) . W_gu[e]
      un-permute         -> d_h[t] = sum over the token's rows (combine with unit weights,
                            fp32 in row order: deterministic, unlike index_add_ on the device)
      gate_up wgrad      -> dW_gu[e] = d(gate_up)_e^T . h[tok]_e, the rows gathered by the kernel's DMA
    """

    @staticmethod
    def forward(ctx, hidden: Tensor, routing_weights: Tensor, gate_up_weight: Tensor, down_weight: Tensor,
                d: "ops.Dispatch"):
        act, gate_up = ops.gate_up_swiglu_save(hidden, d, gate_up_weight)
        y = ops.grouped_gemm_nt(act, down_weight, d.tokens_per_expert)
        out = ops.combine(y, d, routing_weights)
        ctx.save_for_backward(hidden, routing_weights, gate_up_weight, down_weight, act, gate_up, y)
        ctx.d = d
        return out

    @staticmethod
    def backward(ctx, grad_out: Tensor):
        hidden, routing_weights, gate_up_weight, down_weight, act, gate_up, y = ctx.saved_tensors
        d = ctx.d
        tpe = d.tokens_per_expert
        need_h, need_w, need_gu, need_dn = ctx.needs_input_grad[:4]
        grad_out = grad_out.to(hidden.dtype).contiguous()
        d_rows, d_w = ops.combine_backward(grad_out, y, d, routing_weights)
        d_dn = ops.grouped_gemm_tn(d_rows, act, tpe) if need_dn else None
        d_h = d_gu_w = None
        if need_h or need_gu:
            d_gate_up = ops.down_dgrad_swiglu(d_rows, down_weight, tpe, gate_up)
            if need_h:
                d_h_rows = ops.grouped_gemm_nn(d_gate_up, gate_up_weight, tpe)
                d_h = ops.combine(d_h_rows, d, None, top_k=routing_weights.shape[1])
            if need_gu:
                d_gu_w = ops.grouped_gemm_tn_gather(d_gate_up, hidden, d.sorted_token_idx, tpe)
        return d_h, (d_w if need_w else None), d_gu_w, d_dn, None


class SparseMoEGroupedExperts(nn.Module):
    """Expert weights and compute (models/layers.py:248-357, grouped branch).

    Parameters: ``gate_up_weight`` [E, 2I, H] (gate rows 0..I-1, up rows
    I..2I-1) and ``down_weight`` [E, H, I].
    """

    # hidden sizes the fused training kernels accept (they stream K 64 values at a time)
    TRAIN_HIDDEN_MULTIPLE = 64

    def __init__(self, hidden_size: int, intermediate_size: int, num_experts: int, backend: str = "hip",
                 init_std_in=None, init_std_out=None, **kwargs):
        super().__init__()
        if num_experts <= 0:
            raise ValueError(f"num_experts must be positive, got {num_experts}")
        if backend not in ("hip", "triton"):
            raise ValueError(f"Unsupported grouped MoE backend: {backend}; hrm_moe_amd provides the HIP kernels only")
        if init_std_in is None:
            init_std_in = 1.0 / (hidden_size ** 0.5)
        if init_std_out is None:
            init_std_out = 1.0 / (intermediate_size ** 0.5)
        self.num_experts = num_experts
        self.expert_in_one_shard = num_experts
        self.backend = "hip"
        self.gate_up_weight = nn.Parameter(trunc_normal_init_(
            torch.empty((num_experts, 2 * intermediate_size, hidden_size), **kwargs), std=init_std_in))
        self.down_weight = nn.Parameter(trunc_normal_init_(
            torch.empty((num_experts, hidden_size, intermediate_size), **kwargs), std=init_std_out))

    def _needs_autograd(self, hidden_states: Tensor, routing_weights: Tensor) -> bool:
        return torch.is_grad_enabled() and (hidden_states.requires_grad or routing_weights.requires_grad
                                            or self.gate_up_weight.requires_grad or self.down_weight.requires_grad)

    def compute(self, hidden_states: Tensor, selected_experts: Tensor, routing_weights: Tensor) -> Tensor:
        """Expert output [T,H] for tokens routed by ``selected_experts`` / ``routing_weights`` [T,k]."""
        return self._compute(hidden_states, selected_experts, routing_weights)[0]

    def _compute(self, hidden_states: Tensor, selected_experts: Tensor, routing_weights: Tensor,
                 dispatch: Optional["ops.Dispatch"] = None):
        """(expert output [T,H], tokens_per_expert [E] int64 from the dispatch, or None when T == 0).

        ``dispatch``: the permutation of ``selected_experts`` when the caller
        already has it (the router's fused dispatch).
        """
        num_tokens = hidden_states.shape[0]
        dtype = hidden_states.dtype
        gate_up_weight = self.gate_up_weight.to(dtype)
        down_weight = self.down_weight.to(dtype)
        if num_tokens == 0:
            return torch.zeros_like(hidden_states), None
        routing_weights = routing_weights.to(dtype)

        if not self._needs_autograd(hidden_states, routing_weights):
            with record_moe_profile_phase("dispatch"):
                d = dispatch if dispatch is not None else ops.permute(selected_experts, self.num_experts)
            with record_moe_profile_phase("gate_up_gemm"):
                act = ops.gate_up_swiglu(hidden_states, d, gate_up_weight)
            if ops.down_combine_decode_ok(act, down_weight, routing_weights):
                # one or two tokens: down projection and combine in one launch
                with record_moe_profile_phase("down_gemm"):
                    return (ops.down_combine_decode(act, down_weight, d, selected_experts, routing_weights),
                            d.tokens_per_expert)
            with record_moe_profile_phase("down_gemm"):
                y = ops.grouped_gemm_nt(act, down_weight, d.tokens_per_expert)
            with record_moe_profile_phase("combine"):
                return ops.combine(y, d, routing_weights), d.tokens_per_expert

        if hidden_states.shape[1] % self.TRAIN_HIDDEN_MULTIPLE != 0:
            raise NotImplementedError(
                f"training the MoE FFN needs a hidden size that is a multiple of {self.TRAIN_HIDDEN_MULTIPLE} "
                f"(got {hidden_states.shape[1]}); the forward without autograd accepts multiples of 8")
        # HIP forward and backward of the whole expert block
        with record_moe_profile_phase("dispatch"):
            d = dispatch if dispatch is not None else ops.permute(selected_experts, self.num_experts)
        with record_moe_profile_phase("experts"):
            out = _GroupedExpertsFn.apply(hidden_states, routing_weights, gate_up_weight, down_weight, d)
        return out, d.tokens_per_expert

    def forward(self, hidden_states: Tensor, selected_experts: Tensor, routing_weights: Tensor,
                final_hidden_states: Tensor) -> Tensor:
        """Adds the expert output into ``final_hidden_states`` and returns it (models/layers.py:285-335)."""
        if hidden_states.shape[0] == 0:
            return final_hidden_states
        out = self.compute(hidden_states, selected_experts, routing_weights)
        if final_hidden_states.requires_grad or out.requires_grad:
            return final_hidden_states + out
        return final_hidden_states.add_(out)


class SparseMoESwiGLU(nn.Module):
    """Routed SwiGLU MoE FFN (models/layers.py:518-634) on the HIP kernels.

    ``implementation`` accepts "grouped_hip" and, so that existing configs keep
    working, "grouped_triton" (models/layers.py:554-567 with backend triton).
    The reference's other implementations (origin, shard, grouped,
    grouped_cutlass, grouped_ep) are not part of hrm_moe_amd and raise.
    """

    IMPLEMENTATIONS = ("grouped_hip", "grouped_triton")

    def __init__(self, hidden_size: int, intermediate_size: int, num_experts: int, top_k: int,
                 norm_topk_prob: bool, implementation: str = "grouped_hip", expert_in_one_shard: int = 1,
                 init_std_in=None, init_std_out=None, **kwargs):
        super().__init__()
        if num_experts <= 0:
            raise ValueError(f"num_experts must be positive, got {num_experts}")
        if top_k <= 0 or top_k > num_experts:
            raise ValueError(f"top_k must be in [1, num_experts], got top_k={top_k}, num_experts={num_experts}")
        if expert_in_one_shard <= 0 or num_experts % expert_in_one_shard != 0:
            raise ValueError(
                f"expert_in_one_shard must divide num_experts, got "
                f"expert_in_one_shard={expert_in_one_shard}, num_experts={num_experts}")
        if implementation not in self.IMPLEMENTATIONS:
            raise ValueError(f"implementation {implementation!r} is not provided by hrm_moe_amd; "
                             f"use one of {self.IMPLEMENTATIONS}")
        self.hidden_size = hidden_size
        self.num_experts = num_experts
        self.top_k = top_k
        self.norm_topk_prob = norm_topk_prob
        self.implementation = implementation
        self.expert_in_one_shard = expert_in_one_shard
        self.gate = LinearInit(hidden_size, num_experts, bias=False, init_std=init_std_in, **kwargs)
        self.experts = SparseMoEGroupedExperts(hidden_size=hidden_size, intermediate_size=intermediate_size,
                                               num_experts=num_experts, backend="hip", init_std_in=init_std_in,
                                               init_std_out=init_std_out, **kwargs)

    def forward(self, x: Tensor, moe_context: Optional[dict[str, Any]] = None, total_seqlen: Optional[Tensor] = None,
                **_seq_info) -> Tensor:
        original_shape = x.shape
        hidden_states = x.reshape(-1, self.hidden_size)
        want_aux = moe_context is not None and torch.is_grad_enabled()

        dispatch = None
        decoded = None
        with record_moe_profile_phase("router"):
            w_gate = self.gate.weight
            if (torch.is_grad_enabled() and w_gate.requires_grad and self.gate.bias is None
                    and hidden_states.dtype == w_gate.dtype
                    and hidden_states.dtype in (torch.bfloat16, torch.float16) and self.num_experts % 8 == 0
                    and self.hidden_size % 8 == 0):
                router_logits = _GateLinear.apply(hidden_states, w_gate)
            else:
                router_logits = self.gate(hidden_states)
            if torch.is_grad_enabled() and router_logits.requires_grad:
                routing_probs, routing_weights, selected_experts, *dd = _RouterTopK.apply(
                    router_logits, self.top_k, self.norm_topk_prob, hidden_states.dtype)
                dispatch = ops.Dispatch(*dd, None)
            elif self.num_experts <= 128 and self.top_k <= 8 and not self.experts._needs_autograd(
                    hidden_states, router_logits):
                decoded = self._decode_two_launches(hidden_states, router_logits, want_aux)
                if decoded is not None:
                    routing_probs, routing_weights, selected_experts, dispatch, final_hidden_states = decoded
                else:
                    # router and dispatch in two launches
                    routing_probs, routing_weights, selected_experts, dispatch = ops.router_topk_dispatch(
                        router_logits, self.top_k, self.norm_topk_prob, hidden_states.dtype, want_probs=want_aux)
            else:
                routing_probs, routing_weights, selected_experts = ops.router_topk(
                    router_logits, self.top_k, self.norm_topk_prob, hidden_states.dtype, want_probs=want_aux)

        if decoded is not None:
            tokens_per_expert = dispatch.tokens_per_expert
        else:
            final_hidden_states, tokens_per_expert = self.experts._compute(hidden_states, selected_experts,
                                                                           routing_weights, dispatch)

        if want_aux:
            aux_routing_probs = routing_probs
            aux_selected_experts = selected_experts
            counts = tokens_per_expert  # the dispatch's counts equal the reference's bincount over all tokens
            if total_seqlen is not None:
                valid_tokens = int(unwrap_tensor(total_seqlen).item())
                aux_routing_probs = aux_routing_probs[:valid_tokens]
                aux_selected_experts = aux_selected_experts[:valid_tokens]
                counts = None
            with record_moe_profile_phase("aux_metrics"):
                if (counts is not None and aux_routing_probs.is_cuda and aux_routing_probs.dtype == torch.float32
                        and aux_routing_probs.shape[0] > 0 and self.num_experts <= 1024):
                    # loss and counts in two launches instead of torch's chain of small kernels
                    aux_loss, counts_f = _AuxLoss.apply(aux_routing_probs, counts)
                    moe_context.setdefault("aux_losses", []).append(aux_loss)
                    moe_context.setdefault("expert_counts", []).append(counts_f)
                else:
                    aux_loss = load_balancing_loss_func(aux_routing_probs, aux_selected_experts, self.num_experts,
                                                        tokens_per_expert=counts)
                    moe_context.setdefault("aux_losses", []).append(aux_loss)
                    with torch.no_grad():
                        if counts is None:
                            counts = torch.bincount(aux_selected_experts.reshape(-1), minlength=self.num_experts)
                        moe_context.setdefault("expert_counts", []).append(counts.to(torch.float32))

        return final_hidden_states.reshape(original_shape)

    def _decode_two_launches(self, hidden_states: Tensor, router_logits: Tensor, want_probs: bool):
        """(probs, weights, idx, Dispatch, expert output) of one or two tokens: router, dispatch and gate_up in one
        launch, then the down GEMM and combine; None when the call is outside the first launch's limits."""
        if hidden_states.shape[0] > 2 or not hidden_states.is_cuda:
            return None
        dtype = hidden_states.dtype
        gate_up_weight = self.experts.gate_up_weight.to(dtype)
        if not ops.router_gate_up_decode_ok(router_logits, hidden_states, gate_up_weight, self.top_k):
            return None
        down_weight = self.experts.down_weight.to(dtype)
        with record_moe_profile_phase("router_gate_up"):
            probs, w, idx, d, act = ops.router_gate_up_decode(router_logits, hidden_states, gate_up_weight,
                                                               self.top_k, self.norm_topk_prob, want_probs=want_probs)
        with record_moe_profile_phase("down_gemm"):
            if ops.down_combine_decode_ok(act, down_weight, w):
                return probs, w, idx, d, ops.down_combine_decode(act, down_weight, d, idx, w)
            y = ops.grouped_gemm_nt(act, down_weight, d.tokens_per_expert)
        with record_moe_profile_phase("combine"):
            return probs, w, idx, d, ops.combine(y, d, w)
