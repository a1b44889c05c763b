"""Drop-in for models/moe_triton_grouped_gemm.py: grouped linear on gfx950 HIP kernels.

``hip_grouped_linear(input, weight, tokens_per_expert)`` has the contract of the
reference's ``triton_grouped_linear`` (moe_triton_grouped_gemm.py:478-485):

  * rows of ``input`` [M,K] are expert-contiguous in expert order, with
    ``tokens_per_expert[e]`` rows for expert e (any integer dtype, moved to
    the device as int64, never read on the host);
  * ``weight`` is [E,N,K]; the result is [M,N] in the input dtype, fp32
    accumulation, one rounding;
  * bf16 and fp16 only (TypeError otherwise, :350-355); K mismatch raises
    ValueError (:367-368); M == 0 returns ``input @ weight[0].T`` (:479-480);
  * autograd saves (input, weight, tokens_per_expert) and the backward returns
    (grad_input [M,K], grad_weight [E,N,K] in the input dtype, None)
    (:459-475).
  * Forward and backward never synchronise with the host.

Deliberate difference: the reference runs a per-expert torch loop for CPU
tensors (:481-482).  This op needs a ROCm GPU and raises RuntimeError for CPU
tensors: it has no CPU path.

The CU margin knob of the reference (HRM_MOE_TRITON_SM_MARGIN, falling back
to XTUNER_SM_MARGIN, :24-52) is honoured under those names and under
HRM_MOE_HIP_CU_MARGIN, which takes precedence: compute units left out of the
persistent grids.  As in the reference, a value that is not a non-negative
integer raises ValueError when this module is imported.  The kernel library
reads the same variables (include/hrm_moe.h, hrm_moe_reload_config).
"""
from __future__ import annotations

import os
import re

import torch
from torch import Tensor

from . import ops
from .profile import record_moe_profile_phase

MARGIN_VARIABLES = ("HRM_MOE_HIP_CU_MARGIN", "HRM_MOE_TRITON_SM_MARGIN", "XTUNER_SM_MARGIN")
_DECIMAL = re.compile(r"\s*[+-]?[0-9]+\s*")


def cu_margin_from_env(environ=os.environ) -> int:
    """CUs the persistent GEMM grids leave free: the first of MARGIN_VARIABLES that is set and non-empty.

    Every variable that is set must hold a non-negative decimal integer, else
    ValueError (the reference checks both of its names the same way,
    models/moe_triton_grouped_gemm.py:33-47).
    """
    chosen = None
    for name in MARGIN_VARIABLES:
        raw = environ.get(name, "")
        if raw == "":
            continue
        if not _DECIMAL.fullmatch(raw):
            raise ValueError(f"{name} must be a non-negative integer, got {raw!r}")
        value = int(raw)
        if value < 0:
            raise ValueError(f"{name} must be non-negative, got {value}")
        if chosen is None:
            chosen = value
    return 0 if chosen is None else chosen


CU_MARGIN = cu_margin_from_env()


class _HipGroupedLinear(torch.autograd.Function):
    @staticmethod
    def forward(ctx, input: Tensor, weight: Tensor, tokens_per_expert: Tensor) -> Tensor:
        output = ops.grouped_gemm_nt(input, weight, tokens_per_expert)
        ctx.save_for_backward(input, weight, tokens_per_expert)
        return output

    @staticmethod
    def backward(ctx, grad_output: Tensor):
        input, weight, tokens_per_expert = ctx.saved_tensors
        with record_moe_profile_phase("grad_output_contiguous"):
            grad_output = grad_output.contiguous()
        grad_input = grad_weight = None
        if ctx.needs_input_grad[0]:
            with record_moe_profile_phase("grad_input_gemm"):
                grad_input = ops.grouped_gemm_nn(grad_output, weight, tokens_per_expert)
        if ctx.needs_input_grad[1]:
            with record_moe_profile_phase("grad_weight_gemm"):
                grad_weight = ops.grouped_gemm_tn(grad_output, input, tokens_per_expert)
        return grad_input, grad_weight, None


def hip_grouped_linear(input: Tensor, weight: Tensor, tokens_per_expert: Tensor) -> Tensor:
    """Grouped ``F.linear`` over expert-contiguous rows (moe_triton_grouped_gemm.py:478-485)."""
    if input.shape[0] == 0:
        return input @ weight[0].T
    if not input.is_cuda:
        raise RuntimeError("hip_grouped_linear needs tensors on a ROCm GPU; there is no CPU path")
    return _HipGroupedLinear.apply(input, weight, tokens_per_expert)


# The name callers of the reference import.
triton_grouped_linear = hip_grouped_linear
