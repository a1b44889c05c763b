"""hrm_moe_amd: HRM-MoE's routed SwiGLU MoE FFN (grouped_triton path) on MI355X / gfx950.

Public surface, mirroring the reference:
  SparseMoESwiGLU, SparseMoEGroupedExperts, load_balancing_loss_func   (models/layers.py)
  hip_grouped_linear (alias triton_grouped_linear)                       (models/moe_triton_grouped_gemm.py)
  record_moe_profile_phase, reset_moe_profile, pop_moe_profile           (models/moe_profile.py)
  ops: the single-kernel device ops behind them (router_topk, permute,
       grouped_gemm_nt/nn/tn, gate_up_swiglu, combine).
  GraphedMoEForward: HIP-graph replay of the no-autograd forward for a fixed
       token count (decode).
  checkpoint: the release / native key maps and loading MoE layers from a
       local model.safetensors (simple_inference_engine.py:139-145).

The kernels live in libhrm_moe.so (C ABI: include/hrm_moe.h), built by
``build.build_library()``.  Importing the package does not load the library;
the first op does, and raises if it is missing.
"""
from . import _lib, checkpoint, ops  # noqa: F401
from .graph import GraphedMoEForward  # noqa: F401
from .grouped_gemm import hip_grouped_linear, triton_grouped_linear  # noqa: F401
from .layers import (LinearInit, SparseMoEGroupedExperts, SparseMoESwiGLU,  # noqa: F401
                     load_balancing_loss_func, trunc_normal_init_)
from .profile import pop_moe_profile, record_moe_profile_phase, reset_moe_profile  # noqa: F401

__all__ = [
    "SparseMoESwiGLU", "SparseMoEGroupedExperts", "LinearInit", "load_balancing_loss_func", "trunc_normal_init_",
    "hip_grouped_linear", "triton_grouped_linear", "record_moe_profile_phase", "reset_moe_profile",
    "pop_moe_profile", "ops", "GraphedMoEForward", "checkpoint",
]


def load_library():
    """Load libhrm_moe.so now (raises if it is not built)."""
    return _lib.load()
