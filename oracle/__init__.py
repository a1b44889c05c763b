"""CPU oracle for HRM-MoE's routed SwiGLU MoE FFN (grouped_triton path).

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import anything under ``oracle/``, and
only to check results (or as the timed CPU baseline), never as part of the product
path.  The product path (``hrm_moe_amd``) never imports this package and fails
loudly when its HIP library is missing.

Modules:
  synth       deterministic input generator (splitmix64 + Box-Muller)
  moe_oracle  restatement of models/layers.py:163-170,285-335,596-634 and
              models/moe_triton_grouped_gemm.py:55-65,459-485
"""
