"""Write the C1 golden vectors by running the reference MoE module on the CPU.

Runs only in the build container, where the reference checkout is mounted at
/root/reference; the GPU hosts never see it.  The reference's own
equivalence script stubs the attention modules the same way
(scripts/test_moe_shard_equivalence.py:12-18).

Cases (inputs regenerated from the seeds by oracle/synth.py, so the fixture
holds outputs only):
  c1     fp32, T=512, H=256, E=8, I=128, top-2, normalised: the tiny CPU config.
         Module implementations grouped_triton (CPU -> per-expert F.linear,
         models/moe_triton_grouped_gemm.py:55-65,481-482) and origin (origin stores its first 32 output rows).
  bf16s  bf16, T=64, H=128, E=16, I=64, top-4, normalised, grouped_triton:
         pins the bf16 cast points.  The seed is chosen so no two of a token's
         top-(k+1) logits tie, which keeps CPU torch.topk's tie order out of it.

Usage:  python tests/golden/make_c1_golden.py tests/golden/c1_golden.npz
"""
import os
import sys
import types

import numpy as np
import torch

REF = "/root/reference"
HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle import synth  # noqa: E402

sys.path.insert(0, REF)
_stub = types.ModuleType("models.flash_attention_prefixlm_v2")
_stub.flash_attn_varlen_prefixlm = None
sys.modules.setdefault("models.flash_attention_prefixlm_v2", _stub)
_stub2 = types.ModuleType("flash_attn_interface")
_stub2.flash_attn_with_kvcache = None
sys.modules.setdefault("flash_attn_interface", _stub2)
from models.layers import SparseMoESwiGLU  # noqa: E402


def build(impl, h, i, e, k, dtype, wg, wgu, wdn):
    m = SparseMoESwiGLU(hidden_size=h, intermediate_size=i, num_experts=e, top_k=k, norm_topk_prob=True,
                        implementation=impl).to(dtype=dtype)
    with torch.no_grad():
        m.gate.weight.copy_(torch.from_numpy(wg))
        if impl == "origin":
            for ex in range(e):
                m.experts[ex].gate_up_proj.weight.copy_(torch.from_numpy(wgu[ex]))
                m.experts[ex].down_proj.weight.copy_(torch.from_numpy(wdn[ex]))
        else:
            m.experts.gate_up_weight.copy_(torch.from_numpy(wgu))
            m.experts.down_weight.copy_(torch.from_numpy(wdn))
    return m


def run(m, x, grad):
    captured = {}

    def hook(_mod, args):
        captured["selected_experts"] = args[1].detach().clone()
        captured["routing_weights"] = args[2].detach().clone()

    handle = m.experts.register_forward_pre_hook(hook)
    xr = x.clone().requires_grad_(True)
    ctx = {"aux_losses": [], "expert_counts": []}
    out = m(xr, moe_context=ctx)
    handle.remove()
    loss = (out.float() * grad).sum() + torch.stack(ctx["aux_losses"]).sum()
    loss.backward()
    return out.detach(), captured, ctx, xr.grad.detach()


def main(out_path):
    torch.manual_seed(0)
    arrays = {}
    # --- C1: fp32 tiny config -------------------------------------------------
    t, h, e, i, k = 512, 256, 8, 128, 2
    x, wg, wgu, wdn = synth.moe_inputs(11, t, h, e, i)
    grad = torch.from_numpy(synth.normal(12, (t, h)))
    xt = torch.from_numpy(x)
    for impl in ("grouped_triton", "origin"):
        m = build(impl, h, i, e, k, torch.float32, wg, wgu, wdn)
        out, cap, ctx, xg = run(m, xt, grad)
        p = f"c1_{impl}__"
        arrays[p + "out"] = out.numpy() if impl == "grouped_triton" else out[:32].numpy()
        arrays[p + "idx"] = cap["selected_experts"].numpy().astype(np.uint8)
        arrays[p + "weights"] = cap["routing_weights"].numpy()
        arrays[p + "aux_loss"] = ctx["aux_losses"][0].detach().numpy()
        arrays[p + "expert_counts"] = ctx["expert_counts"][0].numpy()
        arrays[p + "x_grad_rows0_15"] = xg[:16].numpy()
        arrays[p + "gate_grad"] = m.gate.weight.grad.numpy()
        arrays[p + "x_grad_sq_sum"] = np.array(float(xg.double().pow(2).sum()))
        if impl == "grouped_triton":
            arrays[p + "gate_up_grad_e0_rows0_3"] = m.experts.gate_up_weight.grad[0, :4].numpy()
            arrays[p + "down_grad_e0_rows0_3"] = m.experts.down_weight.grad[0, :4].numpy()
            arrays[p + "gate_up_grad_sq_sum"] = np.array(float(m.experts.gate_up_weight.grad.double().pow(2).sum()))
            arrays[p + "down_grad_sq_sum"] = np.array(float(m.experts.down_weight.grad.double().pow(2).sum()))
    arrays["c1__shape"] = np.array([t, h, e, i, k, 11, 12])

    # --- bf16 small config, seed without top-(k+1) ties ------------------------
    t, h, e, i, k = 64, 128, 16, 64, 4
    for seed in range(100, 200):
        x, wg, wgu, wdn = synth.moe_inputs(seed, t, h, e, i)
        xb = torch.from_numpy(x).to(torch.bfloat16)
        logits = torch.nn.functional.linear(xb, torch.from_numpy(wg).to(torch.bfloat16)).float()
        top = torch.sort(logits, dim=-1, descending=True).values[:, :k + 1]
        if not (top[:, 1:] == top[:, :-1]).any():
            break
    else:
        raise RuntimeError("no tie-free seed found")
    m = build("grouped_triton", h, i, e, k, torch.bfloat16, wg, wgu, wdn)
    grad = torch.from_numpy(synth.normal(seed * 16 + 9, (t, h)))
    out, cap, ctx, xg = run(m, xb, grad)
    arrays["bf16s__out_bits"] = out.view(torch.int16).numpy().view(np.uint16)
    arrays["bf16s__idx"] = cap["selected_experts"].numpy().astype(np.uint8)
    arrays["bf16s__weights_bits"] = cap["routing_weights"].view(torch.int16).numpy().view(np.uint16)
    arrays["bf16s__aux_loss"] = ctx["aux_losses"][0].detach().float().numpy()
    arrays["bf16s__expert_counts"] = ctx["expert_counts"][0].numpy()
    arrays["bf16s__shape"] = np.array([t, h, e, i, k, seed])
    arrays["torch_version"] = np.array(torch.__version__)
    np.savez_compressed(out_path, **arrays)
    print("wrote", out_path, {k_: v.shape for k_, v in arrays.items()})


if __name__ == "__main__":
    main(sys.argv[1])
