"""Write the torch-on-ROCm top-k tie fixture used to pin the oracle's router.

The reference router calls ``torch.topk(routing_probs, top_k, dim=-1)`` on the
device that holds the activations (models/layers.py:607).  torch leaves the
order of equal values implementation-defined, and the CPU and ROCm kernels
disagree.  This script runs torch.topk on the GPU over tie-heavy inputs and
stores inputs plus the returned indices, so that CPU tests can check the
oracle's tie rule without a GPU.

Inputs are small integer levels (every row is full of exact ties) plus one
case of real router probabilities from bf16 logits.

Usage (needs a ROCm GPU):  python tests/golden/make_topk_ties_rocm.py OUT.npz
"""
import sys

import numpy as np
import torch


CASES = [
    # name, num_experts, top_k, rows, levels
    ("e64_k8_l4", 64, 8, 1024, 4),
    ("e64_k8_l16", 64, 8, 1024, 16),
    ("e64_k4_l6", 64, 4, 512, 6),
    ("e128_k8_l8", 128, 8, 512, 8),
    ("e8_k2_l3", 8, 2, 1024, 3),
    ("e8_k3_l3", 8, 3, 512, 3),
]


def main(out_path: str) -> None:
    assert torch.cuda.is_available(), "needs a ROCm GPU"
    rng = np.random.default_rng(20261201)
    arrays = {}
    for name, num_experts, top_k, rows, levels in CASES:
        lv = rng.integers(0, levels, size=(rows, num_experts), dtype=np.uint8)
        probs = torch.from_numpy(lv.astype(np.float32) * 0.0625 + 0.03125).cuda()
        _, idx = torch.topk(probs, top_k, dim=-1)
        arrays[f"{name}__levels"] = lv
        arrays[f"{name}__gpu_idx"] = idx.cpu().numpy().astype(np.uint8)
        _, cidx = torch.topk(probs.cpu(), top_k, dim=-1)
        arrays[f"{name}__cpu_idx"] = cidx.numpy().astype(np.uint8)

    # Real router statistics: bf16 logits of N(0,1) tokens through an N(0,0.02) gate, H=1280, E=64.
    g = torch.Generator().manual_seed(7)
    x = torch.randn(1024, 1280, generator=g).to(torch.bfloat16)
    wg = (torch.randn(64, 1280, generator=g) * 0.02).to(torch.bfloat16)
    logits = torch.nn.functional.linear(x.cuda(), wg.cuda())
    probs = torch.nn.functional.softmax(logits, dim=-1, dtype=torch.float32)
    _, idx = torch.topk(probs, 8, dim=-1)
    arrays["router_e64_k8__logits_bf16_bits"] = logits.cpu().view(torch.int16).numpy().view(np.uint16)
    arrays["router_e64_k8__gpu_idx"] = idx.cpu().numpy().astype(np.uint8)
    arrays["torch_version"] = np.array(torch.__version__)
    arrays["device_name"] = np.array(torch.cuda.get_device_name(0))
    np.savez_compressed(out_path, **arrays)
    print("wrote", out_path, "torch", torch.__version__, torch.cuda.get_device_name(0))


if __name__ == "__main__":
    main(sys.argv[1])
