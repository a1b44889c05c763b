"""HIP-graph replay of the MoE FFN forward (decode sizes) against eager calls.

Every replay must reproduce the eager forward bit for bit: the kernels are
deterministic and read their routing from the captured input buffer.  Replays
alternate between two inputs, with unrelated eager GPU work and host
synchronisation between them, so a replay that reused stale device state (a
recorded memset or a cached plan) would show.
"""
import pytest
import torch

import hrm_moe_amd
from oracle import synth

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


@pytest.mark.parametrize("t", [1, 8, 64])
def test_graph_replay_matches_eager(cuda, t):
    h, e, i, k = 1536, 64, 512, 8
    x1_, wg, wgu, wdn = synth.moe_inputs(40 + t, t, h, e, i)
    x2_ = synth.normal(90 + t, (t, h))
    layer = hrm_moe_amd.SparseMoESwiGLU(h, i, e, k, True, implementation="grouped_triton").to(cuda, BF)
    with torch.no_grad():
        layer.gate.weight.copy_(torch.from_numpy(wg))
        layer.experts.gate_up_weight.copy_(torch.from_numpy(wgu))
        layer.experts.down_weight.copy_(torch.from_numpy(wdn))
    x1 = torch.from_numpy(x1_).to(cuda, BF)
    x2 = torch.from_numpy(x2_).to(cuda, BF)
    with torch.no_grad():
        e1 = layer(x1).clone()
        e2 = layer(x2).clone()
    assert not torch.equal(e1, e2)
    g = hrm_moe_amd.GraphedMoEForward(layer, x1)
    noise = torch.randn(512, 512, device=cuda)
    for rep in range(6):
        x, ref = (x1, e1) if rep % 2 == 0 else (x2, e2)
        out = g(x).clone()
        noise = noise @ noise.T / 512.0  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {rep} differs from the eager forward"
    # tokens written into the captured input buffer by the caller: no copy, same results
    for rep in range(4):
        x, ref = (x2, e2) if rep % 2 == 0 else (x1, e1)
        g.static_in.copy_(x)
        noise = noise @ noise.T / 512.0
        out = g(g.static_in).clone()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"in-place replay {rep} differs from the eager forward"


def test_graph_rejects_other_shapes(cuda):
    layer = hrm_moe_amd.SparseMoESwiGLU(256, 128, 8, 2, True, implementation="grouped_triton").to(cuda, BF)
    x = torch.randn(4, 256, device=cuda, dtype=BF)
    g = hrm_moe_amd.GraphedMoEForward(layer, x)
    with pytest.raises(ValueError):
        g(torch.randn(5, 256, device=cuda, dtype=BF))
