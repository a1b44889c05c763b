"""Router, dispatch and gate/up + SwiGLU of one or two tokens in one launch.

Parity bar: every output is the same bits as the two launches it replaces, run on the same inputs:
router_topk_dispatch (routing indices and weights, probabilities, the dispatch tensors) and
gate_up_swiglu (act).  Those ops are checked against the oracle in test_gpu_router, test_gpu_permute
and test_gpu_skinny; here the layer output of the module, which takes this launch at one or two tokens,
is also checked against the oracle within bf16 tolerance, and graph replays against eager calls.
"""
import pytest
import torch
import torch.nn.functional as F

import hrm_moe_amd
from hrm_moe_amd import ops
from oracle import moe_oracle as mo
from oracle import synth

pytestmark = pytest.mark.gpu

CASES = [
    # T, H, E, I, k, dtype, logits in fp32
    (1, 1536, 64, 512, 8, torch.bfloat16, False),
    (2, 1536, 64, 512, 8, torch.bfloat16, False),
    (1, 1280, 64, 448, 8, torch.bfloat16, False),
    (2, 1280, 64, 448, 8, torch.float16, False),
    (1, 256, 8, 128, 2, torch.bfloat16, False),
    (2, 512, 32, 64, 4, torch.bfloat16, True),
    (1, 2048, 64, 256, 8, torch.bfloat16, False),
    (2, 128, 16, 48, 2, torch.float16, False),
]


def _inputs(seed, t, h, e, i, dtype, cuda):
    x, wg, wgu, wdn = synth.moe_inputs(seed, t, h, e, i)
    return [torch.from_numpy(a).to(cuda, dtype) for a in (x, wg, wgu, wdn)]


@pytest.mark.parametrize("t,h,e,i,k,dtype,f32_logits", CASES)
@pytest.mark.parametrize("norm", [True, False])
def test_router_gate_up_decode_matches_two_launches(cuda, t, h, e, i, k, dtype, f32_logits, norm):
    print(f"router_gate_up_decode t={t} h={h} e={e} i={i} k={k} {dtype} fp32 logits={f32_logits} norm={norm}",
          flush=True)
    x1, wg, wgu, _ = _inputs(100 + t + h + k, t, h, e, i, dtype, cuda)
    x2 = _inputs(200 + t + h + k, t, h, e, i, dtype, cuda)[0]
    for x in (x1, x2, x1):
        logits = F.linear(x, wg)
        if f32_logits:
            logits = logits.float()
        assert ops.router_gate_up_decode_ok(logits, x, wgu, k)
        probs, w, idx, d, act = ops.router_gate_up_decode(logits, x, wgu, k, norm, want_probs=True,
                                                          want_sort_idx=True)
        cprobs, cw, cidx, cd = ops.router_topk_dispatch(logits, k, norm, x.dtype, want_probs=True, want_sort_idx=True)
        cact = ops.gate_up_swiglu(x, cd, wgu)
        assert torch.equal(idx, cidx), "routing indices"
        assert torch.equal(w, cw), "routing weights"
        assert torch.equal(probs, cprobs), "probabilities"
        for name in ("tokens_per_expert", "expert_offsets", "sorted_token_idx", "slot_to_row", "sort_idx"):
            assert torch.equal(getattr(d, name), getattr(cd, name)), name
        assert torch.equal(act, cact), f"act: max |d| {(act.float() - cact.float()).abs().max().item():.3e}"


@pytest.mark.parametrize("t,k,e", [(1, 8, 64), (2, 8, 64), (2, 4, 32), (1, 2, 8)])
def test_router_gate_up_decode_ties(cuda, t, k, e):
    """Logits on a coarse grid, so many probabilities are equal and the top-k set is decided by ties: the
    kernel's selection (a bitwise search for the k-th largest key, then the lowest indices among the equal
    ones) must give the router's rank-order set, and all outputs the router's bits."""
    h, i = 256, 64
    x, wg, wgu, _ = _inputs(500 + t + k, t, h, e, i, torch.bfloat16, cuda)
    gen = torch.Generator().manual_seed(600 + t + k)
    for levels in (2, 3, 5):
        logits = torch.randint(0, levels, (t, e), generator=gen).to(torch.bfloat16).to(cuda) * 0.5
        probs, w, idx, d, act = ops.router_gate_up_decode(logits, x, wgu, k, True, want_probs=True,
                                                          want_sort_idx=True)
        cprobs, cw, cidx, cd = ops.router_topk_dispatch(logits, k, True, x.dtype, want_probs=True, want_sort_idx=True)
        cact = ops.gate_up_swiglu(x, cd, wgu)
        assert torch.equal(idx, cidx), f"routing indices, {levels} logit levels"
        assert torch.equal(w, cw) and torch.equal(probs, cprobs)
        for name in ("tokens_per_expert", "expert_offsets", "sorted_token_idx", "slot_to_row", "sort_idx"):
            assert torch.equal(getattr(d, name), getattr(cd, name)), name
        assert torch.equal(act, cact)


@pytest.mark.parametrize("t", [1, 2])
def test_decode_module_and_graph(cuda, t):
    """The module takes the fused launch at one or two tokens: its output matches the oracle within bf16
    tolerance and the multi-launch composition bit for bit, and replays of its captured graph (alternating
    inputs, eager work in between) match eager calls bit for bit."""
    h, e, i, k = 1536, 64, 512, 8
    x, wg, wgu, wdn = synth.moe_inputs(300 + t, t, h, e, i)
    layer = hrm_moe_amd.SparseMoESwiGLU(h, i, e, k, True, implementation="grouped_triton").to(cuda, torch.bfloat16)
    with torch.no_grad():
        layer.gate.weight.copy_(torch.from_numpy(wg))
        layer.experts.gate_up_weight.copy_(torch.from_numpy(wgu))
        layer.experts.down_weight.copy_(torch.from_numpy(wdn))
    xs = [torch.from_numpy(x).to(cuda, torch.bfloat16),
          torch.from_numpy(synth.moe_inputs(400 + t, t, h, e, i)[0]).to(cuda, torch.bfloat16)]
    with torch.no_grad():
        eager = [layer(v).clone() for v in xs]
        logits = F.linear(xs[0], layer.gate.weight)
        _, w, idx, d = ops.router_topk_dispatch(logits, k, True, torch.bfloat16, want_probs=False)
        act = ops.gate_up_swiglu(xs[0], d, layer.experts.gate_up_weight)
        composed = ops.down_combine_decode(act, layer.experts.down_weight, d, idx, w)
    assert torch.equal(eager[0], composed), "module output differs from the multi-launch composition"
    cpu = [torch.from_numpy(a).to(torch.bfloat16) for a in (x, wg, wgu, wdn)]
    ref = mo.moe_forward(*cpu, k, True, logits=logits.cpu())
    diff = (eager[0].float().cpu() - ref.float()).abs()
    rel = diff.max().item() / ref.float().abs().max().item()
    print(f"decode module t={t}: max rel err {rel:.3e}, mean abs err {diff.mean().item():.3e}")
    assert rel <= 2e-2
    graphed = hrm_moe_amd.GraphedMoEForward(layer, xs[0])
    for rep in range(6):
        got = graphed(xs[rep % 2]).clone()
        torch.cuda.synchronize()
        assert torch.equal(got, eager[rep % 2]), f"replay {rep}"
        with torch.no_grad():
            again = layer(xs[(rep + 1) % 2])
        assert torch.equal(again, eager[(rep + 1) % 2])
