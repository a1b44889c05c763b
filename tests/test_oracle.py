"""Pins the CPU oracle (oracle/moe_oracle.py) before GPU results are checked against it.

Each oracle function is checked against something it does not restate: the
reference module's own outputs (C1 golden, imported on the CPU), torch.topk
on an MI355X (tie fixture), brute force on tiny inputs, float64 closed forms,
or an independent formulation.  Planted-mistake tests show the fixtures
catch the mistakes they are meant to catch.
"""
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import moe_oracle as mo
from oracle import synth

HERE = os.path.dirname(os.path.abspath(__file__))
TIES = os.path.join(HERE, "golden", "topk_ties_rocm.npz")
C1 = os.path.join(HERE, "golden", "c1_golden.npz")
TIE_CASES = ["e64_k8_l4", "e64_k8_l16", "e64_k4_l6", "e128_k8_l8", "e8_k2_l3", "e8_k3_l3"]


# ---------------------------------------------------------------- synth ----

def test_splitmix64_known_answer():
    # Published splitmix64 stream for state 0 (first two outputs).
    z = synth.splitmix64(0, 2)
    assert int(z[0]) == 0xE220A8397B1DCDAF
    assert int(z[1]) == 0x6E789E6AA1B965F4


def test_normal_moments():
    v = synth.normal(3, (200_000,)).astype(np.float64)
    assert abs(v.mean()) < 0.01 and abs(v.std() - 1.0) < 0.01
    assert np.array_equal(synth.normal(3, (1000,)), synth.normal(3, (1000,)))


def test_logit_bias_folds_into_activations():
    x, wg, _, _ = synth.moe_inputs(9, 64, 96, 8, 16, logit_bias_std=1.5)
    x0, _, _, _ = synth.moe_inputs(9, 64, 96, 8, 16)
    b = (x.astype(np.float64) - x0) @ wg.T.astype(np.float64)
    assert np.allclose(b, b[0:1], atol=1e-4)  # the same per-expert bias on every token
    assert b[0].std() > 0.5


# ----------------------------------------------------------------- topk ----

@pytest.mark.parametrize("case", TIE_CASES)
def test_topk_matches_rocm_fixture(case):
    d = np.load(TIES)
    vals = d[case + "__levels"].astype(np.float32) * 0.0625 + 0.03125
    gpu = d[case + "__gpu_idx"].astype(np.int64)
    _, idx = mo.topk_rocm(vals, gpu.shape[1])
    assert np.array_equal(idx, gpu)


def test_topk_router_rows_match_rocm_fixture():
    d = np.load(TIES)
    logits = torch.from_numpy(d["router_e64_k8__logits_bf16_bits"].view(np.int16)).view(torch.bfloat16)
    probs = mo.softmax_fp32(logits)
    _, idx = mo.topk_rocm(probs.numpy(), 8)
    assert np.array_equal(idx, d["router_e64_k8__gpu_idx"].astype(np.int64))


def test_topk_fixture_rejects_stable_tie_rule():
    # Planted mistake: order ties by ascending index (a stable sort).  The
    # fixture must tell it apart from torch's rule.
    d = np.load(TIES)
    vals = d["e64_k8_l4__levels"].astype(np.float32)
    wrong = np.lexsort((np.broadcast_to(np.arange(64), vals.shape), -vals), axis=-1)[:, :8]
    assert not np.array_equal(wrong, d["e64_k8_l4__gpu_idx"].astype(np.int64))
    # CPU torch is yet another order, which is why the oracle restates the device's.
    assert not np.array_equal(d["e64_k8_l4__cpu_idx"], d["e64_k8_l4__gpu_idx"])


def test_topk_distinct_values_equal_sort():
    rng = np.random.default_rng(1)
    v = rng.permutation(64 * 300).reshape(300, 64).astype(np.float32)
    vals, idx = mo.topk_rocm(v, 8)
    want = np.argsort(-v, axis=1)[:, :8]
    assert np.array_equal(idx, want)
    assert np.array_equal(vals, np.take_along_axis(v, want, 1))


def test_topk_set_is_lowest_index_on_boundary_ties():
    v = np.zeros((1, 16), np.float32)
    v[0, [3, 7, 9, 12]] = 1.0
    v[0, 5] = 2.0
    _, idx = mo.topk_rocm(v, 3)
    assert set(idx[0].tolist()) == {5, 3, 7}
    assert idx[0, 0] == 5


# -------------------------------------------------------------- softmax ----

def test_softmax_closed_form():
    z = torch.from_numpy(synth.normal(4, (128, 64), std=3.0)).to(torch.bfloat16)
    p = mo.softmax_fp32(z).double()
    z64 = z.double()
    ref = torch.exp(z64 - z64.max(-1, keepdim=True).values)
    ref = ref / ref.sum(-1, keepdim=True)
    assert torch.allclose(p, ref, rtol=1e-6, atol=1e-9)


def test_router_normalised_weights_sum_to_one():
    z = torch.from_numpy(synth.normal(5, (256, 64)))
    _, w, idx = mo.router_topk(z, 8, True, torch.float32)
    assert torch.allclose(w.sum(-1), torch.ones(256), atol=1e-6)
    assert all(len(set(r)) == 8 for r in idx.tolist())


# -------------------------------------------------------------- permute ----

def _brute_permute(idx, e):
    t, k = idx.shape
    slots = [(int(idx[s // k, s % k]), s) for s in range(t * k)]
    order = [s for _, s in sorted(slots, key=lambda p: (p[0], p[1]))]
    return np.array(order), np.bincount(idx.reshape(-1), minlength=e)


@pytest.mark.parametrize("t,k,e,seed", [(37, 3, 8, 0), (64, 8, 64, 1), (5, 2, 16, 2), (1, 1, 4, 3)])
def test_permute_brute_force(t, k, e, seed):
    rng = np.random.default_rng(seed)
    idx = np.stack([rng.choice(e, size=k, replace=False) for _ in range(t)])
    p = mo.permute(idx, e)
    order, counts = _brute_permute(idx, e)
    assert np.array_equal(p["sort_idx"], order)
    assert np.array_equal(p["tokens_per_expert"], counts)
    assert np.array_equal(p["sorted_token_idx"], order // k)
    assert np.array_equal(p["slot_to_row"][p["sort_idx"]], np.arange(t * k))
    assert np.array_equal(p["expert_offsets"], np.concatenate([[0], np.cumsum(counts)]))
    assert np.all(np.diff(p["sorted_experts"]) >= 0)


def test_permute_empty_and_skewed():
    idx = np.zeros((10, 1), np.int64)
    p = mo.permute(idx, 4)
    assert p["tokens_per_expert"].tolist() == [10, 0, 0, 0]
    p = mo.permute(np.zeros((0, 2), np.int64), 3)
    assert p["tokens_per_expert"].tolist() == [0, 0, 0] and p["sort_idx"].size == 0


# ------------------------------------------------------- grouped linear ----

def _brute_grouped(a, w, tpe):
    out = np.zeros((a.shape[0], w.shape[1]))
    r = 0
    for e, n in enumerate(tpe):
        for _ in range(n):
            for j in range(w.shape[1]):
                out[r, j] = float(np.dot(a[r].astype(np.float64), w[e, j].astype(np.float64)))
            r += 1
    return out


@pytest.mark.parametrize("tpe", [[3, 0, 5, 1], [9, 0, 0, 0], [0, 0, 0, 4]])
def test_grouped_linear_brute_force(tpe):
    m = sum(tpe)
    a = synth.normal(7, (m, 12))
    w = synth.normal(8, (4, 6, 12))
    got = mo.grouped_linear(torch.from_numpy(a), torch.from_numpy(w), tpe).double().numpy()
    assert np.allclose(got, _brute_grouped(a, w, tpe), rtol=1e-5, atol=1e-5)


def test_grouped_linear_planted_transpose_is_caught():
    tpe = [3, 2]
    a = synth.normal(9, (5, 8))
    w = synth.normal(10, (2, 8, 8))
    wrong = mo.grouped_linear(torch.from_numpy(a), torch.from_numpy(w).transpose(1, 2).contiguous(), tpe)
    assert not np.allclose(wrong.numpy(), _brute_grouped(a, w, tpe), atol=1e-3)


def test_grouped_linear_empty_input():
    a = torch.zeros((0, 8))
    w = torch.from_numpy(synth.normal(11, (3, 5, 8)))
    assert mo.grouped_linear(a, w, [0, 0, 0]).shape == (0, 5)


def test_dgrad_wgrad_adjoint_identities():
    tpe = [4, 0, 7, 2]
    m = sum(tpe)
    a = torch.from_numpy(synth.normal(12, (m, 16))).double()
    w = torch.from_numpy(synth.normal(13, (4, 24, 16))).double()
    g = torch.from_numpy(synth.normal(14, (m, 24))).double()
    y = mo.grouped_linear(a, w, tpe)
    inner = float((g * y).sum())
    da = mo.grouped_linear_dgrad(g, w, tpe)
    dw = mo.grouped_linear_wgrad(g, a, tpe)
    # the oracle accumulates in fp32, as the kernels do
    assert abs(float((da * a).sum()) - inner) < 1e-5 * max(1.0, abs(inner))
    assert abs(float((dw * w).sum()) - inner) < 1e-5 * max(1.0, abs(inner))
    assert torch.count_nonzero(dw[1]) == 0  # expert without rows


def test_dgrad_wgrad_match_autograd():
    tpe = [5, 3]
    a = torch.from_numpy(synth.normal(15, (8, 8))).double().requires_grad_(True)
    w = torch.from_numpy(synth.normal(16, (2, 6, 8))).double().requires_grad_(True)
    y = torch.cat([a[:5] @ w[0].T, a[5:] @ w[1].T])
    g = torch.from_numpy(synth.normal(17, (8, 6))).double()
    y.backward(g)
    assert torch.allclose(mo.grouped_linear_dgrad(g, w.detach(), tpe).double(), a.grad, rtol=1e-5, atol=1e-5)
    assert torch.allclose(mo.grouped_linear_wgrad(g, a.detach(), tpe).double(), w.grad, rtol=1e-5, atol=1e-5)


# ------------------------------------------------------ swiglu, combine ----

def test_swiglu_closed_form():
    gu = torch.from_numpy(synth.normal(18, (7, 10))).double()
    g, u = gu[:, :5], gu[:, 5:]
    assert torch.allclose(mo.swiglu(gu), g / (1 + torch.exp(-g)) * u)


def test_combine_closed_form():
    y = torch.from_numpy(synth.normal(19, (6, 4))).double()
    w = torch.tensor([0.5, 0.25, 1.0, 2.0, -1.0, 0.125], dtype=torch.float64)
    tok = np.array([2, 0, 2, 1, 0, 2])
    out = mo.combine(y, w, tok, 3)
    ref = torch.zeros(3, 4, dtype=torch.float64)
    for r in range(6):
        ref[tok[r]] += w[r] * y[r]
    assert torch.allclose(out, ref)


def test_combine_bf16_accumulates_in_fp32():
    # index_add_ on bf16 CPU tensors sums in fp32 and rounds once.
    y = torch.tensor([[1.0], [2.0 ** -9], [2.0 ** -9]], dtype=torch.bfloat16)
    out = mo.combine(y, torch.ones(3, dtype=torch.bfloat16), np.array([0, 0, 0]), 1)
    assert float(out[0, 0]) == float(torch.tensor(1.0 + 2.0 ** -8, dtype=torch.bfloat16))


# ------------------------------------------------------- whole layer -------

@pytest.fixture(scope="module")
def c1():
    return np.load(C1)


def _c1_inputs(g):
    t, h, e, i, k, s1, _ = [int(v) for v in g["c1__shape"]]
    x, wg, wgu, wdn = synth.moe_inputs(s1, t, h, e, i)
    return [torch.from_numpy(a) for a in (x, wg, wgu, wdn)], k, e


def test_c1_golden_bit_exact(c1):
    (x, wg, wgu, wdn), k, e = _c1_inputs(c1)
    out, im = mo.moe_forward(x, wg, wgu, wdn, k, True, intermediates=True)
    assert torch.equal(out, torch.from_numpy(c1["c1_grouped_triton__out"]))
    assert np.array_equal(im["idx"].numpy(), c1["c1_grouped_triton__idx"].astype(np.int64))
    assert torch.equal(im["weights"], torch.from_numpy(c1["c1_grouped_triton__weights"]))
    aux = mo.load_balancing_loss(im["probs"], im["idx"], e)
    assert abs(float(aux) - float(c1["c1_grouped_triton__aux_loss"])) < 1e-6
    assert np.array_equal(mo.expert_counts(im["idx"], e).numpy(), c1["c1_grouped_triton__expert_counts"])


def test_c1_origin_formulation(c1):
    (x, wg, wgu, wdn), k, _ = _c1_inputs(c1)
    origin = mo.moe_forward_origin(x, wg, wgu, wdn, k)
    assert torch.allclose(origin[:32], torch.from_numpy(c1["c1_origin__out"]), rtol=1e-5, atol=1e-6)
    grouped = mo.moe_forward(x, wg, wgu, wdn, k)
    assert torch.allclose(origin, grouped, rtol=1e-5, atol=1e-6)


def test_c1_planted_gate_up_swap_is_caught(c1):
    (x, wg, wgu, wdn), k, _ = _c1_inputs(c1)
    i = wgu.shape[1] // 2
    swapped = torch.cat([wgu[:, i:], wgu[:, :i]], dim=1)
    out = mo.moe_forward(x, wg, swapped, wdn, k)
    assert not torch.allclose(out, torch.from_numpy(c1["c1_grouped_triton__out"]), atol=1e-4)


def test_bf16_small_golden_bit_exact(c1):
    t, h, e, i, k, seed = [int(v) for v in c1["bf16s__shape"]]
    x, wg, wgu, wdn = synth.moe_inputs(seed, t, h, e, i)
    bf = torch.bfloat16
    out, im = mo.moe_forward(*(torch.from_numpy(a).to(bf) for a in (x, wg, wgu, wdn)), k, True, intermediates=True)
    ref = torch.from_numpy(c1["bf16s__out_bits"].view(np.int16)).view(bf)
    assert torch.equal(out, ref)
    assert np.array_equal(im["idx"].numpy(), c1["bf16s__idx"].astype(np.int64))
    assert np.array_equal(im["weights"].view(torch.int16).numpy().view(np.uint16), c1["bf16s__weights_bits"])


# ------------------------------------------------------------ experts_vjp ----

def test_experts_vjp_matches_c1_golden_weight_grads(c1):
    """Expert weight gradients of the reference module itself (fp32, loss sum(out * grad) + aux)."""
    (x, wg, wgu, wdn), k, e = _c1_inputs(c1)
    t, h = x.shape
    grad = torch.from_numpy(synth.normal(12, (t, h)))
    _, w, idx = mo.router_topk(F.linear(x, wg), k, True, x.dtype)
    r = mo.experts_vjp(x, w, wgu, wdn, idx.numpy(), grad)
    assert torch.equal(r["out"], torch.from_numpy(c1["c1_grouped_triton__out"]))
    for name, got in (("gate_up", r["d_gate_up_weight"]), ("down", r["d_down_weight"])):
        want_rows = torch.from_numpy(c1[f"c1_grouped_triton__{name}_grad_e0_rows0_3"])
        assert torch.allclose(got[0, :4], want_rows, rtol=1e-4, atol=1e-6), name
        sq = float(got.double().pow(2).sum())
        want_sq = float(c1[f"c1_grouped_triton__{name}_grad_sq_sum"])
        assert abs(sq / want_sq - 1.0) < 1e-5, name


def _origin_experts(h, w, wgu, wdn, idx):
    """Per-expert loop (models/layers.py:497-506) on the given routing, differentiable."""
    out = torch.zeros_like(h)
    for e in range(wgu.shape[0]):
        tok, slot = torch.where(idx == e)
        if tok.numel() == 0:
            continue
        gate, up = (h[tok] @ wgu[e].T).chunk(2, dim=-1)
        y = (F.silu(gate) * up) @ wdn[e].T
        out = out.index_add(0, tok, y * w[tok, slot, None])
    return out


def test_experts_vjp_matches_origin_formulation_and_finite_differences():
    t, h, e, i, k = 40, 24, 6, 16, 3
    rng = np.random.default_rng(5)
    idx = np.argsort(rng.random((t, e)), axis=1)[:, :k]
    x, wgu, wdn, w, g = (torch.from_numpy(rng.standard_normal(s)).double() for s in
                         ((t, h), (e, 2 * i, h), (e, h, i), (t, k), (t, h)))
    wgu, wdn = wgu * 0.2, wdn * 0.2
    r = mo.experts_vjp(x, w, wgu, wdn, idx, g)
    leaves = [a.clone().requires_grad_(True) for a in (x, w, wgu, wdn)]
    out = _origin_experts(*leaves, torch.from_numpy(idx))
    assert torch.allclose(out, r["out"], rtol=1e-12, atol=1e-12)
    out.backward(g)
    for name, leaf in zip(("d_hidden", "d_weights", "d_gate_up_weight", "d_down_weight"), leaves):
        assert torch.allclose(r[name], leaf.grad, rtol=1e-10, atol=1e-12), name
    # directional derivative of <g, out> along a random direction of every input
    dirs = [torch.from_numpy(rng.standard_normal(a.shape)) for a in (x, w, wgu, wdn)]
    eps = 1e-6

    def f(s):
        return float((mo.experts_vjp(*(a + s * v for a, v in zip((x, w, wgu, wdn), dirs)), idx, g)["out"] * g).sum())

    fd = (f(eps) - f(-eps)) / (2 * eps)
    an = sum(float((r[n] * v).sum()) for n, v in zip(("d_hidden", "d_weights", "d_gate_up_weight",
                                                       "d_down_weight"), dirs))
    assert abs(fd - an) <= 1e-6 * max(1.0, abs(an))


def test_experts_vjp_planted_wrong_swiglu_grad_is_caught():
    """A transposed gate/up pairing in the backward would fail the origin comparison above:
    check that the comparison discriminates by planting the swap in the forward weights."""
    t, h, e, i, k = 16, 8, 3, 4, 2
    rng = np.random.default_rng(9)
    idx = np.argsort(rng.random((t, e)), axis=1)[:, :k]
    x, wgu, wdn, w, g = (torch.from_numpy(rng.standard_normal(s)).double() for s in
                         ((t, h), (e, 2 * i, h), (e, h, i), (t, k), (t, h)))
    r = mo.experts_vjp(x, w, wgu, wdn, idx, g)
    swapped = torch.cat([wgu[:, i:], wgu[:, :i]], dim=1)
    r2 = mo.experts_vjp(x, w, swapped, wdn, idx, g)
    assert not torch.allclose(r["d_hidden"], r2["d_hidden"], atol=1e-6)


def test_training_chain_reproduces_c1_golden_router_and_input_grads(c1):
    """experts_vjp + router_vjp + the aux loss give the reference module's gate and input gradients."""
    (x, wg, wgu, wdn), k, e = _c1_inputs(c1)
    t, h = x.shape
    grad = torch.from_numpy(synth.normal(12, (t, h)))
    logits = F.linear(x, wg)
    probs, w, idx = mo.router_topk(logits, k, True, x.dtype)
    r = mo.experts_vjp(x, w, wgu, wdn, idx.numpy(), grad)
    p = probs.detach().clone().requires_grad_(True)
    mo.load_balancing_loss(p, idx, e).backward()
    dlogits = mo.router_vjp(logits, True, idx.numpy(), r["d_weights"], p.grad)
    gate_grad = dlogits.T @ x
    x_grad = r["d_hidden"] + dlogits @ wg
    assert torch.allclose(gate_grad, torch.from_numpy(c1["c1_grouped_triton__gate_grad"]), rtol=1e-4, atol=1e-6)
    assert torch.allclose(x_grad[:16], torch.from_numpy(c1["c1_grouped_triton__x_grad_rows0_15"]), rtol=1e-4,
                          atol=1e-6)
    sq = float(x_grad.double().pow(2).sum())
    assert abs(sq / float(c1["c1_grouped_triton__x_grad_sq_sum"]) - 1.0) < 1e-5


def test_router_vjp_finite_differences():
    t, e, k = 12, 10, 3
    rng = np.random.default_rng(3)
    z = torch.from_numpy(rng.standard_normal((t, e)))
    idx = torch.topk(F.softmax(z, -1), k).indices
    gw = torch.from_numpy(rng.standard_normal((t, k)))
    gp = torch.from_numpy(rng.standard_normal((t, e)))
    v = torch.from_numpy(rng.standard_normal((t, e)))
    for norm in (True, False):
        dz = mo.router_vjp(z, norm, idx.numpy(), gw, gp)

        def f(s):
            p = F.softmax(z + s * v, dim=-1, dtype=torch.float64)
            sel = p.gather(1, idx)
            w = sel / sel.sum(-1, keepdim=True) if norm else sel
            return float((w * gw).sum() + (p * gp).sum())

        eps = 1e-6
        fd = (f(eps) - f(-eps)) / (2 * eps)
        assert abs(fd - float((dz * v).sum())) < 1e-6
