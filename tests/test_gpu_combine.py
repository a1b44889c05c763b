"""The combine kernel against the oracle's combine, bit for bit.

The oracle restates models/layers.py:333-334 on the CPU (weighted rows,
index_add_ into zeros), which adds each token's k products in fp32 in
ascending row order and rounds once; the kernel does the same sums, so the
outputs must be identical.  Cases cover the compile-time top-k paths (2, 4, 8),
the generic path (1, 3, 5, 16), token counts that do not fill the last block of
tokens, widths that are not a multiple of the block, and fp16 / fp32 rows.
"""
import numpy as np
import pytest
import torch

from hrm_moe_amd import _lib, ops
from oracle import moe_oracle as mo
from oracle import synth

pytestmark = pytest.mark.gpu


def _distinct_topk(seed, t, e, k):
    rng = np.random.default_rng(seed)
    return np.argsort(rng.random((t, e)), axis=1)[:, :k].astype(np.int64)


@pytest.mark.parametrize("t,h,e,k,dtype", [
    (1, 256, 8, 2, torch.bfloat16),
    (13, 1280, 64, 8, torch.bfloat16),
    (1000, 1536, 64, 8, torch.bfloat16),
    (37, 264, 16, 4, torch.bfloat16),
    (29, 512, 8, 1, torch.bfloat16),
    (50, 1280, 16, 3, torch.bfloat16),
    (45, 520, 32, 5, torch.float16),
    (21, 256, 32, 16, torch.bfloat16),
    (64, 384, 8, 2, torch.float32),
])
def test_combine_bit_exact(cuda, t, h, e, k, dtype):
    idx = _distinct_topk(t * 7 + k, t, e, k)
    d = ops.permute(torch.from_numpy(idx).to(cuda), e)
    perm = mo.permute(idx, e)
    y = torch.from_numpy(synth.normal(t + h, (t * k, h))).to(dtype)
    w = torch.from_numpy(synth.normal(t + 3, (t, k), std=0.3)).to(dtype)
    out = ops.combine(y.to(cuda), d, w.to(cuda))
    sorted_w = w.reshape(-1)[torch.from_numpy(perm["sort_idx"])]
    ref = mo.combine(y, sorted_w, perm["sorted_token_idx"], t)
    assert out.dtype == dtype and out.shape == (t, h)
    assert torch.equal(out.cpu(), ref)


@pytest.mark.parametrize("t,h,e,k,dtype", [(13, 1280, 64, 8, torch.bfloat16), (45, 520, 32, 5, torch.float16),
                                           (64, 384, 8, 2, torch.float32)])
def test_combine_unit_weights(cuda, t, h, e, k, dtype):
    """No weight tensor: the plain sum of each token's rows (the backward's un-permute), checked
    against the oracle's combine with weights of one."""
    idx = _distinct_topk(t * 5 + k, t, e, k)
    d = ops.permute(torch.from_numpy(idx).to(cuda), e)
    perm = mo.permute(idx, e)
    y = torch.from_numpy(synth.normal(t + h + 1, (t * k, h))).to(dtype)
    out = ops.combine(y.to(cuda), d, None, top_k=k)
    ref = mo.combine(y, torch.ones(t * k, dtype=dtype), perm["sorted_token_idx"], t)
    assert torch.equal(out.cpu(), ref)


@pytest.mark.parametrize("t,h,e,i,k,dtype", [
    (1, 1536, 64, 512, 8, torch.bfloat16), (2, 1280, 64, 448, 8, torch.bfloat16), (1, 256, 8, 128, 2, torch.float16),
    (2, 512, 16, 64, 4, torch.bfloat16), (1, 1536, 64, 512, 1, torch.bfloat16), (2, 96, 8, 32, 3, torch.bfloat16),
    (2, 72, 8, 96, 5, torch.float16)])
def test_down_combine_decode(cuda, t, h, e, i, k, dtype):
    """The one-launch down projection + combine for one or two tokens, checked against float64 products of the
    same 16-bit inputs (the reference's math) and against the two-launch path (grouped GEMM, then combine): bit
    for bit where the grouped GEMM runs its skinny kernel, whose dot-product order the fused kernel follows,
    within tolerance where a tiled kernel sums in another order."""
    idx = _distinct_topk(t * 11 + k + i, t, e, k)
    idx_t = torch.from_numpy(idx).to(cuda)
    d = ops.permute(idx_t, e)
    perm = mo.permute(idx, e)
    act = torch.from_numpy(synth.normal(t + i, (t * k, i))).to(dtype)
    wdn = torch.from_numpy(synth.normal(h + i, (e, h, i), std=0.05)).to(dtype)
    w = torch.from_numpy(np.abs(synth.normal(t + 5, (t, k), std=0.3)) + 0.05).to(dtype)
    assert ops.down_combine_decode_ok(act, wdn, w)
    fused = ops.down_combine_decode(act.to(cuda), wdn.to(cuda), d, idx_t, w.to(cuda))
    y = ops.grouped_gemm_nt(act.to(cuda), wdn.to(cuda), d.tokens_per_expert)
    skinny = _lib.last_gemm_kernel(_lib.GEMM_KIND_NT).startswith("mgemm_skinny")
    two = ops.combine(y, d, w.to(cuda))
    # float64 reference: row r of act belongs to sorted position r, whose slot is sort_idx[r]
    sort_idx = perm["sort_idx"]
    rows_e = idx.reshape(-1)[sort_idx]
    yref = torch.einsum("ri,rhi->rh", act.double(), wdn.double()[torch.from_numpy(rows_e)])
    sw = w.reshape(-1)[torch.from_numpy(sort_idx)].double()
    ref = torch.zeros(t, h, dtype=torch.float64).index_add_(0, torch.from_numpy(perm["sorted_token_idx"]).long(),
                                                            yref * sw[:, None])
    got, got2 = fused.double().cpu(), two.double().cpu()
    scale = ref.abs().max().item()
    rel = (got - ref).abs().max().item() / scale
    print(f"down_combine_decode t={t} k={k}: max rel err {rel:.2e} (two-launch "
          f"{(got2 - ref).abs().max().item() / scale:.2e}), fused vs two-launch max |d| "
          f"{(got - got2).abs().max().item():.2e}")
    assert fused.dtype == dtype and fused.shape == (t, h)
    assert rel <= 2e-2
    assert (got - got2).abs().max().item() <= 2e-2 * scale
    assert skinny == (t * k <= e // 4 and h % 16 == 0)
    if skinny:
        assert torch.equal(fused, two)
    again = ops.down_combine_decode(act.to(cuda), wdn.to(cuda), d, idx_t, w.to(cuda))
    assert torch.equal(fused, again)
