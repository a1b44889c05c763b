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

from hrm_moe_amd import ops
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
