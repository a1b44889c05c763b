"""The no-allocation router + dispatch entry point against the workspace entry point, through the C ABI.

hrm_moe_router_topk_dispatch_noalloc has no counterpart in the reference: it
is hrm_moe_router_topk_dispatch (models/layers.py:606-610 and :312-322) with
its scratch in a fixed array inside the library, for callers that cannot
allocate.  Its outputs must equal the workspace entry point's bit for bit.
Calls run back to back, from the largest size the array serves down to small
ones, so each later call finds the previous call's data in the shared array
(nothing in it may need to start zeroed).
"""
import ctypes

import pytest
import torch

from hrm_moe_amd import _lib

pytestmark = pytest.mark.gpu
BF = torch.bfloat16

# T, E, k, norm: the maximum the array serves, then smaller inputs (quad router,
# single-block router, one-wave-per-token router)
CASES = [(32768, 128, 8, True), (4096, 64, 8, True), (700, 64, 8, True), (40, 64, 6, False), (12, 64, 8, True),
         (2048, 128, 4, True), (200, 64, 8, True)]


def _outputs(dev, t, e, k):
    r = t * k
    return dict(probs=torch.full((t, e), -1.0, device=dev), idx=torch.full((t, k), -1, dtype=torch.int64, device=dev),
                w=torch.full((t, k), -1.0, dtype=BF, device=dev),
                tpe=torch.full((e,), -1, dtype=torch.int64, device=dev),
                offs=torch.full((e + 1,), -1, dtype=torch.int32, device=dev),
                sti=torch.full((r,), -1, dtype=torch.int32, device=dev),
                sidx=torch.full((r,), -1, dtype=torch.int64, device=dev),
                s2r=torch.full((r,), -1, dtype=torch.int32, device=dev))


def _run(lib, logits, k, norm, noalloc):
    dev = logits.device
    t, e = logits.shape
    o = _outputs(dev, t, e, k)
    p = _lib.ptr
    args = [p(logits), _lib.dtype_code(logits.dtype), t, e, k, int(norm), p(o["probs"]), p(o["idx"]), p(o["w"]),
            _lib.BF16, p(o["tpe"]), p(o["offs"]), p(o["sti"]), p(o["sidx"]), p(o["s2r"])]
    stream = _lib.stream_of(dev)
    if noalloc:
        st = lib.hrm_moe_router_topk_dispatch_noalloc(*args, stream)
    else:
        ws = torch.empty(lib.hrm_moe_router_dispatch_workspace_size(t, e, k), dtype=torch.uint8, device=dev)
        st = lib.hrm_moe_router_topk_dispatch(*args, p(ws), ws.numel(), stream)
    assert st == _lib.OK, _lib.status_string(st)
    torch.cuda.synchronize()
    return o


def test_noalloc_matches_workspace_entry_point(cuda):
    lib = _lib.load()
    g = torch.Generator(device=cuda).manual_seed(17)
    for t, e, k, norm in CASES:
        print(f"case: noalloc router dispatch T={t} E={e} k={k} norm={norm}", flush=True)
        logits = torch.randn(t, e, device=cuda, generator=g).to(BF)
        logits[: t // 4, :8] = 0.5  # ties at the k / k+1 boundary for a quarter of the tokens
        want = _run(lib, logits, k, norm, noalloc=False)
        for rep in range(2):
            got = _run(lib, logits, k, norm, noalloc=True)
            for name in want:
                assert torch.equal(got[name], want[name]), (t, e, k, name, rep)


def test_noalloc_rejects_sizes_beyond_its_array(cuda):
    lib = _lib.load()
    cap = lib.hrm_moe_router_dispatch_noalloc_max_bytes()
    assert lib.hrm_moe_router_dispatch_workspace_size(32768, 128, 8) <= cap
    assert lib.hrm_moe_router_dispatch_workspace_size(32769, 128, 8) > cap
    buf = ctypes.c_void_p(1 << 20)  # never dereferenced: the call returns before launching
    st = lib.hrm_moe_router_topk_dispatch_noalloc(buf, _lib.BF16, 32769, 128, 8, 1, buf, buf, buf, _lib.BF16, buf,
                                                  buf, buf, buf, buf, None)
    assert st == _lib.ERR_UNSUPPORTED
