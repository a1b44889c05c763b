"""The wgrad work plan under skewed expert loads, on the GPU.

The reference's K-grouped wgrad kernel (models/moe_triton_grouped_gemm.py:
277-347) walks each expert's whole row range per output tile, so a heavily
loaded expert bounds its time.  Here the plan (wgrad_plan_kernel) splits an
expert holding more than twice the mean rows (at least 2048) into row chunks
reduced through fp32 partial sums added in chunk order, cuts the row groups
into 8 runs of about equal rows (one per XCD) and orders each run largest
first.  Checked:
  * the device plan equals a host restatement of those rules (white box: the
    plan is read back from the caller's workspace);
  * weight gradients of split experts, unsplit ones and empty ones against
    the oracle (fp32 accumulation, one rounding): max|d| <= 1e-2 max|ref|,
    mean|d| <= 2e-3 mean|ref|; with splitting against a workspace too small
    for partial slots (no splits), within the same bar; repeated runs are
    bit-identical;
  * with gathered B rows (the gate_up wgrad) the same.
"""
import ctypes

import numpy as np
import pytest
import torch

from hrm_moe_amd import _lib, ops
from oracle import moe_oracle as mo
from oracle import synth

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


def _align(x):
    return (x + 255) & ~255


def plan_model(tpe, m, max_slots):
    """Host restatement of wgrad_plan_kernel: groups (expert, start, end, slot), order, runs, splits."""
    e = len(tpe)
    rows = np.maximum(np.asarray(tpe, np.int64), 0)
    ends = np.cumsum(rows)
    rs = np.minimum(ends - rows, m)
    n = np.minimum(ends, m) - rs
    chunk = max(2048, 2 * ((m + e - 1) // e)) if max_slots > 0 else 1 << 40
    while int(sum((x + chunk - 1) // chunk for x in n if x > chunk)) > max_slots:
        chunk *= 2
    groups, splits, slot = [], [], 0
    for ex in range(e):
        c = (n[ex] + chunk - 1) // chunk if n[ex] > chunk else 1
        if c > 1:
            splits.append((ex, slot, c))
        for j in range(c):
            s0 = rs[ex] + j * chunk
            groups.append((ex, int(s0), int(min(s0 + chunk, rs[ex] + n[ex])), slot + j if c > 1 else -1))
        if c > 1:
            slot += c
    cost = np.array([g[2] - g[1] + 64 for g in groups], np.int64)
    cum = np.cumsum(cost)
    xcd = np.minimum(((cum - cost // 2) * 8) // cum[-1], 7)
    order = sorted(range(len(groups)), key=lambda g: (xcd[g], -cost[g], g))
    runs = [(int(np.searchsorted(xcd[order], x, "left")), int(np.sum(xcd == x))) for x in range(8)]
    runs = [(s if c else 0, c) for s, c in runs]
    return groups, order, runs, splits, rs, n


def skewed_tpe(m, e, seed):
    rng = np.random.default_rng(seed)
    w = rng.lognormal(0.0, 1.2, e)
    w[rng.integers(0, e, 3)] = 0.0
    w[0] = w.sum() * 0.15  # one expert with about 13% of the rows
    tpe = np.floor(w / w.sum() * m).astype(np.int64)
    tpe[1] += m - tpe.sum()
    return tpe


def _wgrad_raw(lib, a, b, tpe_d, e, ws, idx=None, b_rows=0):
    m, na = a.shape
    nb = b.shape[1]
    c = torch.empty((e, na, nb), dtype=a.dtype, device=a.device)
    p = _lib.ptr
    if idx is None:
        st = lib.hrm_moe_grouped_gemm_tn(p(a), p(b), p(tpe_d), m, na, nb, e, _lib.BF16, p(c), p(ws), ws.numel(),
                                         _lib.stream_of(a.device))
    else:
        st = lib.hrm_moe_grouped_gemm_tn_gather(p(a), p(b), p(idx), b_rows, p(tpe_d), m, na, nb, e, _lib.BF16, p(c),
                                                p(ws), ws.numel(), _lib.stream_of(a.device))
    assert st == _lib.OK, _lib.status_string(st)
    torch.cuda.synchronize()
    return c


def _read_plan(ws, m, e, lib):
    """(row_offsets, groups, order, info, splits) from the plan region of a wgrad workspace."""
    base = lib.hrm_moe_grouped_gemm_workspace_size(m, e)
    g = e + e // 2 + 2
    plan_bytes = _align(4 * (e + 1)) + _align(16 * g) + _align(4 * g) + _align(4 * 64) + _align(16 * e)
    raw = ws[base - plan_bytes: base].cpu().numpy()
    off = 0

    def take(nbytes, dtype, count):
        nonlocal off
        arr = raw[off: off + nbytes].view(dtype)[:count]
        off += _align(nbytes)
        return arr
    row_offsets = take(4 * (e + 1), np.int32, e + 1)
    groups = take(16 * g, np.int32, 4 * g).reshape(g, 4)
    order = take(4 * g, np.int32, g)
    info = take(4 * 64, np.int32, 64)
    splits = take(16 * e, np.int32, 4 * e).reshape(e, 4)
    return row_offsets, groups, order, info, splits


CASES = [
    # m, na, nb, e
    (131072, 512, 1536, 64),   # the XL-skew down-projection wgrad shape
    (40000, 256, 512, 16),
    (9000, 256, 256, 8),
]


@pytest.mark.parametrize("m,na,nb,e", CASES)
def test_wgrad_plan_and_split_results(cuda, m, na, nb, e):
    print(f"case: skewed wgrad M={m} Na={na} Nb={nb} E={e}", flush=True)
    lib = _lib.load()
    tpe = skewed_tpe(m, e, m + e)
    tpe_d = torch.from_numpy(tpe).to(cuda)
    a = torch.from_numpy(synth.normal(m + 1, (m, na))).to(BF).to(cuda)
    b = torch.from_numpy(synth.normal(m + 2, (m, nb))).to(BF).to(cuda)
    full = lib.hrm_moe_grouped_wgrad_workspace_size(m, na, nb, e)
    base = lib.hrm_moe_grouped_gemm_workspace_size(m, e)
    assert full > base
    ws = torch.zeros(full, dtype=torch.uint8, device=cuda)
    got = _wgrad_raw(lib, a, b, tpe_d, e, ws)

    max_slots = min(e, (full - base) // (4 * na * nb))
    groups, order, runs, splits, rs, n = plan_model(tpe, m, max_slots)
    row_offsets, dgroups, dorder, info, dsplits = _read_plan(ws, m, e, lib)
    G = len(groups)
    assert info[16] == G and info[17] == len(splits)
    assert np.array_equal(row_offsets[:e], rs) and row_offsets[e] == rs[-1] + n[-1]
    assert np.array_equal(dgroups[:G], np.array(groups, np.int32)), "groups"
    assert np.array_equal(dorder[:G], np.array(order, np.int32)), "order"
    assert [tuple(info[2 * x: 2 * x + 2]) for x in range(8)] == runs, "XCD runs"
    assert np.array_equal(dsplits[: len(splits), :3], np.array(splits, np.int32).reshape(-1, 3)), "splits"
    assert len(splits) >= 1, "the skewed load splits at least its heaviest expert"
    loads = [sum(groups[order[s + j]][2] - groups[order[s + j]][1] for j in range(c)) for s, c in runs]
    print(f"rows per XCD run: {loads}; split experts {[s[0] for s in splits]}")

    # results: split experts, empty experts and the rest against the oracle
    pick = sorted({s[0] for s in splits} | set(np.where(tpe == 0)[0][:1].tolist()) | {1, e // 2, e - 1})
    starts = np.concatenate([[0], np.cumsum(tpe)])
    a_s = torch.cat([a[starts[x]:starts[x + 1]].cpu() for x in pick])
    b_s = torch.cat([b[starts[x]:starts[x + 1]].cpu() for x in pick])
    ref = mo.grouped_linear_wgrad(a_s, b_s, tpe[pick])
    d = (got[pick].float().cpu() - ref).abs()
    print(f"wgrad experts {pick}: max|d|/max|ref| {d.max().item() / ref.abs().max().item():.2e}")
    assert d.max().item() <= 1e-2 * ref.abs().max().item()
    assert d.mean().item() <= 2e-3 * ref.abs().mean().item()
    for x in np.where(tpe == 0)[0]:
        assert torch.count_nonzero(got[x]) == 0

    # no room for partial slots: whole experts, same results within the bar; repeat runs bit-identical
    small = torch.zeros(base, dtype=torch.uint8, device=cuda)
    whole = _wgrad_raw(lib, a, b, tpe_d, e, small)
    d2 = (whole.float() - got.float()).abs()
    assert d2.max().item() <= 1e-2 * got.float().abs().max().item()
    unsplit = [x for x in range(e) if x not in {s[0] for s in splits}]
    assert torch.equal(whole[unsplit], got[unsplit]), "unsplit experts keep their bits"
    assert torch.equal(got, _wgrad_raw(lib, a, b, tpe_d, e, ws)), "not deterministic"


def test_wgrad_gather_split(cuda):
    """Gathered B rows (the gate_up wgrad) with split experts equal the wgrad over materialised rows."""
    m, na, nb, e, b_rows = 65536, 1024, 512, 32, 8192
    print(f"case: skewed gathered wgrad M={m} Na={na} Nb={nb} E={e}", flush=True)
    tpe = skewed_tpe(m, e, 7)
    tpe_d = torch.from_numpy(tpe).to(cuda)
    g = torch.from_numpy(synth.normal(71, (m, na))).to(BF).to(cuda)
    h = torch.from_numpy(synth.normal(72, (b_rows, nb))).to(BF).to(cuda)
    idx = torch.from_numpy(np.random.default_rng(73).integers(0, b_rows, size=m)).to(torch.int32).to(cuda)
    got = ops.grouped_gemm_tn_gather(g, h, idx, tpe_d)
    want = ops.grouped_gemm_tn(g, h.index_select(0, idx.long()), tpe_d)
    assert torch.equal(got, want)
    x = int(np.argmax(tpe))
    starts = np.concatenate([[0], np.cumsum(tpe)])
    rows = slice(int(starts[x]), int(starts[x + 1]))
    ref = mo.grouped_linear_wgrad(g[rows].cpu(), h.index_select(0, idx[rows].long()).cpu(), tpe[[x]])
    d = (got[x].float().cpu() - ref[0]).abs()
    print(f"heaviest expert {x} ({tpe[x]} rows): max|d|/max|ref| {d.max().item() / ref.abs().max().item():.2e}")
    assert d.max().item() <= 1e-2 * ref.abs().max().item()
