"""The router kernel's top-k ordering code, compiled for the host, against the oracle.

hrm-moe_amd/csrc/topk_order.h is shared by the router kernel and
tests/hostcheck/topk_order_check.cpp.  This test builds the latter with g++
and checks every k from 1 to 32 against oracle.topk_rocm, which is pinned to
torch.topk on an MI355X (tests/golden/topk_ties_rocm.npz).
"""
import ctypes
import os
import subprocess

import numpy as np
import pytest

from oracle import moe_oracle as mo

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "hostcheck", "topk_order_check.cpp")
HDR_DIR = os.path.join(os.path.dirname(HERE), "hrm-moe_amd", "csrc")


@pytest.fixture(scope="module")
def host_lib(tmp_path_factory):
    out = str(tmp_path_factory.mktemp("hostcheck") / "libtopk_order_check.so")
    subprocess.run(["g++", "-O1", "-std=c++17", "-shared", "-fPIC", f"-I{HDR_DIR}", SRC, "-o", out], check=True)
    lib = ctypes.CDLL(out)
    lib.topk_order_check.restype = ctypes.c_int
    lib.topk_order_check.argtypes = [ctypes.c_int32, ctypes.c_int64] + [ctypes.c_void_p] * 4 + [ctypes.c_int32]
    return lib


def run_host_order(lib, vals, k, loop_form=0):
    t, e = vals.shape
    order = np.lexsort((np.broadcast_to(np.arange(e), (t, e)), -vals), axis=-1)[:, :k]
    keys = (np.take_along_axis(vals, order, 1).view(np.uint32) + 1).astype(np.uint32)
    sel = order.astype(np.int32)
    out_idx = np.zeros((t, k), np.int32)
    out_sum = np.zeros(t, np.float32)
    rc = lib.topk_order_check(k, t, keys.ctypes.data, sel.ctypes.data, out_idx.ctypes.data, out_sum.ctypes.data,
                              loop_form)
    assert rc == 0
    return out_idx.astype(np.int64), out_sum


@pytest.mark.parametrize("loop_form", [0, 1])
@pytest.mark.parametrize("k", list(range(1, 33)))
def test_ordering_matches_oracle_for_every_k(host_lib, k, loop_form):
    rng = np.random.default_rng(k)
    vals = (rng.integers(0, 4, size=(600, 64)).astype(np.float32) * 0.125 + 0.0625)
    got, got_sum = run_host_order(host_lib, vals, k, loop_form)
    _, want = mo.topk_rocm(vals, k)
    assert np.array_equal(got, want)
    if loop_form:
        _, reg_sum = run_host_order(host_lib, vals, k, 0)
        assert np.array_equal(got_sum, reg_sum)


@pytest.mark.parametrize("k", [2, 4, 8, 16, 32])
def test_compile_time_k_form_matches_oracle(host_lib, k):
    """The router's k == SLOTS specialisation (k fixed at compile time)."""
    rng = np.random.default_rng(100 + k)
    vals = (rng.integers(0, 4, size=(600, 64)).astype(np.float32) * 0.125 + 0.0625)
    got, got_sum = run_host_order(host_lib, vals, k, 2)
    _, want = mo.topk_rocm(vals, k)
    assert np.array_equal(got, want)
    _, reg_sum = run_host_order(host_lib, vals, k, 0)
    assert np.array_equal(got_sum, reg_sum)


def test_ordering_matches_device_fixture(host_lib):
    d = np.load(os.path.join(HERE, "golden", "topk_ties_rocm.npz"))
    for case in ("e64_k8_l4", "e128_k8_l8", "e8_k2_l3", "e8_k3_l3", "e64_k4_l6"):
        vals = d[case + "__levels"].astype(np.float32) * 0.0625 + 0.03125
        gpu = d[case + "__gpu_idx"].astype(np.int64)
        got, _ = run_host_order(host_lib, vals, gpu.shape[1])
        assert np.array_equal(got, gpu), case


def test_weight_sum_order_is_pairwise_for_eight(host_lib):
    rng = np.random.default_rng(3)
    vals = rng.random((500, 64)).astype(np.float32)
    got_idx, got_sum = run_host_order(host_lib, vals, 8)
    w = np.take_along_axis(vals, got_idx, 1)
    pair = ((w[:, 0] + w[:, 1]) + (w[:, 2] + w[:, 3])) + ((w[:, 4] + w[:, 5]) + (w[:, 6] + w[:, 7]))
    assert np.array_equal(got_sum, pair.astype(np.float32))


@pytest.mark.parametrize("loop_form", [0, 2])
@pytest.mark.parametrize("k", [1, 2, 3, 4, 5, 6, 7, 8, 16, 32])
def test_distinct_and_tied_rows_mixed(host_lib, k, loop_form):
    """Rows whose selected keys are all distinct (torch's order is then plain
    descending order) mixed with rows that have ties among them, against the
    oracle and against the loop form's weight sums."""
    if loop_form == 2 and k not in (2, 4, 8, 16, 32):
        pytest.skip("the compile-time form exists for k == SLOTS only")
    rng = np.random.default_rng(500 + k)
    vals = rng.random((800, 64)).astype(np.float32)
    tied = rng.random(800) < 0.3
    vals[tied] = (rng.integers(0, 5, size=(int(tied.sum()), 64)).astype(np.float32) * 0.125 + 0.0625)
    got, got_sum = run_host_order(host_lib, vals, k, loop_form)
    _, want = mo.topk_rocm(vals, k)
    assert np.array_equal(got, want)
    _, mem_sum = run_host_order(host_lib, vals, k, 1)
    assert np.array_equal(got_sum, mem_sum)
    # distinct rows: torch's order is the descending (value, then index) order
    order = np.lexsort((np.broadcast_to(np.arange(64), vals.shape), -vals), axis=-1)[:, :k]
    assert np.array_equal(got[~tied], order[~tied])
