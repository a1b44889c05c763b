"""ctypes binding of the C ABI in include/hrm_moe.h (libhrm_moe.so).

torch is imported before the library is loaded, so the library's
libamdhip64.so.7 dependency resolves to the HIP runtime torch already
loaded: one runtime per process, and torch's streams and device pointers are
valid in the kernels.

There is no fallback: if the library is missing, every op raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (must be loaded before the kernel library)

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "libhrm_moe.so")
ABI_VERSION = 1

OK = 0
ERR_INVALID = -1
ERR_DTYPE = -2
ERR_UNSUPPORTED = -3
ERR_WORKSPACE = -4

BF16, F16, F32 = 0, 1, 2
DTYPE_CODE = {torch.bfloat16: BF16, torch.float16: F16, torch.float32: F32}

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
_INT = ctypes.c_int
_SZ = ctypes.c_size_t

# name -> (restype, argtypes); must match include/hrm_moe.h.
PROTOTYPES = {
    "hrm_moe_abi_version": (_INT, []),
    "hrm_moe_status_string": (ctypes.c_char_p, [_INT]),
    "hrm_moe_reload_config": (_INT, []),
    "hrm_moe_cu_margin": (_INT, []),
    "hrm_moe_last_gemm_kernel": (ctypes.c_char_p, [_INT]),
    "hrm_moe_router_topk": (_INT, [_P, _INT, _I64, _I32, _I32, _I32, _P, _P, _P, _INT, _P]),
    "hrm_moe_permute_workspace_size": (_SZ, [_I64, _I32, _I32]),
    "hrm_moe_permute": (_INT, [_P, _I64, _I32, _I32, _P, _P, _P, _P, _P, _P, _SZ, _P]),
    "hrm_moe_grouped_gemm_workspace_size": (_SZ, [_I64, _I32]),
    "hrm_moe_grouped_wgrad_workspace_size": (_SZ, [_I64, _I64, _I64, _I32]),
    "hrm_moe_grouped_gemm_nt": (_INT, [_P, _P, _P, _I64, _I64, _I64, _I32, _INT, _P, _P, _SZ, _P]),
    "hrm_moe_grouped_gemm_nn": (_INT, [_P, _P, _P, _I64, _I64, _I64, _I32, _INT, _P, _P, _SZ, _P]),
    "hrm_moe_grouped_gemm_tn": (_INT, [_P, _P, _P, _I64, _I64, _I64, _I32, _INT, _P, _P, _SZ, _P]),
    "hrm_moe_gate_up_swiglu": (_INT, [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I32, _INT, _P, _P, _SZ, _P]),
    "hrm_moe_combine": (_INT, [_P, _P, _P, _P, _I64, _I32, _I64, _I32, _INT, _P, _P]),
    "hrm_moe_down_combine_decode": (_INT, [_P, _P, _P, _P, _P, _P, _I64, _I32, _I64, _I64, _I32, _INT, _P, _P]),
    "hrm_moe_router_gate_up_decode_supported": (_INT, [_I64, _I64, _I64, _I32, _I32]),
    "hrm_moe_router_gate_up_decode": (_INT, [_P, _INT, _P, _P, _I64, _I64, _I64, _I32, _I32, _I32, _INT, _P, _P, _P,
                                             _P, _P, _P, _P, _P, _P, _P]),
    "hrm_moe_gate_up_swiglu_save": (_INT, [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I32, _INT, _P, _P, _P, _SZ, _P]),
    "hrm_moe_down_dgrad_swiglu": (_INT, [_P, _P, _P, _P, _I64, _I64, _I64, _I32, _INT, _P, _P, _SZ, _P]),
    "hrm_moe_combine_backward": (_INT, [_P, _P, _P, _P, _P, _I64, _I32, _I64, _I32, _INT, _P, _P, _P]),
    "hrm_moe_router_dispatch_workspace_size": (_SZ, [_I64, _I32, _I32]),
    "hrm_moe_router_topk_dispatch": (_INT, [_P, _INT, _I64, _I32, _I32, _I32, _P, _P, _P, _INT, _P, _P, _P, _P, _P,
                                            _P, _SZ, _P]),
    "hrm_moe_router_dispatch_noalloc_max_bytes": (_SZ, []),
    "hrm_moe_router_topk_dispatch_noalloc": (_INT, [_P, _INT, _I64, _I32, _I32, _I32, _P, _P, _P, _INT, _P, _P, _P,
                                                    _P, _P, _P]),
    "hrm_moe_gate_wgrad_workspace_size": (_SZ, [_I64, _I32, _I64]),
    "hrm_moe_gate_wgrad": (_INT, [_P, _P, _I64, _I32, _I64, _INT, _P, _P, _SZ, _P]),
    "hrm_moe_router_topk_backward": (_INT, [_P, _P, _P, _INT, _P, _I64, _I64, _I32, _I32, _I32, _P, _INT, _P]),
    "hrm_moe_grouped_gemm_tn_gather": (_INT, [_P, _P, _P, _I64, _P, _I64, _I64, _I64, _I32, _INT, _P, _P, _SZ, _P]),
    "hrm_moe_aux_loss_workspace_size": (_SZ, [_I64, _I32]),
    "hrm_moe_aux_loss": (_INT, [_P, _I64, _I32, _P, _P, _P, _P, _P, _SZ, _P]),
    "hrm_moe_aux_loss_backward": (_INT, [_P, _P, _I64, _I32, _P, _P]),
}

_lock = threading.Lock()
_lib = None


class KernelLibraryMissing(RuntimeError):
    pass


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load libhrm_moe.so once and attach the prototypes."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(path):
            raise KernelLibraryMissing(
                f"{path} is not built; build it with `python -c 'import __graft_entry__ as g; g.build()'` "
                "or `python hrm-moe_amd/build.py` (needs hipcc)")
        lib = ctypes.CDLL(path)
        for name, (res, args) in PROTOTYPES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        version = lib.hrm_moe_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"{path} has ABI version {version}, expected {ABI_VERSION}")
        _lib = lib
        return lib


def reload_config() -> None:
    """Make the library re-read its HRM_MOE_* tuning variables (tests switch kernel variants this way)."""
    check(load().hrm_moe_reload_config(), "reload_config")


GEMM_KIND_NT, GEMM_KIND_GATE_UP, GEMM_KIND_NN = 0, 1, 2


def last_gemm_kernel(kind: int) -> str:
    """Kernel instantiation of the latest grouped-GEMM launch of ``kind`` (a profiler kernel-name substring)."""
    return load().hrm_moe_last_gemm_kernel(kind).decode()


def status_string(status: int) -> str:
    return load().hrm_moe_status_string(status).decode()


def check(status: int, what: str) -> None:
    """Map a C ABI status to the exception the reference raises for the same condition."""
    if status == OK:
        return
    msg = f"{what}: {status_string(status)}"
    if status == ERR_DTYPE:
        raise TypeError(msg)
    if status in (ERR_INVALID, ERR_UNSUPPORTED, ERR_WORKSPACE):
        raise ValueError(msg)
    raise RuntimeError(msg)


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return DTYPE_CODE[dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {dtype}") from None


def lib() -> ctypes.CDLL:
    """The loaded library (fast path once loaded)."""
    return _lib if _lib is not None else load()


def ptr(t) -> int:
    """Device address of a tensor (0 for None), as ctypes passes it for void*."""
    return 0 if t is None else t.data_ptr()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(device: torch.device) -> int:
    """torch's current stream on ``device`` as a hipStream_t value."""
    if _raw_stream is not None:
        return _raw_stream(device.index)
    return torch.cuda.current_stream(device).cuda_stream


class _NoGuard:
    def __enter__(self):
        return None

    def __exit__(self, *exc):
        return False


_NO_GUARD = _NoGuard()


def device_guard(device: torch.device):
    """Make ``device`` current for the call (a no-op when it already is)."""
    if device.index is None or device.index == torch.cuda.current_device():
        return _NO_GUARD
    return torch.cuda.device(device)
