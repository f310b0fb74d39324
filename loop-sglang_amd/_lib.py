"""ctypes binding of libloopsgl_tok.so (the C ABI declared in include/loopsgl_tok.h).

There is no CPU fallback: every product entry point calls into the HIP library,
and a missing or unloadable library raises immediately.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_NAME = "libloopsgl_tok.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)

DTYPE_F32, DTYPE_BF16, DTYPE_F16 = 0, 1, 2
OP_EXIT_GATE, OP_REL_CHANGE = 1, 2
ABI_VERSION = 1

# Every symbol the header declares, with its ctypes signature.
_P, _I64, _I32, _F, _SZ = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_float, ctypes.c_size_t
SIGNATURES = {
    "lsg_sample": (ctypes.c_int, [_P, ctypes.c_int, _I64, _I64, _I64, _P, _P, _P, _P, _P, _I64, _P, _P, _P]),
    "lsg_exit_gate": (ctypes.c_int, [_P, ctypes.c_int, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _I32, _F,
                                     _I32, _I32, _I32, _P, _P, _P, _P, _P, _P, _SZ, _P]),
    "lsg_exit_gate_noalloc": (ctypes.c_int, [_P, ctypes.c_int, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P,
                                             _I32, _F, _I32, _I32, _I32, _P, _P, _P, _P, _P, _P]),
    "lsg_exit_gate_route": (ctypes.c_int, [_P, ctypes.c_int, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _I32,
                                           _F, _I32, _I32, _I32, _I32, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                           _SZ, _P]),
    "lsg_cumulative_exit_probability": (ctypes.c_int, [_P, ctypes.c_int, _P, _P, _I64, _P]),
    "lsg_relative_state_change": (ctypes.c_int, [_P, _P, ctypes.c_int, _I64, _I64, _I64, _I64, _F, _F, _P,
                                                 _P, _P, _P, _P, _P, _SZ, _P]),
    "lsg_lm_head": (ctypes.c_int, [_P, _I64, _I64, _I64, _P, _I64, _I64, _P, _I64, _P]),
    "lsg_lm_head_sample": (ctypes.c_int, [_P, _I64, _I64, _I64, _P, _I64, _I64, _P, _P, _P, _P, _P, _SZ, _P, _P]),
    "lsg_lm_head_workspace_bytes": (ctypes.c_size_t, [_I64, _I64]),
    "lsg_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int, _I64]),
    "lsg_last_error": (ctypes.c_char_p, []),
    "lsg_version": (ctypes.c_int, []),
}

_lib = None
_lock = threading.Lock()


def use_library(path: str) -> None:
    """Load `path` (the phase-stamp profiling build) instead of the product
    library; only before the first load()."""
    global LIB_PATH
    if _lib is not None:
        raise RuntimeError(f"{LIB_NAME} is already loaded from {LIB_PATH}")
    LIB_PATH = path


def load() -> ctypes.CDLL:
    """Load the HIP library once; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"{LIB_NAME} is not built ({LIB_PATH} missing); run __graft_entry__.build() "
                    "or python loop-sglang_amd/build.py")
            L = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(L, name)
                fn.restype = res
                fn.argtypes = args
            if L.lsg_version() != ABI_VERSION:
                raise RuntimeError(f"{LIB_NAME} ABI version {L.lsg_version()} != {ABI_VERSION}")
            _lib = L
    return _lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().lsg_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (code {rc}): {msg}")


def dtype_code(t: torch.Tensor) -> int:
    if t.dtype == torch.float32:
        return DTYPE_F32
    if t.dtype == torch.bfloat16:
        return DTYPE_BF16
    if t.dtype == torch.float16:
        return DTYPE_F16
    raise TypeError(f"unsupported dtype {t.dtype} (expected float32, bfloat16 or float16)")


def ptr(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(t: torch.Tensor):
    """The current torch stream of the tensor's device, as a hipStream_t."""
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def require_gpu(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor (the HIP library has no CPU path)")
