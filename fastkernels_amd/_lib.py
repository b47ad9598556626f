"""ctypes binding of libfastkernels_hip.so (declarations in include/fastkernels_hip.h).

The library is loaded lazily, after torch (so the process uses one HIP
runtime).  A missing library raises RuntimeError: there is no CPU fallback.
"""

from __future__ import annotations

import ctypes
import threading
from ctypes import c_float, c_int, c_int64, c_size_t, c_void_p, c_char_p
from pathlib import Path

LIB_NAME = "libfastkernels_hip.so"
LIB_PATH = Path(__file__).resolve().parent / LIB_NAME

FK_DTYPE_F32 = 0
FK_DTYPE_BF16 = 1
FK_DTYPE_I32 = 2
FK_DTYPE_I64 = 3

FK_OK = 0
FK_ERR_INVALID = 1
FK_ERR_DTYPE = 2
FK_ERR_WORKSPACE = 3
FK_ERR_LAUNCH = 4
FK_ERR_UNSUPPORTED = 5
FK_ERR_ALIGNMENT = 6
FK_ERR_DEVICE = 7

P = c_void_p
I = c_int

# name -> (restype, argtypes); mirrors include/fastkernels_hip.h.
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "fk_abi_version": (c_int, []),
    "fk_status_string": (c_char_p, [I]),
    "fk_last_error_detail": (c_char_p, []),
    "fk_workspace_status": (c_int, [P, c_size_t, I, P]),
    "fk_workspace_set_poll_limit": (c_int, [P, c_size_t, ctypes.c_longlong, P]),
    "fk_moe_workspace_bytes": (c_size_t, [I, I, I, I, I]),
    "fk_moe_router": (
        c_int,
        [P, I, P, I, P, I, P, I, I, I, I, I, c_float, c_float, P, P, P, P, c_size_t, P],
    ),
    "fk_moe_align": (c_int, [P, I, P, I, I, I, I, P, c_size_t, P, P, P, P, P]),
    "fk_moe_experts": (
        c_int,
        [P, I, P, P, I, P, P, P, I, I, I, I, I, I, P, P, P, c_size_t, P],
    ),
    "fk_moe_layer": (
        c_int,
        [P, I, P, I, P, I, P, I, P, P, I, P, P, P, I, I, I, I, I, I, c_float, c_float, P, P, P, P, P, P, c_size_t, P],
    ),
    "fk_moe_noalloc_workspace": (c_int, [P, P, P]),
    "fk_moe_layer_noalloc": (
        c_int,
        [P, I, P, I, P, I, P, I, P, P, I, P, P, P, I, I, I, I, I, I, c_float, c_float, P, P, P, P, P, P],
    ),
    "fk_expert_histogram": (c_int, [P, I, c_int64, I, P, P]),
    "fk_fused_swiglu": (c_int, [P, I, c_int64, I, P, P]),
    "fk_residual_add": (c_int, [P, I, P, c_int64, P, P]),
    "fk_stream_read": (c_int, [P, c_size_t, P, P]),
    "fk_attention_workspace_bytes": (c_size_t, [I, I, I, I]),
    "fk_attention_project": (c_int, [P, I, P, I, P, P, P, I, I, I, I, I, c_float, c_float, P, P, P, P]),
    "fk_attention_decode": (
        c_int,
        [P, I, P, I, P, P, P, P, I, P, P, I, P, P, I, I, I, P, I, I, I, I, I, I, c_float, I, c_float, c_float,
         P, P, P, c_size_t, P],
    ),
    "fk_deltanet_project": (
        c_int,
        [P, I, P, I, P, P, P, P, I, I, I, I, I, I, c_float, c_float, P, P, P, P, P],
    ),
    "fk_deltanet_conv": (c_int, [P, I, P, I, P, I, I, I, I, P, P, P]),
    "fk_deltanet_workspace_bytes": (c_size_t, [I, I, I]),
    "fk_deltanet_recurrent_output": (
        c_int,
        [P, P, P, P, P, P, P, P, P, P, P, I, I, I, I, I, c_float, P, P, P, P, c_size_t, P],
    ),
    "fk_deltanet_step_workspace_bytes": (c_size_t, [I, I, I, I]),
    "fk_deltanet_step": (
        c_int,
        [P, P, P, P, P, P, P, P, P, P, P, P, P, P, I, I, I, I, I, I, c_float, P, P, P, P, P, c_size_t, P],
    ),
    "fk_synthetic_moe":(c_int, [P, I, P, P, P, P, P, P, I, I, I, I, I, c_float, P, I, P]),
    "fk_synthetic_deltanet": (
        c_int,
        [P, I, P, I, P, P, P, P, P, P, I, I, I, I, I, c_float, P, P, P],
    ),
    "fk_synthetic_attention": (
        c_int,
        [P, I, P, P, I, P, P, P, P, P, I, I, I, I, I, I, I, I, c_float, P, P],
    ),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class FastKernelsError(RuntimeError):
    """A C-ABI call returned a non-zero status."""

    def __init__(self, fn: str, status: int, detail: str) -> None:
        super().__init__(f"{fn} failed: {status_string(status)} ({detail})")
        self.status = status


def load() -> ctypes.CDLL:
    """Load the kernel library (torch first, so one HIP runtime is shared)."""

    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        import torch  # noqa: F401  (binds the HIP runtime the library links against)

        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m fastkernels_amd.build` "
                "(there is no CPU fallback for the HIP kernels)"
            )
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        version = lib.fk_abi_version()
        if version != 1:
            raise RuntimeError(f"{LIB_PATH} has ABI version {version}, expected 1")
        _lib = lib
        return lib


def status_string(status: int) -> str:
    return load().fk_status_string(status).decode()


def call(name: str, *args: object) -> None:
    """Call an fk_* entry point and raise FastKernelsError on failure."""

    lib = load()
    status = getattr(lib, name)(*args)
    if status != FK_OK:
        detail = lib.fk_last_error_detail().decode()
        raise FastKernelsError(name, status, detail)


def exported_symbols() -> list[str]:
    return sorted(SIGNATURES)
