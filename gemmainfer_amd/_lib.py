"""ctypes binding of libgemmainfer_amd.so (the C ABI in include/gemmainfer_amd.h).

The library is loaded lazily from ``gemmainfer_amd/lib/``.  There is no
fallback: if the library is missing or fails to load, every device entry point
raises ``RuntimeError`` naming the build command.
"""
from __future__ import annotations

import ctypes
import threading
from ctypes import POINTER, c_float, c_int, c_int32, c_int64, c_size_t, c_void_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libgemmainfer_amd.so"

GI_OK = 0
GI_ERR_INVALID_ARG = -1
GI_ERR_UNSUPPORTED = -2
GI_ERR_WORKSPACE = -3
GI_ERR_HIP = -4
GI_ERR_DEVICE = -5

DTYPE_BF16 = 0
DTYPE_FP16 = 1
DTYPE_FP32 = 2
DTYPE_INT32 = 3
DTYPE_INT64 = 4

DEVICE_SPIN_TIMEOUT = 1

# name -> (restype, argtypes); mirrors include/gemmainfer_amd.h and
# include/gemmainfer_amd_probe.h exactly.
SIGNATURES = {
    "gi_last_error": (ctypes.c_char_p, []),
    "gi_abi_version": (c_int, []),
    "gi_moe_route_topk_softmax": (c_int, [c_void_p, c_int, c_void_p, c_int, c_int, c_int,
                                          c_void_p, c_void_p, c_int, c_void_p]),
    "gi_moe_align": (c_int, [c_void_p, c_int, c_int, c_int, c_int, c_void_p, c_void_p,
                             c_void_p, c_void_p, c_void_p, c_void_p]),
    "gi_fused_moe_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int, c_int]),
    "gi_fused_batched_moe": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_int, c_void_p,
                                     c_void_p, c_int, c_void_p, c_int, c_void_p, c_int,
                                     c_void_p, c_int, c_int, c_int, c_int, c_int, c_int,
                                     c_void_p, c_size_t, c_int, c_void_p]),
    "gi_fused_batched_moe_static": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_int, c_void_p,
                                            c_void_p, c_int, c_void_p, c_int, c_void_p, c_int,
                                            c_void_p, c_int, c_int, c_int, c_int, c_int, c_int,
                                            c_int, c_void_p]),
    "gi_fused_batched_moe_static_status": (c_int, [POINTER(c_int32), c_int, c_void_p]),
    "gi_moe_layer_from_logits": (c_int, [c_void_p, c_int, c_void_p, c_int, c_void_p,
                                         c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_int,
                                         c_void_p, c_void_p, c_void_p,
                                         c_int, c_int, c_int, c_int, c_int, c_int,
                                         c_void_p, c_size_t, c_int, c_void_p]),
    "gi_moe_router_logits": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_float, c_void_p,
                                     c_int, c_int, c_int, c_void_p]),
    "gi_moe_layer_from_hidden": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_float, c_void_p,
                                         c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_void_p,
                                         c_int, c_void_p, c_void_p, c_void_p,
                                         c_int, c_int, c_int, c_int, c_int, c_int,
                                         c_void_p, c_size_t, c_int, c_void_p]),
    "gi_workspace_status": (c_int, [c_void_p, c_size_t, POINTER(c_int32), c_void_p]),
    "gi_device_error_flags": (c_int, [c_int, c_int]),
    "gi_w4a16_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int]),
    "gi_w4a16_linear": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_int, c_void_p,
                                c_int, c_int, c_int, c_int, c_float, c_void_p, c_size_t,
                                c_void_p]),
    "gi_w4a16_linear_multi": (c_int, [c_void_p, c_int, c_int, c_void_p, c_void_p, c_void_p, c_void_p,
                                      c_void_p, c_int, c_int, c_int, c_void_p, c_size_t, c_void_p]),
    "gi_w4a16_linear_multi_workspace_bytes": (c_size_t, [c_int, c_void_p, c_int, c_int, c_int]),
    "gi_w4a16_gated_mlp_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int]),
    "gi_w4a16_gated_mlp": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_int,
                                   c_void_p, c_int, c_int, c_int, c_int, c_void_p, c_size_t, c_void_p]),
    "gi_w4a16_ingest": (c_int, [c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_void_p,
                                c_void_p, c_int64, c_void_p]),
    "gi_w4a16_ingest_batched": (c_int, [c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int, c_int64,
                                        c_int64, c_void_p, c_void_p, c_int64, c_int64, c_int64, c_void_p]),
    "gi_softcap_inplace": (c_int, [c_void_p, c_int, c_int64, c_float, c_void_p]),
    "gi_rmsnorm": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int64, c_int, c_float,
                           c_int, c_void_p]),
    "gi_probe_stream_read": (c_int, [c_void_p, c_void_p, c_int, c_int, c_void_p, c_void_p]),
    "gi_probe_decode_timeline": (c_int, [c_void_p, c_size_t]),
    "gi_rope_inplace": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int,
                                c_int, c_int, c_int, c_int, c_int,
                                c_int64, c_int64, c_int64, c_int64, c_int64, c_int64,
                                c_void_p]),
}

_lock = threading.Lock()
_lib = None


class GIError(RuntimeError):
    """A non-OK status from the C ABI; ``code`` is the GI_ERR_* value."""

    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


def load() -> ctypes.CDLL:
    """Load (once) and return the library, with argtypes set from SIGNATURES."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m gemmainfer_amd.build` "
                "(hipcc, gfx950). There is no CPU fallback for device tensors.")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return lib


def check(status: int, what: str) -> None:
    """Raise GIError for a non-OK status, with the library's message."""
    if status != GI_OK:
        msg = load().gi_last_error()
        msg = msg.decode() if msg else ""
        raise GIError(status, f"{what}: {msg} (status {status})")


def exported_symbols() -> list[str]:
    return list(SIGNATURES)
