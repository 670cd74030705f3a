"""ctypes binding of libzmoe_hip.so (declared in include/zmoe.h).

The library is loaded from this directory on first use. There is no fallback:
if it is missing or fails to load, every op raises.
"""

from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libzmoe_hip.so")

DTYPE_F32 = 0
DTYPE_BF16 = 1

_ERR_NAMES = {
    1: "ZMOE_ERR_NULL",
    2: "ZMOE_ERR_SHAPE",
    3: "ZMOE_ERR_DTYPE",
    4: "ZMOE_ERR_ALIGN",
    5: "ZMOE_ERR_WORKSPACE",
    6: "ZMOE_ERR_HIP",
}

P = ctypes.c_void_p
I64 = ctypes.c_int64
I32 = ctypes.c_int
F32 = ctypes.c_float
SZ = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/zmoe.h
SIGNATURES = {
    "zmoe_abi_version": (I32, []),
    "zmoe_status_string": (ctypes.c_char_p, [I32]),
    "zmoe_last_error": (ctypes.c_char_p, []),
    "zmoe_route_topk": (I32, [P, I32, I64, I32, I32, P, I32, P, P, P, P]),
    "zmoe_route_topk_backward": (I32, [P, P, P, I64, I32, I32, P, I64, I32, P]),
    "zmoe_bincount": (I32, [P, I64, I32, P, P]),
    "zmoe_sort_workspace_bytes": (SZ, [I64, I32]),
    "zmoe_flatten_sort_count": (I32, [P, I64, I32, P, P, P, P, P, SZ, P]),
    "zmoe_sort_error_flag": (P, [P]),
    "zmoe_flatten_sort_count_noalloc": (I32, [P, I64, I32, P, P, P, P, P, P]),
    "zmoe_offsets_from_sorted": (I32, [P, I64, I32, P, P]),
    "zmoe_group": (I32, [P, I64, I64, I32, P, I64, I32, P, I32, P, I64, P]),
    "zmoe_scatter2scatter": (I32, [P, I64, P, I64, I64, I64, P, I64, P, P, P, I64, I64, I64, I32, I32, I32, I32,
                                   I32, P, I64, P]),
    "zmoe_group_bwd_w": (I32, [P, I64, P, I64, P, I32, P, I64, I64, I64, I32, I32, I32, P, P, P]),
    "zmoe_group_bwd_w_gather_dy": (I32, [P, I64, P, I32, P, I64, P, I64, I64, I64, I32, I32, I32, P, P]),
    "zmoe_dense_wgrad_workspace_bytes": (SZ, [I64, I64, I32]),
    "zmoe_dense_wgrad": (I32, [P, I64, P, I64, I64, I64, I64, I32, I32, I32, P, P, SZ, P]),
    "zmoe_rowwise_sum_product": (I32, [P, I32, P, I32, I64, I32, I64, P, I32, P]),
    "zmoe_glu_w1_forward": (I32, [P, I64, P, P, P, P, I64, I64, I64, I32, I32, I32, P, P, P]),
    "zmoe_glu_w1_forward_scaled": (I32, [P, I64, P, P, P, P, I64, I64, I64, I32, I32, I32, P, P, P, P]),
    "zmoe_glu_w2_backward_dh": (I32, [P, P, P, P, P, I64, I64, I64, I32, I32, P, P]),
    "zmoe_glu_w2_backward_dh_gates_workspace_bytes": (SZ, [I64, I64]),
    "zmoe_glu_w2_backward_dh_gates": (I32, [P, I64, I32, P, P, P, P, P, P, I64, I64, I32, I32, P, P, P, SZ, P]),
    "zmoe_combine": (I32, [P, P, P, I64, I32, I64, I32, P, P]),
    "zmoe_combine_backward": (I32, [P, P, P, P, I64, I32, I64, I32, P, P, P]),
    "zmoe_combine_rows": (I32, [P, P, P, I64, I32, I64, I32, P, I64, P, P]),
    "zmoe_combine_backward_rows": (I32, [P, P, P, I64, P, P, I64, I32, I64, I32, P, P, P]),
    "zmoe_sum_k": (I32, [P, I64, I32, I64, I32, P, P, I32, P, P]),
    "zmoe_cast_f32_bf16": (I32, [P, I64, P, P]),
    "zmoe_swiglu": (I32, [P, I64, I64, I32, P, P]),
    "zmoe_swiglu_backward": (I32, [P, P, I64, I64, I32, P, I64, P]),
    "zmoe_swiglu_backward_gates": (I32, [P, P, I64, I64, P, P, I32, P, P, P]),
    "zmoe_bias_update": (I32, [P, I32, F32, P, P]),
    "zmoe_rmsnorm_rows": (I32, [P, I64, I64, P, I64, I64, P, I32, F32, I32, P, P, P]),
    "zmoe_rmsnorm_rows_backward_workspace_bytes": (SZ, [I64, I64, I32]),
    "zmoe_rmsnorm_rows_backward": (I32, [P, P, I64, I64, P, I64, I64, P, P, I32, I32, P, I64, P, P, SZ, P]),
    "zmoe_newton_schulz5_workspace_bytes": (SZ, [I64, I64, I64]),
    "zmoe_newton_schulz5": (I32, [P, I64, I64, I64, I32, F32, F32, F32, P, SZ, P]),
}

_lock = threading.Lock()
_lib = None


class ZmoeError(RuntimeError):
    """A libzmoe_hip entry point returned a non-zero status."""


def load():
    """Load libzmoe_hip.so (once) and bind every exported entry point."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"libzmoe_hip.so not found at {LIB_PATH}; build it first "
                "(python architecture-zarelga-superposition_amd/build_lib.py)")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if lib.zmoe_abi_version() != 3:
            raise ImportError("libzmoe_hip.so ABI version mismatch")
        _lib = lib
    return _lib


def call(name, *args):
    """Call entry point ``name``; raise on a non-zero status."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.zmoe_last_error().decode(errors="replace")
        kind = _ERR_NAMES.get(rc, str(rc))
        if rc == 6:
            raise ZmoeError(f"{name}: {kind}: {msg}")
        raise ValueError(f"{name}: {kind}: {msg}")
    return rc
