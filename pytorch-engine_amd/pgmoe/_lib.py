"""ctypes binding of libpgmoe.so (C ABI in include/pgmoe.h).

The library is built in-tree (``make -C pytorch-engine_amd/csrc``) and must be present:
there is no CPU fallback, so every entry point raises if the HIP library is missing.
"""

from __future__ import annotations

import ctypes
import os
from typing import Optional

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libpgmoe.so")
ABI_VERSION = 4

Q4_0, Q4_1, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K = 2, 3, 6, 8, 12, 13, 14
F32, F16, BF16 = 0, 1, 30
FLOAT_QTYPES = (F32, F16, BF16)  # expert tensors held as fp16 (PGMOE_F16), as the reference's fp16 mode
Q2_K, Q3_K, IQ4_NL, IQ4_XS, MXFP4 = 10, 11, 20, 23, 39
# re-quantised at load to Q4_1 blocks with the reference's W4 values (pgmoe_requant_w4)
REQUANT_W4_QTYPES = (Q2_K, Q3_K, IQ4_NL, IQ4_XS, MXFP4)
Q5_1 = 7
# re-quantised at load to fp16 weights with the reference's W8 values (pgmoe_requant_w8_f16)
REQUANT_W8_QTYPES = (Q5_1,)
# GGUF expert formats with a HIP path; Q4_0 is relaid out as Q4_1, Q5_0 as Q8_0 (their values exactly)
SUPPORTED_QTYPES = (Q4_K, Q5_K, Q6_K, Q8_0, Q4_0, Q4_1, Q5_0) + FLOAT_QTYPES + REQUANT_W4_QTYPES + REQUANT_W8_QTYPES

_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64


class Weights(ctypes.Structure):
    _fields_ = [
        ("qtype", _I32),
        ("n_rows", _I32),
        ("n_cols", _I32),
        ("n_mats", _I32),
        ("base", _P),
        ("mat_stride", _I64),
        ("scales", _P),
    ]


class Layer(ctypes.Structure):
    _fields_ = [
        ("hidden", _I32),
        ("n_experts", _I32),
        ("top_k", _I32),
        ("norm_topk", _I32),
        ("router_w", _P),
        ("router_bias", _P),
        ("gate", Weights),
        ("up", Weights),
        ("down", Weights),
        ("has_shared", _I32),
        ("sh_gate", Weights),
        ("sh_up", Weights),
        ("sh_down", Weights),
        ("sh_inp_gate", _P),
        ("act", _I32),
        ("status_host", _P),
    ]


class Dense(ctypes.Structure):
    _fields_ = [
        ("hidden", _I32),
        ("gate", Weights),
        ("up", Weights),
        ("down", Weights),
        ("act", _I32),
    ]


_lib: Optional[ctypes.CDLL] = None


def lib() -> ctypes.CDLL:
    """Load libpgmoe.so once (after torch, so the process shares torch's HIP runtime)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `make -C pytorch-engine_amd/csrc` "
            "(or __graft_entry__.build()); pgmoe has no CPU fallback")
    import torch  # noqa: F401  (loads the HIP runtime torch was built against)

    L = ctypes.CDLL(LIB_PATH)
    L.pgmoe_abi_version.restype = ctypes.c_int
    L.pgmoe_last_error.restype = ctypes.c_char_p
    L.pgmoe_weight_bytes.restype = _I64
    L.pgmoe_weight_bytes.argtypes = [_I32, _I64, _I64]
    L.pgmoe_relayout_weights.argtypes = [_I32, _P, _I64, _I64, _I64, _P, _P]
    L.pgmoe_relayout_weights_padded.argtypes = [_I32, _P, _I64, _I64, _I64, _I64, _I64, _P, _P]
    L.pgmoe_requant_w4.argtypes = [_I32, _P, _I64, _I64, _P, _P]
    L.pgmoe_requant_w8_f16.argtypes = [_I32, _P, _I64, _I64, _I64, _P, _P]
    L.pgmoe_scale_plane_bytes.restype = _I64
    L.pgmoe_scale_plane_bytes.argtypes = [_I32, _I64, _I64]
    L.pgmoe_build_scale_plane.argtypes = [_I32, _P, _I64, _I64, _I64, _I64, _P, _P]
    L.pgmoe_workspace_bytes.restype = ctypes.c_size_t
    L.pgmoe_workspace_bytes.argtypes = [ctypes.POINTER(Layer), _I32]
    L.pgmoe_moe_forward.argtypes = [ctypes.POINTER(Layer), _P, _I32, _P, _P, ctypes.c_size_t, _P]
    L.pgmoe_dense_workspace_bytes.restype = ctypes.c_size_t
    L.pgmoe_dense_workspace_bytes.argtypes = [ctypes.POINTER(Dense), _I32]
    L.pgmoe_dense_forward.argtypes = [ctypes.POINTER(Dense), _P, _I32, _P, _P, ctypes.c_size_t, _P]
    L.pgmoe_moe_forward_timed.argtypes = [ctypes.POINTER(Layer), _P, _I32, _P, _P, ctypes.c_size_t, _P,
                                          ctypes.POINTER(_P), ctypes.POINTER(_P), _I32, ctypes.POINTER(_I32),
                                          ctypes.POINTER(ctypes.c_char_p)]
    L.pgmoe_linear_workspace_bytes.restype = ctypes.c_size_t
    L.pgmoe_linear_workspace_bytes.argtypes = [ctypes.POINTER(Weights), _I32, _I32, _I32]
    L.pgmoe_linear_forward.argtypes = [ctypes.POINTER(Weights), _P, _P, _I32, _P, _I32, _P, ctypes.c_size_t, _P]
    L.pgmoe_dequant_rows.argtypes = [ctypes.POINTER(Weights), _P, _I32, _P, _I32, _P]
    L.pgmoe_add_rmsnorm.argtypes = [_P, _I32, _P, _I32, _P, _I32, _I32, ctypes.c_float, _P, _P, _I32, _P]
    L.pgmoe_moe_forward_noalloc.argtypes = [ctypes.POINTER(Layer), _P, _I32, _P, _P]
    L.pgmoe_moe_routing.argtypes = [ctypes.POINTER(Layer), _I32, _P, ctypes.c_size_t, _P, _P, _P, _P, _P]
    L.pgmoe_moe_status.argtypes = [ctypes.POINTER(Layer), _P, ctypes.c_size_t, ctypes.POINTER(_I32), _I32, _P]
    L.pgmoe_router_topk.argtypes = [_P, _P, _P, _I32, _I32, _I32, _I32, _I32, _P, _P, _P, _P]
    L.pgmoe_dispatch.argtypes = [_P, _I32, _I32, _I32, _I32, _P, _P, _P, _P, _P, _P, _P]
    L.pgmoe_dispatch_ws_bytes.restype = ctypes.c_size_t
    L.pgmoe_dispatch_ws_bytes.argtypes = [_I32, _I32, _I32]
    L.pgmoe_dispatch_ws.argtypes = [_P, _I32, _I32, _I32, _I32, _P, _P, _P, _P, _P, _P, _P, ctypes.c_size_t, _P]
    L.pgmoe_expert_gateup.argtypes = [ctypes.POINTER(Weights), ctypes.POINTER(Weights), _P, _I32, _I32,
                                      _P, _P, _P, _P, _P, _I32, _P, _P]
    L.pgmoe_expert_down.argtypes = [ctypes.POINTER(Weights), _P, _I32, _I32, _P, _P, _P, _P, _P, _P, _I32,
                                    _P, _P, _P, _P]
    L.pgmoe_combine.argtypes = [_P, _P, _I32, _I32, _I32, _P, _P, _P, _P]
    for fn in ("pgmoe_moe_forward", "pgmoe_moe_forward_timed", "pgmoe_router_topk", "pgmoe_dispatch",
               "pgmoe_dispatch_ws", "pgmoe_expert_gateup",
               "pgmoe_expert_down", "pgmoe_combine", "pgmoe_relayout_weights", "pgmoe_relayout_weights_padded",
               "pgmoe_build_scale_plane",
               "pgmoe_dense_forward", "pgmoe_moe_routing", "pgmoe_moe_status", "pgmoe_moe_forward_noalloc",
               "pgmoe_add_rmsnorm", "pgmoe_linear_forward", "pgmoe_dequant_rows", "pgmoe_requant_w4",
               "pgmoe_requant_w8_f16"):
        getattr(L, fn).restype = ctypes.c_int
    ver = L.pgmoe_abi_version()
    if ver != ABI_VERSION:
        raise RuntimeError(f"libpgmoe.so ABI version {ver}, expected {ABI_VERSION}")
    _lib = L
    return L


def check(rc: int, what: str) -> None:
    """Raise RuntimeError with the library's message when a call did not return 0."""
    if rc != 0:
        msg = lib().pgmoe_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (status {rc}): {msg}")


EXPORTS = (
    "pgmoe_abi_version", "pgmoe_last_error", "pgmoe_weight_bytes", "pgmoe_relayout_weights",
    "pgmoe_workspace_bytes", "pgmoe_moe_forward", "pgmoe_router_topk", "pgmoe_dispatch",
    "pgmoe_expert_gateup", "pgmoe_expert_down", "pgmoe_combine", "pgmoe_moe_forward_timed",
    "pgmoe_scale_plane_bytes", "pgmoe_build_scale_plane", "pgmoe_dispatch_ws_bytes", "pgmoe_dispatch_ws",
    "pgmoe_dense_workspace_bytes", "pgmoe_dense_forward", "pgmoe_moe_routing", "pgmoe_moe_status",
    "pgmoe_moe_forward_noalloc", "pgmoe_add_rmsnorm", "pgmoe_linear_workspace_bytes", "pgmoe_linear_forward",
    "pgmoe_dequant_rows", "pgmoe_relayout_weights_padded", "pgmoe_requant_w4", "pgmoe_requant_w8_f16",
)

STATUS_SPIN_TIMEOUT = 1  # PGMOE_STATUS_SPIN_TIMEOUT
ACT_SILU, ACT_GELU_TANH = 0, 1  # PGMOE_ACT_*
