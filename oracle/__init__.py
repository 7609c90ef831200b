"""CPU oracle for the quantized MoE FFN path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may
import this package, and only as the checker.  The product (``pgmoe``) never imports it.

* ``liboracle.so`` (built from ``pgmoe_oracle.c``) restates the reference algorithm:
  GGUF block decode, fixed-order router, top-k, stable dispatch, the per-expert SwiGLU
  loop and the ascending-expert combine (pygguf_engine/model.py:898-937).
* ``torch_port`` restates the reference's CPU execution path (repacked W4/W8 weights,
  chunked fp32 dequant + ``F.linear``; quant_kernels.py:854-1036, :1276-1291,
  :1408-1420, :1467-1475) and is the timed CPU baseline.

Parity pins for each function are listed in ``pgmoe_oracle.c``'s header; none is unpinned.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass
from typing import Any, Optional, Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib: Optional[ctypes.CDLL] = None

Q4_0, Q4_1, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K = 2, 3, 6, 8, 12, 13, 14
F32, F16, BF16 = 0, 1, 30
BLOCK = {Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210), Q8_0: (32, 34), Q4_0: (32, 18),
         Q4_1: (32, 20), Q5_0: (32, 22), F16: (1, 2)}


from .requant import REQUANT_BLOCK, W8_BLOCK, requant_w4, requant_w8_f16  # noqa: E402  (the reference's W4 / W8 re-quantisations)


def fp16_expert_bytes(qtype: int, raw: np.ndarray) -> np.ndarray:
    """The fp16 bytes of an F32 / F16 / BF16 expert tensor as the reference's fp16 expert
    mode holds it (load_float_tensor(..., dtype=torch.float16), quant_kernels.py:1962-1964
    and :1097-1110): F16 as stored, F32 and BF16 (widened exactly to fp32) rounded to fp16
    to nearest even."""
    raw = np.ascontiguousarray(raw).view(np.uint8)
    if qtype == F16:
        return raw.copy()
    if qtype == F32:
        f = raw.view(np.float32)
    elif qtype == BF16:
        f = (raw.view(np.uint16).astype(np.uint32) << 16).view(np.float32)
    else:
        raise ValueError(f"qtype {qtype} is not a float type")
    with np.errstate(over="ignore"):  # beyond fp16's range: inf, as torch's conversion gives
        return f.astype(np.float16).view(np.uint8)

_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64


class _Weights(ctypes.Structure):
    _fields_ = [("qtype", _I), ("n_rows", _I), ("n_cols", _I), ("data", _P)]


def build() -> None:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.or_half_to_float.restype = ctypes.c_float
        L.or_half_to_float.argtypes = [ctypes.c_uint16]
        L.or_float_to_half.restype = ctypes.c_uint16
        L.or_float_to_half.argtypes = [ctypes.c_float]
        L.or_dequant_rows.argtypes = [_I, _I, _P, _I64, _I64, _P]
        L.or_router_logits.argtypes = [_P, _P, _P, _I, _I, _I, _P]
        L.or_topk.argtypes = [_P, _I, _I, _I, _I, _P, _P]
        L.or_dispatch.argtypes = [_P, _I, _I, _I, _P, _P, _P]
        L.or_act_rowscale.argtypes = [_P, _P, _I, _I, _P, _P]
        L.or_act_rowscale.restype = None
        L.or_add_rmsnorm.argtypes = [_P, _I, _P, _I, _P, _I, _I, ctypes.c_float, _P, _P, _I]
        L.or_gelu_tanh.restype = ctypes.c_double
        L.or_gelu_tanh.argtypes = [ctypes.c_double]
        L.or_moe_forward_tokens.argtypes = [_I, _I, _I, _I, _I] + [ctypes.POINTER(_Weights)] * 6 + [
            _P, _P, _P, _P, _P, _I, _P]
        _lib = L
    return _lib


def _ptr(a: Optional[np.ndarray]) -> Optional[int]:
    return None if a is None else a.ctypes.data


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"oracle {what} failed with status {rc}")


# ---------------------------------------------------------------- R9 block decode
def dequant(qtype: int, raw: np.ndarray, rows: int, cols: int, conv: int = 0) -> np.ndarray:
    """Dense fp32 [rows, cols] from GGUF blocks.  conv 0 = ggml-exact, 1 = fp16 sub-scales."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    pb, bb = BLOCK[qtype]
    if raw.nbytes != rows * (cols // pb) * bb:
        raise ValueError("byte count does not match shape")
    out = np.empty((rows, cols), dtype=np.float32)
    _check(lib().or_dequant_rows(qtype, conv, _ptr(raw), rows, cols, _ptr(out)), "dequant")
    return out


# ---------------------------------------------------------------- R1/R2/R3 routing
def router_logits(x: np.ndarray, w: np.ndarray, bias: Optional[np.ndarray] = None) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float16)
    w = np.ascontiguousarray(w, dtype=np.float32)
    M, H = x.shape
    E = w.shape[0]
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    out = np.empty((M, E), dtype=np.float32)
    _check(lib().or_router_logits(_ptr(x), _ptr(w), _ptr(b), M, H, E, _ptr(out)), "router")
    return out


def topk(logits: np.ndarray, k: int, norm: bool):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    M, E = logits.shape
    idx = np.empty((M, k), dtype=np.int32)
    w = np.empty((M, k), dtype=np.float32)
    _check(lib().or_topk(_ptr(logits), M, E, k, int(norm), _ptr(idx), _ptr(w)), "topk")
    return idx, w


def dispatch(idx: np.ndarray, n_experts: int):
    idx = np.ascontiguousarray(idx, dtype=np.int32)
    M, K = idx.shape
    offsets = np.empty(n_experts + 1, dtype=np.int32)
    perm = np.empty(M * K, dtype=np.int32)
    inv = np.empty(M * K, dtype=np.int32)
    _check(lib().or_dispatch(_ptr(idx), M, K, n_experts, _ptr(offsets), _ptr(perm), _ptr(inv)),
           "dispatch")
    return offsets, perm, inv


def act_rowscale(g: np.ndarray, u: np.ndarray):
    g = np.ascontiguousarray(g, dtype=np.float32)
    u = np.ascontiguousarray(u, dtype=np.float32)
    M, I = g.shape
    down_in = np.empty((M, I), dtype=np.float16)
    rs = np.empty((M, 1), dtype=np.float32)
    lib().or_act_rowscale(_ptr(g), _ptr(u), M, I, _ptr(down_in), _ptr(rs))
    return down_in, rs


# ---------------------------------------------------------------- residual add + RMSNorm
_DT = {np.dtype(np.float32): 0, np.dtype(np.float16): 1}


def add_rmsnorm(x: np.ndarray, delta: Optional[np.ndarray], w: np.ndarray, eps: float,
                out_dtype=np.float16, bf16: Sequence[bool] = (False, False)):
    """(h fp32, out) of exec_fused_add_rmsnorm (delta None: exec_fused_rmsnorm, h = f32(x)) in
    the GPU kernel's fixed summation order.  x / delta: fp32 or fp16 arrays, or uint16 bf16
    bits with bf16[i] set."""
    x = np.ascontiguousarray(x)
    R, D = x.shape
    xdt = 30 if bf16[0] else _DT[x.dtype]
    ddt = 0
    if delta is not None:
        delta = np.ascontiguousarray(delta)
        ddt = 30 if bf16[1] else _DT[delta.dtype]
    w = np.ascontiguousarray(w, dtype=np.float32)
    h = np.empty((R, D), dtype=np.float32)
    out = np.empty((R, D), dtype=out_dtype)
    _check(lib().or_add_rmsnorm(_ptr(x), xdt, _ptr(delta), ddt, _ptr(w), R, D, float(eps), _ptr(h), _ptr(out),
                                _DT[np.dtype(out_dtype)]), "add_rmsnorm")
    return h, out


# ---------------------------------------------------------------- layer
@dataclass
class OracleLayer:
    """Everything the oracle needs for one MoE layer, read from a GGUF-like object."""

    hidden: int
    n_experts: int
    top_k: int
    norm_topk: bool
    router_w: np.ndarray
    gate: tuple  # (qtype, n_rows, n_cols, raw bytes)
    up: tuple
    down: tuple
    router_bias: Optional[np.ndarray] = None
    sh_gate: Optional[tuple] = None
    sh_up: Optional[tuple] = None
    sh_down: Optional[tuple] = None
    sh_inp_gate: Optional[np.ndarray] = None
    act: int = 0  # 0 SiLU, 1 GELU-tanh (gemma architectures, model.py:868)

    @classmethod
    def from_gguf(cls, gguf: Any, config: Any, layer_idx: int = 0,
                  router_bias: Optional[np.ndarray] = None) -> "OracleLayer":
        p = f"blk.{layer_idx}"

        def f32(name: str) -> np.ndarray:
            info = gguf.tensors[name]
            raw = gguf.get_tensor_bytes(name)
            if info.qtype == 0:
                return np.frombuffer(raw, dtype=np.float32).reshape(info.shape).copy()
            if info.qtype == 1:
                return np.frombuffer(raw, dtype=np.float16).reshape(info.shape).astype(np.float32)
            if int(info.qtype) in BLOCK:  # quantised: the ggml block values
                shp = tuple(int(v) for v in info.shape)
                rows = int(np.prod(shp[:-1])) if len(shp) > 1 else 1
                return dequant(int(info.qtype), np.asarray(raw), rows, shp[-1]).reshape(shp)
            raise ValueError(f"{name}: oracle reads F32 / F16 / GGUF-block tensors only")

        def q(name: str, mats: bool) -> tuple:
            info = gguf.tensors[name]
            shp = info.shape
            n, k = (shp[1], shp[2]) if mats else (shp[0], shp[1])
            raw = np.ascontiguousarray(gguf.get_tensor_bytes(name))
            if int(info.qtype) in (F32, F16, BF16):  # fp16 expert mode
                return (F16, int(n), int(k), fp16_expert_bytes(int(info.qtype), raw))
            if int(info.qtype) in REQUANT_BLOCK:  # the reference's W4 re-quantisation, as Q4_1 blocks
                rows = int(np.prod([int(v) for v in shp[:-1]]))
                return (Q4_1, int(n), int(k), requant_w4(int(info.qtype), raw, rows, int(k)))
            if int(info.qtype) in W8_BLOCK:  # the reference's W8 re-quantisation, as fp16 weights
                rows = int(np.prod([int(v) for v in shp[:-1]]))
                return (F16, int(n), int(k), requant_w8_f16(int(info.qtype), raw, rows, int(k)))
            return (int(info.qtype), int(n), int(k), raw)

        kw = {}
        if f"{p}.ffn_gate_shexp.weight" in gguf.tensors:
            kw["sh_gate"] = q(f"{p}.ffn_gate_shexp.weight", False)
            kw["sh_up"] = q(f"{p}.ffn_up_shexp.weight", False)
            kw["sh_down"] = q(f"{p}.ffn_down_shexp.weight", False)
            if f"{p}.ffn_gate_inp_shexp.weight" in gguf.tensors:
                kw["sh_inp_gate"] = f32(f"{p}.ffn_gate_inp_shexp.weight").reshape(-1)
        rw = f32(f"{p}.ffn_gate_inp.weight")
        return cls(hidden=rw.shape[1], n_experts=int(config.n_experts),
                   top_k=max(1, int(config.n_experts_used)), norm_topk=bool(config.norm_topk_prob),
                   router_w=rw, gate=q(f"{p}.ffn_gate_exps.weight", True),
                   up=q(f"{p}.ffn_up_exps.weight", True), down=q(f"{p}.ffn_down_exps.weight", True),
                   router_bias=router_bias, act=1 if str(config.arch).startswith("gemma") else 0, **kw)

    def route(self, x: np.ndarray):
        logits = router_logits(x, self.router_w, self.router_bias)
        idx, w = topk(logits, self.top_k, self.norm_topk)
        return logits, idx, w

    def forward_tokens(self, x: np.ndarray, idx: np.ndarray, w: np.ndarray,
                       tokens: Optional[Sequence[int]] = None, conv: int = 0) -> np.ndarray:
        """float64 layer output for `tokens` (all tokens by default) given routing."""
        x = np.ascontiguousarray(x, dtype=np.float16)
        M, H = x.shape
        toks = np.arange(M, dtype=np.int32) if tokens is None else np.asarray(tokens, dtype=np.int32)
        toks = np.ascontiguousarray(toks)
        idx = np.ascontiguousarray(idx, dtype=np.int32)
        w = np.ascontiguousarray(w, dtype=np.float32)
        out = np.empty((len(toks), H), dtype=np.float64)

        def mk(t):
            if t is None:
                return None
            s = _Weights(t[0], t[1], t[2], t[3].ctypes.data)
            return ctypes.pointer(s)

        keep = [self.gate, self.up, self.down, self.sh_gate, self.sh_up, self.sh_down]
        ws = [mk(t) for t in keep]
        sig = None if self.sh_inp_gate is None else np.ascontiguousarray(self.sh_inp_gate, np.float32)
        rc = lib().or_moe_forward_tokens(H, self.n_experts, self.top_k, conv, self.act, *ws, _ptr(sig), _ptr(x),
                                         _ptr(idx), _ptr(w), _ptr(toks), len(toks), _ptr(out))
        _check(rc, "moe_forward_tokens")
        return out


def gelu_tanh(g: float) -> float:
    """The oracle's tanh-approximation GELU (or_gelu_tanh), in double."""
    return float(lib().or_gelu_tanh(float(g)))


def dense_forward(x: np.ndarray, gate: tuple, up: tuple, down: tuple,
                  tokens: Optional[Sequence[int]] = None, conv: int = 0, act: int = 0) -> np.ndarray:
    """float64 output of a dense SwiGLU FFN (GGUFDenseMLP.forward, model.py:839-846) for
    `tokens`: the expert FFN of or_moe_forward_tokens applied as its shared expert to a
    layer with no routed experts.  gate / up / down: (qtype, rows, cols, GGUF bytes)."""
    x = np.ascontiguousarray(x, dtype=np.float16)
    M, H = x.shape
    toks = np.arange(M, dtype=np.int32) if tokens is None else np.asarray(tokens, dtype=np.int32)
    toks = np.ascontiguousarray(toks)
    out = np.empty((len(toks), H), dtype=np.float64)
    keep = [gate, up, down]
    ws = [ctypes.pointer(_Weights(t[0], t[1], t[2], t[3].ctypes.data)) for t in keep]
    none = np.zeros(1, dtype=np.int32)
    rc = lib().or_moe_forward_tokens(H, 0, 0, conv, act, None, None, None, *ws, None, _ptr(x), _ptr(none),
                                     _ptr(none.view(np.float32)), _ptr(toks), len(toks), _ptr(out))
    _check(rc, "moe_forward_tokens (dense)")
    return out


def rel_l2(a: np.ndarray, b: np.ndarray) -> float:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    den = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / den) if den > 0 else float(np.linalg.norm(a - b))


def max_rel(a: np.ndarray, b: np.ndarray) -> float:
    """max|a-b| / max|b| (scale-normalised max-abs)."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    den = np.max(np.abs(b))
    return float(np.max(np.abs(a - b)) / den) if den > 0 else float(np.max(np.abs(a - b)))


def min_topk_margin(logits: np.ndarray, k: int) -> float:
    """Smallest gap between the k-th and (k+1)-th largest logit over tokens."""
    if logits.shape[1] <= k:
        return float("inf")
    s = -np.sort(-logits.astype(np.float64), axis=1)
    return float(np.min(s[:, k - 1] - s[:, k]))
