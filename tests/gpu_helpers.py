"""Helpers shared by the GPU parity tests (layers, oracle runs, error metrics)."""

from __future__ import annotations

import sys
from typing import Optional, Sequence

import numpy as np

import oracle
from pgmoe.synth import CONFIGS, LayerSpec, SyntheticLayer


def log(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def build_pair(spec: LayerSpec, seed: int = 0, scale: float = 1.0):
    """(SyntheticLayer, OracleLayer, HipSparseMoEMLP on cuda:0)."""
    import torch
    from pgmoe import HipSparseMoEMLP

    lay = SyntheticLayer(spec, seed=seed, scale=scale)
    ol = oracle.OracleLayer.from_gguf(lay.gguf, lay.config, router_bias=lay.router_bias)
    mod = HipSparseMoEMLP(lay.gguf, lay.config, 0, torch.device("cuda", 0))
    if lay.router_bias is not None:
        mod.set_router_bias(torch.from_numpy(lay.router_bias))
    return lay, ol, mod


def check_layer_output(got: np.ndarray, ref: np.ndarray, max_rel: float = 2e-2, rel_l2: float = 1e-3,
                       abs_tol: Optional[float] = None) -> dict:
    """rel-L2 <= 1e-3 and max|d| / max|ref| <= 2e-2 against the
    fp64-accumulated oracle; abs_tol additionally bounds max|d| literally."""
    r = oracle.rel_l2(got, ref)
    m = oracle.max_rel(got, ref)
    a = float(np.max(np.abs(got.astype(np.float64) - ref)))
    assert np.all(np.isfinite(got)), "non-finite output"
    assert r <= rel_l2, f"rel_l2 {r:.3e} > {rel_l2}"
    assert m <= max_rel, f"max_rel {m:.3e} > {max_rel}"
    if abs_tol is not None:
        assert a <= abs_tol, f"max abs {a:.3e} > {abs_tol}"
    return {"rel_l2": r, "max_rel": m, "max_abs": a}


def sample_tokens(M: int, n: int, seed: int = 0) -> np.ndarray:
    if M <= n:
        return np.arange(M, dtype=np.int32)
    rng = np.random.default_rng(seed)
    return np.sort(rng.choice(M, size=n, replace=False)).astype(np.int32)


class HipEvents:
    """hipEvent_t handles from the HIP runtime torch loaded (for pgmoe_moe_forward_timed)."""

    def __init__(self, n: int):
        import ctypes
        path = None
        for line in open("/proc/self/maps"):
            if "libamdhip64" in line:
                path = line.split()[-1]
                break
        self.L = ctypes.CDLL(path or "libamdhip64.so")
        self.L.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.L.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.ev = (ctypes.c_void_p * n)()
        for i in range(n):
            h = ctypes.c_void_p()
            assert self.L.hipEventCreate(ctypes.byref(h)) == 0
            self.ev[i] = h.value

    def elapsed_ms(self, a, b) -> float:
        import ctypes
        f = ctypes.c_float()
        assert self.L.hipEventElapsedTime(ctypes.byref(f), a, b) == 0
        return float(f.value)
