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


def oracle_sorted_pairs(idx: np.ndarray, w: np.ndarray, n_experts: int):
    """The oracle's routing in sorted pair order (ascending expert, then token): offsets
    [E+1] and per sorted pair its expert, token and weight, via or_dispatch's stable sort
    of the flat ids t*K + k."""
    M, K = idx.shape
    offsets, perm, _ = oracle.dispatch(idx, n_experts)
    flat_i = idx.reshape(-1)
    flat_w = w.reshape(-1)
    return offsets, flat_i[perm], (perm // K).astype(np.int32), flat_w[perm]


def check_forward_routing(mod, M: int, idx: np.ndarray, w: np.ndarray) -> None:
    """The routing the module's last forward of M tokens produced (read back from its own
    workspace) equals the oracle's: offsets, experts and tokens bit for bit in sorted pair
    order; weights to fp32 rounding (the softmax denominator is summed in another order)."""
    g_off, g_e, g_t, g_w = (t.cpu().numpy() for t in mod.routing(M))
    r_off, r_e, r_t, r_w = oracle_sorted_pairs(idx, w, mod.n_experts)
    assert np.array_equal(g_off, r_off), "expert offsets differ"
    assert np.array_equal(g_e, r_e), "sorted pair experts differ"
    assert np.array_equal(g_t, r_t), "sorted pair tokens differ"
    np.testing.assert_allclose(g_w, r_w, rtol=4e-6, atol=1e-7)


def _dequant_mat(t: tuple, mat: int) -> np.ndarray:
    """fp32 [N, K] of matrix `mat` of a (qtype, N, K, raw bytes of all matrices) tuple,
    by the oracle's GGUF decode (ggml-exact convention)."""
    qtype, n, k, raw = t
    per, bb = oracle.BLOCK[qtype]
    mb = n * (k // per) * bb
    return oracle.dequant(qtype, raw[mat * mb:(mat + 1) * mb], n, k)


def torch_fp32_reference(ol, x: np.ndarray, idx: np.ndarray, w: np.ndarray, dev) -> np.ndarray:
    """Every row of the layer output, from the oracle's routing and its dequantised
    weights, computed with plain torch fp32 products on the GPU (rocBLAS, not pgmoe):
    per active expert silu(x Wg^T) * (x Wu^T) -> Wd, times the top-k weight, accumulated
    in float64; plus the sigmoid-gated shared expert.  The expert weights are decoded on
    host threads (the C oracle releases the GIL) one expert ahead of the GPU."""
    import torch
    import torch.nn.functional as F
    from concurrent.futures import ThreadPoolExecutor

    torch.backends.cuda.matmul.allow_tf32 = False
    M, H = x.shape
    K = idx.shape[1]
    xt = torch.from_numpy(x).to(dev).float()
    out = torch.zeros((M, H), dtype=torch.float64, device=dev)
    experts = [int(e) for e in np.unique(idx)]

    def mats(e):
        return tuple(_dequant_mat(t, e) for t in (ol.gate, ol.up, ol.down))

    def ffn(wg, wu, wd, xe):
        g = xe @ torch.from_numpy(wg).to(dev).T
        u = xe @ torch.from_numpy(wu).to(dev).T
        return (F.silu(g) * u) @ torch.from_numpy(wd).to(dev).T

    with ThreadPoolExecutor(max_workers=8) as pool:
        futs = [pool.submit(mats, e) for e in experts[:8]]
        for i, e in enumerate(experts):
            wg, wu, wd = futs[i].result()
            futs[i] = None
            if i + 8 < len(experts):
                futs.append(pool.submit(mats, experts[i + 8]))
            tok, slot = np.nonzero(idx == e)
            tk = torch.from_numpy(tok.astype(np.int64)).to(dev)
            d = ffn(wg, wu, wd, xt.index_select(0, tk))
            wk = torch.from_numpy(w[tok, slot].astype(np.float64)).to(dev)
            out.index_add_(0, tk, d.double() * wk[:, None])
    if ol.sh_gate is not None:
        so = ffn(_dequant_mat(ol.sh_gate, 0), _dequant_mat(ol.sh_up, 0), _dequant_mat(ol.sh_down, 0), xt).double()
        if ol.sh_inp_gate is not None:
            z = xt.double() @ torch.from_numpy(ol.sh_inp_gate.astype(np.float64)).to(dev)
            so = so * torch.sigmoid(z)[:, None]
        out += so
    return out.cpu().numpy()


def check_rows(got: np.ndarray, ref: np.ndarray, max_rel: float = 2e-2, rel_l2: float = 1e-3) -> dict:
    """The north-star bounds over the whole output (rel-L2, max|d| / max|ref|) and the
    max-abs bound applied row by row (max|d_t| / max|ref_t| <= max_rel for every token t),
    so that one wrong row cannot hide among thousands of right ones."""
    stats = check_layer_output(got, ref, max_rel=max_rel, rel_l2=rel_l2)
    d = np.abs(got.astype(np.float64) - ref).max(axis=1)
    den = np.abs(ref).max(axis=1)
    row = d / np.where(den > 0, den, 1.0)
    worst = int(np.argmax(row))
    rl2_rows = np.linalg.norm(got.astype(np.float64) - ref, axis=1) / np.maximum(np.linalg.norm(ref, axis=1), 1e-300)
    stats.update(rows=len(ref), worst_row=worst, worst_row_max_rel=float(row[worst]),
                 worst_row_rel_l2=float(rl2_rows.max()))
    assert row[worst] <= max_rel, f"row {worst}: max|d|/max|ref| {row[worst]:.3e} > {max_rel}"
    return stats
