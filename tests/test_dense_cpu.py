"""Dense SwiGLU FFN (GGUFDenseMLP, pygguf_engine/model.py:778-846) on the CPU: the oracle's
dense forward pinned against an independent numpy restatement, the synthetic layer's
tensors, and the C-ABI workspace sizing (no GPU needed)."""

import ctypes

import numpy as np
import pytest

import oracle
from pgmoe.synth import DENSE_CONFIGS, DenseSpec, SyntheticDense

Q4_K, Q6_K, Q8_0 = 12, 14, 8


def _mats(lay):
    sp = lay.spec
    H, I = sp.hidden, sp.inter
    shp = {"gate": (I, H), "up": (I, H), "down": (H, I)}
    return [(qt, *shp[p], np.ascontiguousarray(lay.tensor(f"ffn_{p}.weight")))
            for qt, p in zip(sp.qtypes, ("gate", "up", "down"))]


@pytest.mark.parametrize("qtypes", [(Q4_K, Q4_K, Q6_K), (Q8_0, Q8_0, Q8_0), (Q6_K, Q6_K, Q4_K)])
def test_oracle_dense_equals_numpy_restatement(qtypes):
    """silu(G x) * (U x) then D, in float64 on the dequantised matrices (oracle.dequant is
    pinned by the reference's golden vectors): a dropped activation, a swapped gate / up or
    a transposed down fails here."""
    lay = SyntheticDense(DenseSpec("t", 256, 512, qtypes), seed=3)
    g, u, d = _mats(lay)
    x = lay.draw_x(5)
    got = oracle.dense_forward(x, g, u, d)
    G = oracle.dequant(g[0], g[3], g[1], g[2]).astype(np.float64)
    U = oracle.dequant(u[0], u[3], u[1], u[2]).astype(np.float64)
    D = oracle.dequant(d[0], d[3], d[1], d[2]).astype(np.float64)
    xf = x.astype(np.float64)
    gv, uv = xf @ G.T, xf @ U.T
    with np.errstate(over="ignore"):  # silu of large negative inputs is -0
        ref = (gv / (1.0 + np.exp(-gv)) * uv) @ D.T
    assert got.shape == ref.shape
    np.testing.assert_allclose(got, ref, rtol=1e-9, atol=1e-9 * np.abs(ref).max())
    # a token subset gives the same rows
    sub = oracle.dense_forward(x, g, u, d, tokens=[4, 1])
    np.testing.assert_array_equal(sub, got[[4, 1]])


def test_dense_configs_are_well_formed():
    for name, sp in DENSE_CONFIGS.items():
        assert sp.hidden % 256 == 0 and sp.inter % 256 == 0, name
        lay = SyntheticDense(sp, seed=0) if sp.hidden * sp.inter <= 2048 * 5632 else None
        if lay is not None:
            assert lay.gguf.tensors["blk.0.ffn_gate.weight"].shape == (sp.inter, sp.hidden)
            assert lay.gguf.tensors["blk.0.ffn_down.weight"].shape == (sp.hidden, sp.inter)
            assert lay.config.arch == sp.arch


def test_dense_workspace_bytes_and_argument_checks():
    """pgmoe_dense_workspace_bytes sizes decode and prefill workspaces without a GPU and
    returns 0 for malformed layers (no device memory is touched)."""
    from pgmoe._lib import Dense, Weights, lib
    L = lib()

    def w(qt, n, k):
        s = Weights()
        s.qtype, s.n_mats, s.n_rows, s.n_cols = qt, 1, n, k
        s.base = 1 << 20  # never dereferenced: sizing only
        s.mat_stride = L.pgmoe_weight_bytes(qt, n, k)
        s.scales = 1 << 21
        return s

    D = Dense()
    D.hidden = 1024
    D.gate, D.up, D.down = w(Q4_K, 2816, 1024), w(Q4_K, 2816, 1024), w(Q6_K, 1024, 2816)
    dec = L.pgmoe_dense_workspace_bytes(ctypes.byref(D), 4)
    pre = L.pgmoe_dense_workspace_bytes(ctypes.byref(D), 300)
    assert dec >= 4 * 2816 * 4 and pre >= 300 * 2816 * (4 + 2)
    assert L.pgmoe_dense_workspace_bytes(ctypes.byref(D), -1) == 0
    D.down = w(Q6_K, 1024, 2560)  # down's input size must equal gate's rows
    assert L.pgmoe_dense_workspace_bytes(ctypes.byref(D), 4) == 0
