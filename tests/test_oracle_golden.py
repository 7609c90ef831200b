"""Pin the CPU oracle and the torch port against the reference's own outputs.

The vectors in tests/golden/ref_vectors.npz were written by tests/golden/make_golden.py,
which ran the reference's CPU code path (repack, exec_* matmuls, activation, and
GGUFSparseMoEMLP.forward) in the development container.
"""

import numpy as np
import pytest
import torch

import oracle
from oracle import torch_port
from pgmoe.gguf import GGMLType, InMemoryGGUF, MoEConfig

QT = {"q4_k": oracle.Q4_K, "q6_k": oracle.Q6_K, "q8_0": oracle.Q8_0}
ROWS, COLS = 4, 512


@pytest.mark.parametrize("name", ["q4_k", "q6_k", "q8_0"])
@pytest.mark.parametrize("tag", ["big", "small"])
def test_dequant_matches_reference_repack(golden, name, tag):
    raw = golden[f"dq_{name}_{tag}_raw"]
    ref = golden[f"dq_{name}_{tag}_dense"]
    # fp16 sub-scale convention reproduces the reference's dense weights bit for bit
    got = oracle.dequant(QT[name], raw, ROWS, COLS, conv=1)
    assert np.array_equal(got, ref)
    # ggml-exact convention differs only by the fp16 rounding of d*sc and dmin*m
    exact = oracle.dequant(QT[name], raw, ROWS, COLS, conv=0)
    scale = np.abs(exact).max()
    assert np.max(np.abs(exact - ref)) <= scale * 2.0**-10


@pytest.mark.parametrize("name", ["q4_k", "q6_k", "q8_0"])
def test_port_repack_bitwise(golden, name):
    for tag in ("big", "small"):
        raw = golden[f"dq_{name}_{tag}_raw"]
        if QT[name] == oracle.Q4_K:
            qw, sc, zr = torch_port.repack_w4(raw, QT[name], ROWS, COLS)
            assert np.array_equal(zr.numpy().view(np.uint16), golden[f"dq_{name}_{tag}_zeros"].view(np.uint16))
        else:
            qw, sc, _ = torch_port.repack_w8(raw, QT[name], ROWS, COLS)
        assert np.array_equal(qw.numpy(), golden[f"dq_{name}_{tag}_qweight"])
        assert np.array_equal(sc.numpy().view(np.uint16), golden[f"dq_{name}_{tag}_scales"].view(np.uint16))


@pytest.mark.parametrize("name", ["q4_k", "q6_k", "q8_0"])
def test_port_matmul_matches_reference(golden, name):
    raw = golden[f"dq_{name}_small_raw"]
    x = torch.from_numpy(golden["mm_x"])
    if QT[name] == oracle.Q4_K:
        got = torch_port.w4_matmul(x, *torch_port.repack_w4(raw, QT[name], ROWS, COLS))
    else:
        got = torch_port.w8_matmul(x, *torch_port.repack_w8(raw, QT[name], ROWS, COLS))
    ref = golden[f"mm_{name}_out"]
    assert got.dtype == torch.float16
    np.testing.assert_allclose(got.float().numpy(), ref.astype(np.float32), rtol=2e-3, atol=1e-4)
    # and the oracle's dense decode times x agrees to fp16 output rounding
    dense = oracle.dequant(QT[name], raw, ROWS, COLS, conv=1).astype(np.float64)
    y = golden["mm_x"].astype(np.float64) @ dense.T
    np.testing.assert_allclose(ref.astype(np.float64), y, rtol=2e-3, atol=1e-3)


def test_act_rowscale_matches_reference(golden):
    g, u = golden["act_g"].astype(np.float32), golden["act_u"].astype(np.float32)
    din, rs = oracle.act_rowscale(g, u)
    ref_rs = golden["act_row_scale"]
    assert np.all(ref_rs > 1.0)  # the row-scale path is exercised
    np.testing.assert_allclose(rs, ref_rs, rtol=1e-6)
    diff = np.abs(din.astype(np.float32) - golden["act_down_in"].astype(np.float32))
    ulp = np.abs(np.spacing(golden["act_down_in"])).astype(np.float32)
    assert np.all(diff <= ulp)
    pd, pr = torch_port.act_rowscale(torch.from_numpy(g), torch.from_numpy(u), faithful=True)
    np.testing.assert_allclose(pr.numpy(), ref_rs, rtol=1e-6)


def _golden_layer(golden, lname):
    H, E, K, I, norm, Is = (int(v) for v in golden[f"moe_{lname}_meta"])
    arch = {"qwen3moe": "qwen3moe", "qwen2moe": "qwen2moe", "mixtral": "mixtral"}[lname]
    g = InMemoryGGUF({"general.architecture": arch})
    prefix = f"moe_{lname}__"
    shapes = {
        "blk.0.ffn_gate_inp.weight": ((E, H), GGMLType.F32),
        "blk.0.ffn_gate_inp_shexp.weight": ((H,), GGMLType.F32),
    }
    for key in golden:
        if not key.startswith(prefix):
            continue
        tname = key[len(prefix):]
        raw = golden[key]
        if tname in shapes:
            shp, qt = shapes[tname]
        else:
            qt = {"qwen3moe": {"gate": 12, "up": 12, "down": 14}, "qwen2moe": {"gate": 8, "up": 8, "down": 8},
                  "mixtral": {"gate": 12, "up": 12, "down": 12}}[lname][tname.split("_")[1]]
            if "exps" in tname:
                shp = (E, I, H) if "down" not in tname else (E, H, I)
            else:
                shp = (Is, H) if "down" not in tname else (H, Is)
        g.add_tensor(tname, shp, qt, raw)
    cfg = MoEConfig(arch=arch, hidden_size=H, n_experts=E, n_experts_used=K, norm_topk_prob=bool(norm))
    return g, cfg


@pytest.mark.parametrize("lname", ["qwen3moe", "qwen2moe", "mixtral"])
@pytest.mark.parametrize("M", [1, 16])
def test_oracle_layer_matches_reference_block(golden, lname, M):
    g, cfg = _golden_layer(golden, lname)
    L = oracle.OracleLayer.from_gguf(g, cfg)
    x = golden[f"moe_{lname}_M{M}_x"]
    logits, idx, w = L.route(x)
    ref_logits = golden[f"moe_{lname}_M{M}_logits"]
    np.testing.assert_allclose(logits, ref_logits, rtol=1e-5, atol=1e-6)
    assert oracle.min_topk_margin(ref_logits, L.top_k) > 1e-4  # no near-ties in this fixture
    assert np.array_equal(idx, golden[f"moe_{lname}_M{M}_topk_idx"])
    ref = golden[f"moe_{lname}_M{M}_out"].astype(np.float64)
    for conv in (0, 1):
        y = L.forward_tokens(x, idx, w, conv=conv)
        # The reference rounds gate/up, down_in and the down output to fp16, which leaves
        # it ~7e-4 rel-L2 from the exact (double) answer; both bounds cover that.
        assert oracle.rel_l2(y, ref) < 1e-3
        assert oracle.max_rel(y, ref) < 2e-3


@pytest.mark.parametrize("lname", ["qwen3moe", "qwen2moe", "mixtral"])
def test_port_block_matches_reference_block(golden, lname):
    g, cfg = _golden_layer(golden, lname)
    port = torch_port.PortMoE(oracle.OracleLayer.from_gguf(g, cfg))
    for M in (1, 16):
        x = torch.from_numpy(golden[f"moe_{lname}_M{M}_x"])
        ref = golden[f"moe_{lname}_M{M}_out"]
        got = port.forward(x, faithful=True).numpy()
        np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5)
        got_b = port.forward(x, faithful=False).numpy()
        assert oracle.rel_l2(got_b, ref) < 1e-3
