"""CPU-side checks of the C ABI and the host code (no GPU work is launched here):
the library loads and exports every symbol of include/pgmoe.h, argument validation
returns the documented status codes, and the GGUF reader/writer round-trips."""

import ctypes
import os
import re

import numpy as np
import pytest

from pgmoe import _lib
from pgmoe.gguf import GGMLType, GGUFFile, GGUFWriter, InMemoryGGUF
from pgmoe.synth import CONFIGS, SyntheticLayer, random_blocks

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "pgmoe.h")


def test_library_exports_every_header_symbol():
    L = _lib.lib()
    text = open(HEADER).read()
    names = sorted(set(re.findall(r"\b(pgmoe_[a-z_0-9]+)\s*\(", text)))
    assert names, "no declarations parsed"
    for n in names:
        assert hasattr(L, n), f"{n} declared in pgmoe.h but not exported"
    assert set(_lib.EXPORTS) <= set(names)
    assert L.pgmoe_abi_version() == _lib.ABI_VERSION


def test_weight_bytes_are_gguf_bytes_of_64_row_tiles():
    L = _lib.lib()
    for qt, rows, cols, per, bb in [(12, 768, 2048, 256, 144), (14, 2048, 768, 256, 210),
                                    (8, 2560, 3584, 32, 34), (14, 1, 256, 256, 210), (8, 100, 512, 32, 34),
                                    (13, 768, 2048, 256, 176), (13, 5, 512, 256, 176)]:
        padded_rows = (rows + 63) // 64 * 64
        raw = padded_rows * (cols // per) * bb
        assert L.pgmoe_weight_bytes(qt, rows, cols) == (raw + 255) // 256 * 256
        if rows % 64 == 0:  # no padding: exactly the GGUF bytes
            assert L.pgmoe_weight_bytes(qt, rows, cols) == rows * (cols // per) * bb
    assert L.pgmoe_weight_bytes(12, 4, 100) == -1  # not a whole K-quant block row
    assert L.pgmoe_weight_bytes(7, 4, 256) == -1   # Q5_1 is a source format (held as fp16)
    assert L.pgmoe_weight_bytes(10, 4, 256) == -1  # nor Q2_K
    assert L.pgmoe_weight_bytes(3, 64, 256) == 64 * 8 * 20  # Q4_1: the GGUF bytes
    assert L.pgmoe_weight_bytes(6, 4, 256) == L.pgmoe_weight_bytes(8, 4, 256)  # Q5_0 is stored as Q8_0
    assert L.pgmoe_weight_bytes(8, 4, 96) == -1    # rows must be whole 256-weight tiles
    assert L.pgmoe_weight_bytes(8, 4, 320) == -1


def test_dispatch_scratch_bytes():
    """Multi-block dispatch scratch: one int per (workgroup, expert), about 2048 pairs per
    workgroup and at most 64 workgroups."""
    L = _lib.lib()
    assert L.pgmoe_dispatch_ws_bytes(4096, 8, 128) == 16 * 128 * 4
    assert L.pgmoe_dispatch_ws_bytes(1, 8, 128) == 1 * 128 * 4
    assert L.pgmoe_dispatch_ws_bytes(100000, 8, 64) == 64 * 64 * 4
    assert L.pgmoe_dispatch_ws_bytes(4, 8, 0) == 0
    assert L.pgmoe_dispatch_ws(0x1000, 4, 8, 128, 256, 0x2000, 0x3000, 0x4000, 0x5000, 0x6000, 0x7000, 0x8000,
                               16, None) == -3  # scratch too small


def test_scale_plane_bytes_and_argument_checks():
    """Scale plane: one 1 KB chunk per (64-row group, super-block, 64-weight unit) for
    K-quants, none for Q8_0; the builder rejects bad arguments before any device work."""
    L = _lib.lib()
    assert L.pgmoe_scale_plane_bytes(12, 100, 512) == 2 * 2 * 4 * 1024
    assert L.pgmoe_scale_plane_bytes(14, 64, 768) == 1 * 3 * 4 * 1024
    assert L.pgmoe_scale_plane_bytes(8, 64, 256) == 0
    assert L.pgmoe_scale_plane_bytes(12, 4, 100) == -1
    assert L.pgmoe_scale_plane_bytes(2, 4, 256) == -1
    assert L.pgmoe_build_scale_plane(8, 0x1000, 1, 64, 256, 0, 0x2000, None) == -2  # Q8_0: none
    assert L.pgmoe_build_scale_plane(12, 0, 1, 64, 256, 0, 0x2000, None) == -1      # NULL source
    assert L.pgmoe_build_scale_plane(12, 0x1008, 1, 64, 256, 0, 0x2000, None) == -1  # misaligned
    stride = L.pgmoe_weight_bytes(12, 64, 256)
    assert L.pgmoe_build_scale_plane(12, 0x1000, 2, 64, 256, stride - 16, 0x2000, None) == -1


def _fake_layer(E=8, K=2, H=1024, I=512, qt=12, shared=False, shared_inter=None, down_qt=None):
    """A layer struct with aligned fake device pointers (validation never dereferences)."""
    W = _lib.Weights
    down_qt = qt if down_qt is None else down_qt
    stride = _lib.lib().pgmoe_weight_bytes(qt, I, H)
    L = _lib.Layer()
    L.hidden, L.n_experts, L.top_k, L.norm_topk = H, E, K, 1
    L.router_w = 0x10000
    L.gate = W(qt, I, H, E, 0x100000, stride)
    L.up = W(qt, I, H, E, 0x200000, stride)
    L.down = W(down_qt, H, I, E, 0x300000, _lib.lib().pgmoe_weight_bytes(down_qt, H, I))
    if shared:
        Is = shared_inter or 2 * I
        L.has_shared = 1
        L.sh_gate = W(qt, Is, H, 1, 0x400000, 0)
        L.sh_up = W(qt, Is, H, 1, 0x500000, 0)
        L.sh_down = W(qt, H, Is, 1, 0x600000, 0)
    return L


def test_workspace_bytes_never_fall_as_m_grows():
    """A workspace sized for M serves every smaller M: pgmoe_workspace_bytes (and the dense
    and linear sizes) never decrease from M to M + 1, though the split-K scratch of one
    batch can exceed that of a larger one (one more M tile can lower the split count).
    Shapes: Qwen3-30B-A3B, Mixtral-8x7B, Qwen2-57B-A14B with its shared expert."""
    L = _lib.lib()
    layers = {"qwen3": _fake_layer(E=128, K=8, H=2048, I=768, qt=12, down_qt=14),
              "mixtral": _fake_layer(E=8, K=2, H=4096, I=14336, qt=12),
              "qwen2": _fake_layer(E=64, K=8, H=3584, I=2560, qt=8, shared=True, shared_inter=20480)}
    for name, lay in layers.items():
        prev = 0
        for M in range(1, 4097):
            n = L.pgmoe_workspace_bytes(lay, M)
            assert n >= prev, f"{name}: {M} tokens need {n} bytes, {M - 1} needed {prev}"
            prev = n
    W = _lib.Weights
    dense = _lib.Dense()
    dense.hidden = 3584
    dense.gate = W(8, 20480, 3584, 1, 0x100000, 0)
    dense.up = W(8, 20480, 3584, 1, 0x200000, 0)
    dense.down = W(8, 3584, 20480, 1, 0x300000, 0)
    lin = W(8, 20480, 3584, 1, 0x100000, 0)
    prev_d = prev_l = 0
    for M in range(1, 4097):
        nd = L.pgmoe_dense_workspace_bytes(dense, M)
        nl = L.pgmoe_linear_workspace_bytes(lin, M, 1, 0)
        assert nd >= prev_d and nl >= prev_l, M
        prev_d, prev_l = nd, nl


def test_workspace_bytes_and_zero_tokens():
    L = _lib.lib()
    lay = _fake_layer()
    w1 = L.pgmoe_workspace_bytes(lay, 1)
    w16 = L.pgmoe_workspace_bytes(lay, 16)
    assert 0 < w1 < w16
    assert L.pgmoe_workspace_bytes(_fake_layer(shared=True), 16) > w16
    # M = 0 validates and returns without touching the device
    assert L.pgmoe_moe_forward(lay, None, 0, None, None, 0, None) == 0


@pytest.mark.parametrize("mutate,code,msg", [
    (lambda l: setattr(l.gate, "qtype", 2), -2, "qtype"),
    (lambda l: setattr(l.up, "base", 0x200008), -1, "aligned"),
    (lambda l: setattr(l, "top_k", 9), -2, "top_k"),
    (lambda l: setattr(l, "hidden", 1000), -2, "hidden"),
    (lambda l: setattr(l.down, "n_rows", 512), -1, "shapes"),
    (lambda l: setattr(l.gate, "mat_stride", 64), -1, "mat_stride"),
    (lambda l: setattr(l, "n_experts", 600), -2, "n_experts"),
])
def test_forward_validation_errors(mutate, code, msg):
    L = _lib.lib()
    lay = _fake_layer()
    mutate(lay)
    rc = L.pgmoe_moe_forward(lay, 0x1000, 4, 0x2000, 0x3000, 1 << 30, None)
    assert rc == code
    assert msg in L.pgmoe_last_error().decode()


def test_workspace_too_small_reported():
    L = _lib.lib()
    lay = _fake_layer()
    need = L.pgmoe_workspace_bytes(lay, 4)
    rc = L.pgmoe_moe_forward(lay, 0x1000, 4, 0x2000, 0x3000, need - 1, None)
    assert rc == -3 and "workspace" in L.pgmoe_last_error().decode()
    rc = L.pgmoe_moe_forward(lay, 0x1000, 4, 0x2000, 0x3008, need, None)
    assert rc == -1  # misaligned workspace


def test_stage_validation_errors():
    L = _lib.lib()
    assert L.pgmoe_router_topk(0x1000, 0x2000, None, 4, 100, 8, 2, 1, 0x3000, 0x4000, 0x5000, None) == -1
    assert L.pgmoe_router_topk(0x1000, 0x2000, None, 4, 128, 8, 9, 1, 0x3000, 0x4000, 0x5000, None) == -1
    assert L.pgmoe_dispatch(0x1000, 4, 2, 600, 64, 1, 1, 1, 1, 1, 1, None) == -1
    assert L.pgmoe_dispatch(0x1000, 4, 2, 8, 0, 1, 1, 1, 1, 1, 1, None) == -1
    bad = _lib.Weights(12, 100, 300, 1, 0x1000, 0)
    good = _lib.Weights(12, 100, 256, 1, 0x1000, 0)
    assert L.pgmoe_expert_gateup(bad, bad, 0x1000, 1, 1, 1, 1, 1, 1, 1, 0, 0x2000, None) == -2
    q6 = _lib.Weights(14, 100, 256, 1, 0x2000, 0)
    assert L.pgmoe_expert_gateup(good, q6, 0x1000, 1, 1, 1, 1, 1, 1, 1, 0, 0x2000, None) == -2
    assert L.pgmoe_relayout_weights(12, 0x1000, 1, 4, 256, 0x2010, None) == -1
    assert L.pgmoe_relayout_weights(12, 0x1008, 1, 4, 256, 0x2000, None) == -1  # misaligned src
    # zero-padded relayout: [rows, cols] GGUF matrices into [rows_out, cols_out] device ones
    pad = L.pgmoe_relayout_weights_padded
    assert pad(12, 0x1000, 1, 4, 1408, 4, 1536, 0x2000, None) == -2  # K-quant columns are not padded
    assert pad(8, 0x1000, 1, 4, 1400, 4, 1536, 0x2000, None) == -2  # not whole 32-weight blocks
    assert pad(8, 0x1000, 1, 4, 1408, 4, 1408, 0x2000, None) == -2  # device width not a multiple of 256
    assert pad(8, 0x1000, 1, 5, 1408, 4, 1536, 0x2000, None) == -1  # rows > rows_out
    assert pad(8, 0x1000, 1, 4, 1792, 4, 1536, 0x2000, None) == -1  # cols > cols_out
    assert pad(8, 0x1000, 1, 4, 1408, 4, 1536, 0x2010, None) == -1  # misaligned dst
    assert pad(8, 0x1002, 1, 4, 1408, 4, 1536, 0x2000, None) == -1  # misaligned src
    assert pad(8, None, 1, 4, 1408, 4, 1536, 0x2000, None) == -1
    assert L.pgmoe_combine(0x1000, 0x2000, 3, 0, 16, None, None, 0x3000, None) == -1
    # load-time W4 re-quantisation of Q2_K / Q3_K / IQ4_NL / IQ4_XS / MXFP4
    rq = L.pgmoe_requant_w4
    assert rq(12, 0x1000, 4, 256, 0x2000, None) == -2  # Q4_K is kept as it is
    assert "not re-quantised" in L.pgmoe_last_error().decode()
    assert rq(20, 0x1000, 4, 48, 0x2000, None) == -2  # not whole blocks
    assert rq(23, 0x1000, 4, 224, 0x2000, None) == -2  # IQ4_XS blocks are 256 weights
    assert rq(39, 0x1000, 4, 64, 0x2002, None) == -1  # dst not 4-byte aligned
    assert rq(10, None, 4, 256, 0x2000, None) == -1
    assert rq(11, 0x1000, 0, 256, 0x2000, None) == -1
    assert rq(20, 0x1000, 1 << 40, 32, 0x2000, None) == -1  # grid beyond its limit
    # Q5_1 to fp16 weights of the reference's W8 values
    r8 = L.pgmoe_requant_w8_f16
    assert r8(6, 0x1000, 4, 256, 256, 0x2000, None) == -2  # Q5_0 keeps its exact Q8_0 form
    assert r8(7, 0x1000, 4, 48, 64, 0x2000, None) == -2  # not whole blocks
    assert r8(7, 0x1000, 4, 256, 224, 0x2000, None) == -1  # cols_out < cols
    assert r8(7, 0x1000, 4, 64, 80, 0x2000, None) == -1  # cols_out not whole 32-weight blocks
    assert r8(7, 0x1000, 4, 64, 64, 0x2008, None) == -1  # dst not 16-byte aligned
    assert r8(7, None, 4, 64, 64, 0x2000, None) == -1


def test_module_rejects_cpu_device():
    import torch
    from pgmoe import HipSparseMoEMLP
    lay = SyntheticLayer(CONFIGS["tiny"], seed=0, scale=0.01)
    with pytest.raises(ValueError):
        HipSparseMoEMLP(lay.gguf, lay.config, 0, torch.device("cpu"))


def test_gguf_writer_reader_roundtrip(tmp_path):
    rng = np.random.default_rng(0)
    w = GGUFWriter()
    w.add_meta("general.architecture", "qwen3moe")
    w.add_meta("qwen3moe.expert_count", 4)
    w.add_meta("qwen3moe.expert_used_count", 2)
    w.add_meta("qwen3moe.embedding_length", 256)
    q4 = random_blocks(rng, 12, 4 * 128, 256)
    q8 = random_blocks(rng, 8, 256, 64)
    r = rng.standard_normal((4, 256)).astype(np.float32)
    w.add_tensor("blk.0.ffn_gate_exps.weight", (4, 128, 256), 12, q4)
    w.add_tensor("blk.0.ffn_gate_inp.weight", (4, 256), 0, r.view(np.uint8))
    w.add_tensor("x.weight", (256, 64), 8, q8)
    p = tmp_path / "t.gguf"
    w.write(p)
    with GGUFFile(p) as g:
        assert g.version == 3
        info = g.tensors["blk.0.ffn_gate_exps.weight"]
        assert info.shape == (4, 128, 256) and info.ggml_dims == (256, 128, 4) and info.qtype == 12
        assert np.array_equal(g.get_tensor_bytes("blk.0.ffn_gate_exps.weight"), q4)
        assert np.array_equal(g.get_tensor_bytes("x.weight"), q8)
        assert np.array_equal(g.get_tensor_bytes("blk.0.ffn_gate_inp.weight").view(np.float32).reshape(4, 256), r)
        cfg = g.build_model_config()
        assert (cfg.n_experts, cfg.n_experts_used, cfg.norm_topk_prob, cfg.hidden_size) == (4, 2, True, 256)
        assert g.tensor_data_offset % 32 == 0


def test_gguf_reader_rejects_garbage(tmp_path):
    p = tmp_path / "bad.gguf"
    p.write_bytes(b"NOPE" + b"\0" * 64)
    with pytest.raises(ValueError):
        GGUFFile(p)


def test_config_defaults_follow_arch():
    g = InMemoryGGUF({"general.architecture": "qwen2moe", "qwen2moe.expert_count": 64,
                      "qwen2moe.expert_used_count": 8})
    assert g.build_model_config().norm_topk_prob is False
    g2 = InMemoryGGUF({"general.architecture": "mixtral"})
    assert g2.build_model_config().norm_topk_prob is True


def test_synthetic_generator_is_seeded_and_shaped():
    a = SyntheticLayer(CONFIGS["tiny"], seed=1)
    b = SyntheticLayer(CONFIGS["tiny"], seed=1)
    for name in a.gguf.tensors:
        assert np.array_equal(a.gguf.get_tensor_bytes(name), b.gguf.get_tensor_bytes(name))
    assert a.gguf.tensors["blk.0.ffn_down_exps.weight"].shape == (8, 1024, 512)
    x1, x2 = a.draw_x(16), b.draw_x(16)
    assert x1.dtype == np.float16 and np.array_equal(x1, x2)
    blk = a.tensor("ffn_gate_exps.weight").reshape(-1, 144)
    d = blk[:, 0:2].copy().view(np.float16).astype(np.float32)
    assert np.all(d >= 0) and 0.005 < np.median(d) < 0.03  # |N(0,1)| * 0.02


def test_zipf_bias_skews_loads():
    import oracle
    lay = SyntheticLayer(CONFIGS["qwen3_30b_a3b_zipf"], seed=0)
    assert lay.router_bias is not None and lay.router_bias.shape == (128,)
    ol = oracle.OracleLayer.from_gguf(lay.gguf, lay.config, router_bias=lay.router_bias)
    x = lay.draw_x(512)
    _, idx, _ = ol.route(x)
    counts = np.bincount(idx.reshape(-1), minlength=128)
    assert counts.max() > 8 * counts.mean()


def test_add_rmsnorm_argument_checks():
    """pgmoe_add_rmsnorm validates before any device work."""
    L = _lib.lib()
    ok = (0x1000, 0, 0x2000, 0, 0x3000)
    assert L.pgmoe_add_rmsnorm(*ok, 0, 256, 1e-6, None, 0x4000, 1, None) == 0      # no rows: nothing to do
    assert L.pgmoe_add_rmsnorm(*ok, 2, 102, 1e-6, None, 0x4000, 1, None) == -1     # dim not a multiple of 4
    assert L.pgmoe_add_rmsnorm(0x1000, 7, 0x2000, 0, 0x3000, 2, 256, 1e-6, None, 0x4000, 1, None) == -2  # x dtype
    assert L.pgmoe_add_rmsnorm(*ok, 2, 256, 1e-6, None, 0x4000, 30, None) == -2    # bf16 output
    assert L.pgmoe_add_rmsnorm(*ok, 2, 256, -1.0, None, 0x4000, 1, None) == -1     # negative eps
    assert L.pgmoe_add_rmsnorm(None, 0, None, 0, 0x3000, 2, 256, 1e-6, None, 0x4000, 1, None) == -1  # NULL x
    assert L.pgmoe_add_rmsnorm(0x1004, 0, None, 0, 0x3000, 2, 256, 1e-6, None, 0x4000, 1, None) == -1  # misaligned


def test_noalloc_and_routing_argument_checks():
    L = _lib.lib()
    lay = _fake_layer()
    assert L.pgmoe_moe_forward_noalloc(lay, 0x1000, 0, 0x2000, None) == 0           # no tokens
    assert L.pgmoe_moe_forward_noalloc(lay, 0x1000, -1, 0x2000, None) == -1
    assert L.pgmoe_moe_forward_noalloc(lay, None, 4, 0x2000, None) == -1
    assert L.pgmoe_moe_forward_noalloc(lay, 0x1000, 100000, 0x2000, None) == -3     # beyond the fixed scratch
    n = L.pgmoe_workspace_bytes(lay, 4)
    assert L.pgmoe_moe_routing(lay, 4, 0x1000, n - 256, 0x2000, 0x3000, 0x4000, 0x5000, None) == -3
    assert L.pgmoe_moe_routing(lay, 4, 0x1008, n, 0x2000, 0x3000, 0x4000, 0x5000, None) == -1
    st = ctypes.c_int32()
    assert L.pgmoe_moe_status(lay, 0x1000, 16, ctypes.byref(st), 0, None) == -3


def test_padded_widths():
    """The device width of a GGUF matrix: its own when a multiple of 256; the 32-weight
    formats (Q8_0, Q5_0, Q4_0, Q4_1) pad whole 32-weight blocks up to one; -1 otherwise."""
    from pgmoe import ops
    for qt in (8, 6, 2, 3):
        assert ops.padded_width(qt, 1408) == 1536 and ops.padded_width(qt, 96) == 256
        assert ops.padded_width(qt, 2048) == 2048 and ops.padded_width(qt, 1400) == -1
    for qt in (12, 13, 14):
        assert ops.padded_width(qt, 1408) == -1 and ops.padded_width(qt, 2048) == 2048


def test_f16_weight_sizes_and_planes():
    """fp16 expert matrices (PGMOE_F16 = 1): 64-row tiles of 32 chunks a 256-weight
    super-block, no scale plane; widths must be multiples of 256."""
    L = _lib.lib()
    for rows, cols in ((64, 256), (100, 2048), (768, 2048)):
        assert L.pgmoe_weight_bytes(1, rows, cols) == ((rows + 63) // 64) * (cols // 256) * 32 * 1024
        assert L.pgmoe_scale_plane_bytes(1, rows, cols) == 0
    assert L.pgmoe_weight_bytes(1, 64, 320) == -1
    from pgmoe import ops
    assert ops.device_qtype(0) == ops.device_qtype(30) == ops.device_qtype(1) == 1
