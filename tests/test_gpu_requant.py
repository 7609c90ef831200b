"""GPU parity of the formats the reference re-quantises at load: to W4 (Q2_K, Q3_K, IQ4_NL,
IQ4_XS, MXFP4; repack_gguf_to_w4a16, quant_kernels.py:906-942) and to W8 (Q5_1;
repack_gguf_to_w8a16, :1005-1025, held here as the fp16 weights its tensor-core GEMM forms):

* pgmoe_requant_w4's Q4_1 bytes equal the oracle's restatement bit for bit, on random blocks
  and on edge blocks (flat groups, the extremes of each scale field);
* whole MoE layers in these formats (routed and shared experts, a padded I = 1408 down in
  MXFP4) match the oracle, which runs the Q4_1 form, in decode and prefill, with the
  forward's own routing bit-exact;
* GGUFQuantLinear in these formats matches a float64 product of the re-quantised values.
"""

import numpy as np
import pytest

import oracle
from gpu_helpers import build_pair, check_forward_routing, check_layer_output, log, sample_tokens
from oracle.requant import REQUANT_BLOCK, requant_w4, requant_w8_f16
from pgmoe.synth import LayerSpec, random_blocks

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

Q2_K, Q3_K, IQ4_NL, IQ4_XS, MXFP4, Q4_1, Q4_K, Q6_K, Q8_0, Q5_1, F16 = 10, 11, 20, 23, 39, 3, 12, 14, 8, 7, 1


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    yield
    torch.cuda.empty_cache()


_SCALE_AT = {Q2_K: (80, 82), Q3_K: (108,), IQ4_NL: (0,), IQ4_XS: (0,)}  # fp16 scale fields of a block


def _edge_rows(qt, cols):
    """Rows of hand-set blocks: all zero (flat groups, scale 0); the widest ranges (fp16
    scales at 65504, MXFP4 at 2^122, codes alternating between their extremes); the smallest
    scales (fp16 2^-24, MXFP4 2^-128 .. 2^-125, sub-normal in fp32); random codes at scale 1."""
    per, bb = REQUANT_BLOCK[qt]
    nb = cols // per

    def with_scale(b, f16_bits, e):
        if qt == MXFP4:
            b[:, 0] = e
        else:
            for o in _SCALE_AT[qt]:
                b[:, o:o + 2] = np.array([f16_bits], np.uint16).view(np.uint8)
        return b

    wide = with_scale(np.resize(np.array([0x0F, 0xF0], np.uint8), (nb, bb)).copy(), 0x7BFF, 250)
    rng = np.random.default_rng(qt)
    small = rng.integers(0, 256, size=(nb, bb), dtype=np.uint8)
    small = with_scale(small, 0x0001, 0)
    if qt == MXFP4:
        small[:, 0] = np.arange(nb) % 4
    one = with_scale(rng.integers(0, 256, size=(nb, bb), dtype=np.uint8), 0x3C00, 128)
    rows = [np.zeros((nb, bb), np.uint8), wide, small, one]
    return np.concatenate([r.reshape(-1) for r in rows]), len(rows)


@pytest.mark.parametrize("qt", [Q2_K, Q3_K, IQ4_NL, IQ4_XS, MXFP4])
def test_requant_bytes_bit_exact(qt):
    from pgmoe import ops
    cols = 1024
    rows = 300
    raw = random_blocks(np.random.default_rng(qt), qt, rows, cols)
    edge, ne = _edge_rows(qt, cols)
    raw = np.concatenate([raw, edge])
    n = rows + ne
    log(f"requant qt={qt} rows={n} cols={cols}")
    got = ops.requant_w4(qt, torch.from_numpy(raw).to("cuda:0"), n, cols).cpu().numpy()
    with np.errstate(over="ignore", invalid="ignore"):
        ref = requant_w4(qt, raw, n, cols)
    bad = np.nonzero(got != ref)[0]
    assert bad.size == 0, f"{bad.size} bytes differ, first at block {bad[0] // 20} (row {bad[0] // 20 // (cols // 32)})"


def _check(lay, ol, mod, Ms):
    for M in Ms:
        log(f"{lay.spec.name} M={M}")
        x = lay.draw_x(M)
        got = mod(torch.from_numpy(x).to("cuda:0")).cpu().numpy()
        _, idx, w = ol.route(x)
        check_forward_routing(mod, M, idx, w)
        toks = sample_tokens(M, 12)
        check_layer_output(got[toks], ol.forward_tokens(x, idx, w, tokens=toks),
                           abs_tol=2e-2 if M <= 8 else None)


SPECS = {  # (spec, scale: outputs of order 1e-2 .. 1e-1)
    "iq4_xs_q3_k": (LayerSpec("iq4_xs_q3_k", 1024, 16, 4, 512, (IQ4_XS, IQ4_XS, Q3_K)), 0.01),
    "q2_k_iq4_nl_shared": (LayerSpec("q2_k_iq4_nl_shared", 1024, 16, 4, 512, (Q2_K, Q2_K, IQ4_NL), norm_topk=False,
                                     arch="qwen2moe", shared_inter=768, shared_qtypes=(IQ4_XS, MXFP4, Q3_K),
                                     shared_gate=True), 0.01),
    "mxfp4_i1408": (LayerSpec("mxfp4_i1408", 1024, 16, 4, 1408, (MXFP4, MXFP4, MXFP4)), 0.1),
    "q5_1_i1408_shared": (LayerSpec("q5_1_i1408_shared", 1024, 16, 4, 1408, (Q4_K, Q4_K, Q5_1), norm_topk=False,
                                    arch="qwen2moe", shared_inter=1408, shared_qtypes=(Q5_1, Q5_1, Q5_1),
                                    shared_gate=True), 0.1),
}


@pytest.mark.parametrize("name", list(SPECS))
def test_requant_layers(name):
    spec, scale = SPECS[name]
    lay, ol, mod = build_pair(spec, seed=5, scale=scale)
    for t, gq in ((ol.gate, spec.qtypes[0]), (ol.down, spec.qtypes[2])):  # the oracle runs the re-quantised form
        assert t[0] == (F16 if gq == Q5_1 else Q4_1 if gq in REQUANT_BLOCK else gq)
    _check(lay, ol, mod, (1, 2, 8, 300))


@pytest.mark.parametrize("qt,N,K", [(IQ4_NL, 1536, 1024), (Q3_K, 1000, 2048), (MXFP4, 512, 1408)])
@pytest.mark.parametrize("M", [1, 8, 300])
def test_requant_linear(qt, N, K, M):
    from pgmoe import GGUFQuantLinear
    log(f"linear qt={qt} N={N} K={K} M={M}")
    rng = np.random.default_rng(N + qt)
    raw = random_blocks(rng, qt, N, K, 0.01)
    lin = GGUFQuantLinear("w4", K, N, qt, raw=raw, device=torch.device("cuda", 0))
    w = oracle.dequant(Q4_1, requant_w4(qt, raw, N, K), N, K).astype(np.float64)
    x = np.random.default_rng(M).standard_normal((M, K)).astype(np.float16)
    out = lin(torch.from_numpy(x).to("cuda:0").float()).cpu().numpy()
    ref = x.astype(np.float64) @ w.T
    if M <= 8:
        check_layer_output(out, ref, rel_l2=1e-4, max_rel=1e-4)
    else:
        check_layer_output(out, ref)


def _q5_1_edge(cols):
    """Q5_1 rows: all zero; fp16 d and m at +-65504 (the widest range); d and m at the smallest
    fp16 sub-normal; random codes with d = 1, m = -16."""
    nb = cols // 32
    rng = np.random.default_rng(9)
    rows = []
    for d, m in ((0.0, 0.0), (65504.0, -65504.0), (2.0 ** -24, -(2.0 ** -24)), (1.0, -16.0)):
        b = rng.integers(0, 256, size=(nb, 24), dtype=np.uint8) if d else np.zeros((nb, 24), np.uint8)
        b[:, 0:2] = np.array([d], np.float16).view(np.uint8)
        b[:, 2:4] = np.array([m], np.float16).view(np.uint8)
        rows.append(b)
    return np.concatenate([r.reshape(-1) for r in rows]), len(rows)


@pytest.mark.parametrize("cols,cols_out", [(1024, 1024), (1408, 1536)])
def test_requant_w8_f16_bit_exact(cols, cols_out):
    from pgmoe import ops
    rows = 200
    raw = random_blocks(np.random.default_rng(cols), Q5_1, rows, cols)
    edge, ne = _q5_1_edge(cols)
    raw = np.concatenate([raw, edge])
    n = rows + ne
    log(f"requant w8 rows={n} cols={cols} cols_out={cols_out}")
    got = ops.requant_w8_f16(Q5_1, torch.from_numpy(raw).to("cuda:0"), n, cols, cols_out).cpu().numpy()
    got = got.view(np.uint16).reshape(n, cols_out)
    with np.errstate(over="ignore", invalid="ignore"):
        ref = requant_w8_f16(Q5_1, raw, n, cols).view(np.uint16).reshape(n, cols)
    bad = np.argwhere(got[:, :cols] != ref)
    assert bad.size == 0, f"{len(bad)} weights differ, first at (row, col) {tuple(bad[0])}"
    assert np.all(got[:, cols:] == 0)


@pytest.mark.parametrize("M", [1, 8, 300])
def test_requant_w8_linear_and_rows(M):
    from pgmoe import GGUFQuantLinear
    N, K = 640, 1408
    rng = np.random.default_rng(M)
    raw = random_blocks(rng, Q5_1, N, K, 0.1)
    lin = GGUFQuantLinear("w8", K, N, Q5_1, raw=raw, device=torch.device("cuda", 0))
    w16 = requant_w8_f16(Q5_1, raw, N, K).view(np.float16).reshape(N, K)
    x = rng.standard_normal((M, K)).astype(np.float16)
    out = lin(torch.from_numpy(x).to("cuda:0").float()).cpu().numpy()
    ref = x.astype(np.float64) @ w16.astype(np.float64).T
    if M <= 8:
        check_layer_output(out, ref, rel_l2=1e-4, max_rel=1e-4)
    else:
        check_layer_output(out, ref)
    ids = torch.tensor([0, N - 1, 65, 3], dtype=torch.int64)
    rows = lin.embed_lookup(ids).cpu().numpy()  # fp16 rows: the stored weights, bit for bit
    assert np.array_equal(rows.view(np.uint16), w16[ids.numpy()].view(np.uint16))


@pytest.mark.parametrize("M", [1, 8, 300])
def test_requant_dense(M):
    """The dense SwiGLU FFN with IQ4_XS gate, Q3_K up and an I = 1408 Q5_1 down (padded to
    1536): decode GEMVs and the one-group GEMMs against the oracle on the re-quantised
    forms."""
    from pgmoe import HipDenseMLP
    from pgmoe.synth import DenseSpec, SyntheticDense
    sp = DenseSpec("dense_requant", 1024, 1408, (IQ4_XS, Q3_K, Q5_1))
    lay = SyntheticDense(sp, seed=4, scale=0.1)
    mod = HipDenseMLP(lay.gguf, lay.config, 0, torch.device("cuda", 0))
    H, I = sp.hidden, sp.inter
    mats = []
    for qt, p, (n, k) in zip(sp.qtypes, ("gate", "up", "down"), ((I, H), (I, H), (H, I))):
        raw = np.ascontiguousarray(lay.tensor(f"ffn_{p}.weight"))
        mats.append((F16, n, k, requant_w8_f16(qt, raw, n, k)) if qt == Q5_1 else (Q4_1, n, k, requant_w4(qt, raw, n, k)))
    log(f"dense requant M={M}")
    x = lay.draw_x(M)
    got = mod(torch.from_numpy(x).to("cuda:0")).cpu().numpy()
    toks = sample_tokens(M, 8)
    check_layer_output(got[toks], oracle.dense_forward(x, *mats, tokens=toks))
