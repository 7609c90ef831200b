"""GPU parity of the formats the reference re-quantises to W4 at load (Q2_K, Q3_K, IQ4_NL,
IQ4_XS, MXFP4; repack_gguf_to_w4a16, quant_kernels.py:906-942):

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
from oracle.requant import REQUANT_BLOCK, requant_w4
from pgmoe.synth import LayerSpec, random_blocks

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

Q2_K, Q3_K, IQ4_NL, IQ4_XS, MXFP4, Q4_1, Q4_K, Q6_K, Q8_0 = 10, 11, 20, 23, 39, 3, 12, 14, 8


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
}


@pytest.mark.parametrize("name", list(SPECS))
def test_requant_layers(name):
    spec, scale = SPECS[name]
    lay, ol, mod = build_pair(spec, seed=5, scale=scale)
    assert ol.gate[0] == Q4_1 and ol.down[0] == Q4_1  # the oracle runs the re-quantised form
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
