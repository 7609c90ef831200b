"""Expert and FFN intermediate sizes that are not a multiple of 256 (DeepSeek-V2-Lite's
moe_intermediate_size 1408, Qwen1.5-MoE's 1408): with a 32-weight down format (Q8_0, Q5_0,
Q4_0, Q4_1) the layer is loaded zero-padded to the next multiple of 256, gate / up with zero
rows and down with zero columns, and computes the unpadded layer's values.

* the padded relayout gives exactly the device bytes of the same GGUF tensor with zero
  blocks (and zero rows) appended by hand on the host;
* whole MoE layers (E = 16, K = 4, I = 1408; Q8_0 and Q5_0 down, one with an I = 1408 shared
  expert) match the oracle in decode (M <= 8: folded router, GEMV kernels) and prefill
  (grouped GEMMs), with the forward's own routing bit-exact;
* the dense FFN and GGUFQuantLinear at in_features = 1408 match the oracle / a float64
  product of the oracle-decoded weights."""

import numpy as np
import pytest

import oracle
from gpu_helpers import build_pair, check_forward_routing, check_layer_output, log, sample_tokens
from pgmoe.synth import DenseSpec, LayerSpec, SyntheticDense, random_blocks
from test_q4_0_cpu import q4_0_as_q4_1, q5_0_as_q8_0

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

Q4_0, Q4_1, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K = 2, 3, 6, 8, 12, 13, 14
_BLOCK = {Q4_0: (32, 18), Q4_1: (32, 20), Q5_0: (32, 22), Q8_0: (32, 34), Q4_K: (256, 144), Q5_K: (256, 176),
          Q6_K: (256, 210)}

SPECS = {
    "i1408_q8_0": LayerSpec("i1408_q8_0", 2048, 16, 4, 1408, (Q4_K, Q4_K, Q8_0)),
    "i1408_q5_0": LayerSpec("i1408_q5_0", 2048, 16, 4, 1408, (Q8_0, Q8_0, Q5_0), norm_topk=False,
                            arch="qwen2moe", shared_inter=1408, shared_qtypes=(Q8_0, Q8_0, Q5_0),
                            shared_gate=True),
    "i1408_q4_0": LayerSpec("i1408_q4_0", 1024, 16, 4, 1408, (Q4_0, Q4_0, Q4_0)),
}
_cache = {}


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    yield
    _cache.clear()


def _zero_padded(qt, raw, n, rows, cols, rows_out, cols_out):
    """GGUF bytes of n [rows_out, cols_out] matrices: each [rows, cols] source matrix with
    all-zero blocks appended to its rows and all-zero rows after them (the zero block of
    Q8_0, Q4_1 and the K-quants is all-zero bytes)."""
    per, bb = _BLOCK[qt]
    src = raw.reshape(n, rows, cols // per, bb)
    out = np.zeros((n, rows_out, cols_out // per, bb), np.uint8)
    out[:, :rows, :cols // per] = src
    return out.reshape(-1)


@pytest.mark.parametrize("qt,rows,cols,rows_out,cols_out", [
    (Q8_0, 100, 1408, 100, 1536), (Q8_0, 1408, 2048, 1536, 2048), (Q5_0, 70, 1408, 70, 1536),
    (Q4_0, 64, 96, 64, 256), (Q4_1, 130, 1440, 192, 1536), (Q4_K, 1408, 512, 1536, 512),
    (Q5_K, 100, 256, 200, 256), (Q6_K, 1408, 256, 1536, 256)])
def test_padded_relayout_is_the_relayout_of_zero_padded_bytes(qt, rows, cols, rows_out, cols_out):
    """Q4_0 / Q5_0 are compared through their exact Q4_1 / Q8_0 restatements: the zero
    block of the device layout (d = m = 0) is not the relayout of any Q4_0 / Q5_0 block
    bytes (a Q4_0 block with d = 0 has m = -8 d = -0.0)."""
    from pgmoe import ops
    n = 3
    raw = random_blocks(np.random.default_rng(rows + cols + qt), qt, n * rows, cols)
    log(f"padded relayout qt={qt} [{rows}, {cols}] -> [{rows_out}, {cols_out}]")
    got = ops.relayout(qt, torch.from_numpy(raw).cuda(), n, rows, cols, rows_out, cols_out)
    conv, dt = {Q4_0: (q4_0_as_q4_1, Q4_1), Q5_0: (q5_0_as_q8_0, Q8_0)}.get(qt, (None, qt))
    same = conv(raw) if conv else raw
    ref_raw = _zero_padded(dt, same, n, rows, cols, rows_out, cols_out)
    ref = ops.relayout(dt, torch.from_numpy(ref_raw).cuda(), n, rows_out, cols_out)
    torch.cuda.synchronize()
    assert got.shape == ref.shape and torch.equal(got, ref)


def _pair(name):
    if name not in _cache:
        _cache.clear()
        torch.cuda.empty_cache()
        _cache[name] = build_pair(SPECS[name], seed=0)
    return _cache[name]


@pytest.mark.parametrize("name,Ms", [("i1408_q8_0", (1, 4, 8, 40, 600)), ("i1408_q5_0", (1, 2, 8, 300)),
                                     ("i1408_q4_0", (1, 3, 64))])
def test_moe_layer_i1408(name, Ms):
    lay, ol, mod = _pair(name)
    assert mod.inter == 1408 and mod.inter_padded == 1536
    for M in Ms:
        log(f"i1408 layer {name} M={M}")
        x = lay.draw_x(M)
        out = mod(torch.from_numpy(x).to("cuda:0"))
        _, idx, w = ol.route(x)
        check_forward_routing(mod, M, idx, w)
        toks = sample_tokens(M, 16)
        stats = check_layer_output(out.cpu().numpy()[toks], ol.forward_tokens(x, idx, w, tokens=toks))
        log(f"  {name} M={M}: {stats}")
    mod.check_status(sync=True)


@pytest.mark.parametrize("M", [1, 8, 200])
def test_dense_i1408(M):
    from pgmoe import HipDenseMLP
    sp = DenseSpec("dense_i1408", 2048, 1408, (Q4_K, Q4_K, Q8_0))
    lay = SyntheticDense(sp, seed=0)
    mod = HipDenseMLP.from_gguf(lay.gguf, lay.config, 0, torch.device("cuda", 0))
    log(f"dense i1408 M={M}")
    x = lay.draw_x(M)
    got = mod(torch.from_numpy(x).to("cuda:0")).float().cpu().numpy().reshape(M, -1)
    mats = [(qt, *shp, np.ascontiguousarray(lay.tensor(f"ffn_{p}.weight")))
            for qt, p, shp in zip(sp.qtypes, ("gate", "up", "down"), ((1408, 2048), (1408, 2048), (2048, 1408)))]
    toks = sample_tokens(M, 16)
    check_layer_output(got[toks], oracle.dense_forward(x, *mats, tokens=toks))


@pytest.mark.parametrize("qt,N,K", [(Q8_0, 2048, 1408), (Q5_0, 512, 1408), (Q4_0, 300, 96), (Q4_1, 64, 800)])
@pytest.mark.parametrize("M", [1, 8, 256])
def test_linear_padded_in_features(qt, N, K, M):
    from pgmoe import GGUFQuantLinear
    dev = torch.device("cuda", 0)
    rng = np.random.default_rng(N + K + qt)
    raw = random_blocks(rng, qt, N, K, 0.01)
    bias = torch.from_numpy(rng.standard_normal(N).astype(np.float16)).float()
    lin = GGUFQuantLinear("w4" if qt in (Q4_0, Q4_1) else "w8", K, N, qt, raw=raw, bias=bias, device=dev)
    assert lin.cols == (K + 255) // 256 * 256
    log(f"padded linear qt={qt} N={N} K={K} M={M}")
    x = np.random.default_rng(M).standard_normal((M, K)).astype(np.float16)
    out = lin(torch.from_numpy(x).to(dev).float()).cpu().numpy()
    w = oracle.dequant(qt, raw, N, K).astype(np.float64)
    ref = x.astype(np.float64) @ w.T + bias.numpy().astype(np.float64)
    if M <= 8:  # GEMV: fp32 products
        check_layer_output(out, ref, rel_l2=1e-4, max_rel=1e-4)
    else:
        check_layer_output(out, ref)
    ids = torch.tensor([0, N - 1, 7], dtype=torch.int64)
    rows = lin.embed_lookup(ids, dtype=torch.float32)
    assert rows.shape == (3, K)
    dense = oracle.dequant(qt, raw, N, K)
    assert np.array_equal(rows.cpu().numpy().view(np.uint32), dense[ids.numpy()].view(np.uint32))
