"""Q5_K weights on the GPU (the 5-bit K-quant of Q5_K_M files):

* the dequantised rows (embed_lookup) equal the oracle's ggml decode bit for bit (fp32),
  which pins the relayout of the fifth bits and the device decode;
* whole layers with Q5_K experts (gate/up Q5_K with Q6_K or Q5_K down, a Q5_K shared
  expert) on the decode GEMVs (M <= 8) and the MFMA path: routing bit-exact, outputs within
  rel-L2 <= 1e-3 and max|d|/max|ref| <= 2e-2 of the fp64 oracle;
* the quantized linear (GEMV and GEMM) against a float64 product on the decoded weights.
"""

import numpy as np
import pytest

import oracle
from gpu_helpers import build_pair, check_forward_routing, check_layer_output, log, sample_tokens
from pgmoe.synth import LayerSpec, random_blocks

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

Q4_K, Q5_K, Q6_K, Q8_0 = 12, 13, 14, 8


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    yield
    torch.cuda.empty_cache()


def test_q5_k_rows_bit_exact():
    from pgmoe import GGUFQuantLinear
    rng = np.random.default_rng(1)
    for N, K in ((130, 512), (64, 2048), (7, 256)):
        raw = random_blocks(rng, Q5_K, N, K, 1.0)
        lin = GGUFQuantLinear("w8", K, N, Q5_K, raw=raw, device=torch.device("cuda", 0))
        ids = torch.tensor(list(range(N)) + [0, N - 1], dtype=torch.int64)
        got = lin.embed_lookup(ids, dtype=torch.float32).cpu().numpy()
        ref = oracle.dequant(Q5_K, raw, N, K)[ids.numpy()]
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("name", ["q5_k_m", "all_q5_k"])
@pytest.mark.parametrize("scale", [1.0, 0.01])
def test_q5_k_layer(name, scale):
    spec = {"q5_k_m": LayerSpec("q5_k_m", 2048, 64, 8, 768, (Q5_K, Q5_K, Q6_K)),
            "all_q5_k": LayerSpec("all_q5_k", 1024, 16, 4, 512, (Q5_K, Q5_K, Q5_K), arch="qwen2moe",
                                  norm_topk=False, shared_inter=768, shared_qtypes=(Q5_K, Q5_K, Q5_K),
                                  shared_gate=True)}[name]
    lay, ol, mod = build_pair(spec, seed=5, scale=scale)
    for M in (1, 3, 8, 40, 700):
        log(f"q5_k layer {name} scale={scale} M={M}")
        x = lay.draw_x(M)
        got = mod(torch.from_numpy(x).to("cuda:0")).cpu().numpy()
        _, idx, w = ol.route(x)
        check_forward_routing(mod, M, idx, w)
        toks = sample_tokens(M, 10)
        check_layer_output(got[toks], ol.forward_tokens(x, idx, w, tokens=toks),
                           abs_tol=2e-2 if (scale < 1 and M <= 8) else None)


@pytest.mark.parametrize("N,K,bias", [(2048, 2048, False), (1000, 4096, True)])
@pytest.mark.parametrize("M", [1, 8, 300])
def test_q5_k_linear(N, K, bias, M):
    from pgmoe import GGUFQuantLinear
    log(f"q5_k linear N={N} K={K} M={M}")
    rng = np.random.default_rng(N + K + M)
    raw = random_blocks(rng, Q5_K, N, K, 0.01)
    b = torch.from_numpy(rng.standard_normal(N).astype(np.float16)).float() if bias else None
    lin = GGUFQuantLinear("w8", K, N, Q5_K, raw=raw, bias=b, device=torch.device("cuda", 0))
    x = rng.standard_normal((M, K)).astype(np.float16)
    out = lin(torch.from_numpy(x).to("cuda:0").float()).cpu().numpy()
    ref = x.astype(np.float64) @ oracle.dequant(Q5_K, raw, N, K).astype(np.float64).T
    if b is not None:
        ref = ref + b.numpy().astype(np.float64)
    if M <= 8:
        check_layer_output(out, ref, rel_l2=1e-4, max_rel=1e-4)
    else:
        check_layer_output(out, ref)
