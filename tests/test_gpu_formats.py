"""GPU parity of the layer variants beyond SwiGLU with float routers:

* GeGLU experts (gemma architectures: tanh-approximation GELU in place of SiLU,
  model.py:868, quant_kernels.py:1471) on the decode and MFMA paths, with a shared expert,
  and the dense GeGLU FFN (model.py:800);
* quantised router and shared-gate tensors (Q8_0, Q4_K, Q6_K), dequantised at load on the
  device to the ggml block values, as the reference's load_float_tensor does through
  gguf.quants (quant_kernels.py:1111-1114): routing still bit-exact.
"""

import numpy as np
import pytest

import oracle
from gpu_helpers import build_pair, check_forward_routing, check_layer_output, log, sample_tokens
from pgmoe.synth import LayerSpec, random_blocks

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

Q4_K, Q6_K, Q8_0 = 12, 14, 8


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    yield
    torch.cuda.empty_cache()


def _check(lay, ol, mod, Ms, abs_small=False):
    for M in Ms:
        log(f"{lay.spec.name} M={M}")
        x = lay.draw_x(M)
        got = mod(torch.from_numpy(x).to("cuda:0")).cpu().numpy()
        _, idx, w = ol.route(x)
        check_forward_routing(mod, M, idx, w)
        toks = sample_tokens(M, 12)
        check_layer_output(got[toks], ol.forward_tokens(x, idx, w, tokens=toks),
                           abs_tol=2e-2 if (abs_small and M <= 8) else None)


@pytest.mark.parametrize("scale", [1.0, 0.01])
def test_geglu_experts(scale):
    spec = LayerSpec("gemma_moe", 1024, 16, 4, 512, (Q4_K, Q4_K, Q6_K), arch="gemma3", shared_inter=768,
                     shared_qtypes=(Q8_0, Q8_0, Q8_0), shared_gate=True)
    lay, ol, mod = build_pair(spec, seed=11, scale=scale)
    assert mod.use_gelu and ol.act == 1
    _check(lay, ol, mod, (1, 3, 8, 40, 600), abs_small=scale < 1)


def test_geglu_differs_from_swiglu():
    """The same weights under a gemma and a qwen3 architecture give different outputs (the
    activation is really switched), each matching its own oracle."""
    spec_g = LayerSpec("g", 512, 8, 2, 256, (Q4_K, Q4_K, Q4_K), arch="gemma2")
    spec_s = LayerSpec("s", 512, 8, 2, 256, (Q4_K, Q4_K, Q4_K), arch="qwen3moe")
    lg, og, mg = build_pair(spec_g, seed=3, scale=0.01)
    ls, os_, ms = build_pair(spec_s, seed=3, scale=0.01)
    x = lg.draw_x(4)
    a = mg(torch.from_numpy(x).to("cuda:0")).cpu().numpy()
    b = ms(torch.from_numpy(x).to("cuda:0")).cpu().numpy()
    assert not np.allclose(a, b, rtol=1e-3)
    _, idx, w = og.route(x)
    check_layer_output(a, og.forward_tokens(x, idx, w), abs_tol=2e-2)
    _, idx, w = os_.route(x)
    check_layer_output(b, os_.forward_tokens(x, idx, w), abs_tol=2e-2)


def test_dense_geglu():
    from pgmoe import HipDenseMLP
    from pgmoe.synth import DenseSpec, SyntheticDense
    sp = DenseSpec("dense_gemma", 1024, 2816, (Q4_K, Q4_K, Q6_K), arch="gemma3")
    lay = SyntheticDense(sp, seed=2)
    mod = HipDenseMLP(lay.gguf, lay.config, 0, torch.device("cuda", 0))
    assert mod.use_gelu
    mats = [(qt, n, k, np.ascontiguousarray(lay.tensor(f"ffn_{p}.weight")))
            for qt, p, (n, k) in zip(sp.qtypes, ("gate", "up", "down"), ((2816, 1024), (2816, 1024), (1024, 2816)))]
    for M in (1, 6, 300):
        x = lay.draw_x(M)
        got = mod(torch.from_numpy(x).to("cuda:0")).cpu().numpy()
        toks = sample_tokens(M, 8)
        check_layer_output(got[toks], oracle.dense_forward(x, *mats, tokens=toks, act=1))


@pytest.mark.parametrize("rq", [Q8_0, Q4_K, Q6_K])
def test_quantised_router(rq):
    from pgmoe.gguf import GGMLType
    spec = LayerSpec("qrouter", 1024, 32, 4, 256, (Q4_K, Q4_K, Q6_K), arch="qwen2moe", norm_topk=False,
                     shared_inter=512, shared_qtypes=(Q8_0, Q8_0, Q8_0), shared_gate=True)
    from pgmoe.synth import SyntheticLayer
    lay = SyntheticLayer(spec, seed=7, scale=0.01)
    rng = np.random.default_rng(rq)
    lay.gguf.add_tensor("blk.0.ffn_gate_inp.weight", (32, 1024), rq, random_blocks(rng, rq, 32, 1024, 0.5))
    lay.gguf.add_tensor("blk.0.ffn_gate_inp_shexp.weight", (1, 1024), rq, random_blocks(rng, rq, 1, 1024, 0.5))
    ol = oracle.OracleLayer.from_gguf(lay.gguf, lay.config)
    from pgmoe import HipSparseMoEMLP
    mod = HipSparseMoEMLP(lay.gguf, lay.config, 0, torch.device("cuda", 0))
    # the router the module holds is the oracle's decode of the blocks, bit for bit
    assert np.array_equal(mod.router_weight.cpu().numpy().view(np.uint32), ol.router_w.view(np.uint32))
    assert np.array_equal(mod.shared_inp_gate.cpu().numpy().view(np.uint32),
                          ol.sh_inp_gate.reshape(-1).view(np.uint32))
    _check(lay, ol, mod, (1, 5, 64), abs_small=True)
