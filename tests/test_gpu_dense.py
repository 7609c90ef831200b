"""GPU parity of the dense SwiGLU FFN (HipDenseMLP.forward through pgmoe_dense_forward,
the drop-in for GGUFDenseMLP, pygguf_engine/model.py:778-846) against the CPU oracle.

Gates, as for the MoE layer: rel-L2 <= 1e-3 and max|d|/max|ref| <= 2e-2 against the
float64 oracle.  Decode sizes (M <= 8) run the GEMV kernels, larger M the grouped GEMMs
with one group; large M is checked on a token sample (each token's output depends only
on its own input)."""

import numpy as np
import pytest

import oracle
from gpu_helpers import check_layer_output, log, sample_tokens
from pgmoe.synth import DENSE_CONFIGS, DenseSpec, SyntheticDense

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

_cache = {}


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    yield
    _cache.clear()


def _dense(name):
    if name not in _cache:
        from pgmoe import HipDenseMLP
        _cache.clear()
        torch.cuda.empty_cache()
        lay = SyntheticDense(DENSE_CONFIGS[name], seed=0)
        mod = HipDenseMLP.from_gguf(lay.gguf, lay.config, 0, torch.device("cuda", 0))
        _cache[name] = (lay, mod)
    return _cache[name]


def _mats(lay):
    sp = lay.spec
    H, I = sp.hidden, sp.inter
    shp = {"gate": (I, H), "up": (I, H), "down": (H, I)}
    return [(qt, *shp[p], np.ascontiguousarray(lay.tensor(f"ffn_{p}.weight")))
            for qt, p in zip(sp.qtypes, ("gate", "up", "down"))]


def _run(name, M, n_sample):
    lay, mod = _dense(name)
    log(f"dense {name} M={M}")
    x = lay.draw_x(M)
    xd = torch.from_numpy(x).to("cuda:0")
    out = mod(xd.view(1, M, -1))
    torch.cuda.synchronize()
    assert out.dtype == torch.float32 and out.shape == (1, M, lay.spec.hidden)
    got = out.view(M, -1).cpu().numpy()
    toks = sample_tokens(M, n_sample)
    ref = oracle.dense_forward(x, *_mats(lay), tokens=toks)
    stats = check_layer_output(got[toks], ref)
    log(f"  dense {name} M={M}: {stats}")
    return got


@pytest.mark.parametrize("M", [1, 2, 8, 16, 300])
def test_dense_tiny(M):
    _run("dense_tiny", M, 16)


@pytest.mark.parametrize("M", [1, 64])
def test_dense_q8(M):
    _run("dense_q8", M, 8)


# M = 1, 4, 8: the decode gate/up and down loop over row blocks (N = 12288 and 4096)
@pytest.mark.parametrize("M", [1, 4, 8, 4096])
def test_dense_8b(M):
    _run("dense_8b", M, 4)


def test_dense_deterministic_and_graph_replay():
    lay, mod = _dense("dense_tiny")
    for M in (3, 100):
        x = torch.from_numpy(lay.draw_x(M)).to("cuda:0")
        ref = mod(x).clone()
        assert torch.equal(mod(x), ref)
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            mod(x)
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=s):
                out = mod(x)
        torch.cuda.synchronize()
        for _ in range(3):
            other = mod(x[1:])
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, ref) and other.shape[0] == M - 1


def test_dense_zero_tokens_and_contract_errors():
    from pgmoe import HipDenseMLP
    lay, mod = _dense("dense_tiny")
    empty = mod(torch.zeros((0, lay.spec.hidden), dtype=torch.float16, device="cuda:0"))
    assert empty.shape == (0, lay.spec.hidden)
    with pytest.raises(ValueError):
        mod(torch.zeros((2, lay.spec.hidden + 256), dtype=torch.float16, device="cuda:0"))
    gem = SyntheticDense(DenseSpec("g", 256, 512, DENSE_CONFIGS["dense_tiny"].qtypes, arch="gemma2"))
    assert HipDenseMLP(gem.gguf, gem.config, 0, torch.device("cuda", 0)).use_gelu  # GeGLU (model.py:800)
