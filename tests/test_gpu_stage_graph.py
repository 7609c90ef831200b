"""A captured decode stage: the pre-FFN residual add + RMSNorm feeding the MoE block, twice
(layer l's norm -> MoE -> layer l+1's norm -> MoE), with static input buffers, captured
once per token count as one HIP graph and replayed.  This is the capture the reference
switches off for MoE models (model.py:1575 enable_cuda_graph, :1947-1948 verify graphs)
because its MoE block syncs the host; here it runs at M = 1 (decode) and at the verify
sizes 2..8.

Every replay (new inputs copied into the static buffers, eager work between replays) is
checked stage by stage against the oracle, each stage given the GPU's own input to it
(so that no tolerance compounds): the norms bit for bit (or_add_rmsnorm), each MoE
output on every row (rel-L2 <= 1e-3, max|d| / max|ref| <= 2e-2) with its routing from the
oracle; and the replay equals an eager run of the same stage on the same inputs.
"""

import numpy as np
import pytest

import oracle
from gpu_helpers import build_pair, check_layer_output, log
from pgmoe.synth import CONFIGS

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

EPS = 1e-6


@pytest.fixture(scope="module")
def layers():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    spec = CONFIGS["qwen3_30b_a3b"]
    pairs = [build_pair(spec, seed=s) for s in (0, 1)]
    rng = np.random.default_rng(7)
    norms = [(1.0 + 0.1 * rng.standard_normal(spec.hidden)).astype(np.float32) for _ in range(2)]
    yield pairs, norms
    del pairs
    torch.cuda.empty_cache()


def _stage(mods, wts, h, delta):
    from pgmoe.norm import exec_fused_add_rmsnorm
    h1, n1 = exec_fused_add_rmsnorm(h, delta, wts[0], EPS, out_dtype=torch.float16)
    d1 = mods[0](n1)
    h2, n2 = exec_fused_add_rmsnorm(h1, d1, wts[1], EPS, out_dtype=torch.float16)
    d2 = mods[1](n2)
    return n1, h1, d1, n2, h2, d2


def _check_against_oracle(ols, norms, h_np, d_np, outs):
    n1, h1, d1, n2, h2, d2 = (t.cpu().numpy() for t in outs)
    oh1, on1 = oracle.add_rmsnorm(h_np, d_np, norms[0], EPS)
    assert np.array_equal(h1.view(np.uint32), oh1.view(np.uint32)), "norm 1 residual"
    assert np.array_equal(n1.view(np.uint16), on1.view(np.uint16)), "norm 1 output"
    for ol, xin, got in ((ols[0], n1, d1), (ols[1], n2, d2)):
        _, idx, w = ol.route(xin)
        check_layer_output(got, ol.forward_tokens(xin, idx, w))
    oh2, on2 = oracle.add_rmsnorm(h1, d1, norms[1], EPS)
    assert np.array_equal(h2.view(np.uint32), oh2.view(np.uint32)), "norm 2 residual"
    assert np.array_equal(n2.view(np.uint16), on2.view(np.uint16)), "norm 2 output"


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 6, 7, 8])
def test_captured_norm_moe_stage_replays(layers, M):
    pairs, norms = layers
    mods = [p[2] for p in pairs]
    ols = [p[1] for p in pairs]
    dev = torch.device("cuda", 0)
    H = ols[0].hidden
    wts = [torch.from_numpy(w).to(dev) for w in norms]
    rng = np.random.default_rng(100 + M)
    h_in = torch.zeros((M, H), dtype=torch.float32, device=dev)
    d_in = torch.zeros((M, H), dtype=torch.float32, device=dev)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        _stage(mods, wts, h_in, d_in)  # the stream's workspaces exist before capture
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            outs = _stage(mods, wts, h_in, d_in)
    torch.cuda.synchronize()
    log(f"stage graph M={M}: captured")
    for rep in range(3):
        h_np = rng.standard_normal((M, H)).astype(np.float32)
        d_np = rng.standard_normal((M, H)).astype(np.float32)
        h_in.copy_(torch.from_numpy(h_np))
        d_in.copy_(torch.from_numpy(d_np))
        with torch.cuda.stream(s):
            g.replay()
        torch.cuda.synchronize()
        got = [t.clone() for t in outs]
        with torch.cuda.stream(s):
            eager = _stage(mods, wts, h_in, d_in)  # eager work between replays
        torch.cuda.synchronize()
        for a, b in zip(got, eager):
            assert torch.equal(a, b), f"replay {rep} differs from the eager stage"
        _check_against_oracle(ols, norms, h_np, d_np, got)
        log(f"  replay {rep}: norms bit-exact, both MoE outputs within tolerance")
    del g
    for m in mods:
        m.check_status(sync=True)
