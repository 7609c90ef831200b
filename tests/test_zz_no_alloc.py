"""pgmoe_moe_forward_noalloc (the entry point that allocates nothing) against
pgmoe_moe_forward, through the C ABI.

The two run the same kernels, so the outputs must be bit-identical: on two calls in a row
(the second with fewer tokens), across layers of different expert counts sharing the one
device scratch, on the prefill path within the scratch limit, and from a captured graph.
Token counts beyond the fixed scratch are refused before any launch.
"""

import ctypes

import numpy as np
import pytest

from gpu_helpers import build_pair, log
from pgmoe.synth import CONFIGS

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

PGMOE_E_WORKSPACE = -3


@pytest.fixture(scope="module")
def layers():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    out = {name: build_pair(CONFIGS[name], seed=0) for name in ("tiny", "qwen3_30b_a3b")}
    yield out
    out.clear()
    torch.cuda.empty_cache()


def _noalloc(mod, x):
    from pgmoe._lib import check, lib
    M = x.shape[0]
    out = torch.full((M, mod.hidden), float("nan"), dtype=torch.float32, device=x.device)
    stream = torch.cuda.current_stream().cuda_stream
    check(lib().pgmoe_moe_forward_noalloc(mod._layer, x.data_ptr(), M, out.data_ptr(), stream),
          "pgmoe_moe_forward_noalloc")
    return out


def test_noalloc_equals_forward_on_consecutive_calls(layers):
    """Each call against the workspace forward of the same input; the second call of each
    pair has fewer tokens, and layers with E = 8 and E = 128 take turns on the scratch."""
    seq = [("tiny", 8), ("tiny", 1), ("qwen3_30b_a3b", 8), ("qwen3_30b_a3b", 1), ("tiny", 4),
           ("qwen3_30b_a3b", 3), ("qwen3_30b_a3b", 2), ("tiny", 16), ("tiny", 12), ("qwen3_30b_a3b", 64),
           ("qwen3_30b_a3b", 8)]
    for i, (name, M) in enumerate(seq):
        lay, _, mod = layers[name]
        log(f"noalloc call {i}: {name} M={M}")
        x = torch.from_numpy(lay.draw_x(M + i)[i:]).to("cuda:0")
        got = _noalloc(mod, x)
        ref = mod(x)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), (name, M, i)


def test_noalloc_refuses_token_counts_beyond_its_scratch(layers):
    from pgmoe._lib import lib
    lay, _, mod = layers["qwen3_30b_a3b"]
    M = 4096  # ~420 MB of workspace
    x = torch.zeros((M, mod.hidden), dtype=torch.float16, device="cuda:0")
    out = torch.zeros((M, mod.hidden), dtype=torch.float32, device="cuda:0")
    rc = lib().pgmoe_moe_forward_noalloc(mod._layer, x.data_ptr(), M, out.data_ptr(),
                                         torch.cuda.current_stream().cuda_stream)
    assert rc == PGMOE_E_WORKSPACE
    assert b"scratch" in lib().pgmoe_last_error()
    torch.cuda.synchronize()
    assert int(torch.count_nonzero(out)) == 0  # nothing ran


def test_noalloc_graph_replays(layers):
    """A captured allocation-free forward replays to the eager result, with other
    allocation-free calls (other layer, other M) between the replays."""
    lay, _, mod = layers["qwen3_30b_a3b"]
    tl, _, tmod = layers["tiny"]
    x = torch.from_numpy(lay.draw_x(2)).to("cuda:0")
    xt = torch.from_numpy(tl.draw_x(5)).to("cuda:0")
    ref = mod(x).clone()
    ref_t = tmod(xt).clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        _noalloc(mod, x)  # eager first call on this stream (the scratch is already cleared)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            out = _noalloc(mod, x)
    torch.cuda.synchronize()
    for rep in range(3):
        with torch.cuda.stream(s):
            other = _noalloc(tmod, xt)
            g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), rep
        assert torch.equal(other, ref_t), rep
    del g
