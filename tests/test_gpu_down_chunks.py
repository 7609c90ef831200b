"""GPU parity of the decode down + combine when the pairs' SwiGLU rows do not fit in LDS
at once and are staged a chunk of super-block columns at a time (dec_dc_chunk_kernel):
every down format, chunk counts with and without a shorter last chunk, every output row
against the oracle, and the same bits run to run.

With top_k = 8 and I = 1280 (5 super-blocks a row): M = 3 stages all 24 rows at once;
M = 4 (32 rows) takes chunks of 4 + 1 columns; M = 8 (64 rows) chunks of 2 + 2 + 1.

One token in Q4_1 / Q4_K / Q5_K gate/up runs 8-row blocks that leave 8-row sums of the
SwiGLU rows, which the down kernels pair into the 16-row sums their formats use; Q6_K and
Q8_0 gate/up keep 16-row sums.  Both are covered with the rows staged whole (top_k 8,
I = 1280) and in chunks (top_k 16, I = 2560: 16 rows of 10 super-blocks, chunks 8 + 2).
"""

import numpy as np
import pytest

from gpu_helpers import build_pair, check_forward_routing, check_layer_output, log
from pgmoe.synth import LayerSpec

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

Q4_1, Q4_K, Q5_K, Q6_K, Q8_0 = 3, 12, 13, 14, 8


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    yield
    torch.cuda.empty_cache()


@pytest.mark.parametrize("down", [Q4_K, Q6_K, Q8_0, Q5_K, Q4_1])
def test_chunked_down_combine(down):
    spec = LayerSpec(f"chunks_{down}", 512, 32, 8, 1280, (Q4_K, Q4_K, down))
    lay, ol, mod = build_pair(spec, seed=3)
    for M in (3, 4, 8):
        log(f"chunked down qtype {down} M={M}")
        x = lay.draw_x(M)
        xt = torch.from_numpy(x).to("cuda:0")
        got = mod(xt).cpu().numpy()
        _, idx, w = ol.route(x)
        check_forward_routing(mod, M, idx, w)
        check_layer_output(got, ol.forward_tokens(x, idx, w))
        again = mod(xt).cpu().numpy()
        assert np.array_equal(got, again), "not reproducible run to run"
    mod.check_status(sync=True)


@pytest.mark.parametrize("qts", [(Q4_1, Q4_1), (Q4_K, Q6_K), (Q5_K, Q4_K), (Q8_0, Q8_0), (Q6_K, Q5_K)])
@pytest.mark.parametrize("topk,inter", [(8, 1280), (16, 2560)])
def test_one_token_sums(qts, topk, inter):
    gu, down = qts
    spec = LayerSpec(f"one_{gu}_{down}_{topk}", 512, 32, topk, inter, (gu, gu, down))
    lay, ol, mod = build_pair(spec, seed=5)
    xs = lay.draw_x(3)
    for rep in range(3):
        log(f"one token gate/up {gu} down {down} top_k {topk} I {inter} row {rep}")
        x = np.ascontiguousarray(xs[rep:rep + 1])
        got = mod(torch.from_numpy(x).to("cuda:0")).cpu().numpy()
        _, idx, w = ol.route(x)
        check_forward_routing(mod, 1, idx, w)
        check_layer_output(got, ol.forward_tokens(x, idx, w))
    mod.check_status(sync=True)
