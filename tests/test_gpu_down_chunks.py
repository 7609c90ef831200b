"""GPU parity of the decode down + combine when the pairs' SwiGLU rows do not fit in LDS
at once and are staged a chunk of super-block columns at a time (dec_dc_chunk_kernel):
every down format, chunk counts with and without a shorter last chunk, every output row
against the oracle, and the same bits run to run.

With top_k = 8 and I = 1280 (5 super-blocks a row): M = 3 stages all 24 rows at once;
M = 4 (32 rows) takes chunks of 4 + 1 columns; M = 8 (64 rows) chunks of 2 + 2 + 1.
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
    mod.check_status()
