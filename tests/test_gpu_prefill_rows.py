"""Every output row of the prefill configs (C3 M=4096 with the Zipf router bias, C4
Mixtral M=2048, C5 Qwen2 + shared expert M=512) against a plain torch fp32 reference of
the same layer on the GPU (oracle routing and oracle-decoded weights, rocBLAS products,
float64 accumulation).  That reference is itself pinned to the float64 C oracle on a token
sample in the same test.  Bounds: rel-L2 <= 1e-3 over the whole output, and
max|d| / max|ref| <= 2e-2 for the whole output and for every row separately.
"""

import time

import numpy as np
import pytest

import oracle
from gpu_helpers import build_pair, check_forward_routing, check_layer_output, check_rows, log, sample_tokens
from gpu_helpers import torch_fp32_reference
from pgmoe.synth import CONFIGS

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    yield
    torch.cuda.empty_cache()


@pytest.mark.parametrize("name,M", [("qwen3_30b_a3b_zipf", 4096), ("mixtral_8x7b", 2048), ("qwen2_57b_a14b", 512)])
def test_prefill_every_row(name, M):
    t0 = time.time()
    log(f"prefill rows {name} M={M}: building")
    lay, ol, mod = build_pair(CONFIGS[name], seed=0)
    dev = torch.device("cuda", 0)
    x = lay.draw_x(M)
    got = mod(torch.from_numpy(x).to(dev)).cpu().numpy()
    logits, idx, w = ol.route(x)
    check_forward_routing(mod, M, idx, w)
    log(f"  forward + routing checked ({time.time() - t0:.1f} s); torch fp32 reference")
    ref = torch_fp32_reference(ol, x, idx, w, dev)
    toks = sample_tokens(M, 6, seed=1)
    pin = check_layer_output(ref[toks], ol.forward_tokens(x, idx, w, tokens=toks), rel_l2=1e-5, max_rel=1e-5)
    log(f"  torch reference vs float64 oracle on {len(toks)} rows: {pin}")
    stats = check_rows(got, ref)
    log(f"  {name} M={M}, all rows: {stats} ({time.time() - t0:.1f} s)")
    del mod
    torch.cuda.empty_cache()
