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


@pytest.mark.parametrize("name,M", [("qwen3_30b_a3b_zipf", 4096), ("qwen3_30b_a3b", 2048)])
def test_prefill_forward_bit_equal_to_stages(name, M):
    """The forward (multi-block dispatch, the GEMMs in the dispatch's tile order, its own
    workspace) against the stage entry points run one after another (one-block dispatch,
    tiles in expert order, separate buffers): same routing and the same per-tile arithmetic,
    so the outputs must be equal bit for bit, with some tokens scaled up so that their
    SwiGLU rows exceed the fp16-safe 16384 (the row-scale's rs > 1 branch)."""
    from pgmoe import ops
    log(f"forward vs stages {name} M={M}")
    lay, ol, mod = build_pair(CONFIGS[name], seed=3)
    dev = torch.device("cuda", 0)
    x = lay.draw_x(M)
    K, E = mod.top_k, mod.n_experts
    Wg, Wu, Wd = mod.gate_exps.weights(), mod.up_exps.weights(), mod.down_exps.weights()

    def stages(xd):
        _, idx, tw = ops.router_topk(xd, mod.router_weight, mod.router_bias, K, mod.norm_topk_prob)
        disp = ops.dispatch(idx, E, 256)
        inter = ops.expert_gateup(Wg, Wu, xd, K, disp, 1)
        partial = ops.expert_down(Wd, inter, M, K, disp, tw, 1)
        return ops.combine(partial, disp[2], M, K), inter

    _, inter0 = stages(torch.from_numpy(x).to(dev))
    row_max = float(torch.median(inter0.abs().amax(dim=1)))
    f = min(np.sqrt(4 * 16384.0 / max(row_max, 1e-6)), 30000.0 / float(np.abs(x).max()))
    xs = x.copy()
    xs[::5] = (xs[::5].astype(np.float32) * np.float32(f)).astype(np.float16)
    xd = torch.from_numpy(xs).to(dev)
    ref, inter = stages(xd)
    n_big = int((inter.abs().amax(dim=1) > 16384.0).sum())
    got = mod(xd)
    torch.cuda.synchronize()
    log(f"  scale {f:.1f} on every fifth token: {n_big} of {M * K} rows with rs > 1")
    assert n_big > 0
    assert torch.equal(got.view(torch.int32), ref.view(torch.int32))
    del mod
    torch.cuda.empty_cache()
