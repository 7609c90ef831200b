"""The routing the timed forward itself computes, pinned bit for bit against the oracle.

At M <= 8 the forward routes inside the routed gate/up launch (folded router -> radix
top-k selection -> slot derivation -> the published routing descriptor), not through the
stage API's router / top-k / dispatch kernels.  pgmoe_moe_routing reads that descriptor
back from the forward's own workspace (for M > 8, the top-k / dispatch arrays the prefill
forward wrote), so these tests compare the routing of exactly the path bench.py times:
expert offsets, sorted pair experts and tokens bit-exact, ties to the lower expert id
(model.py:903-914; the north star's rule), weights to fp32 rounding.
"""

import numpy as np
import pytest

import oracle
from gpu_helpers import build_pair, check_forward_routing, check_layer_output, log
from pgmoe.synth import CONFIGS, LayerSpec

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

Q4_K, Q6_K, Q8_0 = 12, 14, 8
_cache = {}


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    yield
    _cache.clear()


def _pair(name):
    if name not in _cache:
        _cache.clear()
        torch.cuda.empty_cache()
        _cache[name] = build_pair(CONFIGS[name], seed=0)
    return _cache[name]


@pytest.mark.parametrize("name,Ms", [("tiny", (1, 2, 4, 8, 16)), ("qwen3_30b_a3b", (1, 2, 4, 8, 64)),
                                     ("qwen2_57b_a14b", (1, 2, 4, 8, 24))])
def test_forward_routing_bitexact(name, Ms):
    lay, ol, mod = _pair(name)
    for M in Ms:
        log(f"forward routing {name} M={M}")
        x = lay.draw_x(M)
        out = mod(torch.from_numpy(x).to("cuda:0"))
        logits, idx, w = ol.route(x)
        check_forward_routing(mod, M, idx, w)
        log(f"  min top-k margin {oracle.min_topk_margin(logits, mod.top_k):.2e}")
        if M <= 8:  # the output of the same forward, every row
            check_layer_output(out.cpu().numpy(), ol.forward_tokens(x, idx, w))
    mod.check_status(sync=True)


def _tie_layer(seed=5):
    """E = 16, K = 4 with router rows 1, 2, 4, 6 and 12 identical (and 5x larger than the
    rest): their logits are bitwise equal, and every token's input is signed so that they
    are its five largest.  Four of five tied experts are taken: {1, 2, 4, 6}, never 12."""
    spec = LayerSpec("ties", 512, 16, 4, 256, (Q4_K, Q4_K, Q6_K))
    lay, ol, mod = build_pair(spec, seed=seed, scale=0.01)
    rng = np.random.default_rng(seed)
    W = (rng.standard_normal((16, 512), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    r0 = (W[0] * np.float32(5.0)).astype(np.float32)
    for e in (1, 2, 4, 6, 12):
        W[e] = r0
    with torch.no_grad():
        mod.router_weight.copy_(torch.from_numpy(W))
    ol.router_w = W
    return lay, ol, mod, r0


@pytest.mark.parametrize("M", [1, 3, 8, 40])
def test_forward_routing_ties_lower_id_wins(M):
    lay, ol, mod, r0 = _tie_layer()
    cand = lay.draw_x(16 * M + 64).astype(np.float32)
    s = np.sign(cand @ r0)
    s[s == 0] = 1.0
    cand = (cand * s[:, None]).astype(np.float16)  # exact sign flips: r0's logit is positive
    lc = oracle.router_logits(cand, ol.router_w)
    tied = np.array([1, 2, 4, 6, 12])
    rest = np.setdiff1d(np.arange(16), tied)
    keep = np.nonzero(lc[:, 1] > lc[:, rest].max(axis=1))[0]  # the tied five are the top five
    assert len(keep) >= M
    x = np.ascontiguousarray(cand[keep[:M]])
    logits, idx, w = ol.route(x)
    assert np.all(logits[:, 1] == logits[:, 12]) and np.all(logits[:, 2] == logits[:, 6])
    assert np.all(np.sort(idx, axis=1) == np.array([1, 2, 4, 6], np.int32)), "oracle tie rule"
    log(f"ties M={M}")
    out = mod(torch.from_numpy(x).to("cuda:0"))
    check_forward_routing(mod, M, idx, w)
    check_layer_output(out.cpu().numpy(), ol.forward_tokens(x, idx, w), abs_tol=2e-2 if M <= 8 else None)
    mod.check_status(sync=True)


def test_graph_replay_matches_oracle_qwen3_decode():
    """HIP-graph replays of the C2 decode forward (M = 1..8), each replay checked against
    the oracle on every row and against the eager result, with eager forwards of other
    token counts (on the capture stream, growing its workspace) run between replays."""
    lay, ol, mod = _pair("qwen3_30b_a3b")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    for M in (1, 2, 4, 8):
        log(f"graph replay qwen3 M={M}")
        x_np = lay.draw_x(M)
        x = torch.from_numpy(x_np).to("cuda:0")
        _, idx, w = ol.route(x_np)
        ref = ol.forward_tokens(x_np, idx, w)
        with torch.cuda.stream(s):
            eager = mod(x).clone()
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=s):
                out = mod(x)
        torch.cuda.synchronize()
        for rep in range(3):
            other_M = 8 + 8 * (rep + 1) * M  # prefill-sized calls: the stream's workspace grows
            xo_np = lay.draw_x(other_M)
            with torch.cuda.stream(s):
                other = mod(torch.from_numpy(xo_np).to("cuda:0"))
                g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager), (M, rep)
            check_layer_output(out.cpu().numpy(), ref)
            # the eager call between replays is itself right (its workspace was not disturbed)
            _, oi, ow = ol.route(xo_np)
            toks = np.array([0, other_M - 1], np.int32)
            check_layer_output(other.cpu().numpy()[toks], ol.forward_tokens(xo_np, oi, ow, tokens=toks))
        del g
    mod.check_status(sync=True)
