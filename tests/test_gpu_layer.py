"""GPU parity of the whole layer (HipSparseMoEMLP.forward through pgmoe_moe_forward)
against the CPU oracle, on every BASELINE config at its real shape.

Gates (north star): routing ids bit-exact; rel-L2 <= 1e-3 and max|d|/max|ref| <= 2e-2
against the float64-accumulated oracle (absolute max 2e-2 on the realistic-scale set,
where outputs are O(1); at benchmark scale outputs reach 1e7-1e8, where an absolute
2e-2 is below fp32 resolution).  Large M is checked on a token sample (each token's
output depends only on its own input), routing/dispatch on all tokens.
"""

import numpy as np
import pytest

import oracle
from gpu_helpers import build_pair, check_layer_output, log, sample_tokens
from pgmoe.synth import CONFIGS, LayerSpec

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

_cache = {}


def _pair(name, scale=1.0):
    key = (name, scale)
    if key not in _cache:
        _cache.clear()  # keep one big layer resident at a time
        torch.cuda.empty_cache()
        _cache[key] = build_pair(CONFIGS[name], seed=0, scale=scale)
    return _cache[key]


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    yield
    _cache.clear()


def _run(name, M, n_sample, scale=1.0, abs_tol=None):
    lay, ol, mod = _pair(name, scale)
    log(f"layer {name} M={M} scale={scale}")
    x = lay.draw_x(M)
    xd = torch.from_numpy(x).to("cuda:0").view(1, M, -1)
    out = mod(xd)
    torch.cuda.synchronize()
    assert out.dtype == torch.float32 and out.shape == xd.shape
    got = out.view(M, -1).cpu().numpy()
    logits, idx, w = ol.route(x)
    # routing: GPU top-k ids equal the oracle's
    from pgmoe import ops
    _, gidx, gw = ops.router_topk(xd.view(M, -1), mod.router_weight, mod.router_bias, mod.top_k,
                                  mod.norm_topk_prob)
    assert np.array_equal(gidx.cpu().numpy(), idx)
    margin = oracle.min_topk_margin(logits, mod.top_k)
    toks = sample_tokens(M, n_sample)
    ref = ol.forward_tokens(x, idx, w, tokens=toks)
    stats = check_layer_output(got[toks], ref, abs_tol=abs_tol)
    log(f"  {name} M={M}: {stats} min top-k margin {margin:.2e}")
    return got


@pytest.mark.parametrize("M", [1, 16])
def test_tiny(M):
    _run("tiny", M, 16)


@pytest.mark.parametrize("M", [1, 2, 4, 8])
def test_qwen3_decode(M):
    _run("qwen3_30b_a3b", M, 8)


@pytest.mark.parametrize("M", [1, 4])
def test_qwen3_realistic_scale_absolute(M):
    # decode path keeps fp32 throughout: the literal absolute bound holds
    _run("qwen3_30b_a3b", M, M, scale=0.01, abs_tol=2e-2)


def test_qwen3_realistic_scale_mfma_vs_reference_error():
    """The prefill path feeds fp16 operands to MFMA (dequantised weights, row-scaled fp16
    down input), like the reference's own tl.dot prefill kernel.  At realistic scale the
    outputs reach ~40, where fp16 operand rounding alone is ~1e-3 relative, so the gate
    is: rel-L2 <= 1e-3, max|d|/max|ref| <= 2e-2, and a max-abs error no larger than the
    reference CPU path's own (torch port with the reference's fp16 casts) on the same
    tokens against the same float64 oracle."""
    from oracle import torch_port
    lay, ol, mod = _pair("qwen3_30b_a3b", 0.01)
    M = 64
    got = _run("qwen3_30b_a3b", M, 8, scale=0.01)
    x = lay.draw_x(M)
    _, idx, w = ol.route(x)
    toks = sample_tokens(M, 8)
    ref = ol.forward_tokens(x, idx, w, tokens=toks)
    port = torch_port.PortMoE(ol)
    ref_path = port.forward(torch.from_numpy(x), faithful=True).numpy()[toks]
    ours = float(np.max(np.abs(got[toks] - ref)))
    theirs = float(np.max(np.abs(ref_path - ref)))
    log(f"  realistic M=64 max abs error: ours {ours:.3e}, reference path {theirs:.3e}")
    assert np.all(np.isfinite(ref_path))
    assert ours <= theirs


def test_qwen3_prefill_zipf():
    lay, ol, mod = _pair("qwen3_30b_a3b_zipf")
    M = 4096
    got = _run("qwen3_30b_a3b_zipf", M, 24)
    # skewed loads really happened
    _, idx, _ = ol.route(lay.draw_x(M))
    counts = np.bincount(idx.reshape(-1), minlength=128)
    log(f"  zipf loads: empty={int((counts == 0).sum())} max={int(counts.max())} >500={int((counts > 500).sum())}")
    assert (counts == 0).sum() > 0 and counts.max() > 500


# M = 1..8: N = 14336 gives more gate/up row blocks (and H = 4096 down row blocks) than
# resident blocks, so the decode launches loop over row blocks
@pytest.mark.parametrize("M", [1, 2, 4, 8, 2048])
def test_mixtral(M):
    _run("mixtral_8x7b", M, 6)


@pytest.mark.parametrize("M", [1, 2, 8, 512])
def test_qwen2_shared_expert(M):
    _run("qwen2_57b_a14b", M, 6)


def test_deterministic_repeat():
    lay, ol, mod = _pair("tiny")
    for M in (1, 3, 100):
        xd = torch.from_numpy(lay.draw_x(M)).to("cuda:0")
        a = mod(xd).cpu().numpy()
        b = mod(xd).cpu().numpy()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_zero_tokens_and_zero_input():
    lay, ol, mod = _pair("tiny")
    out = mod(torch.zeros((1, 0, 1024), dtype=torch.float16, device="cuda:0"))
    assert out.shape == (1, 0, 1024)
    z = mod(torch.zeros((5, 1024), dtype=torch.float16, device="cuda:0"))
    assert torch.all(z == 0)


def test_all_tokens_one_expert_and_top_k_equals_e():
    spec = LayerSpec("skew", 512, 4, 4, 256, (12, 12, 14))
    lay, ol, mod = build_pair(spec, seed=3, scale=0.01)
    for M in (7, 300):
        x = lay.draw_x(M)
        got = mod(torch.from_numpy(x).to("cuda:0")).cpu().numpy()
        _, idx, w = ol.route(x)
        # literal absolute bound on the fp32 decode path; MFMA path: relative bounds
        check_layer_output(got, ol.forward_tokens(x, idx, w), abs_tol=2e-2 if M <= 8 else None)
    spec1 = LayerSpec("one", 512, 8, 1, 256, (12, 12, 12))
    lay1, ol1, mod1 = build_pair(spec1, seed=4, scale=0.01)
    bias = np.full(8, -100.0, np.float32)
    bias[6] = 100.0  # every token routes to expert 6
    mod1.set_router_bias(torch.from_numpy(bias))
    ol1.router_bias = bias
    for M in (1, 5, 200):
        x = lay1.draw_x(M)
        got = mod1(torch.from_numpy(x).to("cuda:0")).cpu().numpy()
        _, idx, w = ol1.route(x)
        assert np.all(idx == 6)
        check_layer_output(got, ol1.forward_tokens(x, idx, w), abs_tol=2e-2 if M <= 8 else None)


def test_timed_forward_matches_forward_and_times_every_launch():
    """pgmoe_moe_forward_timed: same bits as the forward; one event pair and one kernel name
    per launch, in the documented order."""
    import ctypes
    from gpu_helpers import HipEvents
    from pgmoe._lib import check, lib
    lay, ol, mod = _pair("tiny")
    starts, stops = HipEvents(16), HipEvents(16)
    # decode: gate/up (router folded in), down + combine; prefill: router, top-k, dispatch,
    # gate/up, row-scale, down, combine, each product possibly followed by its split reduce
    want = {1: ["dec_gu_kernel", "dec_dc_kernel"],
            16: ["router_", "topk_kernel", "dispatch_kernel", ", true,", "rowscale_kernel", ", false,",
                 "combine_kernel"]}
    for M in (1, 16):
        x = torch.from_numpy(lay.draw_x(M)).to("cuda:0")
        ref = mod(x)
        out = torch.empty_like(ref)
        ws = mod._workspace(M)
        n = ctypes.c_int32()
        names = (ctypes.c_char_p * 16)()
        stream = torch.cuda.current_stream().cuda_stream
        check(lib().pgmoe_moe_forward_timed(mod._layer, x.data_ptr(), M, out.data_ptr(), ws.data_ptr(),
                                            ws.numel(), stream, starts.ev, stops.ev, 16, ctypes.byref(n), names),
              "forward_timed")
        torch.cuda.synchronize()
        got = [names[i].decode() for i in range(n.value)]
        main = [g for g in got if "split_reduce" not in g and "dispatch_count" not in g]
        assert len(main) == len(want[M]) and all(w in g for w, g in zip(want[M], main)), got
        assert torch.equal(out, ref)
        if M <= 8:  # decode leaves the router's tagged logits (first in the workspace) at zero
            assert int(ws[:16 * M * mod.n_experts * 8].view(torch.int32).abs().sum().item()) == 0  # 16 copies
        for i in range(n.value):
            d = starts.elapsed_ms(starts.ev[i], stops.ev[i])
            assert 0.0 < d < 50.0, (M, i, d)
        # fewer events than launches: the rest run untimed, same result
        check(lib().pgmoe_moe_forward_timed(mod._layer, x.data_ptr(), M, out.data_ptr(), ws.data_ptr(),
                                            ws.numel(), stream, starts.ev, None, 1, None, None), "forward_timed")
        torch.cuda.synchronize()
        assert torch.equal(out, ref)


def test_one_workspace_across_token_counts():
    """One C-level workspace (sized for the largest M) shared by forwards of different M in
    turn -- decode and prefill -- gives each the bits of a forward on a fresh zeroed
    workspace: the decode router's tagged logits, which persist between forwards, sit at
    the start of the workspace for every M, where no other call writes."""
    from pgmoe._lib import check, lib
    for name in ("tiny", "qwen3_30b_a3b"):
        lay, ol, mod = _pair(name)
        seq = (1, 2, 64, 1, 3, 1, 1)
        nbytes = max(mod.workspace_bytes(M) for M in seq)
        raw = torch.zeros(nbytes + 256, dtype=torch.uint8, device="cuda:0")
        ws = raw[(-raw.data_ptr()) % 256:]
        stream = torch.cuda.current_stream().cuda_stream
        for i, M in enumerate(seq):
            log(f"shared workspace {name}: call {i} M={M}")
            x = torch.from_numpy(lay.draw_x(M + i)[i:]).to("cuda:0")
            out = torch.empty((M, mod.hidden), dtype=torch.float32, device="cuda:0")
            check(lib().pgmoe_moe_forward(mod._layer, x.data_ptr(), M, out.data_ptr(), ws.data_ptr(), ws.numel(),
                                          stream), "forward")
            ref = mod(x)  # its own workspace for this M
            torch.cuda.synchronize()
            assert torch.equal(out, ref), (name, i, M)


def test_graph_replay_equals_eager():
    """A captured forward replays to the eager result, replay after replay, with other
    eager forwards (different inputs) run between the replays."""
    lay, ol, mod = _pair("tiny")
    for M in (1, 16):
        x = torch.from_numpy(lay.draw_x(M)).to("cuda:0")
        x2 = torch.from_numpy(lay.draw_x(M + 1)[1:]).to("cuda:0")
        ref = mod(x).clone()
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
            other = mod(x2)
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, ref)
            assert not torch.equal(other, ref)
