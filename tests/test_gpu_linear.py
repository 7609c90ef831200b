"""GPU parity of the quantized linear (GGUFQuantLinear / FusedLinearPack drop-ins over
pgmoe_linear_forward and pgmoe_dequant_rows).

* the reference's own quantized matmul outputs (golden mm_* vectors written from
  exec_w4a16 / exec_w8a16_matmul's CPU path) through the GEMV (M = 5) and the GEMM (M = 16);
* attention-projection, fused q|k|v and lm_head shapes at M = 1, 8 and 512 against a torch
  fp32 reference on the oracle-decoded weights: rel-L2 <= 1e-3 and max|d|/max|ref| <= 2e-2
  (the GEMV path, fp32 throughout, to 1e-4);
* fusion: a FusedLinearPack's outputs equal the separate modules';
* embed_lookup: rows bit-equal to the oracle's decode (fp32), and its fp16 rounding.
"""

import numpy as np
import pytest

import oracle
from gpu_helpers import check_layer_output, log
from pgmoe.synth import random_blocks

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

Q4_0, Q4_1, Q4_K, Q6_K, Q8_0 = 2, 3, 12, 14, 8
QT = {"q4_k": Q4_K, "q6_k": Q6_K, "q8_0": Q8_0}


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda", 0)


def _lin(qt, N, K, seed, dev, bias=False, scale=0.01):
    from pgmoe import GGUFQuantLinear
    rng = np.random.default_rng(seed)
    raw = random_blocks(rng, qt, N, K, scale)
    b = torch.from_numpy(rng.standard_normal(N).astype(np.float16)).float() if bias else None
    mode = "w4" if qt in (Q4_0, Q4_1, Q4_K) else "w8"
    return GGUFQuantLinear(mode, K, N, qt, raw=raw, bias=b, device=dev), raw, b


def _ref(raw, qt, N, K, x, bias, dev):
    """torch fp32 product on the oracle-decoded weights (float64 on the CPU for small N)."""
    w = oracle.dequant(qt, raw, N, K)
    if N * K <= 1 << 22:
        y = x.astype(np.float64) @ w.astype(np.float64).T
        return y + (bias.numpy().astype(np.float64) if bias is not None else 0.0)
    torch.backends.cuda.matmul.allow_tf32 = False
    y = torch.from_numpy(x).to(dev).float() @ torch.from_numpy(w).to(dev).T
    if bias is not None:
        y = y + bias.to(dev)
    return y.double().cpu().numpy()


@pytest.mark.parametrize("name", ["q4_k", "q6_k", "q8_0"])
def test_reference_matmul_golden(dev, golden, name):
    from pgmoe import GGUFQuantLinear
    raw = golden[f"dq_{name}_small_raw"]
    qt = QT[name]
    lin = GGUFQuantLinear("w4" if qt == Q4_K else "w8", 512, 4, qt, raw=raw, device=dev)
    x = golden["mm_x"]
    ref = golden[f"mm_{name}_out"].astype(np.float32)  # the reference's exec_w*a16_matmul, fp16
    dense = oracle.dequant(qt, raw, 4, 512).astype(np.float64)
    for M in (5, 16):  # GEMV, then the GEMM with the golden rows repeated
        xm = np.concatenate([x] * (M // 5 + 1))[:M]
        out = lin(torch.from_numpy(xm).to(dev))
        assert out.dtype == torch.float16 and out.shape == (M, 4)
        got = out.float().cpu().numpy()
        rows = np.arange(M) % 5
        np.testing.assert_allclose(got, ref[rows], rtol=2e-3, atol=2e-4)
        exact = xm.astype(np.float64) @ dense.T
        if M <= 8:  # GEMV: fp32 products, then the fp16 output rounding
            np.testing.assert_allclose(got, exact, rtol=2e-3, atol=2e-4)
        else:  # MFMA: fp16 weight operands, like the reference's own GPU tl.dot path
            check_layer_output(got, exact)


@pytest.mark.parametrize("qt,N,K,bias", [(Q4_K, 4096, 2048, False), (Q6_K, 512, 2048, True),
                                         (Q8_0, 3584, 3584, True), (Q4_K, 1000, 4096, False),
                                         (Q6_K, 32000, 4096, False), (Q4_0, 2048, 2048, False),
                                         (Q4_1, 1536, 2048, True)])
@pytest.mark.parametrize("M", [1, 8, 512])
def test_linear_shapes(dev, qt, N, K, bias, M):
    log(f"linear qt={qt} N={N} K={K} bias={bias} M={M}")
    lin, raw, b = _lin(qt, N, K, N + K + qt, dev, bias=bias)
    rng = np.random.default_rng(M)
    x = rng.standard_normal((M, K)).astype(np.float16)
    out = lin(torch.from_numpy(x).to(dev).float()).cpu().numpy()  # fp32 in -> fp32 out
    ref = _ref(raw, qt, N, K, x, b, dev)
    if M <= 8:  # GEMV: fp32 products
        check_layer_output(out, ref, rel_l2=1e-4, max_rel=1e-4)
    else:
        check_layer_output(out, ref)
    out16 = lin(torch.from_numpy(x).to(dev))
    assert out16.dtype == torch.float16
    # the fp16 output is the fp32 result rounded (the bias/cast pass or the GEMV epilogue)
    assert np.array_equal(out16.cpu().numpy().view(np.uint16), out.astype(np.float16).view(np.uint16))


def test_fused_pack_equals_separate(dev):
    from pgmoe import FusedLinearPack, GGUFQuantLinear
    q, rq, _ = _lin(Q4_K, 2048, 2048, 1, dev)
    k, rk, bk = _lin(Q4_K, 512, 2048, 2, dev, bias=True)
    v, rv, _ = _lin(Q6_K, 512, 2048, 3, dev)
    o, ro, _ = _lin(Q4_K, 256, 2048, 4, dev)
    pack = FusedLinearPack([q, k, v, o])  # q, k, o fuse (Q4_K); v stays alone (Q6_K)
    assert len(pack.groups) == 2 and not pack.is_single_contiguous
    qk = FusedLinearPack([q, k])
    assert qk.is_single_contiguous
    for M in (1, 8, 300):
        x = torch.from_numpy(np.random.default_rng(M).standard_normal((M, 2048)).astype(np.float16)).to(dev)
        outs = pack(x)
        sep = [m(x) for m in (q, k, v, o)]
        for a, s in zip(outs, sep):
            assert a.shape == s.shape
            if M <= 8:
                assert torch.equal(a, s)
            else:
                torch.testing.assert_close(a.float(), s.float(), rtol=1e-3, atol=1e-3)
        cat = qk.forward_single_concat(x)
        assert cat.shape == (M, 2560)
    with pytest.raises(ValueError):
        GGUFQuantLinear.fuse([q, v])


def test_embed_lookup(dev):
    for qt, N, K in ((Q4_K, 300, 512), (Q6_K, 77, 768), (Q8_0, 129, 256), (Q4_1, 70, 512), (Q4_0, 65, 256)):
        lin, raw, _ = _lin(qt, N, K, qt, dev, scale=1.0)
        ids = torch.tensor([[0, N - 1, 5], [64, 63, 5]], dtype=torch.int64)
        got = lin.embed_lookup(ids, dtype=torch.float32)
        assert got.shape == (2, 3, K)
        dense = oracle.dequant(qt, raw, N, K)
        ref = dense[ids.reshape(-1).numpy()].reshape(2, 3, K)
        assert np.array_equal(got.cpu().numpy().view(np.uint32), ref.view(np.uint32))
        g16 = lin.embed_lookup(ids)
        assert g16.dtype == torch.float16
        assert np.array_equal(g16.cpu().numpy().view(np.uint16), ref.astype(np.float16).view(np.uint16))
        with pytest.raises(IndexError):  # ids on the host are range-checked there
            lin.embed_lookup(torch.tensor([N]))
        # ids on the device are not read back (no host sync): an id out of range is a NaN row
        bad = lin.embed_lookup(torch.tensor([N, 1], device=dev), dtype=torch.float32).cpu().numpy()
        assert np.all(np.isnan(bad[0])) and np.array_equal(bad[1].view(np.uint32), dense[1].view(np.uint32))


def test_embed_lookup_and_linear_replay_from_a_captured_graph(dev):
    """The reference captures embed_lookup and the quantized projections in its decode
    graphs (model.py:1803, :1827, :2039): both drop-ins record without a host sync, and
    every replay (eager work and synchronisations between them) equals the eager result."""
    lin, _, _ = _lin(Q4_K, 300, 512, 11, dev, scale=1.0)
    proj, _, _ = _lin(Q4_K, 256, 512, 12, dev)
    ids = torch.tensor([3, 299, 64], device=dev)
    x = torch.from_numpy(np.random.default_rng(5).standard_normal((1, 512)).astype(np.float16)).to(dev)
    e_ref = lin.embed_lookup(ids).clone()
    y_ref = proj(x).clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        lin.embed_lookup(ids)
        proj(x)  # the stream's workspace exists before capture
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            e_g = lin.embed_lookup(ids)
            y_g = proj(x)
    torch.cuda.synchronize()
    for i in range(3):
        e_g.zero_()
        y_g.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(e_g, e_ref) and torch.equal(y_g, y_ref), f"replay {i}"
        lin.embed_lookup(torch.tensor([i], device=dev))  # eager work between replays
        torch.cuda.synchronize()


def test_unsupported_widths_and_formats(dev):
    from pgmoe import GGUFQuantLinear
    with pytest.raises(NotImplementedError):  # K-quants: a multiple of 256 (32-weight formats are padded)
        GGUFQuantLinear("w4", 320, 4, Q4_K, raw=np.zeros(4 * 144, np.uint8), device=dev)
    with pytest.raises(NotImplementedError):  # 32-weight formats: whole blocks
        GGUFQuantLinear("w8", 80, 4, Q8_0, raw=np.zeros(4 * 3 * 34, np.uint8), device=dev)
    with pytest.raises(NotImplementedError):
        GGUFQuantLinear("w4", 256, 4, 16, raw=np.zeros(4 * 66, np.uint8), device=dev)  # IQ2_XXS
