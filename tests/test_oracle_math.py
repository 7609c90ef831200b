"""Pin the oracle where the golden vectors leave room: closed forms, invariants,
brute force on tiny inputs, and textbook routines (numpy) as independent references."""

import numpy as np
import pytest

import oracle
from pgmoe.synth import random_blocks

L = oracle.lib()


def test_half_conversions_match_numpy():
    allh = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = np.array([L.or_half_to_float(int(h)) for h in allh[::7]], dtype=np.float32)
    ref = allh[::7].view(np.float16).astype(np.float32)
    ok = np.isnan(ref) | (f.view(np.uint32) == ref.view(np.uint32))
    assert ok.all()
    rng = np.random.default_rng(0)
    xs = np.concatenate([
        rng.standard_normal(4000).astype(np.float32) * 10.0 ** rng.integers(-9, 6, 4000),
        np.float32([65504, 65519.99, 65520, -65520, 6.1e-5, 5.96e-8, 2.98e-8, 2.99e-8, 0.0, -0.0]),
    ]).astype(np.float32)
    got = np.array([L.or_float_to_half(float(v)) for v in xs], dtype=np.uint16)
    with np.errstate(over="ignore"):
        ref16 = xs.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref16)


def _pack_k_scales(sc, mn):
    """12-byte K-quant header from eight 6-bit (scale, min) pairs, built bit by bit from
    the ggml layout: bytes 0-3 / 4-7 hold the low 6 bits of sc[0:4] / m[0:4] with the
    high 2 bits of sc[4:8] / m[4:8] on top; bytes 8-11 hold the low nibbles of
    sc[4:8] | m[4:8] << 4."""
    b = np.zeros(12, dtype=np.uint8)
    for j in range(4):
        b[j] = (sc[j] & 63) | ((sc[4 + j] >> 4) << 6)
        b[4 + j] = (mn[j] & 63) | ((mn[4 + j] >> 4) << 6)
        b[8 + j] = (sc[4 + j] & 15) | ((mn[4 + j] & 15) << 4)
    return b


def test_q4k_scale_unpack_roundtrip_all_values():
    # every (sc, m) value in every sub-block position decodes back, via all-zero quants:
    # w = d*sc*0 - dmin*m = -m when dmin = 1, and via all-one quants: w = sc - m when d = 1
    for v in range(64):
        for pos in range(8):
            sc = np.full(8, (v * 7 + pos) % 64, dtype=np.int64)
            mn = np.full(8, (v * 5 + 3 * pos) % 64, dtype=np.int64)
            sc[pos], mn[pos] = v, 63 - v
            blk = np.zeros(144, dtype=np.uint8)
            blk[0:2] = np.array([1.0], dtype=np.float16).view(np.uint8)
            blk[2:4] = np.array([1.0], dtype=np.float16).view(np.uint8)
            blk[4:16] = _pack_k_scales(sc, mn)
            w0 = oracle.dequant(oracle.Q4_K, blk, 1, 256).reshape(8, 32)
            assert np.all(w0 == -mn[:, None])
            blk[16:] = 0x11
            w1 = oracle.dequant(oracle.Q4_K, blk, 1, 256).reshape(8, 32)
            assert np.all(w1 == (sc - mn)[:, None])


def test_q4k_nibble_positions():
    # a single set nibble lights exactly one weight: byte 32c+l, low nibble -> sub-block 2c,
    # high nibble -> sub-block 2c+1, element l
    blk = np.zeros(144, dtype=np.uint8)
    blk[0:2] = np.array([1.0], dtype=np.float16).view(np.uint8)
    blk[4:16] = _pack_k_scales(np.ones(8, np.int64), np.zeros(8, np.int64))
    for byte in (0, 5, 31, 32, 77, 127):
        for hi in (0, 1):
            b = blk.copy()
            b[16 + byte] = 0x1 << (4 * hi)
            w = oracle.dequant(oracle.Q4_K, b, 1, 256).reshape(-1)
            c, l = divmod(byte, 32)
            expect = np.zeros(256, np.float32)
            expect[32 * (2 * c + hi) + l] = 1.0
            assert np.array_equal(w, expect)


def test_q6k_ranges_and_zero_block():
    rng = np.random.default_rng(1)
    raw = random_blocks(rng, oracle.Q6_K, 8, 256)
    blk = raw.reshape(8, 210).copy()
    blk[:, 192:208] = 1  # every sub-scale 1
    blk[:, 208:210] = np.array([1.0], dtype=np.float16).view(np.uint8)
    w = oracle.dequant(oracle.Q6_K, blk.reshape(-1), 8, 256)
    assert w.min() >= -32 and w.max() <= 31 and np.all(w == np.round(w))
    assert len(np.unique(w)) == 64  # all 64 codes appear in 2048 uniform draws
    z = np.zeros(210, dtype=np.uint8)
    z[192:208] = np.arange(16, dtype=np.int8).view(np.uint8) - 8
    z[208:210] = np.array([0.5], dtype=np.float16).view(np.uint8)
    wz = oracle.dequant(oracle.Q6_K, z, 1, 256).reshape(16, 16)
    assert np.all(wz == (-32 * 0.5 * (np.arange(16) - 8))[:, None])


def test_q6k_bit_positions():
    # element n = 128h + 32s + l takes its low nibble from ql[64h + 32(s&1) + l] (shift
    # 4*(s>>1)) and its two high bits from qh[32h + l] (shift 2s)
    base = np.zeros(210, dtype=np.uint8)
    base[192:208] = 1
    base[208:210] = np.array([1.0], dtype=np.float16).view(np.uint8)
    for h in range(2):
        for s in range(4):
            for l in (0, 13, 31):
                n = 128 * h + 32 * s + l
                b = base.copy()
                b[64 * h + 32 * (s & 1) + l] |= 0x5 << (4 * (s >> 1))
                b[128 + 32 * h + l] |= 0x2 << (2 * s)
                w = oracle.dequant(oracle.Q6_K, b, 1, 256).reshape(-1)
                assert w[n] == (0x5 | (0x2 << 4)) - 32
                others = np.delete(w, n)
                assert np.all(others == -32)


def test_q8_0_closed_form():
    rng = np.random.default_rng(2)
    raw = random_blocks(rng, oracle.Q8_0, 3, 64)
    blk = raw.reshape(-1, 34)
    d = blk[:, 0:2].copy().view(np.float16).astype(np.float32)
    q = blk[:, 2:].copy().view(np.int8).astype(np.float32)
    assert np.array_equal(oracle.dequant(oracle.Q8_0, raw, 3, 64).reshape(-1, 32), d * q)


def test_router_logits_close_to_float64_dot():
    rng = np.random.default_rng(3)
    for H in (256, 1024, 3584):
        x = rng.standard_normal((5, H)).astype(np.float16)
        w = (rng.standard_normal((7, H)) * 0.02).astype(np.float32)
        b = rng.standard_normal(7).astype(np.float32)
        got = oracle.router_logits(x, w, b)
        ref = x.astype(np.float64) @ w.astype(np.float64).T + b
        bound = H * 2.0**-23 * (np.abs(x.astype(np.float64)) @ np.abs(w.astype(np.float64)).T) + 1e-6
        assert np.all(np.abs(got - ref) <= bound)


def test_router_order_is_the_documented_tree():
    # One product of 1 in slot 0 and products of 2^-24 in slots 16, 32 and 48: rounding
    # depends on which partial sums meet first, so the result pins the pairing.
    H = 512  # 64 slots x one 8-chunk each
    x = np.zeros((1, H), dtype=np.float16)
    w = np.zeros((1, H), dtype=np.float32)
    vals = {0: 1.0, 32: 2.0**-24, 16: 2.0**-24, 48: 2.0**-24}
    for s, v in vals.items():
        x[0, 8 * s] = 1.0
        w[0, 8 * s] = v
    got = oracle.router_logits(x, w)[0, 0]
    # tree: (p0 + p32) + (p16 + p48) = 1 + 2^-23 (p0+p32 rounds to 1 by ties-to-even)
    assert got == np.float32(1.0) + np.float32(2.0**-23)
    # a left-to-right sum would give ((1 + 2^-24) + 2^-24) + 2^-24 = 1
    assert got != np.float32(1.0)


def _brute_topk(l, k):
    order = sorted(range(len(l)), key=lambda e: (-float(l[e]), e))
    return order[:k]


@pytest.mark.parametrize("E,K", [(8, 2), (16, 4), (128, 8), (5, 5)])
def test_topk_brute_force_and_ties(E, K):
    rng = np.random.default_rng(E * 100 + K)
    logits = rng.standard_normal((50, E)).astype(np.float32)
    logits[0, :] = 0.25  # all equal -> ids 0..K-1
    logits[1, ::2] = 3.0  # ties at the top
    logits[2] = np.round(logits[2])  # many ties
    idx, w = oracle.topk(logits, K, norm=True)
    for m in range(50):
        assert list(idx[m]) == _brute_topk(logits[m], K)
    assert list(idx[0]) == list(range(K))
    np.testing.assert_allclose(w.sum(axis=1), 1.0, rtol=1e-6)
    _, w2 = oracle.topk(logits, K, norm=False)
    p = np.exp(logits.astype(np.float64) - logits.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    np.testing.assert_allclose(w2, np.take_along_axis(p, idx, axis=1), rtol=1e-5)


@pytest.mark.parametrize("M,K,E", [(1, 1, 1), (1, 8, 128), (16, 2, 8), (333, 8, 128), (4096, 8, 128)])
def test_dispatch_is_stable_argsort(M, K, E):
    rng = np.random.default_rng(M)
    idx = np.stack([rng.permutation(E)[:K] for _ in range(M)]).astype(np.int32)
    offsets, perm, inv = oracle.dispatch(idx, E)
    flat = idx.reshape(-1)
    assert np.array_equal(perm, np.argsort(flat, kind="stable"))
    assert np.array_equal(offsets, np.concatenate([[0], np.cumsum(np.bincount(flat, minlength=E))]))
    assert offsets[-1] == M * K
    assert np.array_equal(perm[inv], np.arange(M * K))


def _tiny_layer(qtypes=(12, 12, 14), H=256, I=256, E=4, K=2):
    from pgmoe.synth import LayerSpec, SyntheticLayer

    spec = LayerSpec("t", H, E, K, I, qtypes)
    lay = SyntheticLayer(spec, seed=11, scale=0.01)
    return lay, oracle.OracleLayer.from_gguf(lay.gguf, lay.config)


def test_layer_one_hot_equals_dense_expert():
    lay, L = _tiny_layer()
    x = lay.draw_x(6)
    idx = np.array([[e % 4, (e + 1) % 4] for e in range(6)], dtype=np.int32)
    w = np.zeros((6, 2), dtype=np.float32)
    w[:, 0] = 1.0
    y = L.forward_tokens(x, idx, w)
    xf = x.astype(np.float64)
    for t in range(6):
        e = idx[t, 0]
        g = oracle.dequant(L.gate[0], L.gate[3], 4 * 256, 256)[e * 256:(e + 1) * 256].astype(np.float64)
        u = oracle.dequant(L.up[0], L.up[3], 4 * 256, 256)[e * 256:(e + 1) * 256].astype(np.float64)
        d = oracle.dequant(L.down[0], L.down[3], 4 * 256, 256)[e * 256:(e + 1) * 256].astype(np.float64)
        gv, uv = g @ xf[t], u @ xf[t]
        ref = d @ (gv / (1 + np.exp(-gv)) * uv)
        np.testing.assert_allclose(y[t], ref, rtol=1e-9, atol=1e-12)


def test_layer_zero_input_and_weight_linearity():
    lay, L = _tiny_layer()
    x = lay.draw_x(4)
    _, idx, w = L.route(x)
    assert np.all(L.forward_tokens(np.zeros_like(x), idx, w) == 0)
    y1 = L.forward_tokens(x, idx, w)
    y2 = L.forward_tokens(x, idx, 2 * w)
    np.testing.assert_allclose(y2, 2 * y1, rtol=1e-12)
    # a token subset gives the same rows as the full pass
    ys = L.forward_tokens(x, idx, w, tokens=[3, 1])
    np.testing.assert_allclose(ys, y1[[3, 1]], rtol=0, atol=0)


def test_gelu_tanh_matches_torch_and_kernel_identity():
    """or_gelu_tanh against torch's F.gelu(approximate="tanh") (the reference's CPU branch,
    quant_kernels.py:1471) in float64, and the identity the kernels evaluate,
    0.5 g (1 + tanh z) = g - g / (1 + e^(2z)), on the same points (large |g| included)."""
    import torch
    import torch.nn.functional as F
    g = np.concatenate([np.linspace(-12, 12, 241), [-80.0, -30.0, 0.0, 1e-6, 30.0, 80.0]])
    ours = np.array([oracle.gelu_tanh(v) for v in g])
    ref = F.gelu(torch.from_numpy(g), approximate="tanh").numpy()
    np.testing.assert_allclose(ours, ref, rtol=1e-12, atol=1e-15)
    z = 0.7978845608028654 * (g + 0.044715 * g ** 3)
    with np.errstate(over="ignore"):
        kern = g - g / (1.0 + np.exp(2.0 * z))
    np.testing.assert_allclose(kern, ref, rtol=1e-12, atol=1e-12)
    # a plausible slip (the exact erf GELU) is caught by the same check
    exact = F.gelu(torch.from_numpy(g)).numpy()
    assert not np.allclose(exact, ref, rtol=1e-6, atol=1e-9)


def test_fp16_expert_mode_values():
    """F16 expert tensors decode to their IEEE binary16 values (every bit pattern); F32 and
    BF16 ones are held as the fp16 rounding (to nearest even) of their exact fp32 values,
    as the reference's fp16 expert mode loads them (quant_kernels.py:1962-1964)."""
    allh = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    d = oracle.dequant(oracle.F16, allh.view(np.uint8), 256, 256).reshape(-1)
    ref = allh.view(np.float16).astype(np.float32)
    assert np.all(np.isnan(ref) | (d.view(np.uint32) == ref.view(np.uint32)))
    # BF16 (bit patterns of finite values) -> fp32 exactly (bits << 16) -> fp16 RNE
    b = np.arange(0, 65536, 13, dtype=np.uint32).astype(np.uint16)
    f32 = (b.astype(np.uint32) << 16).view(np.float32)
    fin = np.isfinite(f32)
    with np.errstate(over="ignore"):
        want = f32[fin].astype(np.float16).view(np.uint16)
    got = oracle.fp16_expert_bytes(oracle.BF16, b[fin].view(np.uint8)).view(np.uint16)
    assert np.array_equal(got, want)
    # F32: halfway cases round to even (1 + 2^-11 -> 1, 1 + 3 * 2^-11 -> 1 + 2^-9)
    x = np.float32([1 + 2.0 ** -11, 1 + 3 * 2.0 ** -11, -2.5, 65504.0])
    h = oracle.fp16_expert_bytes(oracle.F32, x.view(np.uint8)).view(np.float16)
    assert h.tolist() == [1.0, 1.0 + 2.0 ** -9, -2.5, 65504.0]
    assert np.array_equal(oracle.fp16_expert_bytes(oracle.F16, x.astype(np.float16).view(np.uint8)),
                          x.astype(np.float16).view(np.uint8))
