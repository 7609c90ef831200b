"""The oracle's restatement of the formats the reference re-quantises to W4 (Q2_K, Q3_K,
IQ4_NL, IQ4_XS, MXFP4; oracle/requant.py), pinned without gguf-py (not importable here):

* decoding: hand-built blocks whose every field is chosen (scales, codes, high bits,
  exponents) against the ggml block definitions' closed forms, so that a swapped nibble, a
  wrong shift, scale index or high-bit position, or a wrong sign or offset changes a value;
* the re-quantisation (quant_kernels.py:920-936): codes in 0..15, the group minimum on code
  0 and the maximum on code 15, every value within half a step (plus the fp16 rounding of
  the step and the minimum) of the Q4_1 value rebuilt from the bytes, zero-width groups,
  and round-half-to-even on quotients that land on .5 exactly;
* Q5_1 and the reference's W8 re-quantisation it takes (quant_kernels.py:1011-1025): nibble
  and fifth-bit positions, each weight within half a step of its group's fp16 scale, the
  largest on code +-127, flat and all-zero groups.
"""

import numpy as np
import pytest

from oracle.requant import (IQ4_NL, IQ4_XS, KVALUES_IQ4NL, KVALUES_MXFP4, MXFP4, Q2_K, Q3_K, REQUANT_BLOCK,
                            ggml_dequant, requant_w4)


def _f16b(v):
    return np.array([v], np.float16).view(np.uint8)


def test_iq4_nl_levels_and_nibbles():
    b = np.zeros(18, np.uint8)
    b[0:2] = _f16b(0.5)
    for j in range(16):
        b[2 + j] = j | ((15 - j) << 4)  # element j: level j, element j + 16: level 15 - j
    w = ggml_dequant(IQ4_NL, b, 1, 32)[0]
    assert np.array_equal(w[:16], 0.5 * KVALUES_IQ4NL)
    assert np.array_equal(w[16:], 0.5 * KVALUES_IQ4NL[::-1])
    assert w[0] == -63.5 and w[15] == 56.5  # kvalues_iq4nl[0] = -127, [15] = 113


@pytest.mark.parametrize("e,scale", [(128, 1.0), (127, 0.5), (130, 4.0), (2, 2.0 ** -126), (0, 2.0 ** -128)])
def test_mxfp4_exponent_and_levels(e, scale):
    b = np.zeros(17, np.uint8)
    b[0] = e
    for j in range(16):
        b[1 + j] = j | (j << 4)
    w = ggml_dequant(MXFP4, b, 1, 32)[0]
    ref = (np.float32(scale) * KVALUES_MXFP4).astype(np.float32)
    assert np.array_equal(w[:16], ref) and np.array_equal(w[16:], ref)
    # the E2M1 values at scale 2^(e - 127): 0, 0.5, 1, 1.5, 2, 3, 4, 6 and their negatives
    assert np.array_equal(KVALUES_MXFP4[:8] / 2, [0, 0.5, 1, 1.5, 2, 3, 4, 6])


def test_iq4_xs_subblock_scales():
    b = np.zeros(136, np.uint8)
    b[0:2] = _f16b(0.25)
    ls = [33 + ib for ib in range(8)]  # dl = d * (ls - 32) = 0.25 (ib + 1)
    sh = 0
    for ib in range(8):
        b[4 + ib // 2] |= (ls[ib] & 15) << (4 * (ib % 2))
        sh |= (ls[ib] >> 4) << (2 * ib)
    b[2], b[3] = sh & 255, sh >> 8
    rng = np.random.default_rng(0)
    codes = rng.integers(0, 16, size=(8, 32))
    for ib in range(8):
        for j in range(16):
            b[8 + 16 * ib + j] = codes[ib, j] | (codes[ib, j + 16] << 4)
    w = ggml_dequant(IQ4_XS, b, 1, 256)[0].reshape(8, 32)
    for ib in range(8):
        assert np.array_equal(w[ib], np.float32(0.25 * (ib + 1)) * KVALUES_IQ4NL[codes[ib]])
    # a negative sub-block scale: ls = 0 -> dl = -32 d
    b2 = b.copy()
    b2[4] &= 0xF0
    b2[2] &= 0xFC
    assert np.array_equal(ggml_dequant(IQ4_XS, b2, 1, 256)[0][:32], np.float32(-8.0) * KVALUES_IQ4NL[codes[0]])


def _q3k_block(d, scales16, codes, high):
    """A Q3_K block from its fields: 16 six-bit scales (packed as ggml packs them), the 2-bit
    codes [8][32] and high bits [8][32] of the eight 32-weight sub-groups."""
    b = np.zeros(110, np.uint8)
    s = np.asarray(scales16)
    for i in range(4):
        b[96 + i] = (s[i] & 15) | ((s[8 + i] & 15) << 4)
        b[100 + i] = (s[4 + i] & 15) | ((s[12 + i] & 15) << 4)
        b[104 + i] = (s[i] >> 4) | ((s[4 + i] >> 4) << 2) | ((s[8 + i] >> 4) << 4) | ((s[12 + i] >> 4) << 6)
    for sg in range(8):  # sub-group sg = (half n, shift j): codes in bits 2j of qs[32n + l], high bit 4n + j of hmask[l]
        n, j = sg // 4, sg % 4
        for l in range(32):
            b[32 + 32 * n + l] |= codes[sg][l] << (2 * j)
            b[l] |= high[sg][l] << (4 * n + j)
    b[108:110] = _f16b(d)
    return b


def test_q3_k_scales_codes_and_high_bits():
    rng = np.random.default_rng(1)
    scales16 = rng.integers(0, 64, size=16)
    codes = rng.integers(0, 4, size=(8, 32))
    high = rng.integers(0, 2, size=(8, 32))
    b = _q3k_block(0.5, scales16, codes, high)
    w = ggml_dequant(Q3_K, b, 1, 256)[0].reshape(8, 32)
    for sg in range(8):
        for l in range(32):
            sc = int(scales16[2 * sg + (l >= 16)]) - 32
            q = int(codes[sg][l]) - (0 if high[sg][l] else 4)
            assert w[sg, l] == np.float32(0.5 * sc * q), (sg, l)


def test_q2_k_scales_mins_and_codes():
    rng = np.random.default_rng(2)
    b = np.zeros(84, np.uint8)
    b[0:16] = rng.integers(0, 256, size=16)
    codes = rng.integers(0, 4, size=(8, 32))
    for sg in range(8):
        n, j = sg // 4, sg % 4
        for l in range(32):
            b[16 + 32 * n + l] |= codes[sg][l] << (2 * j)
    b[80:82] = _f16b(0.25)
    b[82:84] = _f16b(0.125)
    w = ggml_dequant(Q2_K, b, 1, 256)[0].reshape(8, 32)
    for sg in range(8):
        for l in range(32):
            sc = int(b[2 * sg + (l >= 16)])
            ref = np.float32(np.float32(0.25 * (sc & 15)) * codes[sg][l]) - np.float32(0.125 * (sc >> 4))
            assert w[sg, l] == np.float32(ref), (sg, l)


def _q41_values(raw, rows, cols):
    b = raw.reshape(rows, cols // 32, 20)
    d = b[..., 0:2].copy().view(np.float16).astype(np.float32)
    m = b[..., 2:4].copy().view(np.float16).astype(np.float32)
    q = np.concatenate([b[..., 4:20] & 15, b[..., 4:20] >> 4], axis=-1).astype(np.float32)
    return d * q + m, q, d[..., 0], m[..., 0]


@pytest.mark.parametrize("qtype", [Q2_K, Q3_K, IQ4_NL, IQ4_XS, MXFP4])
def test_requant_properties(qtype):
    from pgmoe.synth import random_blocks
    rows, cols = 16, 512
    raw = random_blocks(np.random.default_rng(qtype), qtype, rows, cols)
    w = ggml_dequant(qtype, raw, rows, cols).reshape(rows, cols // 32, 32)
    out = requant_w4(qtype, raw, rows, cols)
    assert out.size == rows * cols // 32 * 20
    rebuilt, q, d, m = _q41_values(out, rows, cols)
    mn, mx = w.min(-1), w.max(-1)
    step = (mx - mn) / 15
    assert np.array_equal(m, mn.astype(np.float16).astype(np.float32))
    assert np.array_equal(d, (((mx - mn) * np.float32(1 / 15)).astype(np.float32)).astype(np.float16).astype(np.float32))
    assert np.all(q[w == mn[..., None]] == 0)
    full = step > 0
    assert np.all(q[full][w[full] == mx[full][..., None]] == 15)
    slack = 0.5 * step + 16 * np.abs(d - step) + np.abs(m - mn) + 1e-6 * np.abs(mn)
    assert np.all(np.abs(rebuilt - w) <= slack[..., None])


def test_requant_flat_group_and_half_even():
    # IQ4_NL blocks with d = 1: one flat group (all 13), one on two levels only
    def block(levels):
        b = np.zeros(18, np.uint8)
        b[0:2] = _f16b(1.0)
        for j in range(16):
            b[2 + j] = levels[j] | (levels[j + 16] << 4)
        return b
    kv = list(KVALUES_IQ4NL)
    flat = block([kv.index(13)] * 32)
    out = requant_w4(IQ4_NL, flat, 1, 32)
    _, q, d, m = _q41_values(out, 1, 32)
    assert d[0, 0] == 0 and m[0, 0] == 13 and np.all(q == 0)
    # min -10 (level 7), max 1 (level 8): step = 11 / 15; w = 1 is code 15, -10 code 0
    lv = [7, 8] * 16
    out = requant_w4(IQ4_NL, block(lv), 1, 32)
    _, q, d, m = _q41_values(out, 1, 32)
    assert np.all(q[0, 0, 0::2] == 0) and np.all(q[0, 0, 1::2] == 15)
    # round half to even, on a Q3_K group whose quotients land on .5 exactly: d = 1, the first 16
    # weights at scale 39 - 32 = 7, the last 16 at 24 - 32 = -8; values -28 (7 * -4), 14 (7 * 2),
    # -14 (7 * -2), 32 (-8 * -4) and zeros, so min -28, max 32, scale 60 * fp32(1/15) = 4 and the
    # quotients 0, 10.5, 3.5, 15, 7: half-even gives codes 0, 10, 4, 15, 7 (half-up: 11 for 10.5)
    scales16 = [39, 24] + [32] * 14
    codes = np.zeros((8, 32), np.int64)
    high = np.ones((8, 32), np.int64)
    codes[0, 1], codes[0, 2] = 2, 2
    high[0, 0], high[0, 2], high[0, 16] = 0, 0, 0
    b = _q3k_block(1.0, scales16, codes, high)
    w = ggml_dequant(Q3_K, b, 1, 256)[0]
    assert list(w[[0, 1, 2, 3, 16, 17]]) == [-28, 14, -14, 0, 32, 0]
    out = requant_w4(Q3_K, b, 1, 256)
    _, q, d, m = _q41_values(out, 1, 256)
    assert d[0, 0] == 4 and m[0, 0] == -28
    assert list(q[0, 0, [0, 1, 2, 3, 16, 17]]) == [0, 10, 4, 7, 15, 7]
    assert np.all(d[0, 1:] == 0) and np.all(m[0, 1:] == 0) and np.all(q[0, 1:] == 0)  # flat zero groups


def test_block_table_matches_the_reference_parser():
    # pygguf_engine/gguf_parser.py:57-91: (weights, bytes) per block
    assert REQUANT_BLOCK == {10: (256, 84), 11: (256, 110), 20: (32, 18), 23: (256, 136), 39: (32, 17)}


def test_q5_1_nibbles_and_fifth_bits():
    from oracle.requant import q5_1_dequant
    b = np.zeros(24, np.uint8)
    b[0:2] = _f16b(0.5)
    b[2:4] = _f16b(-3.0)
    rng = np.random.default_rng(3)
    lo = rng.integers(0, 16, size=32)
    hi = rng.integers(0, 2, size=32)
    for j in range(16):
        b[8 + j] = lo[j] | (lo[j + 16] << 4)
    qh = sum(int(hi[e]) << e for e in range(32))
    b[4:8] = np.array([qh], "<u4").view(np.uint8)
    w = q5_1_dequant(b, 1, 32)[0]
    assert np.array_equal(w, (0.5 * (lo | (hi << 4)) - 3.0).astype(np.float32))
    # one fifth bit at a time lifts exactly its element by 16 d
    for e in (0, 15, 16, 31):
        b2 = b.copy()
        b2[4:8] = np.array([qh ^ (1 << e)], "<u4").view(np.uint8)
        diff = q5_1_dequant(b2, 1, 32)[0] - w
        assert np.count_nonzero(diff) == 1 and abs(diff[e]) == 8.0


def test_requant_w8_properties_and_exact_cases():
    from oracle.requant import Q5_1, q5_1_dequant, requant_w8_f16
    from pgmoe.synth import random_blocks
    rows, cols = 16, 512
    raw = random_blocks(np.random.default_rng(7), Q5_1, rows, cols)
    w = q5_1_dequant(raw, rows, cols).reshape(rows, cols // 16, 16)
    v = requant_w8_f16(Q5_1, raw, rows, cols).view(np.float16).astype(np.float32).reshape(rows, cols // 16, 16)
    amax = np.abs(w).max(-1)
    sc = amax / np.float32(127)
    # within half a step of the fp16 scale plus the fp16 rounding of scale and weight
    bound = 0.5 * sc + 127 * np.abs(sc.astype(np.float16).astype(np.float32) - sc) + 2.0 ** -11 * amax
    assert np.all(np.abs(v - w) <= bound[..., None])
    # the largest magnitude lands on code +-127: its weight is fp16(+-127 fp16(sc))
    i = np.abs(w).argmax(-1)
    top = np.take_along_axis(v, i[..., None], -1)[..., 0]
    s16 = sc.astype(np.float16).astype(np.float32)
    assert np.array_equal(np.abs(top), (127 * s16).astype(np.float16).astype(np.float32))
    # a flat group: d = 1/4, m = -3.875 and every code 31 give 3.875 everywhere, so every code is
    # +127 and every weight fp16(127 fp16(3.875 / 127)); an all-zero block gives +0 weights
    b = np.zeros(24 * 2, np.uint8).reshape(2, 24)
    b[0, 0:2] = _f16b(0.25)
    b[0, 2:4] = _f16b(-3.875)
    b[0, 4:24] = 0xFF
    out = requant_w8_f16(Q5_1, b[0], 1, 32).view(np.float16).astype(np.float32)
    assert np.array_equal(out, np.full(32, np.float16(127 * np.float16(np.float32(3.875) / np.float32(127))),
                                       np.float32))
    out0 = requant_w8_f16(Q5_1, b[1], 1, 32).view(np.uint16)
    assert np.all(out0 == 0)     # +0, not -0
