"""Q4_0 experts (the format of the reference's synthetic qwen35moe test model,
tests/test_pygguf_engine.py:424-440) and Q4_1 / Q5_0: the oracle's decoders pinned by
reduction to the golden-pinned Q8_0 decoder (Q4_0, Q5_0) and to Q4_0 (Q4_1 with m = -8d),
closed forms on exact values, the restated W4 repack of the reference, and the C-ABI sizes
(Q4_0 is stored as Q4_1, Q5_0 as Q8_0)."""

import numpy as np

import oracle
from pgmoe.synth import random_blocks

Q4_0, Q4_1, Q8_0 = 2, 3, 8


def q4_0_as_q8_0(raw: np.ndarray) -> np.ndarray:
    """Q4_0 blocks -> the Q8_0 blocks of the same values: same d, qs = nibble - 8 (weight l
    from the low nibble of byte l, weight 16 + l from its high nibble)."""
    b = raw.reshape(-1, 18)
    out = np.empty((b.shape[0], 34), dtype=np.uint8)
    out[:, 0:2] = b[:, 0:2]
    q = b[:, 2:18]
    out[:, 2:18] = ((q & 15).astype(np.int16) - 8).astype(np.int8).view(np.uint8)
    out[:, 18:34] = ((q >> 4).astype(np.int16) - 8).astype(np.int8).view(np.uint8)
    return out.reshape(-1)


def test_q4_0_decoder_equals_q8_0_of_the_same_values():
    rng = np.random.default_rng(5)
    raw = random_blocks(rng, Q4_0, 6, 256)
    a = oracle.dequant(Q4_0, raw, 6, 256)
    b = oracle.dequant(Q8_0, q4_0_as_q8_0(raw), 6, 256)
    np.testing.assert_array_equal(a, b)
    # closed form on one block: d * (q - 8), low nibbles first
    blk = np.zeros(18, dtype=np.uint8)
    blk[0:2] = np.array([0.5], dtype=np.float16).view(np.uint8)
    blk[2:18] = np.arange(16, dtype=np.uint8) | (np.uint8(15) << 4)
    v = oracle.dequant(Q4_0, blk, 1, 32)
    np.testing.assert_array_equal(v[0, :16], 0.5 * (np.arange(16) - 8))
    np.testing.assert_array_equal(v[0, 16:], np.full(16, 0.5 * 7))


def q4_0_as_q4_1(raw: np.ndarray) -> np.ndarray:
    """Q4_0 blocks -> the Q4_1 blocks of the same values: same d and codes, m = -8d."""
    b = raw.reshape(-1, 18)
    out = np.empty((b.shape[0], 20), dtype=np.uint8)
    out[:, 0:2] = b[:, 0:2]
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32)
    out[:, 2:4] = (-8.0 * d).astype(np.float16).view(np.uint8)
    out[:, 4:20] = b[:, 2:18]
    return out.reshape(-1)


def test_q4_1_decoder():
    rng = np.random.default_rng(8)
    raw = random_blocks(rng, Q4_0, 5, 512)
    np.testing.assert_array_equal(oracle.dequant(Q4_1, q4_0_as_q4_1(raw), 5, 512), oracle.dequant(Q4_0, raw, 5, 512))
    # closed form: d q + m, weight l from the low nibble of byte l, 16 + l from the high one
    blk = np.zeros(20, dtype=np.uint8)
    blk[0:2] = np.array([0.5], dtype=np.float16).view(np.uint8)
    blk[2:4] = np.array([-1.25], dtype=np.float16).view(np.uint8)
    blk[4:20] = np.arange(16, dtype=np.uint8) | (np.uint8(3) << 4)
    v = oracle.dequant(Q4_1, blk, 1, 32)[0]
    np.testing.assert_array_equal(v[:16], 0.5 * np.arange(16) - 1.25)
    np.testing.assert_array_equal(v[16:], np.full(16, 0.5 * 3 - 1.25))


def test_q4_1_and_q4_0_match_the_reference_w4_repack_restated():
    from oracle import torch_port
    rng = np.random.default_rng(9)
    for qt in (Q4_0, Q4_1):
        raw = random_blocks(rng, qt, 6, 512)
        np.testing.assert_array_equal(torch_port.dense_weights((qt, 6, 512, raw)), oracle.dequant(qt, raw, 6, 512))


def test_q4_0_sizes_are_q4_1_sizes():
    from pgmoe._lib import lib
    L = lib()
    for rows, cols in ((64, 256), (100, 2048), (768, 2048)):
        ng, nb = (rows + 63) // 64, cols // 256
        assert L.pgmoe_weight_bytes(Q4_0, rows, cols) == L.pgmoe_weight_bytes(Q4_1, rows, cols) == ng * nb * 10 * 1024
        assert L.pgmoe_scale_plane_bytes(Q4_1, rows, cols) == ng * nb * 4 * 1024
        assert L.pgmoe_scale_plane_bytes(Q4_0, rows, cols) == -1  # a source format only
        assert L.pgmoe_scale_plane_bytes(Q8_0, rows, cols) == 0


Q5_0 = 6


def q5_0_as_q8_0(raw: np.ndarray) -> np.ndarray:
    """Q5_0 blocks -> the Q8_0 blocks of the same values: same d, qs = q - 16 with q the
    nibble plus bit l (bit 16 + l for the high nibbles) of the little-endian qh word."""
    b = raw.reshape(-1, 22)
    out = np.empty((b.shape[0], 34), dtype=np.uint8)
    out[:, 0:2] = b[:, 0:2]
    qh = b[:, 2:6].copy().view("<u4").reshape(-1, 1).astype(np.int64)
    q = b[:, 6:22].astype(np.int64)
    l = np.arange(16)
    lo = (q & 15) | (((qh >> l) & 1) << 4)
    hi = (q >> 4) | (((qh >> (16 + l)) & 1) << 4)
    out[:, 2:18] = (lo - 16).astype(np.int8).view(np.uint8)
    out[:, 18:34] = (hi - 16).astype(np.int8).view(np.uint8)
    return out.reshape(-1)


def test_q5_0_decoder_equals_q8_0_of_the_same_values():
    rng = np.random.default_rng(6)
    raw = random_blocks(rng, Q5_0, 5, 512)
    np.testing.assert_array_equal(oracle.dequant(Q5_0, raw, 5, 512), oracle.dequant(Q8_0, q5_0_as_q8_0(raw), 5, 512))
    # closed form: qh bit l lifts weight l by 16, bit 16 + l weight 16 + l
    blk = np.zeros(22, dtype=np.uint8)
    blk[0:2] = np.array([0.25], dtype=np.float16).view(np.uint8)
    blk[2:6] = np.array([0x0001_8000 | 1], dtype="<u4").view(np.uint8)  # bits 0, 15, 16
    blk[6:22] = 3 | (5 << 4)
    v = oracle.dequant(Q5_0, blk, 1, 32)[0]
    expect = np.array([3 - 16 + (16 if l in (0, 15) else 0) for l in range(16)] +
                      [5 - 16 + (16 if l == 0 else 0) for l in range(16)], dtype=np.float32) * 0.25
    np.testing.assert_array_equal(v, expect)
