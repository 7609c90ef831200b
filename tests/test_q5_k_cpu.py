"""Q5_K (ggml type 13, the 5-bit K-quant of Q5_K_M files): the oracle's decoder pinned
without the reference running --

* with every fifth bit clear, a Q5_K block is the Q4_K block of the same header and qs
  (the Q4_K decoder is pinned by the reference's golden vectors);
* a block of small exact values against the closed form (d*sc_s) (q + 16 bit) - dmin*m_s,
  with the fifth bit of element 32s + l taken from bit s of qh[l] (one bit at a time, so a
  transposed or shifted bit index fails);
* the numpy restatement of the reference's Q5_K -> W8 repack (quant_kernels.py:984-1004)
  against the oracle with fp16 sub-block products (conv = 1);
* the C-ABI sizes of the device layout (11 chunks per row and super-block)."""

import numpy as np

import oracle
from oracle import torch_port
from pgmoe.synth import random_blocks

Q4_K, Q5_K = 12, 13


def q5k_header_qs_as_q4k(raw: np.ndarray) -> np.ndarray:
    b = raw.reshape(-1, 176)
    return np.concatenate([b[:, 0:16], b[:, 48:176]], axis=1).reshape(-1)


def test_q5_k_with_clear_fifth_bits_is_q4_k():
    rng = np.random.default_rng(3)
    raw = random_blocks(rng, Q5_K, 7, 512).reshape(-1, 176)
    raw[:, 16:48] = 0
    for conv in (0, 1):
        np.testing.assert_array_equal(oracle.dequant(Q5_K, raw, 7, 512, conv),
                                      oracle.dequant(Q4_K, q5k_header_qs_as_q4k(raw), 7, 512, conv))


def _block(d, dmin, sc, mn, qs, qh):
    """One Q5_K block from 6-bit scales/mins (ggml's 12-byte packing written out)."""
    b = np.zeros(176, dtype=np.uint8)
    b[0:2] = np.array([d], np.float16).view(np.uint8)
    b[2:4] = np.array([dmin], np.float16).view(np.uint8)
    for j in range(4):
        b[4 + j] = (sc[j] & 63) | ((sc[4 + j] >> 4) << 6)
        b[8 + j] = (mn[j] & 63) | ((mn[4 + j] >> 4) << 6)
        b[12 + j] = (sc[4 + j] & 15) | ((mn[4 + j] & 15) << 4)
    b[16:48] = qh
    b[48:176] = qs
    return b


def test_q5_k_closed_form_one_bit_at_a_time():
    rng = np.random.default_rng(9)
    sc = rng.integers(0, 64, 8)
    mn = rng.integers(0, 64, 8)
    qs = rng.integers(0, 256, 128).astype(np.uint8)
    d, dmin = 0.5, 0.125
    base_q = np.array([(qs[32 * (s // 2) + l] >> (4 * (s % 2))) & 15 for s in range(8) for l in range(32)])
    a = np.repeat(d * sc, 32).astype(np.float64)
    z = np.repeat(dmin * mn, 32).astype(np.float64)
    zero = oracle.dequant(Q5_K, _block(d, dmin, sc, mn, qs, np.zeros(32, np.uint8)), 1, 256)[0]
    np.testing.assert_array_equal(zero, (a * base_q - z).astype(np.float32))
    for s, l in ((0, 0), (1, 31), (2, 5), (5, 17), (7, 30), (6, 0)):
        qh = np.zeros(32, np.uint8)
        qh[l] = 1 << s
        v = oracle.dequant(Q5_K, _block(d, dmin, sc, mn, qs, qh), 1, 256)[0]
        q = base_q.copy()
        q[32 * s + l] += 16
        np.testing.assert_array_equal(v, (a * q - z).astype(np.float32))
        assert np.flatnonzero(v != zero).tolist() == ([32 * s + l] if sc[s] else [])


def test_q5_k_matches_the_reference_repack_restated():
    rng = np.random.default_rng(4)
    rows, cols = 6, 768
    raw = random_blocks(rng, Q5_K, rows, cols)
    port = torch_port.dense_weights((Q5_K, rows, cols, raw))
    np.testing.assert_array_equal(port, oracle.dequant(Q5_K, raw, rows, cols, 1))


def test_q5_k_sizes():
    from pgmoe._lib import lib
    L = lib()
    for rows, cols in ((64, 256), (100, 2048), (768, 2048)):
        ng, nb = (rows + 63) // 64, cols // 256
        assert L.pgmoe_weight_bytes(Q5_K, rows, cols) == ng * nb * 11 * 1024
        assert L.pgmoe_scale_plane_bytes(Q5_K, rows, cols) == L.pgmoe_scale_plane_bytes(Q4_K, rows, cols) > 0
    assert L.pgmoe_weight_bytes(Q5_K, 64, 100) < 0
