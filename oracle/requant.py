"""The reference's W4 re-quantisation of the GGUF formats it reads through gguf-py -- TEST
INFRASTRUCTURE ONLY (imported by ``oracle``; the product never imports it).

For Q2_K, Q3_K, IQ4_NL, IQ4_XS and MXFP4 (members of SUB_5BIT_W4_QTYPES,
quant_kernels.py:28-49, taken by the W4 branch at :1966-1967 and :1812) the reference does
not keep the GGUF values: ``repack_gguf_to_w4a16`` (quant_kernels.py:906-942) decodes each
block with ``gguf.quants.dequantize`` and quantises every 32 weights again to 4 bits,
asymmetric, with an fp16 scale and zero:

    w_min, w_max = min, max of the 32 fp32 values
    scale = (w_max - w_min) * (1 / 15)                      (fp32)
    q     = clip(round((w - w_min) / (scale or 1)), 0, 15)  (fp32 ops, round half to even)
    stored: q, fp16(scale), fp16(-w_min); the W4 value is q * scale16 - zero16

which is exactly a Q4_1 block (d = fp16(scale), m = fp16(w_min) = -fp16(-w_min), codes q,
element j in the low nibble of byte j and element j + 16 in its high nibble).  A zero minimum
is stored as +0: numpy's min may keep either zero (it depends on the reduction order), and the
values d q + m are the same for both.
``requant_w4`` restates that on the decoded values; ``ggml_dequant`` restates the decoding.

Q5_1 takes the reference's W8 fallback instead (quant_kernels.py:1005-1025: per 16 weights,
symmetric int8 at max|w| / 127, fp16 scales); ``requant_w8_f16`` restates it as the fp16
weights fp16(scale16 * code) that its tensor-core GEMM forms, which this build stores.

gguf-py (llama.cpp's ``gguf`` package; the reference pins no version and it is not
importable here) decodes these blocks as ggml's ``dequantize_row_*`` (ggml-quants.c) do.
Its published block definitions, restated per format below, give every value exactly in
fp32 (each is a product of an fp16 and small integers that fits 24 bits, less one exactly
rounded subtraction for Q2_K), so any correct decoding gives the same bits.  The byte
positions of the fp16 scale agree with the reference's own fixtures, which write it to
bytes 0-1 of IQ4_XS / IQ4_NL blocks and to the last two bytes of Q3_K blocks
(tests/test_pygguf_engine.py:367-378).  What pins the restatement: the closed forms and
bit-layout cases of tests/test_requant_cpu.py; no gguf-py output exists here to compare
with, so the decoding itself is "parity unpinned" against gguf-py.
"""

from __future__ import annotations

import numpy as np

Q2_K, Q3_K, IQ4_NL, IQ4_XS, MXFP4 = 10, 11, 20, 23, 39
# (weights, bytes) of one GGUF block
REQUANT_BLOCK = {Q2_K: (256, 84), Q3_K: (256, 110), IQ4_NL: (32, 18), IQ4_XS: (256, 136), MXFP4: (32, 17)}

# ggml's kvalues_iq4nl: the 16 non-linear levels of IQ4_NL / IQ4_XS
KVALUES_IQ4NL = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], np.float32)
# ggml's kvalues_mxfp4: twice the E2M1 values (the block scale is 2^(e - 128), half of 2^(e - 127))
KVALUES_MXFP4 = np.array([0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12], np.float32)


def _f16(b: np.ndarray) -> np.ndarray:
    """fp16 fields (two little-endian bytes, last axis) -> fp32."""
    return np.ascontiguousarray(b).view(np.float16).astype(np.float32)[..., 0]


def _nibbles32(qs: np.ndarray) -> np.ndarray:
    """[..., 16] bytes -> [..., 32] codes: element j the low nibble of byte j, element j + 16
    its high nibble (the Q4_0 / IQ4_NL / MXFP4 arrangement)."""
    return np.concatenate([qs & 15, qs >> 4], axis=-1)


def ggml_dequant(qtype: int, raw: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """fp32 [rows, cols] values of a GGUF matrix in one of the formats above."""
    per, nbytes = REQUANT_BLOCK[qtype]
    if cols % per:
        raise ValueError(f"{cols} columns are not whole {per}-weight blocks")
    b = np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1, nbytes)
    nb = b.shape[0]
    if qtype == IQ4_NL:  # block_iq4_nl {fp16 d; u8 qs[16]}: d * kvalues[code]
        d = _f16(b[:, 0:2].reshape(nb, 1, 2))
        y = d * KVALUES_IQ4NL[_nibbles32(b[:, 2:18])]
    elif qtype == MXFP4:  # block_mxfp4 {u8 e; u8 qs[16]}: 2^(e - 128) * kvalues[code]
        scale = np.ldexp(np.float32(1.0), b[:, 0].astype(np.int32) - 128).astype(np.float32).reshape(nb, 1)
        y = scale * KVALUES_MXFP4[_nibbles32(b[:, 1:17])]
    elif qtype == IQ4_XS:  # {fp16 d; u16 scales_h; u8 scales_l[4]; u8 qs[128]}
        d = _f16(b[:, 0:2].reshape(nb, 1, 2))
        sh = b[:, 2].astype(np.uint32) | (b[:, 3].astype(np.uint32) << 8)
        ib = np.arange(8)
        lo = (b[:, 4 + ib // 2] >> (4 * (ib % 2))) & 15                      # [nb, 8]
        hi = (sh[:, None] >> (2 * ib)) & 3
        ls = (lo.astype(np.int32) | (hi.astype(np.int32) << 4)) - 32          # sub-block scales
        dl = d * ls.astype(np.float32)                                       # [nb, 8]
        codes = _nibbles32(b[:, 8:136].reshape(nb, 8, 16))                   # [nb, 8, 32]
        y = dl[:, :, None] * KVALUES_IQ4NL[codes]
    elif qtype == Q3_K:  # {u8 hmask[32]; u8 qs[64]; u8 scales[12]; fp16 d}
        d = _f16(b[:, 108:110].reshape(nb, 1, 2))
        aux = np.ascontiguousarray(b[:, 96:108]).view("<u4").astype(np.uint32)  # [nb, 3]
        a0, a1, tmp = aux[:, 0], aux[:, 1], aux[:, 2]
        k1, k2 = np.uint32(0x03030303), np.uint32(0x0F0F0F0F)
        s = np.stack([(a0 & k2) | (((tmp >> 0) & k1) << 4), (a1 & k2) | (((tmp >> 2) & k1) << 4),
                      ((a0 >> 4) & k2) | (((tmp >> 4) & k1) << 4), ((a1 >> 4) & k2) | (((tmp >> 6) & k1) << 4)],
                     axis=1).astype("<u4")
        sc = np.ascontiguousarray(s).view(np.uint8).reshape(nb, 16).astype(np.int32) - 32  # 16 scales
        hm, qs = b[:, 0:32], b[:, 32:96]
        y = np.empty((nb, 256), np.float32)
        for s_ in range(8):  # 32-weight sub-block s_ = (half n, shift j)
            n, j = s_ // 4, s_ % 4
            q = ((qs[:, 32 * n:32 * n + 32] >> (2 * j)) & 3).astype(np.int32)
            high = (hm[:, 0:32] >> (4 * n + j)) & 1
            v = q - 4 * (1 - high.astype(np.int32))
            dl = d * np.stack([sc[:, 2 * s_], sc[:, 2 * s_ + 1]], axis=1).astype(np.float32)  # [nb, 2]
            y[:, 32 * s_:32 * s_ + 32] = np.repeat(dl, 16, axis=1) * v.astype(np.float32)
    elif qtype == Q2_K:  # {u8 scales[16]; u8 qs[64]; fp16 d; fp16 dmin}
        d = _f16(b[:, 80:82].reshape(nb, 1, 2))
        dmin = _f16(b[:, 82:84].reshape(nb, 1, 2))
        sc, qs = b[:, 0:16], b[:, 16:80]
        y = np.empty((nb, 256), np.float32)
        for s_ in range(8):
            n, j = s_ // 4, s_ % 4
            q = ((qs[:, 32 * n:32 * n + 32] >> (2 * j)) & 3).astype(np.float32)
            bt = np.repeat(np.stack([sc[:, 2 * s_], sc[:, 2 * s_ + 1]], axis=1), 16, axis=1)
            dl = d * (bt & 15).astype(np.float32)
            ml = dmin * (bt >> 4).astype(np.float32)
            y[:, 32 * s_:32 * s_ + 32] = dl * q - ml
    else:
        raise ValueError(f"qtype {qtype} is not re-quantised")
    return np.asarray(y, np.float32).reshape(rows, cols)


Q5_1 = 7
W8_BLOCK = {Q5_1: (32, 24)}


def q5_1_dequant(raw: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """fp32 [rows, cols] of Q5_1 blocks {fp16 d; fp16 m; u32 qh; u8 qs[16]}: d q + m with
    q = nibble | fifth bit << 4; element j: low nibble of qs[j], bit j of qh; element j + 16:
    high nibble of qs[j], bit j + 16 (ggml's dequantize_row_q5_1); product and sum rounded
    separately in fp32."""
    if cols % 32:
        raise ValueError(f"{cols} columns are not whole 32-weight blocks")
    b = np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1, 24)
    nb = b.shape[0]
    d = _f16(b[:, 0:2].reshape(nb, 1, 2))
    m = _f16(b[:, 2:4].reshape(nb, 1, 2))
    qh = np.ascontiguousarray(b[:, 4:8]).view("<u4").astype(np.uint32)          # [nb, 1]
    hi = ((qh >> np.arange(32, dtype=np.uint32)) & 1).astype(np.uint8)          # [nb, 32]
    q = (_nibbles32(b[:, 8:24]) | (hi << 4)).astype(np.float32)
    return (d * q + m).astype(np.float32).reshape(rows, cols)


def requant_w8_f16(qtype: int, raw: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """The fp16 weights (bytes of [rows, cols]) of the reference's W8 re-quantisation of a Q5_1
    matrix (repack_gguf_to_w8a16's fallback, quant_kernels.py:1011-1025): per 16 weights
    sc = max|w| / 127 (1 for an all-zero group), int8 codes clip(round(w / sc), -127, 127),
    the fp16 scale fp16(sc); each weight fp16(fp16(sc) * code), the operand its tensor-core
    GEMM forms (``(q_grp * s).to(tl.float16)``, quant_kernels.py:553-620)."""
    if qtype != Q5_1:
        raise ValueError(f"qtype {qtype} is not re-quantised to W8")
    g = q5_1_dequant(raw, rows, cols).reshape(rows, cols // 16, 16)
    amax = np.max(np.abs(g), axis=-1, keepdims=True)
    sc = np.where(amax == np.float32(0.0), np.float32(1.0), amax / np.float32(127.0)).astype(np.float32)
    q = np.clip(np.round(g / sc), -127, 127).astype(np.int8)
    s16 = sc.astype(np.float16).astype(np.float32)
    return (q.astype(np.float32) * s16).astype(np.float16).view(np.uint8).reshape(-1)


def requant_w4(qtype: int, raw: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """The Q4_1 GGUF bytes (rows x cols / 32 blocks of 20 bytes) of the reference's W4
    re-quantisation (quant_kernels.py:920-936) of a matrix in one of the formats above."""
    w = ggml_dequant(qtype, raw, rows, cols).reshape(rows, cols // 32, 32)
    w_min = np.min(w, axis=-1, keepdims=True)
    w_max = np.max(w, axis=-1, keepdims=True)
    scale = (w_max - w_min) * np.float32(1.0 / 15.0)
    scale_safe = np.where(scale == np.float32(0.0), np.float32(1.0), scale).astype(np.float32)
    q = np.clip(np.round((w - w_min) / scale_safe), 0, 15).astype(np.uint8)
    out = np.empty((rows, cols // 32, 20), np.uint8)
    out[..., 0:2] = scale.astype(np.float16).view(np.uint8).reshape(rows, cols // 32, 2)
    # a zero minimum as +0: which zero a min reduction keeps depends on its order, the value does not
    out[..., 2:4] = (w_min + np.float32(0.0)).astype(np.float16).view(np.uint8).reshape(rows, cols // 32, 2)
    out[..., 4:20] = q[..., :16] | (q[..., 16:] << 4)
    return out.reshape(-1)
