// Load-time W4 re-quantisation of the GGUF formats the reference reads through gguf-py
// (Q2_K, Q3_K, IQ4_NL, IQ4_XS, MXFP4; below it, the W8 one of Q5_1, quant_kernels.py:1005-1025,
// written as fp16 weights): each 32-weight group is decoded exactly in fp32 and
// quantised again to 4 bits as repack_gguf_to_w4a16 does (quant_kernels.py:906-942):
//   scale = (max - min) * fp32(1/15), q = clip(rint((w - min) / (scale or 1)), 0, 15),
//   stored as a Q4_1 block: d = fp16(scale), m = fp16(min) (the reference's zero is
//   fp16(-min), its value q * scale16 - zero16), codes q (element j in the low nibble of
//   byte j, element j + 16 in its high nibble).
// The result then takes the Q4_1 relayout and kernels.  Block definitions (ggml's
// dequantize_row_*, which gguf-py's dequantize mirrors): every decoded value is a product
// of an fp16 and small integers that fits fp32 exactly (Q2_K: less one rounded subtraction).
#include "common.h"
#include "launch.h"

namespace pgmoe {

// Every product and difference below is rounded on its own, as numpy's are (Q2_K's d sc q - dmin m
// fused into one FMA would round once and can move a group's scale by an fp16 ulp).  Plain
// operators under this pragma: header helpers such as __fmul_rn carry their own contraction
// setting into the inlined code.
#pragma clang fp contract(off)

__constant__ float kIq4nl[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};
__constant__ float kMxfp4[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};

template <int QT> struct GgmlBlock;
template <> struct GgmlBlock<PGMOE_Q2_K> { static constexpr int per = 256, bytes = 84; };
template <> struct GgmlBlock<PGMOE_Q3_K> { static constexpr int per = 256, bytes = 110; };
template <> struct GgmlBlock<PGMOE_IQ4_NL> { static constexpr int per = 32, bytes = 18; };
template <> struct GgmlBlock<PGMOE_IQ4_XS> { static constexpr int per = 256, bytes = 136; };
template <> struct GgmlBlock<PGMOE_MXFP4> { static constexpr int per = 32, bytes = 17; };

__device__ __forceinline__ float f16_at(const uint8_t* p) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(p[0] | (p[1] << 8)));
}
__device__ __forceinline__ uint32_t u32_at(const uint8_t* p) {
    return p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

// The 32 values of sub-group s (weights 32 s .. 32 s + 31) of the GGUF block at b.
template <int QT>
__device__ void decode32(const uint8_t* b, int s, float (&w)[32]) {
    if constexpr (QT == PGMOE_IQ4_NL || QT == PGMOE_MXFP4) {
        // {fp16 d; u8 qs[16]} / {u8 e; u8 qs[16]}: scale * kvalues[code]
        const float sc = QT == PGMOE_IQ4_NL ? f16_at(b) : __builtin_ldexpf(1.0f, (int)b[0] - 128);
        const uint8_t* qs = b + (QT == PGMOE_IQ4_NL ? 2 : 1);
        const float* kv = QT == PGMOE_IQ4_NL ? kIq4nl : kMxfp4;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            w[j] = sc * kv[qs[j] & 15];
            w[j + 16] = sc * kv[qs[j] >> 4];
        }
    } else if constexpr (QT == PGMOE_IQ4_XS) {
        // {fp16 d; u16 scales_h; u8 scales_l[4]; u8 qs[128]}: d (ls - 32) kvalues[code]
        const float d = f16_at(b);
        const uint32_t sh = b[2] | ((uint32_t)b[3] << 8);
        const int ls = ((b[4 + s / 2] >> (4 * (s % 2))) & 15) | (((sh >> (2 * s)) & 3) << 4);
        const float dl = d * (float)(ls - 32);
        const uint8_t* qs = b + 8 + 16 * s;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            w[j] = dl * kIq4nl[qs[j] & 15];
            w[j + 16] = dl * kIq4nl[qs[j] >> 4];
        }
    } else if constexpr (QT == PGMOE_Q3_K) {
        // {u8 hmask[32]; u8 qs[64]; u8 scales[12]; fp16 d}: d (sc - 32) (q - 4 [high bit clear]);
        // sub-group s = (half n, shift j): codes bits 2j of qs[32 n + l], high bit 4n + j of hmask[l]
        const float d = f16_at(b + 108);
        const uint32_t a0 = u32_at(b + 96), a1 = u32_at(b + 100), tmp = u32_at(b + 104);
        const uint32_t k1 = 0x03030303u, k2 = 0x0f0f0f0fu;
        const uint32_t aux[4] = {(a0 & k2) | (((tmp >> 0) & k1) << 4), (a1 & k2) | (((tmp >> 2) & k1) << 4),
                                 ((a0 >> 4) & k2) | (((tmp >> 4) & k1) << 4),
                                 ((a1 >> 4) & k2) | (((tmp >> 6) & k1) << 4)};
        const int n = s >> 2, j = s & 3;
        const int i0 = 2 * s, i1 = 2 * s + 1;  // the sub-group's two 16-weight scales
        const int sc0 = (int)((aux[i0 >> 2] >> (8 * (i0 & 3))) & 0xff) - 32;
        const int sc1 = (int)((aux[i1 >> 2] >> (8 * (i1 & 3))) & 0xff) - 32;
        const float dl0 = d * (float)sc0, dl1 = d * (float)sc1;
        const uint8_t* hm = b;
        const uint8_t* qs = b + 32 + 32 * n;
#pragma unroll
        for (int l = 0; l < 32; ++l) {
            const int q = ((qs[l] >> (2 * j)) & 3) - (((hm[l] >> (4 * n + j)) & 1) ? 0 : 4);
            w[l] = (l < 16 ? dl0 : dl1) * (float)q;
        }
    } else {
        static_assert(QT == PGMOE_Q2_K, "format");
        // {u8 scales[16]; u8 qs[64]; fp16 d; fp16 dmin}: d (sc & 15) q - dmin (sc >> 4)
        const float d = f16_at(b + 80), dmin = f16_at(b + 82);
        const int n = s >> 2, j = s & 3;
        const uint8_t* qs = b + 16 + 32 * n;
#pragma unroll
        for (int l = 0; l < 32; ++l) {
            const uint8_t sc = b[2 * s + (l >> 4)];
            const float dl = d * (float)(sc & 15), ml = dmin * (float)(sc >> 4);
            w[l] = dl * (float)((qs[l] >> (2 * j)) & 3) - ml;
        }
    }
}

// One thread per 32-weight group (row, g) of a [rows, cols] matrix -> one Q4_1 block.
template <int QT>
__global__ void requant_w4_kernel(const uint8_t* __restrict__ src, int64_t rows, int cols,
                                  uint8_t* __restrict__ dst) {
    const int gpr = cols / 32;
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= rows * gpr) return;
    const int64_t row = gid / gpr;
    const int g = (int)(gid - row * gpr);
    using B = GgmlBlock<QT>;
    constexpr int SUB = B::per / 32;  // 32-weight groups of a block
    const uint8_t* blk = src + (row * (cols / B::per) + g / SUB) * B::bytes;
    float w[32];
    decode32<QT>(blk, g % SUB, w);
    float mn = w[0], mx = w[0];
#pragma unroll
    for (int i = 1; i < 32; ++i) {
        mn = fminf(mn, w[i]);
        mx = fmaxf(mx, w[i]);
    }
    float scale = (mx - mn) * (1.0f / 15.0f);
    // Rounded to fp32 first, then to fp16, as numpy does: without this the product and its fp16
    // conversion merge into one mixed-precision FMA that rounds once (different on fp16 ties).
    asm volatile("" : "+v"(scale));
    const float safe = scale == 0.0f ? 1.0f : scale;
    uint32_t qw[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const float ql = fminf(fmaxf(rintf((w[j] - mn) / safe), 0.0f), 15.0f);
        const float qh = fminf(fmaxf(rintf((w[j + 16] - mn) / safe), 0.0f), 15.0f);
        qw[j >> 2] |= ((uint32_t)ql | ((uint32_t)qh << 4)) << (8 * (j & 3));
    }
    uint32_t* o = reinterpret_cast<uint32_t*>(dst + gid * 20);
    // m = fp16(min) with a zero minimum stored as +0 (which of +0 / -0 a min reduction keeps
    // depends on its order; the value d q + m does not)
    o[0] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)scale) |
           ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(mn + 0.0f)) << 16);
    o[1] = qw[0];
    o[2] = qw[1];
    o[3] = qw[2];
    o[4] = qw[3];
}

// Q5_1 {fp16 d; fp16 m; u32 qh; u8 qs[16]}: d q + m with q = nibble | fifth bit << 4
// (element j: low nibble of qs[j] and bit j of qh; element j + 16: high nibble, bit j + 16).
__device__ void decode_q5_1(const uint8_t* b, float (&w)[32]) {
    const float d = f16_at(b), m = f16_at(b + 2);
    const uint32_t qh = u32_at(b + 4);
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        w[j] = d * (float)((b[8 + j] & 15) | (((qh >> j) & 1) << 4)) + m;
        w[j + 16] = d * (float)((b[8 + j] >> 4) | (((qh >> (j + 16)) & 1) << 4)) + m;
    }
}

// One thread per 32-weight block (row, g) of the fp16 [rows, cols_out] output: the
// reference's W8 values of Q5_1 block g (two 16-weight groups: sc = max|w| / 127, or 1 when
// the group is all zero; q = clip(rint(w / sc), -127, 127); fp16(sc) q rounded to fp16, the
// product being exact in fp32), or zeros for g past the source's cols.
__global__ void requant_w8_f16_kernel(const uint8_t* __restrict__ src, int64_t rows, int cols, int cols_out,
                                      uint8_t* __restrict__ dst) {
    const int gpo = cols_out / 32, gpr = cols / 32;
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= rows * gpo) return;
    const int64_t row = gid / gpo;
    const int g = (int)(gid - row * gpo);
    uint32_t h[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) h[i] = 0u;
    if (g < gpr) {
        float w[32];
        decode_q5_1(src + (row * gpr + g) * 24, w);
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            float amax = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(w[16 * half + i]));
            float sc = amax == 0.0f ? 1.0f : amax / 127.0f;
            asm volatile("" : "+v"(sc));  // sc itself in fp32, then its fp16 rounding
            const float s16 = (float)(_Float16)sc;
#pragma unroll
            for (int i = 0; i < 16; i += 2) {  // codes through int, as the reference stores int8 (no -0)
                const float q0 = (float)(int)fminf(fmaxf(rintf(w[16 * half + i] / sc), -127.0f), 127.0f);
                const float q1 = (float)(int)fminf(fmaxf(rintf(w[16 * half + i + 1] / sc), -127.0f), 127.0f);
                // the fp32 products themselves (exact): a mixed FMA with a +0 addend would turn the
                // -0 of fp16(sc) = 0 times a negative code into +0
                float v0 = s16 * q0, v1 = s16 * q1;
                asm volatile("" : "+v"(v0), "+v"(v1));
                h[8 * half + i / 2] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v0) |
                                      ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v1) << 16);
            }
        }
    }
    uint4* o = reinterpret_cast<uint4*>(dst + (row * cols_out + 32 * (int64_t)g) * 2);
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = make_uint4(h[4 * i], h[4 * i + 1], h[4 * i + 2], h[4 * i + 3]);
}

int launch_requant_w8_f16(int qtype, const uint8_t* src, int64_t rows, int cols, int cols_out, uint8_t* dst,
                          hipStream_t st) {
    if (qtype != PGMOE_Q5_1) return fail(PGMOE_E_UNSUPPORTED, "requant w8: qtype %d", qtype);
    const int64_t n = rows * (cols_out / 32);
    if (n == 0) return PGMOE_OK;
    const int threads = 256;
    PG_LAUNCH(requant_w8_f16_kernel, dim3((unsigned)div_up(n, threads)), dim3(threads), 0, st, src, rows, cols,
              cols_out, dst);
    return check_launch("requant_w8_f16");
}

int requant_w4_block(int qtype, int* per, int* bytes) {
    switch (qtype) {
    case PGMOE_Q2_K: *per = 256; *bytes = 84; return 0;
    case PGMOE_Q3_K: *per = 256; *bytes = 110; return 0;
    case PGMOE_IQ4_NL: *per = 32; *bytes = 18; return 0;
    case PGMOE_IQ4_XS: *per = 256; *bytes = 136; return 0;
    case PGMOE_MXFP4: *per = 32; *bytes = 17; return 0;
    }
    return -1;
}

int launch_requant_w4(int qtype, const uint8_t* src, int64_t rows, int cols, uint8_t* dst, hipStream_t st) {
    const int64_t n = rows * (cols / 32);
    if (n == 0) return PGMOE_OK;
    const int threads = 256;
    const dim3 grid((unsigned)div_up(n, threads));
    switch (qtype) {
    case PGMOE_Q2_K: PG_LAUNCH(requant_w4_kernel<PGMOE_Q2_K>, grid, dim3(threads), 0, st, src, rows, cols, dst); break;
    case PGMOE_Q3_K: PG_LAUNCH(requant_w4_kernel<PGMOE_Q3_K>, grid, dim3(threads), 0, st, src, rows, cols, dst); break;
    case PGMOE_IQ4_NL: PG_LAUNCH(requant_w4_kernel<PGMOE_IQ4_NL>, grid, dim3(threads), 0, st, src, rows, cols, dst); break;
    case PGMOE_IQ4_XS: PG_LAUNCH(requant_w4_kernel<PGMOE_IQ4_XS>, grid, dim3(threads), 0, st, src, rows, cols, dst); break;
    case PGMOE_MXFP4: PG_LAUNCH(requant_w4_kernel<PGMOE_MXFP4>, grid, dim3(threads), 0, st, src, rows, cols, dst); break;
    default: return fail(PGMOE_E_UNSUPPORTED, "requant: qtype %d", qtype);
    }
    return check_launch("requant_w4");
}

}  // namespace pgmoe
