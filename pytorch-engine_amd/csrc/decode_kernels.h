// Decode path (M <= 8 tokens), three launches per layer (five with a shared expert), no
// host sync:
//   router logits (router.hip, fixed order, also the 16-element sums of x) ->
//   gate/up + SwiGLU, each block routing the tokens itself from the logits ->
//   down + combine fused (every block owns a few output rows across all active experts).
// Work is spread one quarter super-block (64 weights) per lane: a layer's active weights
// cover ~200K lanes, every lane has its 3-5 weight loads in flight at once, and the
// activations (every token row, staged in LDS before the block knows its expert) are
// read as wave-uniform broadcasts.  The 64-row tile layout keeps each load instruction
// on whole 128-byte lines.
//   gate/up: fp16 magic-number dequant (1024 + code) feeding v_dot2_f32_f16
//   down   : fp32 FMA on the fp32 SwiGLU output
// The per-expert down kernel (stage API, shared expert, many pairs) streams whole
// super-blocks per lane.
// Reference: pygguf_engine/model.py:898-937; quant_kernels.py:68-311 (GEMV kernels it
// replaces), :1423-1475 (SwiGLU + row-scale).
#pragma once
#include <utility>

#include "common.h"
#include "launch.h"

namespace pgmoe {

constexpr int kDecTM = 8;  // token rows per expert chunk

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, a), __builtin_bit_cast(half2_t, b), c, false);
}

// (v.byte[i], v.byte[j]) -> fp16 pair (1024 + byte_i, 1024 + byte_j): byte into the low
// mantissa bits under exponent 0x64 (value 1024, ulp 1).
constexpr uint32_t kSel01 = 0x04010400u, kSel23 = 0x04030402u;
__device__ __forceinline__ uint32_t magic2(uint32_t v, uint32_t sel) {
    return __builtin_amdgcn_perm(0x64646464u, v, sel);
}

__device__ __forceinline__ uint32_t ld32(const uint16_t* p) { return *(const uint32_t*)p; }

// Q6_K 6-bit codes (0..63) of elements 128h + 32s + 4k + 0..3, one per byte.
__device__ __forceinline__ uint32_t q6_word(uint32_t qlA, uint32_t qlB, uint32_t qh, int s) {
    const uint32_t lo = (s & 1 ? qlB : qlA) >> (4 * (s >> 1));
    const uint32_t hi = s == 0 ? qh << 4 : s == 1 ? qh << 2 : s == 2 ? qh : qh >> 2;
    return (lo & 0x0f0f0f0fu) | (hi & 0x30303030u);
}

// ============================================================================ tiles
// Raw 16-byte chunks of one (row, 256-weight super-block), loaded ahead of their use.
template <int QT> struct Raw;
template <> struct Raw<PGMOE_Q4_1> { uint4 c[10]; };
template <> struct Raw<PGMOE_Q4_K> { uint4 c[9]; };
template <> struct Raw<PGMOE_Q5_K> { uint4 c[11]; };
template <> struct Raw<PGMOE_Q6_K> { uint4 c[13]; uint32_t d; };
template <> struct Raw<PGMOE_Q8_0> { uint4 c[17]; };
template <> struct Raw<PGMOE_F16> { uint4 c[32]; };

template <int QT>
__device__ __forceinline__ void load_raw(Raw<QT>& r, const uint8_t* mat, int N, int nb, int row, int b) {
    const uint8_t* t = tile_ptr<QT>(mat, nb, row >> 6, b) + (row & 63) * 16;
#pragma unroll
    for (int c = 0; c < Tile<QT>::CH; ++c) r.c[c] = *(const uint4*)(t + c * 1024);
    if constexpr (QT == PGMOE_Q6_K) {
        const int64_t dpl = (int64_t)row_groups(N) * nb * 13 * 1024;
        r.d = *(const uint16_t*)(mat + dpl + (((int64_t)(row >> 6) * nb + b) * 64 + (row & 63)) * 2);
    }
}

// ---------------------------------------------------------------- quarter super-blocks
// The routed decode kernels give every lane one quarter (64 weights) of one 256-weight
// super-block of one row, so a layer's active weights spread over ~200K lanes (a dozen
// waves per CU) and each lane issues 3-5 independent 16-byte loads.  Quarter p of a
// super-block:
//   Q4_K: elements 64p .. 64p+63 (sub-blocks 2p: low nibbles, 2p+1: high nibbles of
//         qs[32p .. 32p+31]) -> chunks 0 (d, dmin, scales), 1+2p, 2+2p
//   Q5_K: as Q4_K, plus the quarter's 8 bytes of fifth bits (chunk 9 + (p >> 1))
//   Q4_1: as Q4_K, with the codes in chunks 2+2p, 3+2p and, in place of the header, the
//         fp16 d and m of blocks 2p, 2p+1 (chunk 0 / chunk 1, bytes 4p .. 4p+3)
//   Q6_K: (h, g) = (p >> 1, p & 1): elements 128h + 32s + 16g + [0, 16) for s = 0..3
//         (sub-blocks 8h + 2s + g) -> ql chunks 4h+g, 4h+2+g, qh chunk 8+2h+g, scale
//         bytes 8h .. 8h+7 and d
//   Q8_0: Q8_0 blocks 2p, 2p+1 = elements 64p .. 64p+63 -> chunks 4p .. 4p+3 and the two
//         fp16 scales at chunk 16 bytes 4p .. 4p+3
//   F16:  elements 64p .. 64p+63 -> chunks 8p .. 8p+7 (the weights themselves)
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ u32x4 ldq(const uint8_t* p) { return *(const u32x4*)p; }

template <int QT> struct Qtr;
template <> struct Qtr<PGMOE_Q4_1> { uint32_t dw, mw; u32x4 a, b; };
template <> struct Qtr<PGMOE_Q4_K> { u32x4 h, a, b; };
template <> struct Qtr<PGMOE_Q5_K> { u32x4 h, a, b; u32x2 hb; };
template <> struct Qtr<PGMOE_Q6_K> { u32x4 la, lb, qh; u32x2 sc; uint32_t d; };
template <> struct Qtr<PGMOE_Q8_0> { u32x4 c0, c1, c2, c3; uint32_t d; };
template <> struct Qtr<PGMOE_F16> { u32x4 c[8]; };

template <int QT>
__device__ __forceinline__ void load_qtr(Qtr<QT>& q, const uint8_t* mat, int N, int nb, int row, int j, int p) {
    const uint8_t* t = tile_ptr<QT>(mat, nb, row >> 6, j) + (row & 63) * 16;
    if constexpr (QT == PGMOE_Q4_1) {
        q.dw = *(const uint32_t*)(t + 4 * p);
        q.mw = *(const uint32_t*)(t + 1024 + 4 * p);
        q.a = ldq(t + (2 + 2 * p) * 1024);
        q.b = ldq(t + (3 + 2 * p) * 1024);
    } else if constexpr (QT == PGMOE_Q4_K || QT == PGMOE_Q5_K) {
        q.h = ldq(t);
        q.a = ldq(t + (1 + 2 * p) * 1024);
        q.b = ldq(t + (2 + 2 * p) * 1024);
        if constexpr (QT == PGMOE_Q5_K) q.hb = *(const u32x2*)(t + (9 + (p >> 1)) * 1024 + 8 * (p & 1));
    } else if constexpr (QT == PGMOE_Q6_K) {
        const int h = p >> 1, g = p & 1;
        q.la = ldq(t + (4 * h + g) * 1024);
        q.lb = ldq(t + (4 * h + 2 + g) * 1024);
        q.qh = ldq(t + (8 + 2 * h + g) * 1024);
        q.sc = *(const u32x2*)(t + 12 * 1024 + 8 * h);
        const int64_t dpl = (int64_t)row_groups(N) * nb * 13 * 1024;
        q.d = *(const uint16_t*)(mat + dpl + (((int64_t)(row >> 6) * nb + j) * 64 + (row & 63)) * 2);
    } else if constexpr (QT == PGMOE_F16) {
#pragma unroll
        for (int i = 0; i < 8; ++i) q.c[i] = ldq(t + (8 * p + i) * 1024);
    } else {
        q.c0 = ldq(t + (4 * p) * 1024);
        q.c1 = ldq(t + (4 * p + 1) * 1024);
        q.c2 = ldq(t + (4 * p + 2) * 1024);
        q.c3 = ldq(t + (4 * p + 3) * 1024);
        q.d = *(const uint32_t*)(t + 16 * 1024 + 4 * p);
    }
}

// Staged activations: row element e of a token at unit (e >> 6) * XU + (e & 63), with
// XU = 72 halves (gate/up, fp16) or 68 floats (down, fp32) per 64-element unit; the
// padding puts the four quarters' units of one super-block on different LDS banks.
constexpr int kXuH = 72, kXuF = 68;
__device__ __forceinline__ int xpos_h(int e) { return (e >> 6) * kXuH + (e & 63); }
__device__ __forceinline__ int xpos_f(int e) { return (e >> 6) * kXuF + (e & 63); }

// Token t of a lane's pair list: 4-bit fields of `toks`.
__device__ __forceinline__ int tok_of(uint32_t toks, int t) { return (toks >> (4 * t)) & 15; }

// 16 fp16 x values (32 bytes) at xr as 8 half2 words.
__device__ __forceinline__ void ldx16(const uint16_t* xr, uint32_t (&v)[8]) {
    const u32x4 a = *(const u32x4*)xr, b = *(const u32x4*)(xr + 8);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

// ---------------------------------------------------------------- gate/up quarter (fp16 x)
// acc[t] += x_tok(t) . w(row, quarter p of super-block j) for the cnt <= TM pairs.  xs: the
// staged fp16 token rows (row stride xrs halves), xss: their 16-element sums (row stride
// srs).  Codes enter v_dot2_f32_f16 as fp16 (1024 + code); the offset returns through the
// 16-element sums, as in the whole-super-block path.
// Q4_K / Q5_K / Q4_1: weight a q - z with (a0, z0) for sub-block 2p (the low nibbles) and
// (a1, z1) for 2p+1 (the high nibbles).  HB: the fifth bits (Q5_K), word hb.x for
// sub-block 2p, hb.y for 2p+1; bits k, 8+k, 16+k, 24+k of a word belong to elements
// 4k .. 4k+3.
template <int TM, bool HB>
__device__ __forceinline__ void gu_qtr_k(float a0, float z0, float a1, float z1, const u32x4& qa, const u32x4& qb,
                                         const u32x2& hb, int j, int p, const uint16_t* xs, int xrs,
                                         const float* xss, int srs, uint32_t toks, int cnt, float* acc) {
    const float b0 = z0 + 1024.0f * a0, b1 = z1 + 1024.0f * a1;
    const uint32_t w8[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
    uint32_t lo[16], hi[16];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        uint32_t l = w8[k] & 0x0f0f0f0fu, hh = (w8[k] >> 4) & 0x0f0f0f0fu;
        if constexpr (HB) {
            l |= ((hb.x >> k) & 0x01010101u) << 4;
            hh |= ((hb.y >> k) & 0x01010101u) << 4;
        }
        lo[2 * k] = magic2(l, kSel01);
        lo[2 * k + 1] = magic2(l, kSel23);
        hi[2 * k] = magic2(hh, kSel01);
        hi[2 * k + 1] = magic2(hh, kSel23);
    }
    const int xo = xpos_h(256 * j + 64 * p), so = 16 * j + 4 * p;
#pragma unroll
    for (int t = 0; t < TM; ++t) {
        if (t < cnt) {
            const int m = tok_of(toks, t);
            const uint16_t* xr = xs + m * xrs + xo;
            float tl = 0.f, th = 0.f;
#pragma unroll
            for (int h16 = 0; h16 < 2; ++h16) {
                uint32_t xl[8], xh[8];
                ldx16(xr + 16 * h16, xl);
                ldx16(xr + 32 + 16 * h16, xh);
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    tl = dot2(lo[8 * h16 + k], xl[k], tl);
                    th = dot2(hi[8 * h16 + k], xh[k], th);
                }
            }
            const float* sx = xss + m * srs + so;
            acc[t] += a0 * tl - b0 * (sx[0] + sx[1]) + a1 * th - b1 * (sx[2] + sx[3]);
        }
    }
}

// (a, z) of K-quant sub-blocks 2p, 2p+1 from the header chunk: a = d sc, z = dmin m.
__device__ __forceinline__ void kq_scales(const u32x4& h, int p, float& a0, float& z0, float& a1, float& z1) {
    const float dd = lo_half(h.x), dm = hi_half(h.x);
    int s0, m0, s1, m1;
    kscale(h.y, h.z, h.w, 2 * p, s0, m0);
    kscale(h.y, h.z, h.w, 2 * p + 1, s1, m1);
    a0 = dd * (float)s0;
    z0 = dm * (float)m0;
    a1 = dd * (float)s1;
    z1 = dm * (float)m1;
}

template <int TM>
__device__ __forceinline__ void gu_qtr(const Qtr<PGMOE_Q4_K>& q, int j, int p, const uint16_t* xs, int xrs,
                                       const float* xss, int srs, uint32_t toks, int cnt, float* acc) {
    float a0, z0, a1, z1;
    kq_scales(q.h, p, a0, z0, a1, z1);
    gu_qtr_k<TM, false>(a0, z0, a1, z1, q.a, q.b, u32x2{0u, 0u}, j, p, xs, xrs, xss, srs, toks, cnt, acc);
}
template <int TM>
__device__ __forceinline__ void gu_qtr(const Qtr<PGMOE_Q5_K>& q, int j, int p, const uint16_t* xs, int xrs,
                                       const float* xss, int srs, uint32_t toks, int cnt, float* acc) {
    float a0, z0, a1, z1;
    kq_scales(q.h, p, a0, z0, a1, z1);
    gu_qtr_k<TM, true>(a0, z0, a1, z1, q.a, q.b, q.hb, j, p, xs, xrs, xss, srs, toks, cnt, acc);
}
// Q4_1: a = d, z = -m of blocks 2p, 2p+1.
template <int TM>
__device__ __forceinline__ void gu_qtr(const Qtr<PGMOE_Q4_1>& q, int j, int p, const uint16_t* xs, int xrs,
                                       const float* xss, int srs, uint32_t toks, int cnt, float* acc) {
    gu_qtr_k<TM, false>(lo_half(q.dw), -lo_half(q.mw), hi_half(q.dw), -hi_half(q.mw), q.a, q.b, u32x2{0u, 0u}, j,
                        p, xs, xrs, xss, srs, toks, cnt, acc);
}

// fp16 value 1024 + q6 (6-bit code), weight = d * sc * (q6 - 32).
template <int TM>
__device__ __forceinline__ void gu_qtr(const Qtr<PGMOE_Q6_K>& q, int j, int p, const uint16_t* xs, int xrs,
                                       const float* xss, int srs, uint32_t toks, int cnt, float* acc) {
    const float d = h2f((uint16_t)q.d);
    const int h = p >> 1, g = p & 1;
    const uint32_t la[4] = {q.la.x, q.la.y, q.la.z, q.la.w};
    const uint32_t lb[4] = {q.lb.x, q.lb.y, q.lb.z, q.lb.w};
    const uint32_t qh[4] = {q.qh.x, q.qh.y, q.qh.z, q.qh.w};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        uint32_t mm[8];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t code = q6_word(la[k], lb[k], qh[k], s);
            mm[2 * k] = magic2(code, kSel01);
            mm[2 * k + 1] = magic2(code, kSel23);
        }
        const int bi = 2 * s + g;  // scale byte within bytes 8h .. 8h+7
        const uint32_t sw = bi < 4 ? q.sc.x : q.sc.y;
        const float a = d * (float)(int8_t)((sw >> (8 * (bi & 3))) & 0xff);
        const int e0 = 256 * j + 128 * h + 32 * s + 16 * g;
        const int xo = xpos_h(e0);
#pragma unroll
        for (int t = 0; t < TM; ++t) {
            if (t < cnt) {
                const int m = tok_of(toks, t);
                uint32_t xv[8];
                ldx16(xs + m * xrs + xo, xv);
                float T = 0.f;
#pragma unroll
                for (int k = 0; k < 8; ++k) T = dot2(mm[k], xv[k], T);
                acc[t] += a * (T - 1056.0f * xss[m * srs + (e0 >> 4)]);
            }
        }
    }
}

// Q8_0 code q in [-128, 127]: byte ^ 0x80 = q + 128, so the fp16 value is 1152 + q.
template <int TM>
__device__ __forceinline__ void gu_qtr(const Qtr<PGMOE_Q8_0>& q, int j, int p, const uint16_t* xs, int xrs,
                                       const float* xss, int srs, uint32_t toks, int cnt, float* acc) {
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
        const float d = jj ? hi_half(q.d) : lo_half(q.d);
        const u32x4 ca = jj ? q.c2 : q.c0, cb = jj ? q.c3 : q.c1;
        const uint32_t w8[8] = {ca.x, ca.y, ca.z, ca.w, cb.x, cb.y, cb.z, cb.w};
        uint32_t mm[16];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t v = w8[k] ^ 0x80808080u;
            mm[2 * k] = magic2(v, kSel01);
            mm[2 * k + 1] = magic2(v, kSel23);
        }
        const int e0 = 256 * j + 64 * p + 32 * jj;
        const int xo = xpos_h(e0);
#pragma unroll
        for (int t = 0; t < TM; ++t) {
            if (t < cnt) {
                const int m = tok_of(toks, t);
                const uint16_t* xr = xs + m * xrs + xo;
                float T = 0.f;
#pragma unroll
                for (int h16 = 0; h16 < 2; ++h16) {
                    uint32_t xv[8];
                    ldx16(xr + 16 * h16, xv);
#pragma unroll
                    for (int k = 0; k < 8; ++k) T = dot2(mm[8 * h16 + k], xv[k], T);
                }
                const float* sx = xss + m * srs + (e0 >> 4);
                acc[t] += d * (T - 1152.0f * (sx[0] + sx[1]));
            }
        }
    }
}

// F16: the weights enter v_dot2_f32_f16 as they are (no scale, no offset sums).
template <int TM>
__device__ __forceinline__ void gu_qtr(const Qtr<PGMOE_F16>& q, int j, int p, const uint16_t* xs, int xrs,
                                       const float* xss, int srs, uint32_t toks, int cnt, float* acc) {
    const int xo = xpos_h(256 * j + 64 * p);
#pragma unroll
    for (int t = 0; t < TM; ++t) {
        if (t < cnt) {
            const uint16_t* xr = xs + tok_of(toks, t) * xrs + xo;
            float T = 0.f;
#pragma unroll
            for (int h16 = 0; h16 < 4; ++h16) {  // elements 16 h16 .. +16: chunks 2 h16, 2 h16 + 1
                uint32_t xv[8];
                ldx16(xr + 16 * h16, xv);
                const u32x4 a = q.c[2 * h16], b = q.c[2 * h16 + 1];
                const uint32_t w8[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
                for (int k = 0; k < 8; ++k) T = dot2(w8[k], xv[k], T);
            }
            acc[t] += T;
        }
    }
}

// ---------------------------------------------------------------- down quarter (fp32 x)
// part[c] = inter_(p0+c) . w(row, quarter p of super-block j) for c < cnt <= TM; xs: the
// staged fp32 inter rows from pair p0 on (row stride xrs floats), iss: their 16-element
// sums (row stride srs).
__device__ __forceinline__ void bytes_f(uint32_t v, float* f) {
    f[0] = (float)(v & 0xff);
    f[1] = (float)((v >> 8) & 0xff);
    f[2] = (float)((v >> 16) & 0xff);
    f[3] = (float)(v >> 24);
}

template <int N>
__device__ __forceinline__ float dotf(const float* qf, const float* xr) {
    float T = 0.f;
#pragma unroll
    for (int i = 0; i < N; i += 4) {
        const floatx4 v = *(const floatx4*)(xr + i);
        T = __builtin_fmaf(qf[i], v.x, T);
        T = __builtin_fmaf(qf[i + 1], v.y, T);
        T = __builtin_fmaf(qf[i + 2], v.z, T);
        T = __builtin_fmaf(qf[i + 3], v.w, T);
    }
    return T;
}

template <int TM, bool HB>
__device__ __forceinline__ void dn_qtr_k(float a0, float z0, float a1, float z1, const u32x4& qa, const u32x4& qb,
                                         const u32x2& hb, int j, int p, const float* xs, int xrs, const float* iss,
                                         int srs, int cnt, float* part) {
    const uint32_t w8[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
#pragma unroll
    for (int hi = 0; hi < 2; ++hi) {
        const float a = hi ? a1 : a0, bm = hi ? z1 : z0;
        float qf[32];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            uint32_t v = (w8[k] >> (4 * hi)) & 0x0f0f0f0fu;
            if constexpr (HB) v |= (((hi ? hb.y : hb.x) >> k) & 0x01010101u) << 4;
            bytes_f(v, qf + 4 * k);
        }
        const int e0 = 256 * j + 64 * p + 32 * hi;
        const int xo = xpos_f(e0);
#pragma unroll
        for (int c = 0; c < TM; ++c) {
            if (c < cnt) {
                const float T = dotf<32>(qf, xs + c * xrs + xo);
                const float* sx = iss + c * srs + (e0 >> 4);
                part[c] += a * T - bm * (sx[0] + sx[1]);
            }
        }
    }
}

template <int TM>
__device__ __forceinline__ void dn_qtr(const Qtr<PGMOE_Q4_K>& q, int j, int p, const float* xs, int xrs,
                                       const float* iss, int srs, int cnt, float* part) {
    float a0, z0, a1, z1;
    kq_scales(q.h, p, a0, z0, a1, z1);
    dn_qtr_k<TM, false>(a0, z0, a1, z1, q.a, q.b, u32x2{0u, 0u}, j, p, xs, xrs, iss, srs, cnt, part);
}
template <int TM>
__device__ __forceinline__ void dn_qtr(const Qtr<PGMOE_Q5_K>& q, int j, int p, const float* xs, int xrs,
                                       const float* iss, int srs, int cnt, float* part) {
    float a0, z0, a1, z1;
    kq_scales(q.h, p, a0, z0, a1, z1);
    dn_qtr_k<TM, true>(a0, z0, a1, z1, q.a, q.b, q.hb, j, p, xs, xrs, iss, srs, cnt, part);
}
template <int TM>
__device__ __forceinline__ void dn_qtr(const Qtr<PGMOE_Q4_1>& q, int j, int p, const float* xs, int xrs,
                                       const float* iss, int srs, int cnt, float* part) {
    dn_qtr_k<TM, false>(lo_half(q.dw), -lo_half(q.mw), hi_half(q.dw), -hi_half(q.mw), q.a, q.b, u32x2{0u, 0u}, j,
                        p, xs, xrs, iss, srs, cnt, part);
}

template <int TM>
__device__ __forceinline__ void dn_qtr(const Qtr<PGMOE_Q6_K>& q, int j, int p, const float* xs, int xrs,
                                       const float* iss, int srs, int cnt, float* part) {
    const float d = h2f((uint16_t)q.d);
    const int h = p >> 1, g = p & 1;
    const uint32_t la[4] = {q.la.x, q.la.y, q.la.z, q.la.w};
    const uint32_t lb[4] = {q.lb.x, q.lb.y, q.lb.z, q.lb.w};
    const uint32_t qh[4] = {q.qh.x, q.qh.y, q.qh.z, q.qh.w};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        float qf[16];
#pragma unroll
        for (int k = 0; k < 4; ++k) bytes_f(q6_word(la[k], lb[k], qh[k], s), qf + 4 * k);
        const int bi = 2 * s + g;
        const uint32_t sw = bi < 4 ? q.sc.x : q.sc.y;
        const float a = d * (float)(int8_t)((sw >> (8 * (bi & 3))) & 0xff);
        const int e0 = 256 * j + 128 * h + 32 * s + 16 * g;
        const int xo = xpos_f(e0);
#pragma unroll
        for (int c = 0; c < TM; ++c) {
            if (c < cnt) {
                const float T = dotf<16>(qf, xs + c * xrs + xo);
                part[c] += a * (T - 32.0f * iss[c * srs + (e0 >> 4)]);
            }
        }
    }
}

template <int TM>
__device__ __forceinline__ void dn_qtr(const Qtr<PGMOE_Q8_0>& q, int j, int p, const float* xs, int xrs,
                                       const float* iss, int srs, int cnt, float* part) {
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
        const float d = jj ? hi_half(q.d) : lo_half(q.d);
        const u32x4 ca = jj ? q.c2 : q.c0, cb = jj ? q.c3 : q.c1;
        const uint32_t w8[8] = {ca.x, ca.y, ca.z, ca.w, cb.x, cb.y, cb.z, cb.w};
        float qf[32];
#pragma unroll
        for (int k = 0; k < 8; ++k) bytes_f(w8[k] ^ 0x80808080u, qf + 4 * k);  // q + 128 per byte
        const int e0 = 256 * j + 64 * p + 32 * jj;
        const int xo = xpos_f(e0);
#pragma unroll
        for (int c = 0; c < TM; ++c) {
            if (c < cnt) {
                const float T = dotf<32>(qf, xs + c * xrs + xo);
                const float* sx = iss + c * srs + (e0 >> 4);
                part[c] += d * (T - 128.0f * (sx[0] + sx[1]));
            }
        }
    }
}

template <int TM>
__device__ __forceinline__ void dn_qtr(const Qtr<PGMOE_F16>& q, int j, int p, const float* xs, int xrs,
                                       const float* iss, int srs, int cnt, float* part) {
#pragma unroll
    for (int h16 = 0; h16 < 4; ++h16) {  // elements 16 h16 .. +16 of the quarter
        const u32x4 a = q.c[2 * h16], b = q.c[2 * h16 + 1];
        const uint32_t w8[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        float qf[16];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            qf[2 * k] = lo_half(w8[k]);
            qf[2 * k + 1] = hi_half(w8[k]);
        }
        const int xo = xpos_f(256 * j + 64 * p + 16 * h16);
#pragma unroll
        for (int c = 0; c < TM; ++c)
            if (c < cnt) part[c] += dotf<16>(qf, xs + c * xrs + xo);
    }
}

// ---------------------------------------------------------------- down (fp32)
// acc[t] += inter_t . w(row, block); x = global fp32 rows (stride K, wave-uniform)
// offset to the block, isum = LDS 16-element sums (stride K/16) offset to the block.
template <int TM>
__device__ __forceinline__ void dn_compute(const Raw<PGMOE_Q6_K>& r, const float* x, const float* isum, int K,
                                           int me, float* acc) {
    const float d = h2f((uint16_t)r.d);
    const uint32_t scw[4] = {r.c[12].x, r.c[12].y, r.c[12].z, r.c[12].w};
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                float qf[16];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const int kk = 4 * half + k;
                    const int wa = 16 * h + kk, wb = 16 * h + 8 + kk, wq = 8 * h + kk;
                    const uint32_t qa = ((const uint32_t*)&r.c[wa >> 2])[wa & 3];
                    const uint32_t qb = ((const uint32_t*)&r.c[wb >> 2])[wb & 3];
                    const uint32_t qh = ((const uint32_t*)&r.c[8 + (wq >> 2)])[wq & 3];
                    const uint32_t q = q6_word(qa, qb, qh, s);
                    qf[4 * k + 0] = (float)(q & 0xff);
                    qf[4 * k + 1] = (float)((q >> 8) & 0xff);
                    qf[4 * k + 2] = (float)((q >> 16) & 0xff);
                    qf[4 * k + 3] = (float)(q >> 24);
                }
                const int sb = 8 * h + 2 * s + half;
                const float a = d * (float)(int8_t)((scw[sb >> 2] >> (8 * (sb & 3))) & 0xff);
#pragma unroll
                for (int t = 0; t < TM; ++t) {
                    if (t < me) {
                        const float* xr = x + (int64_t)t * K + 128 * h + 32 * s + 16 * half;
                        float T = 0.f;
#pragma unroll
                        for (int i = 0; i < 16; ++i) T = __builtin_fmaf(qf[i], xr[i], T);
                        acc[t] += a * (T - 32.0f * isum[t * (K >> 4) + sb]);
                    }
                }
            }
}

template <int TM, int QT>
__device__ __forceinline__ void dn_compute_k(const Raw<QT>& r, const float* x, const float* isum, int K, int me,
                                             float* acc) {
    const uint4 hd = r.c[0];
    const float dd = lo_half(hd.x), dm = hi_half(hd.x);
    constexpr int QC = QT == PGMOE_Q4_1 ? 2 : 1;  // first code chunk
#pragma unroll
    for (int s = 0; s < 8; ++s) {  // sub-block s: qs bytes 32(s/2).., nibble s&1 (Q5_K: fifth-bit word s)
        float a, bm;
        if constexpr (QT == PGMOE_Q4_1) {  // d, m: fp16 word s of chunks 0, 1
            const uint32_t dwd = (s >> 1) == 0 ? r.c[0].x : (s >> 1) == 1 ? r.c[0].y : (s >> 1) == 2 ? r.c[0].z : r.c[0].w;
            const uint32_t mwd = (s >> 1) == 0 ? r.c[1].x : (s >> 1) == 1 ? r.c[1].y : (s >> 1) == 2 ? r.c[1].z : r.c[1].w;
            a = (s & 1) ? hi_half(dwd) : lo_half(dwd);
            bm = -((s & 1) ? hi_half(mwd) : lo_half(mwd));
        } else {
            int sc, mn;
            kscale(hd.y, hd.z, hd.w, s, sc, mn);
            a = dd * (float)sc;
            bm = dm * (float)mn;
        }
        const int c2 = s >> 1, sh = 4 * (s & 1);
        const uint4 qa = r.c[QC + 2 * c2], qb = r.c[QC + 1 + 2 * c2];
        const uint32_t w8[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
        float qf[32];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            uint32_t v = (w8[k] >> sh) & 0x0f0f0f0fu;
            if constexpr (QT == PGMOE_Q5_K) {  // word s at chunk 9 + (s >> 2), dword s & 3
                const uint4 hc = r.c[9 + (s >> 2)];
                const uint32_t hw = (s & 3) == 0 ? hc.x : (s & 3) == 1 ? hc.y : (s & 3) == 2 ? hc.z : hc.w;
                v |= ((hw >> k) & 0x01010101u) << 4;
            }
            qf[4 * k + 0] = (float)(v & 0xff);
            qf[4 * k + 1] = (float)((v >> 8) & 0xff);
            qf[4 * k + 2] = (float)((v >> 16) & 0xff);
            qf[4 * k + 3] = (float)(v >> 24);
        }
#pragma unroll
        for (int t = 0; t < TM; ++t) {
            if (t < me) {
                const float* xr = x + (int64_t)t * K + 32 * s;
                float T = 0.f;
#pragma unroll
                for (int i = 0; i < 32; ++i) T = __builtin_fmaf(qf[i], xr[i], T);
                const float* sx = isum + t * (K >> 4) + 2 * s;
                acc[t] += a * T - bm * (sx[0] + sx[1]);
            }
        }
    }
}

template <int TM>
__device__ __forceinline__ void dn_compute(const Raw<PGMOE_Q4_K>& r, const float* x, const float* isum, int K,
                                           int me, float* acc) {
    dn_compute_k<TM, PGMOE_Q4_K>(r, x, isum, K, me, acc);
}
template <int TM>
__device__ __forceinline__ void dn_compute(const Raw<PGMOE_Q5_K>& r, const float* x, const float* isum, int K,
                                           int me, float* acc) {
    dn_compute_k<TM, PGMOE_Q5_K>(r, x, isum, K, me, acc);
}
template <int TM>
__device__ __forceinline__ void dn_compute(const Raw<PGMOE_Q4_1>& r, const float* x, const float* isum, int K,
                                           int me, float* acc) {
    dn_compute_k<TM, PGMOE_Q4_1>(r, x, isum, K, me, acc);
}

template <int TM>
__device__ __forceinline__ void dn_compute(const Raw<PGMOE_Q8_0>& r, const float* x, const float* isum, int K,
                                           int me, float* acc) {
    const uint32_t dw[4] = {r.c[16].x, r.c[16].y, r.c[16].z, r.c[16].w};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const float d = (j & 1) ? hi_half(dw[j >> 1]) : lo_half(dw[j >> 1]);
        const uint4 qa = r.c[2 * j], qb = r.c[2 * j + 1];
        const uint32_t w8[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
        float qf[32];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t v = w8[k] ^ 0x80808080u;  // q + 128 per byte
            qf[4 * k + 0] = (float)(v & 0xff);
            qf[4 * k + 1] = (float)((v >> 8) & 0xff);
            qf[4 * k + 2] = (float)((v >> 16) & 0xff);
            qf[4 * k + 3] = (float)(v >> 24);
        }
#pragma unroll
        for (int t = 0; t < TM; ++t) {
            if (t < me) {
                const float* xr = x + (int64_t)t * K + 32 * j;
                float T = 0.f;
#pragma unroll
                for (int i = 0; i < 32; ++i) T = __builtin_fmaf(qf[i], xr[i], T);
                const float* sx = isum + t * (K >> 4) + 2 * j;
                acc[t] += d * (T - 128.0f * (sx[0] + sx[1]));
            }
        }
    }
}

// Sum over the KS = 64/RB lanes that share a row (lanes r, r+RB, r+2RB, ...).
template <int RB>
__device__ __forceinline__ float kslot_sum(float v) {
    if constexpr (RB < 64) {
        v += xor_lane<RB>(v);
        return kslot_sum<2 * RB>(v);
    } else {
        return v;
    }
}

// ============================================================================ routing in a block
// Decode forward: the lowest gate/up blocks compute the router logits [M][E] and every
// gate/up block re-derives the top-k sets of the M <= 8 tokens from them (wave m selects
// token m with scalar ballot arithmetic, about half a microsecond, instead of a launch and
// its dependent global round trips), and block (0, 0) also publishes a compact routing
// descriptor for the fused down + combine kernel:
//   int32 words: [0] n_active; slot a at kDescSlot + 4a = {expert, first sorted pair,
//   pair count, 0}; sorted pair p at kDescPair + 2p = {token, weight bits}.
// Active slots are in ascending expert id; the pairs of an expert in ascending token
// order (the order of the reference's torch.where over the expert mask, model.py:912-914).
constexpr int kDescSlot = 16;
constexpr int kDescPair = kDescSlot + 4 * 128;
constexpr int kDescWords = kDescPair + 2 * 128;

struct RouteShared {
    uint32_t pres[kDecTM][16];  // token x expert membership bits (E <= 512)
    uint32_t used[16];          // union of pres over the tokens
    int wc[16];                 // active experts in the words before q
    int wp[16];                 // (token, expert) pairs in the words before q
    int mem_e[kDecTM * 16];     // the K members of token m at [m*K, m*K+K), ascending id
    float mem_w[kDecTM * 16];   // their combine weights (publishing block only)
    int n_act;                  // active experts
};

// Selection key of (logit v, expert e): larger key = earlier in (logit desc, id asc).
// -0.0 is folded into +0.0 first so that the key order equals the float order.
__device__ __forceinline__ uint64_t route_key(float v, int e) {
    const uint32_t u = __builtin_bit_cast(uint32_t, v + 0.0f);
    const uint32_t o = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)o << 9) | (uint64_t)(511 - e);
}

// Block-wide copy of n elements: element i moves from src(i) to dst(i), U loads in flight
// per thread before the first store (expanded over an index sequence so the staging
// values stay in registers).
template <typename T, typename Src, typename Dst, int... I>
__device__ __forceinline__ void copy_step(int i0, int n, int nth, Src src, Dst dst, std::integer_sequence<int, I...>) {
    T v[sizeof...(I)];
    ((v[I] = (i0 + I * nth < n) ? *src(i0 + I * nth) : T{}), ...);
    ((i0 + I * nth < n ? (void)(*dst(i0 + I * nth) = v[I]) : (void)0), ...);
}

template <int U, typename T, typename Src, typename Dst>
__device__ __forceinline__ void copy_idx(int n, int tid, int nth, Src src, Dst dst) {
    for (int i0 = tid; i0 < n; i0 += U * nth) copy_step<T>(i0, n, nth, src, dst, std::make_integer_sequence<int, U>{});
}

template <int U, typename T>
__device__ __forceinline__ void copy_words(T* dst, const T* __restrict__ src, int n, int tid, int nth) {
    copy_idx<U, T>(n, tid, nth, [=](int i) { return src + i; }, [=](int i) { return dst + i; });
}

// A threshold with exactly K of the distinct keys of one token at or above it (lane l
// holds experts l + 64r): a radix descent on the 41 key bits.  The threshold and the
// counts are wave-uniform (scalar registers); each step is one vector compare per key
// word and a popcount of the resulting lane mask.  Steps go in unrolled groups of 8 with
// one exit test a group: the descent may stop once a candidate with exactly K keys at or
// above it was taken (with random logits after about a dozen steps), and a step past that
// point keeps such a threshold (a higher candidate with K keys is as good), so the test
// need not follow every step.  Measured in a one-wave microbenchmark (MI355X, E = 128,
// K = 8): 1,550-1,680 cycles with a test and a branch after every step, 644 with the
// groups of 8 (a step's VALU -> SALU hand-off and branch cost ~130 cycles).
template <int RE>
__device__ __forceinline__ uint64_t kth_key_radix(const uint64_t (&key)[RE], int K) {
    uint64_t thr = 0;
    int last = 0;  // keys at or above the last candidate taken
    for (int b0 = 40; b0 >= 0; b0 -= 8) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int b = b0 - i;
            if (b >= 0) {
                const uint64_t cand = thr | (1ull << b);
                int cnt = 0;
#pragma unroll
                for (int r = 0; r < RE; ++r) cnt += __popcll(__ballot(key[r] >= cand));
                thr = cnt >= K ? cand : thr;
                last = cnt >= K ? cnt : last;
            }
        }
        if (last == K) break;
    }
    return thr;
}

// Ready-tagged logits: word [m][e] = (1 << 32) | float bits once the router wave of
// expert e has stored it, 0 before (the forward's last kernel clears the words again).
// Stores and polls are relaxed agent-scope atomics, so a consumer sees each word either
// unwritten or final, from any XCD, with no fence and no cache invalidation.
// kRlogCopies replicas of the words ([copy][M][E]): every block polls copy
// (block id % kRlogCopies), so the few cache lines of one copy are not hammered by every
// polling wave of the grid (polls go past the per-XCD L2s, to the memory side).
constexpr int kRlogCopies = 16;
__device__ __forceinline__ void put_logit(uint64_t* p, float v) {
    __hip_atomic_store(p, (1ull << 32) | __builtin_bit_cast(uint32_t, v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
constexpr int kSpinMax = 1 << 20;  // polls before a waiting wave gives up (no hang; see below)
// Bit of the workspace status word set by a wave whose bounded wait gave up: the layer's
// output is then wrong, and pgmoe_moe_status reports it to the host.
constexpr int32_t kStatusSpinTimeout = PGMOE_STATUS_SPIN_TIMEOUT;

// Logits of token m for lane l (experts l + 64r; -inf past E): polls the tagged words
// (a bounded spin with short sleeps) until every one of the wave's is written.  A wave that
// gives up after kSpinMax polls sets kStatusSpinTimeout in *status (vector atomic OR) and,
// when the caller gave one, in its host-mapped word *status_host (system scope, so the
// host sees it without synchronising the stream).
template <int RE>
__device__ __forceinline__ void load_logits(const uint64_t* rlog, int m, int E, int lane, float (&v)[RE],
                                            int32_t* status, int32_t* status_host) {
    uint64_t q[RE];
    int n = 0;
    for (;;) {
        bool ready = true;
#pragma unroll
        for (int r = 0; r < RE; ++r) {
            const int e = lane + 64 * r;
            q[r] = e < E ? __hip_atomic_load(rlog + (int64_t)m * E + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                         : 1ull << 32;
            ready = ready && (q[r] >> 32) != 0;
        }
        if (__all(ready)) break;
        if (++n >= kSpinMax) {
            if (lane == 0 && status) __hip_atomic_fetch_or(status, kStatusSpinTimeout, __ATOMIC_RELAXED,
                                                           __HIP_MEMORY_SCOPE_AGENT);
            if (lane == 0 && status_host)
                __hip_atomic_fetch_or(status_host, kStatusSpinTimeout, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
#pragma unroll
    for (int r = 0; r < RE; ++r) v[r] = lane + 64 * r < E ? __builtin_bit_cast(float, (uint32_t)q[r]) : -INFINITY;
}

// Top-k membership of token m (one wave; v = load_logits): the members are exactly the
// keys at or above the radix threshold (keys are distinct).  Lane 0 writes the
// membership words R.pres[m][*], the members write their ids to R.mem_e; with `weights`,
// also their softmax weights
// (max-subtracted, denominator over all E, optional renorm; model.py:903-907) in
// ascending id order to R.mem_e / R.mem_w.
template <int RE>
__device__ __forceinline__ void route_token(const float (&v)[RE], int m, int E, int K, RouteShared& R, bool weights,
                                            int norm, int lane) {
    uint64_t key[RE];
#pragma unroll
    for (int r = 0; r < RE; ++r) key[r] = lane + 64 * r < E ? route_key(v[r], lane + 64 * r) : 0ull;
    const uint64_t thr = kth_key_radix<RE>(key, K);
    float top = -INFINITY, den = 0.f;
    if (weights) {
#pragma unroll
        for (int r = 0; r < RE; ++r) top = fmaxf(top, v[r]);
        top = wave_max(top);
#pragma unroll
        for (int r = 0; r < RE; ++r)
            if (lane + 64 * r < E) den += expf(v[r] - top);
        den = group_sum<64>(den);
    }
    int base = 0;
    float psel = 0.f;
#pragma unroll
    for (int r = 0; r < RE; ++r) {
        const bool in = key[r] >= thr && lane + 64 * r < E;
        const uint64_t mask = __ballot(in);
        if (lane == 0) {
            R.pres[m][2 * r] = (uint32_t)mask;
            R.pres[m][2 * r + 1] = (uint32_t)(mask >> 32);
        }
        const int pos = base + __popcll(mask & ((1ull << lane) - 1ull));
        if (in && pos < K) {  // exactly K members unless logits hold NaNs
            R.mem_e[m * K + pos] = lane + 64 * r;
            if (weights) {
                const float pr = expf(v[r] - top) / den;
                R.mem_w[m * K + pos] = pr;
                psel += pr;
            }
        }
        base += __popcll(mask);
    }
    if (weights && norm) {
        psel = group_sum<64>(psel);
        for (int i = lane; i < K; i += 64) R.mem_w[m * K + i] = R.mem_w[m * K + i] / fmaxf(psel, 1e-20f);
    }
    if (lane < 16 && lane >= 2 * RE) R.pres[m][lane] = 0u;
}

// Active slot a of the routing in R (after the barrier that follows route_token): every
// wave derives it on its own from the membership words (lane q < 16 holds word q of every
// token), with DPP row scans and lane reads instead of LDS round trips, so no further
// barrier is needed.  With store_words, the per-word prefix counts used / wc / wp and
// n_act also go to R (for publish_route).
struct SlotInfo {
    int n_act, e, p_begin, count;
    uint32_t toks;  // the count tokens of expert e, ascending, 4 bits each
};

// Inclusive prefix sum over each 16-lane DPP row.
__device__ __forceinline__ int row_scan16(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);  // row_shr:1
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);  // row_shr:2
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);  // row_shr:4
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);  // row_shr:8
    return v;
}

template <int TM>
__device__ __forceinline__ SlotInfo slot_info(RouteShared& R, int M, int a, int lane, bool store_words) {
    uint32_t wm[TM];
    uint32_t u = 0;
    int pc = 0;
#pragma unroll
    for (int m = 0; m < TM; ++m) {
        wm[m] = (m < M && lane < 16) ? R.pres[m][lane & 15] : 0u;
        u |= wm[m];
        pc += __popc(wm[m]);
    }
    const int ca = row_scan16(__popc(u)), cp = row_scan16(pc);
    const int wc = ca - __popc(u), wp = cp - pc;
    if (store_words && lane < 16) {
        R.used[lane] = u;
        R.wc[lane] = wc;
        R.wp[lane] = wp;
    }
    SlotInfo si;
    si.n_act = __builtin_amdgcn_readlane(ca, 15);
    if (store_words && lane == 0) R.n_act = si.n_act;
    si.e = -1;
    si.p_begin = si.count = 0;
    si.toks = 0;
    if (a >= si.n_act) return si;
    const uint64_t hit = __ballot(lane < 16 && a >= wc && a < ca);
    const int q = __ffsll((unsigned long long)hit) - 1;
    uint32_t uq = __builtin_amdgcn_readlane(u, q);
    const int skip = a - __builtin_amdgcn_readlane(wc, q);
    for (int i = 0; i < skip; ++i) uq &= uq - 1u;
    const int bit = __ffs(uq) - 1;
    si.e = 32 * q + bit;
    const uint32_t below = (1u << bit) - 1u;
    int pb = __builtin_amdgcn_readlane(wp, q), c = 0;
    uint32_t toks = 0;
#pragma unroll
    for (int m = 0; m < TM; ++m) {
        const uint32_t w = __builtin_amdgcn_readlane(wm[m], q);  // 0 past M
        pb += __popc(w & below);
        if ((w >> bit) & 1u) {
            toks |= (uint32_t)m << (4 * c);
            ++c;
        }
    }
    si.p_begin = pb;
    si.count = c;
    si.toks = toks;
    return si;
}

// Active slot a of a single token's routing: its a-th member in ascending id (R.mem_e),
// sorted pair a; the token has exactly K members.
__device__ __forceinline__ SlotInfo slot_info1(const RouteShared& R, int a, int K) {
    SlotInfo si;
    si.n_act = K;
    si.e = a < K ? R.mem_e[a] : -1;
    si.p_begin = a;
    si.count = 1;
    si.toks = 0;
    return si;
}

// Expert e's active-slot index (or -1), its first sorted pair and pair count.
__device__ __forceinline__ int route_expert(const RouteShared& R, int M, int e, int& p_begin, int& count) {
    const int q = e >> 5;
    const uint32_t bit = 1u << (e & 31), below = bit - 1u;
    if (!(R.used[q] & bit)) return -1;
    p_begin = R.wp[q];
    count = 0;
    for (int m = 0; m < M; ++m) {
        p_begin += __popc(R.pres[m][q] & below);
        count += (R.pres[m][q] & bit) ? 1 : 0;
    }
    return R.wc[q] + __popc(R.used[q] & below);
}

// Flat routing arrays of a counting-sort dispatch (the stage API's layout), written by the
// routing block when the down stage runs per expert: offsets [E+1], perm / inv / w [M*K]
// (pair f = token*K + i, members i in ascending expert id), active [n_active], n_active.
struct FlatRoute {
    int32_t *offsets, *perm, *inv, *active, *n_active;
    float* w;
};

// Publish the routing descriptor (block (0, 0) only; R holds the weights and the word
// prefix counts), and the flat arrays when fl.offsets is set.  One thread per expert, then
// one per pair.
__device__ __forceinline__ void publish_route(const RouteShared& R, int M, int E, int K, int32_t* __restrict__ desc,
                                              const FlatRoute& fl) {
    const int tid = threadIdx.x, nth = blockDim.x;
    for (int e = tid; e < E; e += nth) {
        int pb = 0, c = 0;
        const int a = route_expert(R, M, e, pb, c);
        if (a >= 0) {
            desc[kDescSlot + 4 * a] = e;
            desc[kDescSlot + 4 * a + 1] = pb;
            desc[kDescSlot + 4 * a + 2] = c;
            if (fl.offsets) fl.active[a] = e;
        }
        if (fl.offsets) {  // pairs of the experts below e
            const int q = e >> 5;
            int o = R.wp[q];
            for (int m = 0; m < M; ++m) o += __popc(R.pres[m][q] & ((1u << (e & 31)) - 1u));
            fl.offsets[e] = o;
        }
    }
    for (int f = tid; f < M * K; f += nth) {
        const int m = f / K, e = R.mem_e[f], q = e >> 5;
        const uint32_t bit = 1u << (e & 31);
        int pos = R.wp[q];
        for (int m2 = 0; m2 < M; ++m2) {
            pos += __popc(R.pres[m2][q] & (bit - 1u));
            pos += (m2 < m && (R.pres[m2][q] & bit)) ? 1 : 0;
        }
        desc[kDescPair + 2 * pos] = m;
        desc[kDescPair + 2 * pos + 1] = __builtin_bit_cast(int32_t, R.mem_w[f]);
        if (fl.offsets) {
            fl.perm[pos] = f;
            fl.inv[f] = pos;
            fl.w[f] = R.mem_w[f];
        }
    }
    if (tid == 0) {
        desc[0] = R.n_act;
        if (fl.offsets) {
            fl.offsets[E] = M * K;
            *fl.n_active = R.n_act;
        }
    }
}


// ============================================================================ kernels
// Where a decode expert kernel finds its pairs:
//   kDispatch: offsets / perm / active / n_active of a counting-sort dispatch (stage API);
//   kRoute   : derived in the block from the router logits (decode forward; block (0, 0)
//              also publishes the routing descriptor);
//   kIdent   : one expert (matrix 0) applied to every token with weight 1 (shared expert);
//   kLinear  : kIdent with a single matrix (gate/up launch only): y = x . W^T (+ bias),
//              the quantized linear (GGUFQuantLinear.forward, quant_kernels.py:1826).
enum DecMode { kDispatch = 0, kRoute = 1, kIdent = 2, kLinear = 3 };

struct DecDisp {
    int mode;  // DecMode
    const int32_t *offsets, *perm, *active, *n_active;
    const uint64_t* rlog; // kRoute: ready-tagged router logits [kRlogCopies][M][E] (put_logit)
    int32_t* desc;        // kRoute: published by block (0, 0)
    int32_t* status;      // kRoute: workspace status word (kStatusSpinTimeout), or null
    int M, E, norm;       // M: tokens (every mode)
    FlatRoute flat;       // kRoute: optional flat arrays, published by block (0, 0)
    const float* bias;    // kLinear: [N] added to the outputs, or null
    int out_f16;          // kLinear: outputs as fp16 (round to nearest even) instead of fp32
    int act;              // gate activation PGMOE_ACT_* of the gate/up epilogue
    int32_t* status_host; // kRoute: the caller's host-mapped status word (pgmoe_layer.status_host), or null
};

// Router work folded into the routed gate/up launch: with R = ceil(rows / blocks) (1
// unless the grid is small), wave w < R of block b computes logits row b * R + w (all
// tokens; row E is the shared expert's gate) and stores it as tagged words (put_logit);
// every block's routing waves poll the words of their tokens.  The producers sit in the
// lowest blocks, which are dispatched first, and never wait.
struct RouterIn {
    const float* W;        // [E][H] fp32 router weights; null: logits come from a router launch
    const float* bias;     // [E] or null
    const float* extra_w;  // shared expert gate row [H] or null
    float* extra_out;      // [M] its logits
    float* xsum_out;       // [M][H/16] 16-element sums of x for the shared expert's launches, or null
};

// Active slot a of the dispatch or identity modes (a token meets an expert at most once,
// so count <= M <= 8).
template <int MODE>
__device__ __forceinline__ SlotInfo slot_plain(const DecDisp& dp, int a, int topk) {
    SlotInfo si;
    si.e = -1;
    si.p_begin = si.count = 0;
    si.toks = 0;
    if constexpr (MODE == kIdent || MODE == kLinear) {
        si.n_act = 1;
        if (a > 0) return si;
        si.e = 0;
        si.count = dp.M;
        for (int m = 0; m < dp.M; ++m) si.toks |= (uint32_t)m << (4 * m);
        return si;
    }
    si.n_act = *dp.n_active;
    if (a >= si.n_act) return si;
    si.e = dp.active[a];
    si.p_begin = dp.offsets[si.e];
    si.count = min(dp.offsets[si.e + 1] - si.p_begin, dp.M);
    for (int t = 0; t < si.count; ++t) si.toks |= (uint32_t)(dp.perm[si.p_begin + t] / topk) << (4 * t);
    return si;
}

// Gate/up + SwiGLU.  Block = 16 rows (8 for one routed token in the gu_rows8 formats, set
// out in the kernel) of the experts of active slots blockIdx.y,
// + gridDim.y, ...; W (even) waves: wave w owns the items it = w, w + W, ... of the
// 2 * (K/256) (matrix = it & 1, super-block j = it >> 1), lane = (row r = lane & 15,
// quarter p = lane >> 4).  Every token row is staged in LDS (fp16, padded units) while the
// block routes, once for all its slots; each lane then loads the quarters of two items at
// once and accumulates one partial per pair of the expert.  inter / isum rows are indexed
// by sorted pair p_begin + t.
// Dynamic LDS: xs [M][K/64][72] fp16 | xss [M][K/16] f32.
// xsum (optional): 16-element sums of the x rows [M][K/16] (else computed from xs);
// isum (optional output): 16-element sums of the inter rows [P][N/16] (8-row blocks: 8-element
// sums [P][N/8]).
template <int RE>
__device__ __forceinline__ void route_waves(const DecDisp& dp, int topk, RouteShared& R, bool pub, int lane, int w,
                                            int nw, [[maybe_unused]] unsigned long long& t_ready) {
    float v[RE];
    const int copy = (blockIdx.y * gridDim.x + blockIdx.x) % kRlogCopies;
    const uint64_t* rlog = dp.rlog + (int64_t)copy * dp.M * dp.E;
    for (int m = w; m < dp.M; m += nw) {
        load_logits<RE>(rlog, m, dp.E, lane, v, dp.status, dp.status_host);
#ifdef PG_TRACE
        if (m == 0) t_ready = wall_clock64();
#endif
        route_token<RE>(v, m, dp.E, topk, R, pub, dp.norm, lane);
    }
}

// Issue priority from the slots a block has left after the current one.  Blocks of up to 8
// waves share a CU two at a time (the 128-register bound allows 16 waves); the older
// one's waves win the issue arbitration and it runs ahead, and the kernel then ends on
// the other.  Lowering a block's priority as it nears its end lets the other catch up.
// Measured with 2+ tokens: C2 (8 waves) M = 4 / 8 37.0 / 63.0 -> 35.5 / 60.3 us; blocks
// of 14-16 waves, alone on their CU, were 1-2 % slower with it, so they keep priority 0.
__device__ __forceinline__ void slot_prio(int left) {
    if (left >= 3)
        __builtin_amdgcn_s_setprio(3);
    else if (left == 2)
        __builtin_amdgcn_s_setprio(2);
    else if (left == 1)
        __builtin_amdgcn_s_setprio(1);
    else
        __builtin_amdgcn_s_setprio(0);
}

// The one-token routed gate/up runs 8-row blocks (and leaves 8-row sums) for the formats
// of at most 11 chunks a tile (Q4_1, Q4_K, Q5_K); Q6_K and Q8_0 keep 16-row blocks, which
// measured faster for their larger rows.
template <int QT> constexpr bool gu_rows8() { return Tile<QT>::CH <= 11; }
// MODE: DecMode (fixed per instantiation, so each kernel holds only its own path); RE:
// logit words per lane of the routing waves (kRoute: E <= 64 * RE); RL: the grid is one
// round of resident blocks and each block loops over row blocks blockIdx.x, + gridDim.x,
// ... (launched so when the row blocks outnumber the resident blocks).
template <int QT, int TM, int MODE, int RE, bool RL>
__global__ __launch_bounds__(1024) void dec_gu_kernel(const uint8_t* __restrict__ gbase,
                                                      const uint8_t* __restrict__ ubase, int64_t gstride,
                                                      int64_t ustride, int N, int K, const uint16_t* __restrict__ x,
                                                      const float* __restrict__ xsum, int topk, DecDisp dp,
                                                      RouterIn rt, float* __restrict__ inter,
                                                      float* __restrict__ isum) {
    constexpr int RB = 16, XR = 4;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    __shared__ RouteShared R;
    __shared__ float red[16][TM][RB];  // per-wave row partials
    // With 4+ tokens (blocks then take several slots) the first pass of the next slot is
    // loaded before this slot's epilogue, so its weights stream during the reduction and
    // the inter stores; with fewer the registers this takes cost more than it saves (and
    // Q5_K's fifth-bit words, or F16's 32-register quarters, leave no room for it within 128
    // registers).  With 4+ tokens
    // the wave index is made scalar, which frees registers.
    constexpr bool pf = TM >= 4 && QT != PGMOE_Q5_K && QT != PGMOE_F16 && (MODE == kRoute || MODE == kDispatch);
    const int tid = threadIdx.x, lane = tid & 63, nth = blockDim.x, nw = nth >> 6;
    const int w = TM >= 4 ? __builtin_amdgcn_readfirstlane(tid >> 6) : tid >> 6;
    const int M = dp.M;
    const int nb = K >> 8, xrs = (K >> 6) * kXuH, srs = K >> 4;
    const bool pub = MODE == kRoute && blockIdx.x == 0 && blockIdx.y == 0;
    uint16_t* xs = (uint16_t*)smem;
    float* xss = (float*)(smem + (size_t)M * xrs * 2);
    PG_DECL;
    PG_MARK(1, 0);
    unsigned long long t_ready = 0;  // profiling builds: when wave 0 had its token's logits
    constexpr bool fused = MODE == kRoute;  // kRoute always carries the router (rt)
    const int rows = dp.E + (rt.extra_w ? 1 : 0);
    // 0. folded router: logits rows spread one per block where the grid allows (the host
    //    sizes the grid so that rows per block <= waves), producers in the lowest blocks
    const int bid = blockIdx.y * gridDim.x + blockIdx.x;
    const int rpb = (rows + gridDim.x * gridDim.y - 1) / (gridDim.x * gridDim.y);  // router rows per block
    //    With TM >= 4 tokens, TM / 2 waves share a row, two tokens each (the logits are per
    //    (token, row), so the split changes no value; a wave then keeps all of its chunk
    //    loads in flight at once).
    constexpr int TS = TM < 4 ? TM : 4, TH = TM / TS;  // router waves per row, tokens per wave
    for (int gi = w; fused && gi < rpb * TS; gi += nw) {  // (row, token group) gi; a block with
        const int e = bid * rpb + gi / TS, t0 = (gi % TS) * TH;  // fewer waves takes several
        if (e < rows && t0 < M) {
            constexpr int PF = TH <= 2 ? 4 : TH == 4 ? 2 : 1;
            float lg[TH][1];
            router_tile<TH, 1, PF>(x, rt.W, rt.extra_w, M, K, dp.E, t0, e, lane, lg);
            // every lane holds the totals: lane c stores copy c
#pragma unroll
            for (int t = 0; t < TH; ++t) {
                const int tt = t0 + t;
                if (tt < M) {
                    if (e < dp.E) {
                        float v = lg[t][0];
                        if (rt.bias) v = v + rt.bias[e];
                        if (lane < kRlogCopies)
                            put_logit((uint64_t*)dp.rlog + ((int64_t)lane * M + tt) * dp.E + e, v);
                    } else if (lane == 0) {
                        rt.extra_out[tt] = lg[t][0];
                    }
                }
            }
            PG_MARK(1, 3);
        }
    }
    // 1. token rows (and their 16-element sums) to registers, behind the logits of the
    //    wave's token (or, with the folded router, while it runs); the selection then
    //    waits for the logits only
    const int npc = M * (K >> 3);  // 16-byte pieces of the x rows
    const int nps = xsum ? M * (K >> 6) : 0;
    u32x4 xr[XR];
    floatx4 sr;
    auto issue = [&]() {
#pragma unroll
        for (int k = 0; k < XR; ++k) {
            const int i = tid + k * nth;
            if (i < npc) xr[k] = *(const u32x4*)(x + 8 * (int64_t)i);
        }
        if (tid < nps) sr = *(const floatx4*)(xsum + 4 * tid);
    };
    issue();
    // 2. rows to LDS (pieces past XR per thread are copied directly), before the routing:
    //    the copies overlap the wait for the logits
    const int kp = K >> 3;
#pragma unroll
    for (int k = 0; k < XR; ++k) {
        const int i = tid + k * nth;
        if (i < npc) *(u32x4*)(xs + (i / kp) * xrs + xpos_h(8 * (i % kp))) = xr[k];
    }
    for (int i = tid + XR * nth; i < npc; i += nth)
        *(u32x4*)(xs + (i / kp) * xrs + xpos_h(8 * (i % kp))) = *(const u32x4*)(x + 8 * (int64_t)i);
    if (tid < nps) *(floatx4*)(xss + 4 * tid) = sr;
    for (int i = tid + nth; i < nps; i += nth) *(floatx4*)(xss + 4 * i) = *(const floatx4*)(xsum + 4 * i);
    if (!xsum) {
        __syncthreads();
        for (int i = tid; i < M * srs; i += nth) {
            const uint16_t* pp = xs + (i / srs) * xrs + xpos_h(16 * (i % srs));
            float sm = 0.f;
#pragma unroll
            for (int k = 0; k < 16; ++k) sm += h2f(pp[k]);
            xss[i] = sm;
        }
    }
    PG_MARK(1, 1);
    if constexpr (fused) route_waves<RE>(dp, topk, R, pub, lane, w, nw, t_ready);
    __syncthreads();  // the rows, their sums and the routing
    PG_MARK(1, 6);
    if (rt.xsum_out && blockIdx.x == 0 && blockIdx.y == 0)
        for (int i = tid; i < M * srs; i += nth) rt.xsum_out[i] = xss[i];
    // 3. the block's active slots a = blockIdx.y, + gridDim.y, ...: expert and pairs (the
    //    same in every wave), items, then the SwiGLU rows
    const int r = lane & 15, p = lane >> 4;
    const int row = blockIdx.x * RB + r;  // < row_groups(N) * 64: padded tile rows are readable
    constexpr bool lin = MODE == kLinear;  // one matrix: item = super-block, every wave on it
    const int nit = lin ? nb : 2 * nb;
    auto slot_at = [&](int a) -> SlotInfo {
        if constexpr (MODE == kRoute && TM == 1)
            return pub ? slot_info<1>(R, M, a, lane, w == 0 && a == 0) : slot_info1(R, a, topk);
        else if constexpr (MODE == kRoute)
            return slot_info<TM>(R, M, a, lane, w == 0 && pub && a == 0);
        else
            return slot_plain<MODE>(dp, a, topk);
    };
    // One or two tokens (h8): 8-row blocks of half the waves (for C2 with one token, 768
    // blocks three a CU, where 384 16-row blocks left half the CUs with two, which ended
    // last).  Lane = (row r of 8, quarter p, matrix u = lane >> 5 (0 gate, 1 up)); wave w
    // takes super-blocks w, w + W, ... of both matrices, two at a time.  The inter rows'
    // sums go out as 8-row sums (isum [P][N/8]).
    constexpr bool h8 = MODE == kRoute && TM <= 2 && gu_rows8<QT>();
    // One row block per block (the grid covers the rows), or (RL) row blocks blockIdx.x,
    // + gridDim.x, ... per block: the two forms are kept apart so the first compiles as
    // it does without the second.
    if constexpr (!RL) {
        if constexpr (h8) {
            const int r8 = lane & 7, p8 = (lane >> 3) & 3, u8 = lane >> 5;
            const int row8 = blockIdx.x * 8 + r8;
            float* red8 = &red[0][0][0];  // [W][2][TM][8]
            for (int a = blockIdx.y;; a += gridDim.y) {
                const SlotInfo si = slot_at(a);
                if (si.e < 0) break;  // uniform over the block
                PG_MARK(1, 2);
                const uint8_t* mat = u8 ? ubase + (int64_t)si.e * ustride : gbase + (int64_t)si.e * gstride;
                float acc[TM];
#pragma unroll
                for (int t = 0; t < TM; ++t) acc[t] = 0.f;
                for (int j = w; j < nb; j += 2 * nw) {
                    const int j1 = j + nw;
                    Qtr<QT> l0, l1;
                    load_qtr<QT>(l0, mat, N, nb, row8, j, p8);
                    load_qtr<QT>(l1, mat, N, nb, row8, min(j1, nb - 1), p8);
                    gu_qtr<TM>(l0, j, p8, xs, xrs, xss, srs, si.toks, si.count, acc);
                    if (j1 < nb) gu_qtr<TM>(l1, j1, p8, xs, xrs, xss, srs, si.toks, si.count, acc);
                }
                PG_MARK(1, 4);
                // quarters -> rows (lanes r, r+8, r+16, r+24 of each half); waves in LDS
#pragma unroll
                for (int t = 0; t < TM; ++t) {
                    float v8 = acc[t];
                    v8 += xor_lane<8>(v8);
                    v8 += xor_lane<16>(v8);
                    if (p8 == 0) red8[((w * 2 + u8) * TM + t) * 8 + r8] = v8;
                }
                __syncthreads();
                // (one token: tid < 8, t = 0, the count is 1)
                if (TM == 1 ? tid < 8 : tid < TM * 8 && (tid >> 3) < si.count) {  // row rr of token t
                    const int t = TM == 1 ? 0 : tid >> 3, rr = TM == 1 ? tid : tid & 7;
                    float gs = 0.f, us = 0.f;
                    for (int ww = 0; ww < nw; ++ww) {
                        gs += red8[((ww * 2) * TM + t) * 8 + rr];
                        us += red8[((ww * 2 + 1) * TM + t) * 8 + rr];
                    }
                    const float v = gate_act(dp.act, gs) * us;
                    const int orow = blockIdx.x * 8 + rr;
                    const int64_t pr = si.p_begin + t;
                    if (orow < N) inter[pr * N + orow] = v;
                    if (isum) {
                        const float sm = group_sum<8>(v);
                        if (rr == 0 && orow < N) isum[pr * (N >> 3) + (orow >> 3)] = sm;
                    }
                }
                if (a + (int)gridDim.y >= si.n_act) break;  // the block's last slot
                __syncthreads();                           // red is rewritten by the next slot
            }
        }
        if constexpr (!h8) {
            auto mat_of = [&](int e) {  // wave w's matrix of expert e (odd waves: up)
                return (!lin && (w & 1)) ? ubase + (int64_t)e * ustride : gbase + (int64_t)e * gstride;
            };
            // items, two per wave at a time (both quarters' loads in flight together): pass `it`
            // holds items it and it + nw (the second clamped to a readable item past the end);
            // q0, q1: the prefetched pass
            Qtr<QT> q0, q1;
            auto load_pass = [&](const uint8_t* mat, int it) {
                const int it1 = min(it + nw, nit - 1);
                load_qtr<QT>(q0, mat, N, nb, row, lin ? it : it >> 1, p);
                load_qtr<QT>(q1, mat, N, nb, row, lin ? it1 : it1 >> 1, p);
            };
            int a = blockIdx.y;
            SlotInfo si = slot_at(a);
            if constexpr (pf)
                if (si.e >= 0 && w < nit) load_pass(mat_of(si.e), w);
            while (si.e >= 0) {  // uniform over the block
                PG_MARK(1, 2);
                if constexpr (MODE == kRoute && TM >= 2)
                    if (nw <= 8) slot_prio((si.n_act - 1 - a) / (int)gridDim.y);  // two blocks a CU
                const uint8_t* mat = mat_of(si.e);
                float acc[TM];
        #pragma unroll
                for (int t = 0; t < TM; ++t) acc[t] = 0.f;
                for (int it = w; it < nit; it += 2 * nw) {
                    const int it1 = it + nw;
                    const int j0 = lin ? it : it >> 1, j1 = lin ? min(it1, nit - 1) : min(it1, nit - 1) >> 1;
                    if constexpr (pf) {
                        if (it != w) load_pass(mat, it);
                        gu_qtr<TM>(q0, j0, p, xs, xrs, xss, srs, si.toks, si.count, acc);
                        if (it1 < nit) gu_qtr<TM>(q1, j1, p, xs, xrs, xss, srs, si.toks, si.count, acc);
                    } else {
                        Qtr<QT> l0, l1;
                        load_qtr<QT>(l0, mat, N, nb, row, j0, p);
                        load_qtr<QT>(l1, mat, N, nb, row, j1, p);
                        gu_qtr<TM>(l0, j0, p, xs, xrs, xss, srs, si.toks, si.count, acc);
                        if (it1 < nit) gu_qtr<TM>(l1, j1, p, xs, xrs, xss, srs, si.toks, si.count, acc);
                    }
                }
                PG_MARK(1, 4);
                SlotInfo sn;
                if constexpr (pf) {
                    sn = slot_at(a + gridDim.y);
                    if (sn.e >= 0 && w < nit) load_pass(mat_of(sn.e), w);
                }
                // quarters -> rows (lanes r, r+16, r+32, r+48); waves -> gate (even) / up (odd)
        #pragma unroll
                for (int t = 0; t < TM; ++t) acc[t] = kslot_sum<RB>(acc[t]);
                if (p == 0) {
        #pragma unroll
                    for (int t = 0; t < TM; ++t)
                        if (t < si.count) red[w][t][r] = acc[t];
                }
                __syncthreads();
                // thread (t, rr) = (tid / 16, tid % 16): whole 16-lane groups, so the 16-row sum
                // of a token is a shuffle reduction inside its group
                const int cnt = si.count, p0 = si.p_begin;
                if (lin && tid < cnt * RB) {  // every wave's partial of the one matrix, in wave order
                    const int t = tid >> 4, rr = tid & 15;
                    const int orow = blockIdx.x * RB + rr;
                    float v = red[0][t][rr];
                    for (int ww = 1; ww < nw; ++ww) v = v + red[ww][t][rr];
                    if (orow < N) {
                        if (dp.bias) v = v + dp.bias[orow];
                        if (dp.out_f16)
                            ((half_t*)inter)[(int64_t)(p0 + t) * N + orow] = (half_t)v;
                        else
                            inter[(int64_t)(p0 + t) * N + orow] = v;
                    }
                } else if (tid < cnt * RB) {
                    const int t = tid >> 4, rr = tid & 15;
                    float g = 0.f, u = 0.f;
                    for (int ww = 0; ww < nw; ww += 2) {
                        g += red[ww][t][rr];
                        u += red[ww + 1][t][rr];
                    }
                    const float v = gate_act(dp.act, g) * u;
                    const int orow = blockIdx.x * RB + rr;
                    if (orow < N) inter[(int64_t)(p0 + t) * N + orow] = v;
                    if (isum) {
                        const float sm = group_sum<16>(v);
                        if (rr == 0 && orow < N) isum[(int64_t)(p0 + t) * (N >> 4) + (orow >> 4)] = sm;
                    }
                }
                if (a + (int)gridDim.y >= si.n_act) break;  // the block's last slot
                __syncthreads();                           // red is rewritten by the next slot
                a += gridDim.y;
                if constexpr (pf)
                    si = sn;
                else
                    si = slot_at(a);
            }
        }
    } else {
        // Items (slot a, row block bx), slot-major, i = a * nrb + bx: block b takes items b,
        // b + G, b + 2G, ... (G = gridDim.x; the host launches one round of resident blocks,
        // gridDim.y = 1), so every block gets the same number of items to within one.
        const int nrb = (N + (h8 ? 7 : RB - 1)) / (h8 ? 8 : RB);
        const int n_items = nrb * slot_at(0).n_act;
        if constexpr (h8) {
            const int r8 = lane & 7, p8 = (lane >> 3) & 3, u8 = lane >> 5;
            float* red8 = &red[0][0][0];  // [W][2][TM][8]
            for (int i = blockIdx.x; i < n_items; i += gridDim.x) {
                const int a = i / nrb, bx = i - a * nrb;
                const int row8 = bx * 8 + r8;
                const SlotInfo si = slot_at(a);
                PG_MARK(1, 2);
                const uint8_t* mat = u8 ? ubase + (int64_t)si.e * ustride : gbase + (int64_t)si.e * gstride;
                float acc[TM];
#pragma unroll
                for (int t = 0; t < TM; ++t) acc[t] = 0.f;
                for (int j = w; j < nb; j += 2 * nw) {
                    const int j1 = j + nw;
                    Qtr<QT> l0, l1;
                    load_qtr<QT>(l0, mat, N, nb, row8, j, p8);
                    load_qtr<QT>(l1, mat, N, nb, row8, min(j1, nb - 1), p8);
                    gu_qtr<TM>(l0, j, p8, xs, xrs, xss, srs, si.toks, si.count, acc);
                    if (j1 < nb) gu_qtr<TM>(l1, j1, p8, xs, xrs, xss, srs, si.toks, si.count, acc);
                }
                PG_MARK(1, 4);
#pragma unroll
                for (int t = 0; t < TM; ++t) {
                    float v8 = acc[t];
                    v8 += xor_lane<8>(v8);
                    v8 += xor_lane<16>(v8);
                    if (p8 == 0) red8[((w * 2 + u8) * TM + t) * 8 + r8] = v8;
                }
                __syncthreads();
                // (one token: tid < 8, t = 0, the count is 1)
                if (TM == 1 ? tid < 8 : tid < TM * 8 && (tid >> 3) < si.count) {  // row rr of token t
                    const int t = TM == 1 ? 0 : tid >> 3, rr = TM == 1 ? tid : tid & 7;
                    float gs = 0.f, us = 0.f;
                    for (int ww = 0; ww < nw; ++ww) {
                        gs += red8[((ww * 2) * TM + t) * 8 + rr];
                        us += red8[((ww * 2 + 1) * TM + t) * 8 + rr];
                    }
                    const float v = gate_act(dp.act, gs) * us;
                    const int orow = bx * 8 + rr;
                    const int64_t pr = si.p_begin + t;
                    if (orow < N) inter[pr * N + orow] = v;
                    if (isum) {
                        const float sm = group_sum<8>(v);
                        if (rr == 0 && orow < N) isum[pr * (N >> 3) + (orow >> 3)] = sm;
                    }
                }
                if (i + (int)gridDim.x < n_items) __syncthreads();  // red is rewritten by the next item
            }
        }
        if constexpr (!h8) {
            auto mat_of = [&](int e) {  // wave w's matrix of expert e (odd waves: up)
                return (!lin && (w & 1)) ? ubase + (int64_t)e * ustride : gbase + (int64_t)e * gstride;
            };
            // passes of two items (matrix / super-block) a wave, as in the one-round form;
            // q0, q1: the prefetched pass of row rw
            Qtr<QT> q0, q1;
            auto load_pass = [&](const uint8_t* mat, int rw, int it) {
                const int it1 = min(it + nw, nit - 1);
                load_qtr<QT>(q0, mat, N, nb, rw, lin ? it : it >> 1, p);
                load_qtr<QT>(q1, mat, N, nb, rw, lin ? it1 : it1 >> 1, p);
            };
            int i = blockIdx.x;
            SlotInfo si;
            if (i < n_items) {
                si = slot_at(i / nrb);
                if constexpr (pf)
                    if (w < nit) load_pass(mat_of(si.e), (i % nrb) * RB + r, w);
            }
            constexpr bool one = MODE == kIdent || MODE == kLinear;  // one slot: item = row block
            while (i < n_items) {  // uniform over the block
                const int a = one ? 0 : i / nrb, bx = i - a * nrb;
                const int row = bx * RB + r;
                PG_MARK(1, 2);
                const uint8_t* mat = mat_of(si.e);
                float acc[TM];
#pragma unroll
                for (int t = 0; t < TM; ++t) acc[t] = 0.f;
                for (int it = w; it < nit; it += 2 * nw) {
                    const int it1 = it + nw;
                    const int j0 = lin ? it : it >> 1, j1 = lin ? min(it1, nit - 1) : min(it1, nit - 1) >> 1;
                    if constexpr (pf) {
                        if (it != w) load_pass(mat, row, it);
                        gu_qtr<TM>(q0, j0, p, xs, xrs, xss, srs, si.toks, si.count, acc);
                        if (it1 < nit) gu_qtr<TM>(q1, j1, p, xs, xrs, xss, srs, si.toks, si.count, acc);
                    } else {
                        Qtr<QT> l0, l1;
                        load_qtr<QT>(l0, mat, N, nb, row, j0, p);
                        load_qtr<QT>(l1, mat, N, nb, row, j1, p);
                        gu_qtr<TM>(l0, j0, p, xs, xrs, xss, srs, si.toks, si.count, acc);
                        if (it1 < nit) gu_qtr<TM>(l1, j1, p, xs, xrs, xss, srs, si.toks, si.count, acc);
                    }
                }
                PG_MARK(1, 4);
                // the next item's slot, and (pf) its first pass before this item's epilogue
                const int in = i + (int)gridDim.x;
                SlotInfo sn;
                if (in < n_items) {
                    sn = one ? si : slot_at(in / nrb);
                    if constexpr (pf)
                        if (w < nit) load_pass(mat_of(sn.e), (in % nrb) * RB + r, w);
                }
                // quarters -> rows (lanes r, r+16, r+32, r+48); waves -> gate (even) / up (odd)
#pragma unroll
                for (int t = 0; t < TM; ++t) acc[t] = kslot_sum<RB>(acc[t]);
                if (p == 0) {
#pragma unroll
                    for (int t = 0; t < TM; ++t)
                        if (t < si.count) red[w][t][r] = acc[t];
                }
                __syncthreads();
                const int cnt = si.count, p0 = si.p_begin;
                if (lin && tid < cnt * RB) {  // every wave's partial of the one matrix, in wave order
                    const int t = tid >> 4, rr = tid & 15;
                    const int orow = bx * RB + rr;
                    float v = red[0][t][rr];
                    for (int ww = 1; ww < nw; ++ww) v = v + red[ww][t][rr];
                    if (orow < N) {
                        if (dp.bias) v = v + dp.bias[orow];
                        if (dp.out_f16)
                            ((half_t*)inter)[(int64_t)(p0 + t) * N + orow] = (half_t)v;
                        else
                            inter[(int64_t)(p0 + t) * N + orow] = v;
                    }
                } else if (tid < cnt * RB) {
                    const int t = tid >> 4, rr = tid & 15;
                    float g = 0.f, u = 0.f;
                    for (int ww = 0; ww < nw; ww += 2) {
                        g += red[ww][t][rr];
                        u += red[ww + 1][t][rr];
                    }
                    const float v = gate_act(dp.act, g) * u;
                    const int orow = bx * RB + rr;
                    if (orow < N) inter[(int64_t)(p0 + t) * N + orow] = v;
                    if (isum) {
                        const float sm = group_sum<16>(v);
                        if (rr == 0 && orow < N) isum[(int64_t)(p0 + t) * (N >> 4) + (orow >> 4)] = sm;
                    }
                }
                if (in >= n_items) break;
                __syncthreads();  // red is rewritten by the next item
                i = in;
                si = sn;
            }
        }
    }
    // block (0, 0) publishes the routing last: its stores then stay off the block's own
    // critical path (a barrier would wait for them)
    if constexpr (fused)
        if (pub) publish_route(R, M, dp.E, topk, dp.desc, dp.flat);
    PG_MARK(1, 5);
    PG_SET(7, t_ready);
    PG_FLUSH(1);
}

// Fused down + combine.  Block = 8 output rows for all M tokens; lane = (row r = lane & 7,
// quarter p = (lane >> 3) & 3, u = lane >> 5); the items (active slot a, super-block j),
// it = a * (K/256) + j, go two per wave per pass (it = 2w + u, 2w + 2W + u, then + 4W),
// each lane accumulating w_(t,a) * (inter_(t,a) . d_a,row) per token; a fixed shuffle +
// LDS tree sums the lanes and waves.  out[t, row] = that sum (+ shared[t, row] *
// sigmoid(shared_logit[t])).  Inputs: the routing descriptor (P = M*K pairs) and the inter
// / isum rows in sorted pair order, all staged in LDS at once (the host uses this kernel
// only when they fit).  A null descriptor is the identity: one slot, matrix 0, pair p =
// token p with weight 1 (a dense FFN or the shared expert alone, P = M).  The item order
// depends only on the routing, so results are reproducible run to run.
// Dynamic LDS: xs [P][K/64][68] f32 | iss [P][K/16] f32.
template <int QT, int TM>
__device__ __forceinline__ void dc_item(const Qtr<QT>& q, bool valid, int it, int nb, int p, const float* xs, int xrs,
                                        const float* iss, int srs, const int* d_pb, const int* d_cnt,
                                        const int* d_tok, const float* d_w, float* acc) {
    if (!valid) return;
    const int a = it / nb, j = it % nb;
    const int pb = d_pb[a], cnt = min(d_cnt[a], TM);
    float part[TM];
#pragma unroll
    for (int c = 0; c < TM; ++c) part[c] = 0.f;
    dn_qtr<TM>(q, j, p, xs + pb * xrs, xrs, iss + pb * srs, srs, cnt, part);
#pragma unroll
    for (int c = 0; c < TM; ++c) {
        if (c < cnt) {
            const int tq = d_tok[pb + c];
            const float v = d_w[pb + c] * part[c];
#pragma unroll
            for (int t = 0; t < TM; ++t)
                if (t == tq) acc[t] += v;
        }
    }
}

// Lanes -> rows (lanes r + 8k), waves -> tokens' outputs: out[t, row] = the block's sum
// (+ shared[t, row] * sigmoid(shared_logit[t])).  red: [16][TM][8] LDS.
template <int TM>
__device__ __forceinline__ void dc_finish(float* acc, float (*red)[TM][8], int M, int N,
                                          const float* __restrict__ shared, const float* __restrict__ shared_logit,
                                          float* __restrict__ out, int bx) {
    constexpr int RB = 8;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, nth = blockDim.x, nw = nth >> 6;
#pragma unroll
    for (int t = 0; t < TM; ++t) acc[t] = kslot_sum<RB>(acc[t]);
    if (lane < RB) {
#pragma unroll
        for (int t = 0; t < TM; ++t) red[w][t][lane] = acc[t];
    }
    __syncthreads();
    for (int i = tid; i < M * RB; i += nth) {
        const int t = i / RB, rr = i % RB;
        float v = 0.f;
        for (int ww = 0; ww < nw; ++ww) v += red[ww][t][rr];
        const int orow = bx * RB + rr;
        if (orow < N) {
            if (shared) {
                const float g = shared_logit ? 1.0f / (1.0f + expf(-shared_logit[t])) : 1.0f;
                v += shared[(int64_t)t * N + orow] * g;
            }
            out[(int64_t)t * N + orow] = v;
        }
    }
}

template <int QT, int TM, bool RL>
__global__ __launch_bounds__(1024) void dec_dc_kernel(const uint8_t* __restrict__ dbase, int64_t dstride, int N,
                                                      int K, const float* __restrict__ inter,
                                                      const float* __restrict__ isum, int isum8,
                                                      const int32_t* __restrict__ desc,
                                                      int M, int P, const float* __restrict__ shared,
                                                      const float* __restrict__ shared_logit,
                                                      float* __restrict__ out, uint64_t* __restrict__ clear,
                                                      int n_clear) {
    constexpr int RB = 8;
    clear_words(clear, n_clear);  // the gate/up launch is done with them
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    __shared__ int d_pb[128], d_cnt[128], d_tok[128];
    __shared__ float d_w[128];
    __shared__ float red[16][TM][RB];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, nth = blockDim.x, nw = nth >> 6;
    const int nb = K >> 8, xrs = (K >> 6) * kXuF, srs = K >> 4;
    float* xs = (float*)smem;
    float* iss = xs + P * xrs;
    const int r = lane & 7, p = (lane >> 3) & 3, u = lane >> 5;
    // RL: row blocks bx = blockIdx.x, + gridDim.x, ..., all on the rows staged once
    const int nrb = (N + RB - 1) / RB;
    int bx = blockIdx.x, row = bx * RB + r;
    PG_DECL;
    PG_MARK(3, 0);
    // 0. the first IR pieces per thread of the inter rows, and of their sums, into
    //    registers before anything else: their addresses (sorted pairs 0 .. P-1) do not
    //    depend on the descriptor, so these loads overlap its round trip instead of
    //    following it (one token: every piece).  Measured on Qwen3 (same box, two A/B
    //    pairs): down + combine M = 1 7.3-7.4 -> 6.9 us, M = 2 10.2-10.3 -> 9.9-10.0 us,
    //    M = 4 16.2-16.6 -> 15.9 us.
    constexpr int IR = 2;
    const int kq = K >> 2;
    const int n_in = P * kq;                                  // 16-byte pieces of the inter rows
    const int n_is = isum8 ? P * (K >> 4) : P * (K >> 6);    // 8-byte / 16-byte pieces of the sums
    u32x4 ir[IR];
#pragma unroll
    for (int k = 0; k < IR; ++k)
        if (tid + k * nth < n_in) ir[k] = *(const u32x4*)(inter + 4 * (int64_t)(tid + k * nth));
    float s0 = 0.f, s1 = 0.f;       // isum8: the two 8-row sums of 16-row group tid
    u32x4 sr = {0u, 0u, 0u, 0u};   // else: 16-byte piece tid of the 16-row sums
    if (tid < n_is) {
        if (isum8) {
            s0 = isum[2 * tid];
            s1 = isum[2 * tid + 1];
        } else {
            sr = *(const u32x4*)(isum + 4 * tid);
        }
    }
    // 1. the experts of this lane's first two items straight from the descriptor, then
    //    their weights, then the pair table and the staging of the inter rows
    const bool ident = desc == nullptr;
    const int S = (ident ? 1 : desc[0]) * nb;  // items (active slot a, super-block j), it = a * nb + j
    int it0 = 2 * w + u, it1 = it0 + 2 * nw;
    int e0 = ident ? 0 : desc[kDescSlot + 4 * min(it0 / nb, 127)];
    int e1 = ident ? 0 : desc[kDescSlot + 4 * min(it1 / nb, 127)];
    Qtr<QT> q0, q1;
    load_qtr<QT>(q0, dbase + (int64_t)(it0 < S ? e0 : 0) * dstride, N, nb, row, it0 % nb, p);
    load_qtr<QT>(q1, dbase + (int64_t)(it1 < S ? e1 : 0) * dstride, N, nb, row, it1 % nb, p);
    for (int i = tid; i < P; i += nth) {
        d_pb[i] = ident ? 0 : desc[kDescSlot + 4 * i + 1];
        d_cnt[i] = ident ? P : desc[kDescSlot + 4 * i + 2];
        d_tok[i] = ident ? i : desc[kDescPair + 2 * i];
        d_w[i] = ident ? 1.0f : __builtin_bit_cast(float, desc[kDescPair + 2 * i + 1]);
    }
#pragma unroll
    for (int k = 0; k < IR; ++k) {
        const int i = tid + k * nth;
        if (i < n_in) *(u32x4*)(xs + (i / kq) * xrs + xpos_f(4 * (i % kq))) = ir[k];
    }
    if (n_in > IR * nth)
        copy_idx<4, u32x4>(
            n_in - IR * nth, tid, nth, [=](int i) { return (const u32x4*)(inter + 4 * (int64_t)(i + IR * nth)); },
            [=](int i) {
                const int j = i + IR * nth;
                return (u32x4*)(xs + (j / kq) * xrs + xpos_f(4 * (j % kq)));
            });
    if (isum8) {  // 8-row sums (the one-token gate/up): pairs of them
        if (tid < n_is) iss[tid] = s0 + s1;
        for (int i = tid + nth; i < n_is; i += nth) iss[i] = isum[2 * i] + isum[2 * i + 1];
    } else {
        if (tid < n_is) ((u32x4*)iss)[tid] = sr;
        if (n_is > nth)
            copy_words<2>((u32x4*)iss + nth, (const u32x4*)isum + nth, n_is - nth, tid, nth);
    }
    __syncthreads();
    PG_MARK(3, 1);
    // 2. items, two per lane per pass (row block after row block)
    for (;;) {
        float acc[TM];
#pragma unroll
        for (int t = 0; t < TM; ++t) acc[t] = 0.f;
        for (;;) {
            dc_item<QT, TM>(q0, it0 < S, it0, nb, p, xs, xrs, iss, srs, d_pb, d_cnt, d_tok, d_w, acc);
            dc_item<QT, TM>(q1, it1 < S, it1, nb, p, xs, xrs, iss, srs, d_pb, d_cnt, d_tok, d_w, acc);
            it0 += 4 * nw;
            it1 += 4 * nw;
            if (it0 - u >= S) break;  // wave-uniform (it0 - u is the pass's first item): no item left
            // (rare) more items than lanes: next pass
            e0 = ident ? 0 : desc[kDescSlot + 4 * min(it0 / nb, 127)];
            e1 = ident ? 0 : desc[kDescSlot + 4 * min(it1 / nb, 127)];
            load_qtr<QT>(q0, dbase + (int64_t)(it0 < S ? e0 : 0) * dstride, N, nb, row, it0 % nb, p);
            load_qtr<QT>(q1, dbase + (int64_t)(it1 < S ? e1 : 0) * dstride, N, nb, row, it1 % nb, p);
        }
        PG_MARK(3, 2);
        // the next row block's first pass goes out before this one's sums are formed
        const int bn = bx + (int)gridDim.x;
        if (RL && bn < nrb) {
            it0 = 2 * w + u;
            it1 = it0 + 2 * nw;
            e0 = ident ? 0 : desc[kDescSlot + 4 * min(it0 / nb, 127)];
            e1 = ident ? 0 : desc[kDescSlot + 4 * min(it1 / nb, 127)];
            const int rown = bn * RB + r;
            load_qtr<QT>(q0, dbase + (int64_t)(it0 < S ? e0 : 0) * dstride, N, nb, rown, it0 % nb, p);
            load_qtr<QT>(q1, dbase + (int64_t)(it1 < S ? e1 : 0) * dstride, N, nb, rown, it1 % nb, p);
        }
        dc_finish<TM>(acc, red, M, N, shared, shared_logit, out, bx);
        if (!RL || bn >= nrb) break;
        bx = bn;
        row = bx * RB + r;
        __syncthreads();  // red is rewritten by the next row block
    }
    PG_MARK(3, 4);
    PG_FLUSH(3);
}

// Fused down + combine when the inter / isum rows do not fit in LDS at once: the same
// block, lanes and sums as dec_dc_kernel, with the rows staged one chunk of JC super-block
// columns at a time (the host picks the most that fit).  In a chunk of JCc columns
// starting at super-block j0, the items (active slot a, super-block j0 + jj),
// it = a * JCc + jj, go two per wave per pass as in dec_dc_kernel; the first pass of the
// next chunk is loaded before that chunk is staged.  Each lane's item order depends only
// on the routing and JC, so results are reproducible run to run.
// Dynamic LDS: xs [P][JC*4][68] f32 | iss [P][JC*16] f32.
template <int QT, int TM>
__global__ __launch_bounds__(1024) void dec_dc_chunk_kernel(const uint8_t* __restrict__ dbase, int64_t dstride,
                                                            int N, int K, int JC, const float* __restrict__ inter,
                                                            const float* __restrict__ isum, int isum8,
                                                            const int32_t* __restrict__ desc, int M, int P,
                                                            const float* __restrict__ shared,
                                                            const float* __restrict__ shared_logit,
                                                            float* __restrict__ out, uint64_t* __restrict__ clear,
                                                            int n_clear) {
    constexpr int RB = 8;
    clear_words(clear, n_clear);  // the gate/up launch is done with them
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    __shared__ int d_pb[128], d_cnt[128], d_tok[128];
    __shared__ float d_w[128];
    __shared__ float red[16][TM][RB];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, nth = blockDim.x, nw = nth >> 6;
    const int nb = K >> 8, xrs = JC * 4 * kXuF, srs = JC * 16;
    float* xs = (float*)smem;
    float* iss = xs + P * xrs;
    const int r = lane & 7, p = (lane >> 3) & 3, u = lane >> 5;
    const int row = blockIdx.x * RB + r;
    // 1. the experts of this lane's first two items, their weights, then the pair table
    //    (prefetching the first chunk's rows ahead of the descriptor, as dec_dc_kernel does,
    //    spilled here: this kernel's registers are at the 128 bound)
    const bool ident = desc == nullptr;
    const int A = ident ? 1 : desc[0];  // active slots
    int j0 = 0, JCc = JC < nb ? JC : nb;
    Qtr<QT> q0, q1;
    auto load_pass = [&](int it0, int it1) {  // items it0, it1 of the current chunk (any)
        const int a0 = it0 / JCc, a1 = it1 / JCc;
        const int e0 = ident ? 0 : desc[kDescSlot + 4 * min(a0, 127)];  // both slots first
        const int e1 = ident ? 0 : desc[kDescSlot + 4 * min(a1, 127)];
        load_qtr<QT>(q0, dbase + (int64_t)(a0 < A ? e0 : 0) * dstride, N, nb, row, j0 + it0 % JCc, p);
        load_qtr<QT>(q1, dbase + (int64_t)(a1 < A ? e1 : 0) * dstride, N, nb, row, j0 + it1 % JCc, p);
    };
    int it0 = 2 * w + u, it1 = it0 + 2 * nw;
    load_pass(it0, it1);
    for (int i = tid; i < P; i += nth) {
        d_pb[i] = ident ? 0 : desc[kDescSlot + 4 * i + 1];
        d_cnt[i] = ident ? P : desc[kDescSlot + 4 * i + 2];
        d_tok[i] = ident ? i : desc[kDescPair + 2 * i];
        d_w[i] = ident ? 1.0f : __builtin_bit_cast(float, desc[kDescPair + 2 * i + 1]);
    }
    float acc[TM];
#pragma unroll
    for (int t = 0; t < TM; ++t) acc[t] = 0.f;
    for (;;) {
        {  // stage the chunk: columns [256 j0, 256 (j0 + JCc)) of every pair's rows and sums
            const int kq = JCc * 64, sq = JCc * 4;  // 16-byte words of a row's chunk, of its sums
            const float* src = inter + 256 * j0;
            copy_idx<4, u32x4>(
                P * kq, tid, nth, [=](int i) { return (const u32x4*)(src + (int64_t)(i / kq) * K + 4 * (i % kq)); },
                [=](int i) { return (u32x4*)(xs + (i / kq) * xrs + xpos_f(4 * (i % kq))); });
            if (isum8) {  // 8-row sums (the one-token gate/up): pairs of them
                const int sc = JCc * 16;
                for (int i = tid; i < P * sc; i += nth) {
                    const int pr = i / sc, c = i - pr * sc;
                    const float* s8 = isum + (int64_t)pr * (K >> 3) + 32 * j0 + 2 * c;
                    iss[pr * srs + c] = s8[0] + s8[1];
                }
            } else {
                const float* ssrc = isum + 16 * j0;
                copy_idx<2, u32x4>(
                    P * sq, tid, nth,
                    [=](int i) { return (const u32x4*)(ssrc + (int64_t)(i / sq) * (K >> 4) + 4 * (i % sq)); },
                    [=](int i) { return (u32x4*)(iss + (i / sq) * srs + 4 * (i % sq)); });
            }
        }
        __syncthreads();
        // 2. the chunk's items, two per lane per pass
        const int S = A * JCc;
        for (;;) {
            dc_item<QT, TM>(q0, it0 < S, it0, JCc, p, xs, xrs, iss, srs, d_pb, d_cnt, d_tok, d_w, acc);
            dc_item<QT, TM>(q1, it1 < S, it1, JCc, p, xs, xrs, iss, srs, d_pb, d_cnt, d_tok, d_w, acc);
            it0 += 4 * nw;
            it1 += 4 * nw;
            if (it0 - u >= S) break;  // wave-uniform (it0 - u is the pass's first item): no item left
            load_pass(it0, it1);      // (rare) more items than lanes: next pass
        }
        if (j0 + JCc >= nb) break;
        // the next chunk's first pass, then (once every wave is done with this chunk) its rows
        j0 += JCc;
        JCc = JC < nb - j0 ? JC : nb - j0;
        it0 = 2 * w + u;
        it1 = it0 + 2 * nw;
        load_pass(it0, it1);
        __syncthreads();
    }
    // 3. lanes and waves -> the tokens' outputs
    dc_finish<TM>(acc, red, M, N, shared, shared_logit, out, blockIdx.x);
}

// Per-expert down GEMV: partial[p, row] = w[perm[p]] * (inter_p . d_row) for the pairs of
// one active expert (stage API; kIdent: the shared expert, weight 1, partial = its output).
// The K loop steps JW = KS*W super-blocks at a time; each step stages the matching
// column chunk of the TM inter rows of the chunk in LDS (fp32), and the next step's
// weights are loaded before the current step is computed.  isum (optional input):
// 16-element sums of inter rows [P][K/16]; otherwise computed from the staged chunk.
// LDS: xs [TM][JW*256] f32 | iss [TM][JW*16] f32 | red [W][TM][RB] f32.
template <int QT, int RB, int W, int TM>
__global__ __launch_bounds__(W * 64) void dec_down_kernel(const uint8_t* __restrict__ dbase, int64_t dstride, int N,
                                                          int K, const float* __restrict__ inter,
                                                          const float* __restrict__ isum_in, DecDisp dp,
                                                          const float* __restrict__ topk_w,
                                                          float* __restrict__ partial) {
    constexpr int KS = 64 / RB;
    constexpr int JW = KS * W;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int a = blockIdx.y;
    const int MODE = dp.mode;
    int e, p_begin, p_end;
    if (MODE == kIdent) {
        e = 0;
        p_begin = 0;
        p_end = dp.M;
    } else {
        if (a >= *dp.n_active) return;
        e = dp.active[a];
        p_begin = dp.offsets[e];
        p_end = dp.offsets[e + 1];
    }
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int r = lane % RB, ks = lane / RB;
    const int row = blockIdx.x * RB + r;
    const int nb = K >> 8;
    const int j0 = ks + KS * w;  // this lane's super-block within a step
    float* xs = (float*)smem;
    float* iss = xs + TM * JW * 256;
    float* red = iss + TM * JW * 16;
    const uint8_t* dm = dbase + (int64_t)e * dstride;
    for (int p0 = p_begin; p0 < p_end; p0 += TM) {
        const int me = min(TM, p_end - p0);
        float acc[TM];
#pragma unroll
        for (int t = 0; t < TM; ++t) acc[t] = 0.f;
        Raw<QT> rw;
        if (j0 < nb) load_raw<QT>(rw, dm, N, nb, row, j0);
        for (int jb = 0; jb < nb; jb += JW) {
            const int nbj = min(JW, nb - jb);
            __syncthreads();  // the previous step's LDS reads are done
            {
                const int n4 = nbj * 64;  // 16-byte words of one row chunk
                copy_idx<8, uint4>(
                    me * n4, tid, W * 64,
                    [=](int i) { return (const uint4*)(inter + (int64_t)(p0 + i / n4) * K + 256 * jb + 4 * (i % n4)); },
                    [=](int i) { return (uint4*)(xs + (i / n4) * (JW * 256) + 4 * (i % n4)); });
                if (isum_in) {
                    for (int i = tid; i < me * nbj * 16; i += W * 64) {
                        const int t = i / (nbj * 16), c = i % (nbj * 16);
                        iss[t * (JW * 16) + c] = isum_in[(int64_t)(p0 + t) * (K >> 4) + 16 * jb + c];
                    }
                }
            }
            __syncthreads();
            if (!isum_in) {
                for (int i = tid; i < me * nbj * 16; i += W * 64) {
                    const int t = i / (nbj * 16), c = i % (nbj * 16);
                    const float* p = xs + t * (JW * 256) + 16 * c;
                    float sm = 0.f;
#pragma unroll
                    for (int k = 0; k < 16; ++k) sm += p[k];
                    iss[t * (JW * 16) + c] = sm;
                }
                __syncthreads();
            }
            const int j = jb + j0;
            Raw<QT> rn;
            if (j + JW < nb) load_raw<QT>(rn, dm, N, nb, row, j + JW);
            if (j < nb) dn_compute<TM>(rw, xs + 256 * j0, iss + 16 * j0, JW * 256, me, acc);
            rw = rn;
        }
#pragma unroll
        for (int t = 0; t < TM; ++t) acc[t] = kslot_sum<RB>(acc[t]);
        if (ks == 0) {
#pragma unroll
            for (int t = 0; t < TM; ++t)
                if (t < me) red[(w * TM + t) * RB + r] = acc[t];
        }
        __syncthreads();
        for (int i = tid; i < me * RB; i += W * 64) {
            const int t = i / RB, rr = i % RB;
            float v = 0.f;
#pragma unroll
            for (int ww = 0; ww < W; ++ww) v += red[(ww * TM + t) * RB + rr];
            const int orow = blockIdx.x * RB + rr;
            if (orow < N) partial[(int64_t)(p0 + t) * N + orow] = MODE == kIdent ? v : topk_w[dp.perm[p0 + t]] * v;
        }
    }
}

// ============================================================================ launch plumbing
// Per-expert down (stage API / shared expert): block shapes (rows per block RB, waves
// W <= 4 so every wave may use up to 512 VGPRs): one super-block per lane when nb equals
// KS * W for one of them, else (16, 4) with a K loop.
struct DecShape {
    int RB, W;
};

inline DecShape pick_shape(int nb) {
    static const DecShape menu[] = {{16, 1}, {16, 2}, {16, 4}, {32, 1}, {64, 1}, {64, 3}};
    for (const DecShape& s : menu)
        if ((64 / s.RB) * s.W == nb) return s;
    return {16, 4};
}

// Down: per K step, t rows of JW super-blocks staged as fp32 (1088 bytes a super-block
// with its sums) plus the [W][t][RB] partials; t halves while that exceeds 60 KB.
inline size_t down_lds_bytes(int t, int RB, int W) { return (size_t)t * (64 / RB) * W * 1088 + (size_t)W * t * RB * 4; }
inline int down_tile_tokens(int M, const DecShape& sp) {
    int t = M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8;
    while (t > 1 && down_lds_bytes(t, sp.RB, sp.W) > 60 * 1024) t >>= 1;
    return t;
}

// Token bound of the routed kernels: the smallest of 1, 2, 4, 8 that is >= M.
inline int tm_bucket(int M) { return M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8; }

// Gate/up: waves = K/256 rounded up to even (at most two items per wave up to 16
// super-blocks), 2..16.
inline int gu_waves(int nb) {
    const int w = nb + (nb & 1);
    return w < 2 ? 2 : w > 16 ? 16 : w;
}
inline size_t gu_lds_bytes(int M, int K) { return (size_t)M * (K / 64) * kXuH * 2 + (size_t)M * (K / 16) * 4; }
// Gate/up grid rows: active slots per block column, at most 16 (blocks then take several
// slots, routing and staging the tokens once).
inline int gu_slot_blocks(int max_active) { return max_active < 16 ? max_active : 16; }
// Fused down + combine: two items per wave per pass, so (items + 1) / 2 waves up to 16.
inline int dc_waves(int items) {
    const int w = (items + 1) / 2;
    return w < 1 ? 1 : w > 16 ? 16 : w;
}
// Its staging: JC super-block columns of P inter rows (padded units) and their sums.
inline size_t dc_lds_bytes(int P, int JC) { return (size_t)P * JC * (4 * kXuF * 4 + 16 * 4); }
size_t dec_lds_limit();
// Columns per staging chunk of the fused down + combine: all K / 256 when the rows fit
// (dec_dc_kernel); else, for rows of at most 32 super-blocks, the most that fit
// (dec_dc_chunk_kernel); 0: neither (the per-expert down and combine kernels instead,
// measured faster for longer rows: with K = 14336 and few experts they stream each
// expert's rows with more blocks).
inline int dc_chunk(int P, int K) {
    const int nb = K >> 8;
    const int jc = (int)(dec_lds_limit() / dc_lds_bytes(P, 1));
    return jc >= nb ? nb : nb <= 32 ? jc : 0;
}

// Dynamic LDS a block of the current device may take beside the kernels' static arrays.
// Of gy slot rows of gx blocks each, how many fit in one round of resident blocks of
// `kernel` on the current device (at least 1): a grid past that waits a whole block
// duration for its last round.
int resident_rows(const void* kernel, int threads, size_t lds, int gx, int gy);
// Blocks of `kernel` resident on the current device at once (at least 1).
int resident_blocks(const void* kernel, int threads, size_t lds);

template <int QT, int TM>
inline void gu_launch(const Mats& g, const Mats& u, const uint16_t* x, const float* xsum, int topk, const DecDisp& dp,
                      const RouterIn& rt, int max_active, float* inter, float* isum, hipStream_t st) {
    // a linear has half the items of a gate/up pair: two per wave as well
    // the one-token routed launch: 8-row blocks, ceil(K/512) waves (both matrices a wave)
    const bool h8 = dp.mode == kRoute && TM <= 2 && gu_rows8<QT>();
    const int nbk = g.K >> 8, W8 = (nbk + 1) / 2;
    const int W = h8 ? (W8 > 16 ? 16 : W8) : gu_waves(dp.mode == kLinear ? (nbk + 1) / 2 : nbk);
    int gx = div_up(g.N, h8 ? 8 : 16);
    const int gy = gu_slot_blocks(max_active);
    // every router row needs a wave (TM / 2 with 4+ tokens)
    const int rrows = dp.mode == kRoute ? (dp.E + (rt.extra_w ? 1 : 0)) * (TM < 4 ? TM : 4) : 0;
    const size_t sh = gu_lds_bytes(dp.M, g.K);
    // slot rows: as many as fit in one round of resident blocks (blocks loop over the rest)
#define PG_GU(MODE, RE)                                                                                         \
    do {                                                                                                        \
        int gyr = resident_rows((const void*)dec_gu_kernel<QT, TM, MODE, RE, false>, 64 * W, sh, gx, gy);       \
        const int res = resident_blocks((const void*)dec_gu_kernel<QT, TM, MODE, RE, true>, 64 * W, sh);        \
        /* not two slot rows in one round: one round of blocks taking (slot, row block) items */               \
        const int gxr = gx * gy < res ? gx * gy : res;                                                          \
        const bool rl = gyr == 1 && (gy > 1 || gx > res) && gxr * W >= rrows; /* a wave per router row */      \
        if (rl) gx = gxr;                                                                                       \
        const int gmin = rrows ? div_up(rrows, gx * W) : 1;                                                     \
        gyr = rl ? 1 : gyr > gmin ? gyr : gmin;                                                                 \
        if (rl)                                                                                                 \
            PG_LAUNCH((dec_gu_kernel<QT, TM, MODE, RE, true>), dim3(gx, gyr), dim3(64 * W), sh, st, g.base,     \
                      u.base, g.stride, u.stride, g.N, g.K, x, xsum, topk, dp, rt, inter, isum);                \
        else                                                                                                    \
            PG_LAUNCH((dec_gu_kernel<QT, TM, MODE, RE, false>), dim3(gx, gyr), dim3(64 * W), sh, st, g.base,    \
                      u.base, g.stride, u.stride, g.N, g.K, x, xsum, topk, dp, rt, inter, isum);                \
    } while (0)
    if (dp.mode == kRoute) {
        if (dp.E <= 128)
            PG_GU(kRoute, 2);
        else
            PG_GU(kRoute, 8);
    } else if (dp.mode == kIdent) {
        PG_GU(kIdent, 1);
    } else if (dp.mode == kLinear) {
        PG_GU(kLinear, 1);
    } else {
        PG_GU(kDispatch, 1);
    }
#undef PG_GU
}

template <int QT, int RB, int W, int TM>
inline void dn_launch(const Mats& d, const float* inter, const float* isum, const DecDisp& dp, int max_active,
                      const float* topk_w, float* partial, hipStream_t st) {
    const size_t sh = down_lds_bytes(TM, RB, W);
    PG_LAUNCH((dec_down_kernel<QT, RB, W, TM>), dim3(div_up(d.N, RB), max_active), dim3(64 * W), sh,
                       st, d.base, d.stride, d.N, d.K, inter, isum, dp, topk_w, partial);
}

template <int QT, int TM>
inline void dc_launch(const Mats& d, const float* inter, const float* isum, int isum8, const int32_t* desc, int M,
                      int P, int max_active, const float* shared, const float* shared_logit, float* out,
                      uint64_t* clear, int n_clear, hipStream_t st) {
    const int nb = d.K >> 8, JC = dc_chunk(P, d.K);
    const int W = dc_waves(max_active * JC);  // items of a chunk
    if (JC >= nb) {
        // two or more row blocks per resident block: one round, each block looping over rows
        // on the rows it staged once (fewer: the loop's registers cost more than it saves)
        const int rb = div_up(d.N, 8);
        const int res = resident_blocks((const void*)dec_dc_kernel<QT, TM, true>, 64 * W, dc_lds_bytes(P, nb));
        if (rb >= 2 * res)
            PG_LAUNCH((dec_dc_kernel<QT, TM, true>), dim3(res), dim3(64 * W), dc_lds_bytes(P, nb), st, d.base,
                      d.stride, d.N, d.K, inter, isum, isum8, desc, M, P, shared, shared_logit, out, clear, n_clear);
        else
            PG_LAUNCH((dec_dc_kernel<QT, TM, false>), dim3(rb), dim3(64 * W), dc_lds_bytes(P, nb), st, d.base,
                      d.stride, d.N, d.K, inter, isum, isum8, desc, M, P, shared, shared_logit, out, clear, n_clear);
    }
    else
        PG_LAUNCH((dec_dc_chunk_kernel<QT, TM>), dim3(div_up(d.N, 8)), dim3(64 * W), dc_lds_bytes(P, JC), st,
                  d.base, d.stride, d.N, d.K, JC, inter, isum, isum8, desc, M, P, shared, shared_logit, out, clear,
                  n_clear);
}

#define PG_TM(F, QT, RB, W, ...)                   \
    switch (TM) {                                 \
    case 1: F<QT, RB, W, 1>(__VA_ARGS__); break;  \
    case 2: F<QT, RB, W, 2>(__VA_ARGS__); break;  \
    case 4: F<QT, RB, W, 4>(__VA_ARGS__); break;  \
    default: F<QT, RB, W, 8>(__VA_ARGS__); break; \
    }

#define PG_TM2(F, QT, ...)                   \
    switch (tm_bucket(M)) {                  \
    case 1: F<QT, 1>(__VA_ARGS__); break;    \
    case 2: F<QT, 2>(__VA_ARGS__); break;    \
    case 4: F<QT, 4>(__VA_ARGS__); break;    \
    default: F<QT, 8>(__VA_ARGS__); break;   \
    }

// Block shapes for the per-expert down kernel: the shapes pick_shape returns.
#define PG_SHAPES(F, QT, ...)                                  \
    switch (sp.RB * 16 + sp.W) {                               \
    case 16 * 16 + 1: PG_TM(F, QT, 16, 1, __VA_ARGS__); break; \
    case 16 * 16 + 2: PG_TM(F, QT, 16, 2, __VA_ARGS__); break; \
    case 32 * 16 + 1: PG_TM(F, QT, 32, 1, __VA_ARGS__); break; \
    case 64 * 16 + 1: PG_TM(F, QT, 64, 1, __VA_ARGS__); break; \
    case 64 * 16 + 3: PG_TM(F, QT, 64, 3, __VA_ARGS__); break; \
    default: PG_TM(F, QT, 16, 4, __VA_ARGS__); break;          \
    }

// Per-qtype launchers (instantiated by decode_inst.hip, one object per format and stage).
template <int QT>
int dec_gateup_q(const Mats& g, const Mats& u, const uint16_t* x, const float* xsum, int topk, int M,
                 const DecDisp& dp, const RouterIn& rt, int max_active, float* inter, float* isum, hipStream_t st);
template <int QT>
int dec_down_q(const Mats& d, const float* inter, const float* isum, int M, int mode, const DecDisp& dp,
               int max_active, const float* topk_w, float* partial, hipStream_t st);
template <int QT>
int dec_down_combine_q(const Mats& d, const float* inter, const float* isum, int isum8, const int32_t* desc, int M,
                       int P, int max_active, const float* shared, const float* shared_logit, float* out,
                       uint64_t* clear, int n_clear, hipStream_t st);

#define PG_DEFINE_DECODE_GATEUP(QT)                                                                                  \
    template <>                                                                                                     \
    int dec_gateup_q<QT>(const Mats& g, const Mats& u, const uint16_t* x, const float* xsum, int topk, int M,      \
                         const DecDisp& dp, const RouterIn& rt, int max_active, float* inter, float* isum,          \
                         hipStream_t st) {                                                                          \
        if (M < 1 || M > kDecTM) return fail(PGMOE_E_UNSUPPORTED, "decode gate/up: 1..%d tokens (got %d)", kDecTM, M); \
        if (gu_lds_bytes(M, g.K) > dec_lds_limit())                                           \
            return fail(PGMOE_E_UNSUPPORTED, "decode gate/up: %d tokens of %d inputs exceed LDS", M, g.K);          \
        PG_TM2(gu_launch, QT, g, u, x, xsum, topk, dp, rt, max_active, inter, isum, st);                             \
        return check_launch("dec_gateup");                                                                          \
    }

#define PG_DEFINE_DECODE_DOWN(QT)                                                                                    \
    template <>                                                                                                     \
    int dec_down_q<QT>(const Mats& d, const float* inter, const float* isum, int M, int mode, const DecDisp& dp,   \
                       int max_active, const float* topk_w, float* partial, hipStream_t st) {                       \
        const DecShape sp = pick_shape(d.K >> 8);                                                                   \
        const int TM = down_tile_tokens(M, sp);                                                                     \
        PG_SHAPES(dn_launch, QT, d, inter, isum, dp, max_active, topk_w, partial, st);                   \
        return check_launch("dec_down");                                                                            \
    }

#define PG_DEFINE_DECODE_DOWN_COMBINE(QT)                                                                            \
    template <>                                                                                                     \
    int dec_down_combine_q<QT>(const Mats& d, const float* inter, const float* isum, int isum8,                    \
                               const int32_t* desc, int M, int P, int max_active, const float* shared,              \
                               const float* shared_logit, float* out, uint64_t* clear, int n_clear,                 \
                               hipStream_t st) {                                                                    \
        if (P > 128 || dc_chunk(P, d.K) < 1)                                                                        \
            return fail(PGMOE_E_UNSUPPORTED, "decode down + combine: %d pairs of %d inputs exceed LDS", P, d.K);    \
        PG_TM2(dc_launch, QT, d, inter, isum, isum8, desc, M, P, max_active, shared, shared_logit, out, clear,   \
               n_clear, st);                                                                                        \
        return check_launch("dec_down_combine");                                                                    \
    }

}  // namespace pgmoe
