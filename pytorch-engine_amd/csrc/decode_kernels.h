// Decode path (M <= 8 tokens), three launches per layer (five with a shared expert), no
// host sync:
//   router logits (router.hip, fixed order, also the 16-element sums of x) ->
//   gate/up + SwiGLU, each block routing the tokens itself from the logits ->
//   down + combine fused (every block owns a few output rows across all active experts).
// Per-expert kernels: a block owns RB rows of one active expert; lane = (row, K-slice), so
// each lane streams whole 256-weight super-blocks of one row from the 64-row tile
// layout (coalesced 16-byte chunks), activations are wave-uniform (LDS / broadcast),
// and partial sums meet through a few shuffles and one LDS pass.  Weight loads are
// issued before the activation staging so both latencies overlap.
//   gate/up: fp16 magic-number dequant (1024 + code) feeding v_dot2_f32_f16
//   down   : fp32 FMA on the fp32 SwiGLU output
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

// K-quant 6-bit (scale, min) of sub-block s from the 12 scale bytes (words D, Mb, MD).
__device__ __forceinline__ void kscale(uint32_t D, uint32_t Mb, uint32_t MD, int s, int& sc, int& mn) {
    if (s < 4) {
        sc = (D >> (8 * s)) & 63;
        mn = (Mb >> (8 * s)) & 63;
    } else {
        const int j = s - 4;
        const uint32_t md = (MD >> (8 * j)) & 0xff;
        sc = (md & 0x0f) | (((D >> (8 * j)) >> 2) & 0x30);
        mn = (md >> 4) | (((Mb >> (8 * j)) >> 2) & 0x30);
    }
}

// Q6_K 6-bit codes (0..63) of elements 128h + 32s + 4k + 0..3, one per byte.
__device__ __forceinline__ uint32_t q6_word(uint32_t qlA, uint32_t qlB, uint32_t qh, int s) {
    const uint32_t lo = (s & 1 ? qlB : qlA) >> (4 * (s >> 1));
    const uint32_t hi = s == 0 ? qh << 4 : s == 1 ? qh << 2 : s == 2 ? qh : qh >> 2;
    return (lo & 0x0f0f0f0fu) | (hi & 0x30303030u);
}

// ============================================================================ tiles
// Raw 16-byte chunks of one (row, 256-weight super-block), loaded ahead of their use.
template <int QT> struct Raw;
template <> struct Raw<PGMOE_Q4_K> { uint4 c[9]; };
template <> struct Raw<PGMOE_Q6_K> { uint4 c[13]; uint32_t d; };
template <> struct Raw<PGMOE_Q8_0> { uint4 c[17]; };

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

// ---------------------------------------------------------------- gate/up (fp16 dot2)
// acc[t] += x_t . w(row, block) for t < me (TM a compile-time bound); xs = LDS fp16 x rows
// (stride K) offset to the block; xsum = 16-element sums of those rows (stride K/16)
// offset to the block.
__device__ __forceinline__ uint4 ld128(const uint16_t* p) { return *(const uint4*)p; }

template <int TM>
__device__ __forceinline__ void gu_compute(const Raw<PGMOE_Q4_K>& r, const uint16_t* xs, const float* xsum, int K,
                                           int me, float* acc) {
    const uint4 h = r.c[0];
    const float dd = lo_half(h.x), dm = hi_half(h.x);
#pragma unroll
    for (int c2 = 0; c2 < 4; ++c2) {  // qs bytes 32c2..32c2+31: sub-blocks 2c2 (low), 2c2+1 (high)
        int s0, m0, s1, m1;
        kscale(h.y, h.z, h.w, 2 * c2, s0, m0);
        kscale(h.y, h.z, h.w, 2 * c2 + 1, s1, m1);
        const float a0 = dd * (float)s0, b0 = dm * (float)m0 + 1024.0f * a0;
        const float a1 = dd * (float)s1, b1 = dm * (float)m1 + 1024.0f * a1;
        const uint4 qa = r.c[1 + 2 * c2], qb = r.c[2 + 2 * c2];
        const uint32_t w8[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
        uint32_t lo[16], hi[16];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t l = w8[k] & 0x0f0f0f0fu, hh = (w8[k] >> 4) & 0x0f0f0f0fu;
            lo[2 * k] = magic2(l, kSel01);
            lo[2 * k + 1] = magic2(l, kSel23);
            hi[2 * k] = magic2(hh, kSel01);
            hi[2 * k + 1] = magic2(hh, kSel23);
        }
#pragma unroll
        for (int t = 0; t < TM; ++t) {
            if (t < me) {
                const uint16_t* xr = xs + t * K + 64 * c2;
                uint32_t xl[16], xh[16];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const uint4 v = ld128(xr + 8 * q), u = ld128(xr + 32 + 8 * q);
                    xl[4 * q] = v.x; xl[4 * q + 1] = v.y; xl[4 * q + 2] = v.z; xl[4 * q + 3] = v.w;
                    xh[4 * q] = u.x; xh[4 * q + 1] = u.y; xh[4 * q + 2] = u.z; xh[4 * q + 3] = u.w;
                }
                float tl = 0.f, th = 0.f;
#pragma unroll
                for (int k = 0; k < 16; ++k) {
                    tl = dot2(lo[k], xl[k], tl);
                    th = dot2(hi[k], xh[k], th);
                }
                const float* sx = xsum + t * (K >> 4) + 4 * c2;
                acc[t] += a0 * tl - b0 * (sx[0] + sx[1]) + a1 * th - b1 * (sx[2] + sx[3]);
            }
        }
    }
}

// Q8_0 code q in [-128, 127]: byte ^ 0x80 = q + 128, so the fp16 value is 1152 + q.
template <int TM>
__device__ __forceinline__ void gu_compute(const Raw<PGMOE_Q8_0>& r, const uint16_t* xs, const float* xsum, int K,
                                           int me, float* acc) {
    const uint32_t dw[4] = {r.c[16].x, r.c[16].y, r.c[16].z, r.c[16].w};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const float d = (j & 1) ? hi_half(dw[j >> 1]) : lo_half(dw[j >> 1]);
        const uint4 qa = r.c[2 * j], qb = r.c[2 * j + 1];
        const uint32_t w8[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
        uint32_t m[16];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t v = w8[k] ^ 0x80808080u;
            m[2 * k] = magic2(v, kSel01);
            m[2 * k + 1] = magic2(v, kSel23);
        }
#pragma unroll
        for (int t = 0; t < TM; ++t) {
            if (t < me) {
                const uint16_t* xr = xs + t * K + 32 * j;
                uint32_t xv[16];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const uint4 v = ld128(xr + 8 * q);
                    xv[4 * q] = v.x; xv[4 * q + 1] = v.y; xv[4 * q + 2] = v.z; xv[4 * q + 3] = v.w;
                }
                float T = 0.f;
#pragma unroll
                for (int k = 0; k < 16; ++k) T = dot2(m[k], xv[k], T);
                const float* sx = xsum + t * (K >> 4) + 2 * j;
                acc[t] += d * (T - 1152.0f * (sx[0] + sx[1]));
            }
        }
    }
}

// fp16 value 1024 + q6 (6-bit code), weight = d * sc * (q6 - 32).
template <int TM>
__device__ __forceinline__ void gu_compute(const Raw<PGMOE_Q6_K>& r, const uint16_t* xs, const float* xsum, int K,
                                           int me, float* acc) {
    const float d = h2f((uint16_t)r.d);
    const uint32_t scw[4] = {r.c[12].x, r.c[12].y, r.c[12].z, r.c[12].w};
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            uint32_t m[16];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const int wa = 16 * h + k, wb = 16 * h + 8 + k, wq = 8 * h + k;  // word indices
                const uint32_t qa = ((const uint32_t*)&r.c[wa >> 2])[wa & 3];
                const uint32_t qb = ((const uint32_t*)&r.c[wb >> 2])[wb & 3];
                const uint32_t qh = ((const uint32_t*)&r.c[8 + (wq >> 2)])[wq & 3];
                const uint32_t q = q6_word(qa, qb, qh, s);
                m[2 * k] = magic2(q, kSel01);
                m[2 * k + 1] = magic2(q, kSel23);
            }
            const int sb = 8 * h + 2 * s;
            const float a0 = d * (float)(int8_t)((scw[sb >> 2] >> (8 * (sb & 3))) & 0xff);
            const float a1 = d * (float)(int8_t)((scw[(sb + 1) >> 2] >> (8 * ((sb + 1) & 3))) & 0xff);
#pragma unroll
            for (int t = 0; t < TM; ++t) {
                if (t < me) {
                    const uint16_t* xr = xs + t * K + 128 * h + 32 * s;
                    uint32_t xv[16];
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const uint4 v = ld128(xr + 8 * q);
                        xv[4 * q] = v.x; xv[4 * q + 1] = v.y; xv[4 * q + 2] = v.z; xv[4 * q + 3] = v.w;
                    }
                    float T0 = 0.f, T1 = 0.f;
#pragma unroll
                    for (int k = 0; k < 8; ++k) T0 = dot2(m[k], xv[k], T0);
#pragma unroll
                    for (int k = 8; k < 16; ++k) T1 = dot2(m[k], xv[k], T1);
                    const float* sx = xsum + t * (K >> 4) + sb;
                    acc[t] += a0 * (T0 - 1056.0f * sx[0]) + a1 * (T1 - 1056.0f * sx[1]);
                }
            }
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

template <int TM>
__device__ __forceinline__ void dn_compute(const Raw<PGMOE_Q4_K>& r, const float* x, const float* isum, int K,
                                           int me, float* acc) {
    const uint4 hd = r.c[0];
    const float dd = lo_half(hd.x), dm = hi_half(hd.x);
#pragma unroll
    for (int s = 0; s < 8; ++s) {  // sub-block s: qs bytes 32(s/2).., nibble s&1
        int sc, mn;
        kscale(hd.y, hd.z, hd.w, s, sc, mn);
        const float a = dd * (float)sc, bm = dm * (float)mn;
        const int c2 = s >> 1, sh = 4 * (s & 1);
        const uint4 qa = r.c[1 + 2 * c2], qb = r.c[2 + 2 * c2];
        const uint32_t w8[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
        float qf[32];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t v = (w8[k] >> sh) & 0x0f0f0f0fu;
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
#pragma unroll
    for (int s = RB; s < 64; s <<= 1) v += __shfl_xor(v, s, 64);
    return v;
}

// ============================================================================ routing in a block
// Decode forward: the router kernel writes logits [M][E]; every gate/up block re-derives
// the top-k sets of the M <= 8 tokens from them (about a microsecond of register work
// instead of a launch and its dependent global round trips), and block (0, 0) also
// publishes a compact routing descriptor for the fused down + combine kernel:
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
    int n_act, e, p_begin, count;
    int tok[kDecTM];
    uint64_t wbuf[4][64];       // per-wave selection scratch
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

// K-th largest of the distinct keys of one token held by a wave (lane l: experts l + 64r),
// by a 41-step radix descent on the key bits (ballot counts).  Exact for any keys; used
// when the candidate select below has too many candidates.
template <int RE>
__device__ __forceinline__ uint64_t kth_key_radix(const uint64_t (&key)[RE], int K) {
    uint64_t thr = 0;
    for (int b = 40; b >= 0; --b) {
        const uint64_t cand = thr | (1ull << b);
        int cnt = 0;
#pragma unroll
        for (int r = 0; r < RE; ++r) cnt += __popcll(__ballot(key[r] >= cand));
        thr = cnt >= K ? cand : thr;
    }
    return thr;
}

// Rank of v among n 64-bit values in LDS (number strictly greater), n even.
__device__ __forceinline__ int lds_rank(const uint64_t* buf, int n, uint64_t v) {
    int c = 0;
    for (int j = 0; j < n; j += 2) {
        const uint64_t a = buf[j], b = buf[j + 1];
        c += a > v ? 1 : 0;
        c += b > v ? 1 : 0;
    }
    return c;
}

// K-th largest key of one token (keys distinct, at least K of them nonzero; 1 <= K <= 16).
// 1. T = the K-th largest of the 64 lane maxima.  At most K lanes have a maximum >= the
//    K-th largest key k* (each such maximum is a distinct key >= k*), so T <= k*.
// 2. The candidates (keys >= T) hold the K largest keys; they are ranked among
//    themselves and the one of rank K-1 is k*.  More than 64 candidates (keys bunched in
//    few lanes) take the radix descent instead.
// wbuf: this wave's 64-word LDS scratch.
template <int RE>
__device__ __forceinline__ uint64_t kth_key(const uint64_t (&key)[RE], int K, int lane, uint64_t* wbuf) {
    uint64_t lm = 0;
#pragma unroll
    for (int r = 0; r < RE; ++r) lm = key[r] > lm ? key[r] : lm;
    wbuf[lane] = lm;
    __builtin_amdgcn_wave_barrier();
    const int c1 = lds_rank(wbuf, 64, lm);
    const uint64_t b1 = __ballot(lm != 0 && c1 == K - 1);
    const int l1 = __ffsll((unsigned long long)b1) - 1;
    const uint64_t T = ((uint64_t)__shfl(uint32_t(lm >> 32), l1, 64) << 32) | __shfl(uint32_t(lm), l1, 64);
    int C = 0;
#pragma unroll
    for (int r = 0; r < RE; ++r) C += __popcll(__ballot(key[r] >= T));
    if (C > 64) return kth_key_radix<RE>(key, K);
    __builtin_amdgcn_wave_barrier();
    int base = 0;
#pragma unroll
    for (int r = 0; r < RE; ++r) {
        const bool in = key[r] >= T;
        const uint64_t mk = __ballot(in);
        if (in) wbuf[base + __popcll(mk & ((1ull << lane) - 1ull))] = key[r];
        base += __popcll(mk);
    }
    if ((C & 1) && lane == C) wbuf[C] = 0;  // pad to an even count (0 is below every key)
    __builtin_amdgcn_wave_barrier();
    const uint64_t ci = lane < C ? wbuf[lane] : 0;
    const int c2 = lds_rank(wbuf, (C + 1) & ~1, ci);
    const uint64_t b2 = __ballot(lane < C && c2 == K - 1);
    const int l2 = __ffsll((unsigned long long)b2) - 1;
    return ((uint64_t)__shfl(uint32_t(ci >> 32), l2, 64) << 32) | __shfl(uint32_t(ci), l2, 64);
}

// Top-k membership of NT tokens handled by one wave (tokens m = wv + nw*i, i < NT; those
// >= M are skipped).  Lane l holds the keys of experts l + 64r, r < RE; the members of a
// token are exactly its keys at or above its K-th largest key (keys are distinct).  With
// `weights`, also the softmax weights of the members (max-subtracted, denominator over
// all E, optional renorm; model.py:903-907).
template <int RE, int NT>
__device__ __forceinline__ void route_tokens(const float* sl, int M, int E, int K, RouteShared& R, bool weights,
                                             int norm, int wv, int nw, int lane) {
    uint64_t key[NT][RE];
    uint64_t thr[NT];
#pragma unroll
    for (int i = 0; i < NT; ++i) {
        const int m = wv + nw * i;
#pragma unroll
        for (int r = 0; r < RE; ++r) {
            const int e = lane + 64 * r;
            key[i][r] = (m < M && e < E) ? route_key(sl[m * E + e], e) : 0ull;
        }
    }
#pragma unroll
    for (int i = 0; i < NT; ++i) thr[i] = wv + nw * i < M ? kth_key<RE>(key[i], K, lane, R.wbuf[wv]) : ~0ull;
    if (wv == 0) PG_MARK(1, 7);
#pragma unroll
    for (int i = 0; i < NT; ++i) {
        const int m = wv + nw * i;
        if (m >= M) continue;
        float top = -INFINITY, den = 0.f;
        if (weights) {
#pragma unroll
            for (int r = 0; r < RE; ++r)
                if (lane + 64 * r < E) top = fmaxf(top, sl[m * E + lane + 64 * r]);
#pragma unroll
            for (int s = 32; s >= 1; s >>= 1) top = fmaxf(top, __shfl_xor(top, s, 64));
#pragma unroll
            for (int r = 0; r < RE; ++r)
                if (lane + 64 * r < E) den += expf(sl[m * E + lane + 64 * r] - top);
            den = group_sum<64>(den);
        }
        int base = 0;
        float psel = 0.f;
#pragma unroll
        for (int r = 0; r < RE; ++r) {
            const bool in = key[i][r] >= thr[i] && lane + 64 * r < E;
            const uint64_t mask = __ballot(in);
            if (lane == 0) {
                R.pres[m][2 * r] = (uint32_t)mask;
                R.pres[m][2 * r + 1] = (uint32_t)(mask >> 32);
            }
            const int pos = base + __popcll(mask & ((1ull << lane) - 1ull));
            if (in && pos < K) {  // exactly K members unless logits hold NaNs
                R.mem_e[m * K + pos] = lane + 64 * r;
                if (weights) {
                    const float p = expf(sl[m * E + lane + 64 * r] - top) / den;
                    R.mem_w[m * K + pos] = p;
                    psel += p;
                }
            }
            base += __popcll(mask);
        }
        if (weights && norm) {
            psel = group_sum<64>(psel);
            for (int j = lane; j < K; j += 64) R.mem_w[m * K + j] = R.mem_w[m * K + j] / fmaxf(psel, 1e-20f);
        }
        if (lane < 16 && lane >= 2 * RE) R.pres[m][lane] = 0u;
    }
}

// Routing of the M <= 8 tokens in one block from the logits [M][E] (sl: LDS scratch of
// M*E floats), then the per-word prefix counts: used / wc / wp / n_act.  Every thread of
// the block calls this.  NT = tokens per wave, a compile-time bound >= ceil(M / waves).
template <int NT>
__device__ __forceinline__ void route_in_block(const float* __restrict__ logits, int M, int E, int K, float* sl,
                                               RouteShared& R, bool weights, int norm) {
    const int tid = threadIdx.x, nth = blockDim.x, lane = tid & 63, wv = tid >> 6, nw = nth >> 6;
    copy_words<8>(sl, logits, M * E, tid, nth);
    __syncthreads();
    PG_MARK(1, 6);
    if (E <= 64)
        route_tokens<1, NT>(sl, M, E, K, R, weights, norm, wv, nw, lane);
    else if (E <= 128)
        route_tokens<2, NT>(sl, M, E, K, R, weights, norm, wv, nw, lane);
    else if (E <= 256)
        route_tokens<4, NT>(sl, M, E, K, R, weights, norm, wv, nw, lane);
    else
        route_tokens<8, NT>(sl, M, E, K, R, weights, norm, wv, nw, lane);
    __syncthreads();
    if (wv == 0) {  // lane q: word q of the expert bitmaps; wave prefix sums over the words
        uint32_t u = 0;
        int pc = 0;
        if (lane < 16) {
            for (int m = 0; m < M; ++m) {
                const uint32_t w = R.pres[m][lane];
                u |= w;
                pc += __popc(w);
            }
        }
        int ca = __popc(u), cp = pc;
#pragma unroll
        for (int s = 1; s < 16; s <<= 1) {
            const int oa = __shfl_up(ca, s, 64), op = __shfl_up(cp, s, 64);
            if (lane >= s) {
                ca += oa;
                cp += op;
            }
        }
        if (lane < 16) {
            R.used[lane] = u;
            R.wc[lane] = ca - __popc(u);
            R.wp[lane] = cp - pc;
        }
        if (lane == 15) R.n_act = ca;
    }
    __syncthreads();
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

// Publish the routing descriptor (block (0, 0) only; R holds the weights), and the flat
// arrays when fl.offsets is set.  One thread per expert, then one per pair.
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
//   kIdent   : one expert (matrix 0) applied to every token with weight 1 (shared expert).
enum DecMode { kDispatch = 0, kRoute = 1, kIdent = 2 };

struct DecDisp {
    int mode;  // DecMode
    const int32_t *offsets, *perm, *active, *n_active;
    const float* logits;  // kRoute
    int32_t* desc;        // kRoute: published by block (0, 0)
    int M, E, norm;       // M: tokens (kRoute, kIdent)
    FlatRoute flat;       // kRoute: optional flat arrays, published by block (0, 0)
};

// Gate/up + SwiGLU.  Block = RB rows of one active expert, W waves; lane (r, ks):
// row = RB*blockIdx.x + r, super-blocks j = ks + KS*w, + KS*W, ...  Pairs of the expert
// are taken TM at a time.  inter / isum rows are indexed by sorted pair.
// Dynamic LDS: max(xs [TM][K] fp16 + xs_sum [TM][K/16] f32, logits [M][E] f32 (kRoute),
// partials [W][TM][2][RB] + SwiGLU row [TM][RB]).
// xsum (optional): 16-element sums of x rows [M][K/16]; isum (optional output):
// 16-element sums of inter rows [P][N/16].
template <int QT, int RB, int W, int TM>
__global__ __launch_bounds__(W * 64) void dec_gateup_kernel(const uint8_t* __restrict__ gbase,
                                                            const uint8_t* __restrict__ ubase, int64_t gstride,
                                                            int64_t ustride, int N, int K,
                                                            const uint16_t* __restrict__ x,
                                                            const float* __restrict__ xsum, int topk, DecDisp dp,
                                                            float* __restrict__ inter, float* __restrict__ isum) {
    constexpr int KS = 64 / RB;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    __shared__ RouteShared R;
    const int a = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int MODE = dp.mode;
    int e, p_begin, p_end;
    PG_MARK(1, 0);
    if (MODE == kRoute) {
        const bool pub = blockIdx.x == 0 && a == 0;
        // tokens per wave: sized from TM, or for kDecTM when the LDS limit made TM < M
        if (dp.M <= ((TM + W - 1) / W) * W)
            route_in_block<(TM + W - 1) / W>(dp.logits, dp.M, dp.E, topk, (float*)smem, R, pub, dp.norm);
        else
            route_in_block<(kDecTM + W - 1) / W>(dp.logits, dp.M, dp.E, topk, (float*)smem, R, pub, dp.norm);
        PG_MARK(1, 1);
        if (a >= R.n_act) return;  // uniform: every block computed the same n_act
        for (int ee = tid; ee < dp.E; ee += W * 64) {  // the expert of this block's slot
            int pb = 0, c = 0;
            if (route_expert(R, dp.M, ee, pb, c) == a) {
                R.e = ee;
                R.p_begin = pb;
                R.count = c;
                int n = 0;
                for (int m = 0; m < dp.M; ++m)
                    if ((R.pres[m][ee >> 5] >> (ee & 31)) & 1u) R.tok[n++] = m;
            }
        }
        __syncthreads();
        PG_MARK(1, 2);
        e = R.e;
        p_begin = R.p_begin;
        p_end = p_begin + R.count;
    } else if (MODE == kIdent) {
        e = 0;
        p_begin = 0;
        p_end = dp.M;
    } else {
        if (a >= *dp.n_active) return;
        e = dp.active[a];
        p_begin = dp.offsets[e];
        p_end = dp.offsets[e + 1];
    }
    const int r = lane % RB, ks = lane / RB;
    const int row = blockIdx.x * RB + r;  // < row_groups(N) * 64: padded tile rows are readable
    const int nb = K >> 8;
    const int j0 = ks + KS * w;
    uint16_t* xs = (uint16_t*)smem;
    float* xss = (float*)(smem + (size_t)TM * K * 2);
    float* red = (float*)smem;           // [W][TM][2][RB] after the K loop
    float* act = red + W * TM * 2 * RB;  // [TM][RB] SwiGLU values
    const uint8_t* gm = gbase + (int64_t)e * gstride;
    const uint8_t* um = ubase + (int64_t)e * ustride;
    for (int p0 = p_begin; p0 < p_end; p0 += TM) {
        const int me = min(TM, p_end - p0);
        Raw<QT> rg, ru;
        if (j0 < nb) {  // weights first: their latency overlaps the activation staging
            load_raw<QT>(rg, gm, N, nb, row, j0);
            load_raw<QT>(ru, um, N, nb, row, j0);
        }
        __syncthreads();
        for (int i = tid; i < me * (K >> 3); i += W * 64) {
            const int t = i / (K >> 3), c = i % (K >> 3);
            const int tok = MODE == kRoute ? R.tok[p0 - p_begin + t] : MODE == kIdent ? p0 + t : dp.perm[p0 + t] / topk;
            *(uint4*)(xs + t * K + 8 * c) = *(const uint4*)(x + (int64_t)tok * K + 8 * c);
        }
        if (xsum) {
            for (int i = tid; i < me * (K >> 4); i += W * 64) {
                const int t = i / (K >> 4), c = i % (K >> 4);
                const int tok =
                    MODE == kRoute ? R.tok[p0 - p_begin + t] : MODE == kIdent ? p0 + t : dp.perm[p0 + t] / topk;
                xss[i] = xsum[(int64_t)tok * (K >> 4) + c];
            }
        }
        __syncthreads();
        if (!xsum) {
            for (int i = tid; i < me * (K >> 4); i += W * 64) {
                const uint16_t* p = xs + (i / (K >> 4)) * K + 16 * (i % (K >> 4));
                float sm = 0.f;
#pragma unroll
                for (int k = 0; k < 16; ++k) sm += h2f(p[k]);
                xss[i] = sm;
            }
            __syncthreads();
        }
        PG_MARK(1, 3);
        float ag[TM], au[TM];
#pragma unroll
        for (int t = 0; t < TM; ++t) ag[t] = au[t] = 0.f;
        for (int j = j0; j < nb; j += KS * W) {
            if (j != j0) {
                load_raw<QT>(rg, gm, N, nb, row, j);
                load_raw<QT>(ru, um, N, nb, row, j);
            }
            gu_compute<TM>(rg, xs + 256 * j, xss + 16 * j, K, me, ag);
            gu_compute<TM>(ru, xs + 256 * j, xss + 16 * j, K, me, au);
        }
        PG_MARK(1, 4);
#pragma unroll
        for (int t = 0; t < TM; ++t) {
            ag[t] = kslot_sum<RB>(ag[t]);
            au[t] = kslot_sum<RB>(au[t]);
        }
        __syncthreads();  // xs is dead: reuse it for the cross-wave partials
        if (ks == 0) {
#pragma unroll
            for (int t = 0; t < TM; ++t)
                if (t < me) {
                    red[((w * TM + t) * 2 + 0) * RB + r] = ag[t];
                    red[((w * TM + t) * 2 + 1) * RB + r] = au[t];
                }
        }
        __syncthreads();
        for (int i = tid; i < me * RB; i += W * 64) {
            const int t = i / RB, rr = i % RB;
            float g = 0.f, u = 0.f;
#pragma unroll
            for (int ww = 0; ww < W; ++ww) {
                g += red[((ww * TM + t) * 2 + 0) * RB + rr];
                u += red[((ww * TM + t) * 2 + 1) * RB + rr];
            }
            const float v = silu(g) * u;
            act[t * RB + rr] = v;
            const int orow = blockIdx.x * RB + rr;
            if (orow < N) inter[(int64_t)(p0 + t) * N + orow] = v;
        }
        if (isum) {
            __syncthreads();
            for (int i = tid; i < me * (RB / 16); i += W * 64) {
                const int t = i / (RB / 16), g16 = i % (RB / 16);
                const int grow = blockIdx.x * RB + 16 * g16;
                if (grow < N) {
                    float sm = 0.f;
#pragma unroll
                    for (int k = 0; k < 16; ++k) sm += act[t * RB + 16 * g16 + k];
                    isum[(int64_t)(p0 + t) * (N >> 4) + (grow >> 4)] = sm;
                }
            }
        }
    }
    // block (0, 0) publishes the routing last: its stores then stay off the block's own
    // critical path (a barrier would wait for them)
    if (MODE == kRoute && blockIdx.x == 0 && a == 0) publish_route(R, dp.M, dp.E, topk, dp.desc, dp.flat);
    PG_MARK(1, 5);
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

// Fused down + combine.  Block = RB output rows for all M tokens; its W waves x KS lane
// groups walk the slices (active slot a, super-block j), slice s = ks + KS*w + KS*W*i, each
// lane accumulating w_(t,a) * (inter_(t,a) . d_a,row(j)) per token, with the next slice's
// weights loaded before the current one is computed; a fixed shuffle + LDS tree sums the
// slices.  out[t, row] = that sum (+ shared[t, row] * sigmoid(shared_logit[t])).
// Inputs: the routing descriptor (P = M*K pairs), inter / isum rows in sorted pair order,
// all P rows staged in LDS together with the descriptor (the host uses this kernel only
// when P*K*4 + P*K/16*4 fits).  The slice order depends only on the routing, so results
// are reproducible run to run.
// Dynamic LDS: xs [P][K] f32 | iss [P][K/16] f32.
template <int QT, int RB, int W, int TM>
__global__ __launch_bounds__(W * 64) void dec_down_combine_kernel(
    const uint8_t* __restrict__ dbase, int64_t dstride, int N, int K, const float* __restrict__ inter,
    const float* __restrict__ isum, const int32_t* __restrict__ desc, int M, int P, const float* __restrict__ shared,
    const float* __restrict__ shared_logit, float* __restrict__ out) {
    constexpr int KS = 64 / RB;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    __shared__ int d_slot[128 * 3];
    __shared__ int d_tok[128];
    __shared__ float d_w[128];
    __shared__ float red[W][TM][RB];
    __shared__ int s_nact;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    float* xs = (float*)smem;
    float* iss = xs + P * K;
    PG_MARK(3, 0);
    {
        int v[5] = {0, 0, 0, 0, 0};
        const bool has = tid < P;
        if (has) {
            v[0] = desc[kDescSlot + 4 * tid];
            v[1] = desc[kDescSlot + 4 * tid + 1];
            v[2] = desc[kDescSlot + 4 * tid + 2];
            v[3] = desc[kDescPair + 2 * tid];
            v[4] = desc[kDescPair + 2 * tid + 1];
        }
        const int n0 = tid == 0 ? desc[0] : 0;
        copy_words<8>((uint4*)xs, (const uint4*)inter, P * (K >> 2), tid, W * 64);
        copy_words<4>((uint4*)iss, (const uint4*)isum, P * (K >> 6), tid, W * 64);
        if (has) {
            d_slot[3 * tid] = v[0];
            d_slot[3 * tid + 1] = v[1];
            d_slot[3 * tid + 2] = v[2];
            d_tok[tid] = v[3];
            d_w[tid] = __builtin_bit_cast(float, v[4]);
        }
        if (tid == 0) s_nact = n0;
    }
    __syncthreads();
    PG_MARK(3, 1);
    const int nact = s_nact;
    const int r = lane % RB, ks = lane / RB;
    const int row = blockIdx.x * RB + r;
    const int nb = K >> 8;
    const int S = nact * nb;
    float acc[TM];
#pragma unroll
    for (int t = 0; t < TM; ++t) acc[t] = 0.f;
    int s = ks + KS * w;
    Raw<QT> rw;
    if (s < S) load_raw<QT>(rw, dbase + (int64_t)d_slot[3 * (s / nb)] * dstride, N, nb, row, s % nb);
    while (s < S) {
        const int sn = s + KS * W;
        Raw<QT> rn;
        if (sn < S) load_raw<QT>(rn, dbase + (int64_t)d_slot[3 * (sn / nb)] * dstride, N, nb, row, sn % nb);
        const int a = s / nb, j = s % nb;
        const int p0 = d_slot[3 * a + 1], cnt = d_slot[3 * a + 2];
        float part[TM];
#pragma unroll
        for (int t = 0; t < TM; ++t) part[t] = 0.f;
        dn_compute<TM>(rw, xs + p0 * K + 256 * j, iss + p0 * (K >> 4) + 16 * j, K, cnt, part);
#pragma unroll
        for (int q = 0; q < TM; ++q) {
            if (q < cnt) {
                const int tq = d_tok[p0 + q];
                const float v = d_w[p0 + q] * part[q];
#pragma unroll
                for (int t = 0; t < TM; ++t)
                    if (t == tq) acc[t] += v;
            }
        }
        rw = rn;
        s = sn;
        PG_MARK(3, 2);
    }
    PG_MARK(3, 3);
#pragma unroll
    for (int t = 0; t < TM; ++t) acc[t] = kslot_sum<RB>(acc[t]);
    if (ks == 0) {
#pragma unroll
        for (int t = 0; t < TM; ++t) red[w][t][r] = acc[t];
    }
    __syncthreads();
    for (int i = tid; i < M * RB; i += W * 64) {
        const int t = i / RB, rr = i % RB;
        float v = 0.f;
#pragma unroll
        for (int ww = 0; ww < W; ++ww) v += red[ww][t][rr];
        const int orow = blockIdx.x * RB + rr;
        if (orow < N) {
            if (shared) {
                const float g = shared_logit ? 1.0f / (1.0f + expf(-shared_logit[t])) : 1.0f;
                v += shared[(int64_t)t * N + orow] * g;
            }
            out[(int64_t)t * N + orow] = v;
        }
    }
    PG_MARK(3, 4);
}

// LDS bytes the fused down + combine kernel stages (all P inter rows and their sums).
inline size_t dc_stage_bytes(int P, int K) { return (size_t)P * K * 4 + (size_t)P * (K / 16) * 4; }
constexpr size_t kDcStageMax = 52 * 1024;

// ============================================================================ launch plumbing
// Block shapes (rows per block RB, waves W <= 4 so every wave may use up to 512 VGPRs):
// one super-block per lane when nb equals KS * W for one of them, else (16, 4) with a
// K loop.
struct DecShape {
    int RB, W;
};

inline DecShape pick_shape(int nb) {
    static const DecShape menu[] = {{16, 1}, {16, 2}, {16, 4}, {32, 1}, {64, 1}, {64, 3}};
    for (const DecShape& s : menu)
        if ((64 / s.RB) * s.W == nb) return s;
    return {16, 4};
}

// Token tile: the smallest power of two >= M (max 8), halved while the gate/up LDS stage
// (TM fp16 rows of K plus their 16-element sums) would exceed 60 KB.
inline int tile_tokens(int M, int K) {
    int t = M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8;
    while (t > 1 && (size_t)t * K * 2 + (size_t)t * (K / 16) * 4 > 60 * 1024) t >>= 1;
    return t;
}

// Down: per K step, t rows of JW super-blocks staged as fp32 (1088 bytes a super-block
// with its sums) plus the [W][t][RB] partials; t halves while that exceeds 60 KB.
inline size_t down_lds_bytes(int t, int RB, int W) { return (size_t)t * (64 / RB) * W * 1088 + (size_t)W * t * RB * 4; }
inline int down_tile_tokens(int M, const DecShape& sp) {
    int t = M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8;
    while (t > 1 && down_lds_bytes(t, sp.RB, sp.W) > 60 * 1024) t >>= 1;
    return t;
}

template <int QT, int RB, int W, int TM>
inline void gu_launch(const Mats& g, const Mats& u, const uint16_t* x, const float* xsum, int topk, const DecDisp& dp,
                      int max_active, float* inter, float* isum, hipStream_t st) {
    const size_t stage = (size_t)TM * g.K * 2 + (size_t)TM * (g.K / 16) * 4;
    const size_t tail = (size_t)W * TM * 2 * RB * 4 + (size_t)TM * RB * 4;
    const size_t logits = dp.mode == kRoute ? (size_t)dp.M * dp.E * 4 : 0;
    size_t sh = stage > tail ? stage : tail;
    sh = sh > logits ? sh : logits;
    PG_LAUNCH((dec_gateup_kernel<QT, RB, W, TM>), dim3(div_up(g.N, RB), max_active), dim3(64 * W), sh,
                       st, g.base, u.base, g.stride, u.stride, g.N, g.K, x, xsum, topk, dp, inter, isum);
}

template <int QT, int RB, int W, int TM>
inline void dn_launch(const Mats& d, const float* inter, const float* isum, const DecDisp& dp, int max_active,
                      const float* topk_w, float* partial, hipStream_t st) {
    const size_t sh = down_lds_bytes(TM, RB, W);
    PG_LAUNCH((dec_down_kernel<QT, RB, W, TM>), dim3(div_up(d.N, RB), max_active), dim3(64 * W), sh,
                       st, d.base, d.stride, d.N, d.K, inter, isum, dp, topk_w, partial);
}

template <int QT, int RB, int W, int TM>
inline void dc_launch(const Mats& d, const float* inter, const float* isum, const int32_t* desc, int M, int P,
                      const float* shared, const float* shared_logit, float* out, hipStream_t st) {
    PG_LAUNCH((dec_down_combine_kernel<QT, RB, W, TM>), dim3(div_up(d.N, RB)), dim3(64 * W),
                       dc_stage_bytes(P, d.K), st, d.base,
                       d.stride, d.N, d.K, inter, isum, desc, M, P, shared, shared_logit, out);
}

#define PG_TM(F, QT, RB, W, ...)                   \
    switch (TM) {                                 \
    case 1: F<QT, RB, W, 1>(__VA_ARGS__); break;  \
    case 2: F<QT, RB, W, 2>(__VA_ARGS__); break;  \
    case 4: F<QT, RB, W, 4>(__VA_ARGS__); break;  \
    default: F<QT, RB, W, 8>(__VA_ARGS__); break; \
    }

// Block shapes for the per-expert kernels: the shapes pick_shape returns.
#define PG_SHAPES(F, QT, ...)                                  \
    switch (sp.RB * 16 + sp.W) {                               \
    case 16 * 16 + 1: PG_TM(F, QT, 16, 1, __VA_ARGS__); break; \
    case 16 * 16 + 2: PG_TM(F, QT, 16, 2, __VA_ARGS__); break; \
    case 32 * 16 + 1: PG_TM(F, QT, 32, 1, __VA_ARGS__); break; \
    case 64 * 16 + 1: PG_TM(F, QT, 64, 1, __VA_ARGS__); break; \
    case 64 * 16 + 3: PG_TM(F, QT, 64, 3, __VA_ARGS__); break; \
    default: PG_TM(F, QT, 16, 4, __VA_ARGS__); break;          \
    }

// Fused down + combine: rows per block and waves chosen so the grid has >= 256 blocks
// where the output allows it and each lane walks few slices.
struct DcShape {
    int RB, W;
};
inline DcShape pick_dc_shape(int N, int slices) {
    const int rb = N >= 256 * 16 ? 16 : 8;
    const int ks = 64 / rb;
    int w = (slices + ks - 1) / ks;
    w = w < 1 ? 1 : w > 4 ? 4 : w;
    return {rb, w};
}

#define PG_DC_SHAPES(QT, ...)                                    \
    switch (dsp.RB * 16 + dsp.W) {                               \
    case 8 * 16 + 1: PG_TM(dc_launch, QT, 8, 1, __VA_ARGS__); break;  \
    case 8 * 16 + 2: PG_TM(dc_launch, QT, 8, 2, __VA_ARGS__); break;  \
    case 8 * 16 + 3: PG_TM(dc_launch, QT, 8, 3, __VA_ARGS__); break;  \
    case 8 * 16 + 4: PG_TM(dc_launch, QT, 8, 4, __VA_ARGS__); break;  \
    case 16 * 16 + 1: PG_TM(dc_launch, QT, 16, 1, __VA_ARGS__); break; \
    case 16 * 16 + 2: PG_TM(dc_launch, QT, 16, 2, __VA_ARGS__); break; \
    case 16 * 16 + 3: PG_TM(dc_launch, QT, 16, 3, __VA_ARGS__); break; \
    default: PG_TM(dc_launch, QT, 16, 4, __VA_ARGS__); break;          \
    }

// Per-qtype launchers (defined in decode_q4k.hip / decode_q6k.hip / decode_q8_0.hip).
template <int QT>
int dec_gateup_q(const Mats& g, const Mats& u, const uint16_t* x, const float* xsum, int topk, int M, int mode,
                 const DecDisp& dp, int max_active, float* inter, float* isum, hipStream_t st);
template <int QT>
int dec_down_q(const Mats& d, const float* inter, const float* isum, int M, int mode, const DecDisp& dp,
               int max_active, const float* topk_w, float* partial, hipStream_t st);
template <int QT>
int dec_down_combine_q(const Mats& d, const float* inter, const float* isum, const int32_t* desc, int M, int P,
                       int max_active, const float* shared, const float* shared_logit, float* out, hipStream_t st);

#define PG_DEFINE_DECODE_GATEUP(QT)                                                                                  \
    template <>                                                                                                     \
    int dec_gateup_q<QT>(const Mats& g, const Mats& u, const uint16_t* x, const float* xsum, int topk, int M,      \
                         int mode, const DecDisp& dp, int max_active, float* inter, float* isum, hipStream_t st) {  \
        const DecShape sp = pick_shape(g.K >> 8);                                                                   \
        const int TM = tile_tokens(M, g.K);                                                                         \
        if ((size_t)TM * g.K * 2 + (size_t)TM * (g.K / 16) * 4 > 64 * 1024)                                        \
            return fail(PGMOE_E_UNSUPPORTED, "decode gate/up: %d inputs exceed the LDS stage", g.K);                \
        PG_SHAPES(gu_launch, QT, g, u, x, xsum, topk, dp, max_active, inter, isum, st);                  \
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
    int dec_down_combine_q<QT>(const Mats& d, const float* inter, const float* isum, const int32_t* desc, int M,   \
                               int P, int max_active, const float* shared, const float* shared_logit, float* out,   \
                               hipStream_t st) {                                                                    \
        const DcShape dsp = pick_dc_shape(d.N, max_active * (d.K >> 8));                                            \
        const int TM = tile_tokens(M, 0);                                                                           \
        if (dc_stage_bytes(P, d.K) > kDcStageMax)                                                                   \
            return fail(PGMOE_E_UNSUPPORTED, "decode down + combine: %d pairs of %d inputs exceed LDS", P, d.K);    \
        PG_DC_SHAPES(QT, d, inter, isum, desc, M, P, shared, shared_logit, out, st);                                 \
        return check_launch("dec_down_combine");                                                                    \
    }

}  // namespace pgmoe
