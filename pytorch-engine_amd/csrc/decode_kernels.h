// Decode path (M <= 8 tokens), five short launches per layer, no host sync:
//   router logits (router.hip, fixed order) -> top-k + dispatch (one block) ->
//   gate/up + SwiGLU -> down -> combine (experts.hip, ascending expert id).
// Expert kernels: a block owns RB rows of one active expert; lane = (row, K-slice), so
// each lane streams whole 256-weight super-blocks of one row from the 64-row tile
// layout (coalesced 16-byte chunks), activations are wave-uniform (LDS / broadcast),
// and partial sums meet through a few shuffles and one LDS pass.  Weight loads are
// issued before the activation staging so both latencies overlap.
//   gate/up: fp16 magic-number dequant (1024 + code) feeding v_dot2_f32_f16
//   down   : fp32 FMA on the fp32 SwiGLU output
// Reference: pygguf_engine/model.py:898-937; quant_kernels.py:68-311 (GEMV kernels it
// replaces), :1423-1475 (SwiGLU + row-scale).
#pragma once
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

// ============================================================================ kernels
// Block = RB rows of one active expert, W waves; lane (r, ks): row = RB*blockIdx.x + r,
// super-blocks j = ks + KS*w, + KS*W, ...  Pairs of the expert are taken TM at a time.
// LDS: xs [TM][K] fp16 | xs_sum [TM][K/16] f32; partials and the SwiGLU row reuse xs.
// xsum (optional): 16-element sums of x rows, [M][K/16]; isum (optional output):
// 16-element sums of the inter rows, [P][N/16].
template <int QT, int RB, int W, int TM>
__global__ __launch_bounds__(W * 64) void dec_gateup_kernel(const uint8_t* __restrict__ gbase,
                                                            const uint8_t* __restrict__ ubase, int64_t gstride,
                                                            int64_t ustride, int N, int K,
                                                            const uint16_t* __restrict__ x,
                                                            const float* __restrict__ xsum, int topk,
                                                            const int32_t* __restrict__ offsets,
                                                            const int32_t* __restrict__ perm,
                                                            const int32_t* __restrict__ active,
                                                            const int32_t* __restrict__ n_active,
                                                            float* __restrict__ inter, float* __restrict__ isum) {
    constexpr int KS = 64 / RB;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int a = blockIdx.y;
    if (a >= *n_active) return;
    const int e = active[a];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int r = lane % RB, ks = lane / RB;
    const int row = blockIdx.x * RB + r;  // < row_groups(N) * 64: padded tile rows are readable
    const int nb = K >> 8;
    const int j0 = ks + KS * w;
    uint16_t* xs = (uint16_t*)smem;
    float* xss = (float*)(smem + (size_t)TM * K * 2);
    float* red = (float*)smem;            // [W][TM][2][RB] after the K loop
    float* act = red + W * TM * 2 * RB;   // [TM][RB] SwiGLU values
    const uint8_t* gm = gbase + (int64_t)e * gstride;
    const uint8_t* um = ubase + (int64_t)e * ustride;
    const int p_begin = offsets[e], p_end = offsets[e + 1];
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
            const int tok = perm[p0 + t] / topk;
            *(uint4*)(xs + t * K + 8 * c) = *(const uint4*)(x + (int64_t)tok * K + 8 * c);
        }
        if (xsum) {
            for (int i = tid; i < me * (K >> 4); i += W * 64) {
                const int t = i / (K >> 4), c = i % (K >> 4);
                xss[i] = xsum[(int64_t)(perm[p0 + t] / topk) * (K >> 4) + c];
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
}

// partial[p, row] = w[perm[p]] * (inter_p . d_row) for the pairs of one active expert.
// isum (optional input): 16-element sums of inter rows [P][K/16]; otherwise computed.
// LDS: isum staging [TM][K/16] f32 (only without isum) | red [W][TM][RB] f32.
template <int QT, int RB, int W, int TM>
__global__ __launch_bounds__(W * 64) void dec_down_kernel(const uint8_t* __restrict__ dbase, int64_t dstride, int N,
                                                          int K, const float* __restrict__ inter,
                                                          const float* __restrict__ isum_in,
                                                          const int32_t* __restrict__ offsets,
                                                          const int32_t* __restrict__ perm,
                                                          const int32_t* __restrict__ active,
                                                          const int32_t* __restrict__ n_active,
                                                          const float* __restrict__ topk_w,
                                                          float* __restrict__ partial) {
    constexpr int KS = 64 / RB;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int a = blockIdx.y;
    if (a >= *n_active) return;
    const int e = active[a];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int r = lane % RB, ks = lane / RB;
    const int row = blockIdx.x * RB + r;
    const int nb = K >> 8;
    const int j0 = ks + KS * w;
    float* iss = (float*)smem;
    float* red = (float*)(smem + (isum_in ? 0 : (size_t)TM * (K >> 4) * 4));
    const uint8_t* dm = dbase + (int64_t)e * dstride;
    const int p_begin = offsets[e], p_end = offsets[e + 1];
    for (int p0 = p_begin; p0 < p_end; p0 += TM) {
        const int me = min(TM, p_end - p0);
        Raw<QT> rw;
        if (j0 < nb) load_raw<QT>(rw, dm, N, nb, row, j0);
        const float* sums = isum_in ? isum_in + (int64_t)p0 * (K >> 4) : iss;
        if (!isum_in) {
            __syncthreads();
            for (int i = tid; i < me * (K >> 4); i += W * 64) {
                const float* p = inter + (int64_t)(p0 + i / (K >> 4)) * K + 16 * (i % (K >> 4));
                float sm = 0.f;
#pragma unroll
                for (int k = 0; k < 16; ++k) sm += p[k];
                iss[i] = sm;
            }
            __syncthreads();
        }
        float acc[TM];
#pragma unroll
        for (int t = 0; t < TM; ++t) acc[t] = 0.f;
        for (int j = j0; j < nb; j += KS * W) {
            if (j != j0) load_raw<QT>(rw, dm, N, nb, row, j);
            dn_compute<TM>(rw, inter + (int64_t)p0 * K + 256 * j, sums + 16 * j, K, me, acc);
        }
#pragma unroll
        for (int t = 0; t < TM; ++t) acc[t] = kslot_sum<RB>(acc[t]);
        __syncthreads();
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
            if (orow < N) partial[(int64_t)(p0 + t) * N + orow] = topk_w[perm[p0 + t]] * v;
        }
    }
}

// ============================================================================ launch plumbing
// Block shapes (rows per block RB, waves W <= 4 so every wave may use up to 512 VGPRs):
// one super-block per lane when nb equals KS * W for one of them, else (16, 4) with a
// K loop.
struct DecShape {
    int RB, W;
};

inline DecShape pick_shape(int nb) {
    static const DecShape menu[] = {{16, 1}, {16, 2}, {16, 4}, {32, 1}, {32, 2}, {32, 4},
                                    {64, 1}, {64, 2}, {64, 3}, {64, 4}};
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

template <int QT, int RB, int W, int TM>
inline void gu_launch(const Mats& g, const Mats& u, const uint16_t* x, const float* xsum, int topk,
                      const int32_t* offsets, const int32_t* perm, const int32_t* active, const int32_t* n_active,
                      int max_active, float* inter, float* isum, hipStream_t st) {
    const size_t stage = (size_t)TM * g.K * 2 + (size_t)TM * (g.K / 16) * 4;
    const size_t tail = (size_t)W * TM * 2 * RB * 4 + (size_t)TM * RB * 4;
    const size_t sh = stage > tail ? stage : tail;
    hipLaunchKernelGGL((dec_gateup_kernel<QT, RB, W, TM>), dim3(div_up(g.N, RB), max_active), dim3(64 * W), sh, st,
                       g.base, u.base, g.stride, u.stride, g.N, g.K, x, xsum, topk, offsets, perm, active, n_active,
                       inter, isum);
}

template <int QT, int RB, int W, int TM>
inline void dn_launch(const Mats& d, const float* inter, const float* isum, const int32_t* offsets,
                      const int32_t* perm, const int32_t* active, const int32_t* n_active, int max_active,
                      const float* topk_w, float* partial, hipStream_t st) {
    const size_t sh = (isum ? 0 : (size_t)TM * (d.K / 16) * 4) + (size_t)W * TM * RB * 4;
    hipLaunchKernelGGL((dec_down_kernel<QT, RB, W, TM>), dim3(div_up(d.N, RB), max_active), dim3(64 * W), sh, st,
                       d.base, d.stride, d.N, d.K, inter, isum, offsets, perm, active, n_active, topk_w, partial);
}

#define PG_TM(F, QT, RB, W, ...)                   \
    switch (TM) {                                 \
    case 1: F<QT, RB, W, 1>(__VA_ARGS__); break;  \
    case 2: F<QT, RB, W, 2>(__VA_ARGS__); break;  \
    case 4: F<QT, RB, W, 4>(__VA_ARGS__); break;  \
    default: F<QT, RB, W, 8>(__VA_ARGS__); break; \
    }

#define PG_SHAPES(F, QT, ...)                                  \
    switch (sp.RB * 16 + sp.W) {                               \
    case 16 * 16 + 1: PG_TM(F, QT, 16, 1, __VA_ARGS__); break; \
    case 16 * 16 + 2: PG_TM(F, QT, 16, 2, __VA_ARGS__); break; \
    case 32 * 16 + 1: PG_TM(F, QT, 32, 1, __VA_ARGS__); break; \
    case 32 * 16 + 2: PG_TM(F, QT, 32, 2, __VA_ARGS__); break; \
    case 32 * 16 + 4: PG_TM(F, QT, 32, 4, __VA_ARGS__); break; \
    case 64 * 16 + 1: PG_TM(F, QT, 64, 1, __VA_ARGS__); break; \
    case 64 * 16 + 2: PG_TM(F, QT, 64, 2, __VA_ARGS__); break; \
    case 64 * 16 + 3: PG_TM(F, QT, 64, 3, __VA_ARGS__); break; \
    case 64 * 16 + 4: PG_TM(F, QT, 64, 4, __VA_ARGS__); break; \
    default: PG_TM(F, QT, 16, 4, __VA_ARGS__); break;          \
    }

// Per-qtype launchers (defined in decode_q4k.hip / decode_q6k.hip / decode_q8_0.hip).
template <int QT>
int dec_gateup_q(const Mats& g, const Mats& u, const uint16_t* x, const float* xsum, int topk, int M,
                 const int32_t* offsets, const int32_t* perm, const int32_t* active, const int32_t* n_active,
                 int max_active, float* inter, float* isum, hipStream_t st);
template <int QT>
int dec_down_q(const Mats& d, const float* inter, const float* isum, int M, const int32_t* offsets,
               const int32_t* perm, const int32_t* active, const int32_t* n_active, int max_active,
               const float* topk_w, float* partial, hipStream_t st);

#define PG_DEFINE_DECODE_LAUNCHERS(QT)                                                                                \
    template <>                                                                                                      \
    int dec_gateup_q<QT>(const Mats& g, const Mats& u, const uint16_t* x, const float* xsum, int topk, int M,       \
                         const int32_t* offsets, const int32_t* perm, const int32_t* active,                        \
                         const int32_t* n_active, int max_active, float* inter, float* isum, hipStream_t st) {      \
        const DecShape sp = pick_shape(g.K >> 8);                                                                    \
        const int TM = tile_tokens(M, g.K);                                                                          \
        if ((size_t)TM * g.K * 2 + (size_t)TM * (g.K / 16) * 4 > 64 * 1024)                                         \
            return fail(PGMOE_E_UNSUPPORTED, "decode gate/up: %d inputs exceed the LDS stage", g.K);                 \
        PG_SHAPES(gu_launch, QT, g, u, x, xsum, topk, offsets, perm, active, n_active, max_active, inter, isum, st);  \
        return check_launch("dec_gateup");                                                                           \
    }                                                                                                                \
    template <>                                                                                                      \
    int dec_down_q<QT>(const Mats& d, const float* inter, const float* isum, int M, const int32_t* offsets,         \
                       const int32_t* perm, const int32_t* active, const int32_t* n_active, int max_active,         \
                       const float* topk_w, float* partial, hipStream_t st) {                                        \
        const DecShape sp = pick_shape(d.K >> 8);                                                                    \
        const int TM = tile_tokens(M, 0);                                                                            \
        if (!isum && (size_t)TM * (d.K / 16) * 4 + (size_t)sp.W * TM * sp.RB * 4 > 64 * 1024)                        \
            return fail(PGMOE_E_UNSUPPORTED, "decode down: LDS stage too large");                                    \
        PG_SHAPES(dn_launch, QT, d, inter, isum, offsets, perm, active, n_active, max_active, topk_w, partial, st);   \
        return check_launch("dec_down");                                                                             \
    }

}  // namespace pgmoe
