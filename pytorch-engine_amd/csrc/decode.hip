// Decode path (M <= 8 tokens): three launches per layer.
//   route   : router logits (fixed order), top-k, softmax, dispatch -- the last block
//             finishing its logits does top-k and the counting sort (no host sync)
//   gate/up : per active expert, 64 rows per block, lane = row, wave = K-slice;
//             fp16 magic-number dequant feeding v_dot2_f32_f16, SwiGLU in the epilogue
//   down    : same structure in fp32 on the SwiGLU output; the last block per row group
//             sums the token's experts in ascending id (deterministic combine)
// Reference: pygguf_engine/model.py:898-937; quant_kernels.py:68-311 (GEMV kernels it
// replaces), :1423-1475 (SwiGLU + row-scale).
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

// ============================================================================ gate/up
// acc_g[t] += x_t . g_row(block b), acc_u[t] += x_t . u_row(block b) for one 256-weight
// block; tg/tu point at this lane's row inside the tiles; xs = LDS fp16 x rows (row
// stride K) already offset to the block; xsum = LDS 16-element sums (stride K/16),
// offset to the block.
template <int QT> struct GateUp;

template <> struct GateUp<PGMOE_Q4_K> {
    __device__ static __forceinline__ void block(const uint8_t* tg, const uint8_t* tu, const uint16_t* xs,
                                                 const float* xsum, int K, int me, float* ag, float* au) {
        uint4 hg = *(const uint4*)tg, hu = *(const uint4*)tu;
        uint4 qg[8], qu[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            qg[c] = *(const uint4*)(tg + (1 + c) * 1024);
            qu[c] = *(const uint4*)(tu + (1 + c) * 1024);
        }
        const float dg = lo_half(hg.x), mg = hi_half(hg.x), du = lo_half(hu.x), mu = hi_half(hu.x);
#pragma unroll
        for (int c2 = 0; c2 < 4; ++c2) {  // qs bytes 32c2..32c2+31: sub-blocks 2c2 (low), 2c2+1 (high)
            int s0, m0, s1, m1;
            kscale(hg.y, hg.z, hg.w, 2 * c2, s0, m0);
            kscale(hg.y, hg.z, hg.w, 2 * c2 + 1, s1, m1);
            const float ga0 = dg * (float)s0, gb0 = mg * (float)m0 + 1024.0f * ga0;
            const float ga1 = dg * (float)s1, gb1 = mg * (float)m1 + 1024.0f * ga1;
            kscale(hu.y, hu.z, hu.w, 2 * c2, s0, m0);
            kscale(hu.y, hu.z, hu.w, 2 * c2 + 1, s1, m1);
            const float ua0 = du * (float)s0, ub0 = mu * (float)m0 + 1024.0f * ua0;
            const float ua1 = du * (float)s1, ub1 = mu * (float)m1 + 1024.0f * ua1;
            uint32_t gw[8], uw[8];
            gw[0] = qg[2 * c2].x; gw[1] = qg[2 * c2].y; gw[2] = qg[2 * c2].z; gw[3] = qg[2 * c2].w;
            gw[4] = qg[2 * c2 + 1].x; gw[5] = qg[2 * c2 + 1].y; gw[6] = qg[2 * c2 + 1].z; gw[7] = qg[2 * c2 + 1].w;
            uw[0] = qu[2 * c2].x; uw[1] = qu[2 * c2].y; uw[2] = qu[2 * c2].z; uw[3] = qu[2 * c2].w;
            uw[4] = qu[2 * c2 + 1].x; uw[5] = qu[2 * c2 + 1].y; uw[6] = qu[2 * c2 + 1].z; uw[7] = qu[2 * c2 + 1].w;
            uint32_t gl[16], gh[16], ul[16], uh[16];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const uint32_t a = gw[k] & 0x0f0f0f0fu, b = (gw[k] >> 4) & 0x0f0f0f0fu;
                gl[2 * k] = magic2(a, kSel01);
                gl[2 * k + 1] = magic2(a, kSel23);
                gh[2 * k] = magic2(b, kSel01);
                gh[2 * k + 1] = magic2(b, kSel23);
                const uint32_t c = uw[k] & 0x0f0f0f0fu, d = (uw[k] >> 4) & 0x0f0f0f0fu;
                ul[2 * k] = magic2(c, kSel01);
                ul[2 * k + 1] = magic2(c, kSel23);
                uh[2 * k] = magic2(d, kSel01);
                uh[2 * k + 1] = magic2(d, kSel23);
            }
            for (int t = 0; t < me; ++t) {
                const uint16_t* xr = xs + t * K + 64 * c2;
                float tgl = 0.f, tgh = 0.f, tul = 0.f, tuh = 0.f;
#pragma unroll
                for (int k = 0; k < 16; ++k) {
                    const uint32_t xl = ld32(xr + 2 * k), xh = ld32(xr + 32 + 2 * k);
                    tgl = dot2(gl[k], xl, tgl);
                    tgh = dot2(gh[k], xh, tgh);
                    tul = dot2(ul[k], xl, tul);
                    tuh = dot2(uh[k], xh, tuh);
                }
                const float* sx = xsum + t * (K >> 4) + 4 * c2;
                const float S0 = sx[0] + sx[1], S1 = sx[2] + sx[3];
                ag[t] += ga0 * tgl - gb0 * S0 + ga1 * tgh - gb1 * S1;
                au[t] += ua0 * tul - ub0 * S0 + ua1 * tuh - ub1 * S1;
            }
        }
    }
};

template <> struct GateUp<PGMOE_Q8_0> {
    // Q8_0 code q in [-128, 127]: byte ^ 0x80 = q + 128, so the fp16 value is 1152 + q.
    __device__ static __forceinline__ void one(const uint8_t* t, const uint16_t* xs, const float* xsum, int K,
                                               int me, float* acc) {
        uint4 q[16];
#pragma unroll
        for (int c = 0; c < 16; ++c) q[c] = *(const uint4*)(t + c * 1024);
        const uint4 dv0 = *(const uint4*)(t + 16 * 1024);
        const uint32_t dw[4] = {dv0.x, dv0.y, dv0.z, dv0.w};
#pragma unroll
        for (int j = 0; j < 8; ++j) {  // Q8_0 block j: chunks 2j, 2j+1
            const float d = (j & 1) ? hi_half(dw[j >> 1]) : lo_half(dw[j >> 1]);
            const uint32_t w8[8] = {q[2 * j].x, q[2 * j].y, q[2 * j].z, q[2 * j].w,
                                    q[2 * j + 1].x, q[2 * j + 1].y, q[2 * j + 1].z, q[2 * j + 1].w};
            uint32_t m[16];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const uint32_t v = w8[k] ^ 0x80808080u;
                m[2 * k] = magic2(v, kSel01);
                m[2 * k + 1] = magic2(v, kSel23);
            }
            for (int tt = 0; tt < me; ++tt) {
                const uint16_t* xr = xs + tt * K + 32 * j;
                float T = 0.f;
#pragma unroll
                for (int k = 0; k < 16; ++k) T = dot2(m[k], ld32(xr + 2 * k), T);
                const float* sx = xsum + tt * (K >> 4) + 2 * j;
                acc[tt] += d * (T - 1152.0f * (sx[0] + sx[1]));
            }
        }
    }
    __device__ static __forceinline__ void block(const uint8_t* tg, const uint8_t* tu, const uint16_t* xs,
                                                 const float* xsum, int K, int me, float* ag, float* au) {
        one(tg, xs, xsum, K, me, ag);
        one(tu, xs, xsum, K, me, au);
    }
};

template <> struct GateUp<PGMOE_Q6_K> {
    // fp16 value 1024 + q6 (q6 = 6-bit code), weight = d*sc*(q6 - 32).
    __device__ static __forceinline__ void one(const uint8_t* t, const uint8_t* dptr, const uint16_t* xs,
                                               const float* xsum, int K, int me, float* acc) {
        uint4 c[13];
#pragma unroll
        for (int i = 0; i < 13; ++i) c[i] = *(const uint4*)(t + i * 1024);
        const float d = h2f(*(const uint16_t*)dptr);
        const uint32_t ql[32] = {c[0].x, c[0].y, c[0].z, c[0].w, c[1].x, c[1].y, c[1].z, c[1].w,
                                 c[2].x, c[2].y, c[2].z, c[2].w, c[3].x, c[3].y, c[3].z, c[3].w,
                                 c[4].x, c[4].y, c[4].z, c[4].w, c[5].x, c[5].y, c[5].z, c[5].w,
                                 c[6].x, c[6].y, c[6].z, c[6].w, c[7].x, c[7].y, c[7].z, c[7].w};
        const uint32_t qh[16] = {c[8].x, c[8].y, c[8].z, c[8].w, c[9].x, c[9].y, c[9].z, c[9].w,
                                 c[10].x, c[10].y, c[10].z, c[10].w, c[11].x, c[11].y, c[11].z, c[11].w};
        const uint32_t scw[4] = {c[12].x, c[12].y, c[12].z, c[12].w};
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                uint32_t m[16];
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    const uint32_t q = q6_word(ql[16 * h + k], ql[16 * h + 8 + k], qh[8 * h + k], s);
                    m[2 * k] = magic2(q, kSel01);
                    m[2 * k + 1] = magic2(q, kSel23);
                }
                const int sb = 8 * h + 2 * s;  // sub-scales sb (k < 4) and sb + 1 (k >= 4)
                const float a0 = d * (float)(int8_t)((scw[sb >> 2] >> (8 * (sb & 3))) & 0xff);
                const float a1 = d * (float)(int8_t)((scw[(sb + 1) >> 2] >> (8 * ((sb + 1) & 3))) & 0xff);
                for (int tt = 0; tt < me; ++tt) {
                    const uint16_t* xr = xs + tt * K + 128 * h + 32 * s;
                    float T0 = 0.f, T1 = 0.f;
#pragma unroll
                    for (int k = 0; k < 8; ++k) T0 = dot2(m[k], ld32(xr + 2 * k), T0);
#pragma unroll
                    for (int k = 8; k < 16; ++k) T1 = dot2(m[k], ld32(xr + 2 * k), T1);
                    const float* sx = xsum + tt * (K >> 4) + 8 * h + 2 * s;
                    acc[tt] += a0 * (T0 - 1056.0f * sx[0]) + a1 * (T1 - 1056.0f * sx[1]);
                }
            }
    }
};

template <int QT>
__device__ __forceinline__ void gateup_block(const uint8_t* gm, const uint8_t* um, int N, int nb, int rg, int b,
                                             int lane, const uint16_t* xs, const float* xsum, int K, int me,
                                             float* ag, float* au) {
    const uint8_t* tg = tile_ptr<QT>(gm, nb, rg, b) + lane * 16;
    const uint8_t* tu = tile_ptr<QT>(um, nb, rg, b) + lane * 16;
    if constexpr (QT == PGMOE_Q6_K) {
        const int64_t dpl = (int64_t)row_groups(N) * nb * 13 * 1024 + (((int64_t)rg * nb + b) * 64 + lane) * 2;
        GateUp<QT>::one(tg, gm + dpl, xs + 256 * b, xsum + 16 * b, K, me, ag);
        GateUp<QT>::one(tu, um + dpl, xs + 256 * b, xsum + 16 * b, K, me, au);
    } else {
        GateUp<QT>::block(tg, tu, xs + 256 * b, xsum + 16 * b, K, me, ag, au);
    }
}

// Block = one row group (64 rows) of one active expert; WPB waves split the K blocks.
// LDS: xs [tmc][K] fp16 | xsum [tmc][K/16] f32; the cross-wave partials reuse xs.
template <int QT, int WPB>
__global__ __launch_bounds__(WPB * 64) void dec_gateup_kernel(const uint8_t* __restrict__ gbase,
                                                              const uint8_t* __restrict__ ubase, int64_t gstride,
                                                              int64_t ustride, int N, int K, int tmc,
                                                              const uint16_t* __restrict__ x, int topk,
                                                              const int32_t* __restrict__ offsets,
                                                              const int32_t* __restrict__ perm,
                                                              const int32_t* __restrict__ active,
                                                              const int32_t* __restrict__ n_active,
                                                              float* __restrict__ inter) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int a = blockIdx.y;
    if (a >= *n_active) return;
    const int e = active[a];
    const int rg = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int nb = K >> 8;
    uint16_t* xs = (uint16_t*)smem;
    float* xsum = (float*)(smem + (size_t)tmc * K * 2);
    float* red = (float*)smem;  // [WPB][tmc][2][64], used after the K loop
    const uint8_t* gm = gbase + (int64_t)e * gstride;
    const uint8_t* um = ubase + (int64_t)e * ustride;
    const int p_begin = offsets[e], p_end = offsets[e + 1];
    for (int p0 = p_begin; p0 < p_end; p0 += tmc) {
        const int me = min(tmc, p_end - p0);
        __syncthreads();
        for (int i = tid; i < me * (K >> 3); i += WPB * 64) {
            const int t = i / (K >> 3), c = i % (K >> 3);
            const int tok = perm[p0 + t] / topk;
            *(uint4*)(xs + t * K + 8 * c) = *(const uint4*)(x + (int64_t)tok * K + 8 * c);
        }
        __syncthreads();
        for (int i = tid; i < me * (K >> 4); i += WPB * 64) {
            const int t = i / (K >> 4), j = i % (K >> 4);
            const uint16_t* p = xs + t * K + 16 * j;
            float s = 0.f;
#pragma unroll
            for (int k = 0; k < 16; ++k) s += h2f(p[k]);
            xsum[i] = s;
        }
        __syncthreads();
        float ag[kDecTM], au[kDecTM];
#pragma unroll
        for (int t = 0; t < kDecTM; ++t) ag[t] = au[t] = 0.f;
        for (int b = w; b < nb; b += WPB) gateup_block<QT>(gm, um, N, nb, rg, b, lane, xs, xsum, K, me, ag, au);
        __syncthreads();  // all waves done with xs before it is reused for partials
#pragma unroll
        for (int t = 0; t < kDecTM; ++t) {
            if (t < me) {
                red[((w * tmc + t) * 2 + 0) * 64 + lane] = ag[t];
                red[((w * tmc + t) * 2 + 1) * 64 + lane] = au[t];
            }
        }
        __syncthreads();
        for (int i = tid; i < me * 64; i += WPB * 64) {
            const int t = i >> 6, r = i & 63;
            float g = 0.f, u = 0.f;
#pragma unroll
            for (int ww = 0; ww < WPB; ++ww) {
                g += red[((ww * tmc + t) * 2 + 0) * 64 + r];
                u += red[((ww * tmc + t) * 2 + 1) * 64 + r];
            }
            const int row = 64 * rg + r;
            if (row < N) inter[(int64_t)(p0 + t) * N + row] = silu(g) * u;
        }
    }
}

// ============================================================================ down
// acc[t] += inter_t . d_row(block b) in fp32.  x = inter rows (global, wave-uniform),
// isum = LDS 16-element sums of those rows (stride K/16), both offset to the block.
template <int QT> struct Down;

template <> struct Down<PGMOE_Q6_K> {
    __device__ static __forceinline__ void block(const uint8_t* t, const uint8_t* dptr, const float* x,
                                                 const float* isum, int K, int me, float* acc) {
        uint4 c[13];
#pragma unroll
        for (int i = 0; i < 13; ++i) c[i] = *(const uint4*)(t + i * 1024);
        const float d = h2f(*(const uint16_t*)dptr);
        const uint32_t ql[32] = {c[0].x, c[0].y, c[0].z, c[0].w, c[1].x, c[1].y, c[1].z, c[1].w,
                                 c[2].x, c[2].y, c[2].z, c[2].w, c[3].x, c[3].y, c[3].z, c[3].w,
                                 c[4].x, c[4].y, c[4].z, c[4].w, c[5].x, c[5].y, c[5].z, c[5].w,
                                 c[6].x, c[6].y, c[6].z, c[6].w, c[7].x, c[7].y, c[7].z, c[7].w};
        const uint32_t qh[16] = {c[8].x, c[8].y, c[8].z, c[8].w, c[9].x, c[9].y, c[9].z, c[9].w,
                                 c[10].x, c[10].y, c[10].z, c[10].w, c[11].x, c[11].y, c[11].z, c[11].w};
        const uint32_t scw[4] = {c[12].x, c[12].y, c[12].z, c[12].w};
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
                        const uint32_t q = q6_word(ql[16 * h + kk], ql[16 * h + 8 + kk], qh[8 * h + kk], s);
                        qf[4 * k + 0] = (float)(q & 0xff);
                        qf[4 * k + 1] = (float)((q >> 8) & 0xff);
                        qf[4 * k + 2] = (float)((q >> 16) & 0xff);
                        qf[4 * k + 3] = (float)(q >> 24);
                    }
                    const int sb = 8 * h + 2 * s + half;
                    const float a = d * (float)(int8_t)((scw[sb >> 2] >> (8 * (sb & 3))) & 0xff);
                    for (int tt = 0; tt < me; ++tt) {
                        const float* xr = x + (int64_t)tt * K + 128 * h + 32 * s + 16 * half;
                        float T = 0.f;
#pragma unroll
                        for (int i = 0; i < 16; ++i) T = __builtin_fmaf(qf[i], xr[i], T);
                        acc[tt] += a * (T - 32.0f * isum[tt * (K >> 4) + sb]);
                    }
                }
    }
};

template <> struct Down<PGMOE_Q4_K> {
    __device__ static __forceinline__ void block(const uint8_t* t, const uint8_t*, const float* x,
                                                 const float* isum, int K, int me, float* acc) {
        const uint4 hd = *(const uint4*)t;
        uint4 q[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) q[c] = *(const uint4*)(t + (1 + c) * 1024);
        const float dd = lo_half(hd.x), dm = hi_half(hd.x);
#pragma unroll
        for (int s = 0; s < 8; ++s) {  // sub-block s: qs bytes 32(s/2).. nibble s&1
            int sc, mn;
            kscale(hd.y, hd.z, hd.w, s, sc, mn);
            const float a = dd * (float)sc, bm = dm * (float)mn;
            const int c2 = s >> 1, sh = 4 * (s & 1);
            const uint32_t w8[8] = {q[2 * c2].x, q[2 * c2].y, q[2 * c2].z, q[2 * c2].w,
                                    q[2 * c2 + 1].x, q[2 * c2 + 1].y, q[2 * c2 + 1].z, q[2 * c2 + 1].w};
            float qf[32];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const uint32_t v = (w8[k] >> sh) & 0x0f0f0f0fu;
                qf[4 * k + 0] = (float)(v & 0xff);
                qf[4 * k + 1] = (float)((v >> 8) & 0xff);
                qf[4 * k + 2] = (float)((v >> 16) & 0xff);
                qf[4 * k + 3] = (float)(v >> 24);
            }
            for (int tt = 0; tt < me; ++tt) {
                const float* xr = x + (int64_t)tt * K + 32 * s;
                float T = 0.f;
#pragma unroll
                for (int i = 0; i < 32; ++i) T = __builtin_fmaf(qf[i], xr[i], T);
                const float* sx = isum + tt * (K >> 4) + 2 * s;
                acc[tt] += a * T - bm * (sx[0] + sx[1]);
            }
        }
    }
};

template <> struct Down<PGMOE_Q8_0> {
    __device__ static __forceinline__ void block(const uint8_t* t, const uint8_t*, const float* x,
                                                 const float* isum, int K, int me, float* acc) {
        uint4 q[16];
#pragma unroll
        for (int c = 0; c < 16; ++c) q[c] = *(const uint4*)(t + c * 1024);
        const uint4 dv = *(const uint4*)(t + 16 * 1024);
        const uint32_t dw[4] = {dv.x, dv.y, dv.z, dv.w};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float d = (j & 1) ? hi_half(dw[j >> 1]) : lo_half(dw[j >> 1]);
            const uint32_t w8[8] = {q[2 * j].x, q[2 * j].y, q[2 * j].z, q[2 * j].w,
                                    q[2 * j + 1].x, q[2 * j + 1].y, q[2 * j + 1].z, q[2 * j + 1].w};
            float qf[32];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const uint32_t v = w8[k] ^ 0x80808080u;  // q + 128 per byte
                qf[4 * k + 0] = (float)(v & 0xff);
                qf[4 * k + 1] = (float)((v >> 8) & 0xff);
                qf[4 * k + 2] = (float)((v >> 16) & 0xff);
                qf[4 * k + 3] = (float)(v >> 24);
            }
            for (int tt = 0; tt < me; ++tt) {
                const float* xr = x + (int64_t)tt * K + 32 * j;
                float T = 0.f;
#pragma unroll
                for (int i = 0; i < 32; ++i) T = __builtin_fmaf(qf[i], xr[i], T);
                const float* sx = isum + tt * (K >> 4) + 2 * j;
                acc[tt] += d * (T - 128.0f * (sx[0] + sx[1]));
            }
        }
    }
};

// Block = one row group (64 output rows) of one active expert.  Writes
// partial[p, row] = w[perm[p]] * (inter_p . d_row).  With `out` set, the last block of
// the row group (across all active experts) then writes
// out[t, row] = sum of the token's partials in ascending expert id (+ shared * gate).
template <int QT, int WPB>
__global__ __launch_bounds__(WPB * 64) void dec_down_kernel(
    const uint8_t* __restrict__ dbase, int64_t dstride, int N, int K, int tmc, const float* __restrict__ inter,
    const int32_t* __restrict__ offsets, const int32_t* __restrict__ perm, const int32_t* __restrict__ active,
    const int32_t* __restrict__ n_active, const float* __restrict__ topk_w, float* __restrict__ partial, int M,
    int topk, const int32_t* __restrict__ inv, const float* __restrict__ shared,
    const float* __restrict__ shared_logit, float* __restrict__ out, int32_t* __restrict__ counters) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    __shared__ int last;
    const int a = blockIdx.y;
    const int nact = *n_active;
    const bool live = a < nact;
    const int rg = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int nb = K >> 8;
    float* isum = (float*)smem;                         // [tmc][K/16]
    float* red = (float*)(smem + (size_t)tmc * (K >> 4) * 4);  // [WPB][tmc][64]
    if (live) {
        const int e = active[a];
        const uint8_t* dm = dbase + (int64_t)e * dstride;
        const int64_t dpl = (int64_t)row_groups(N) * nb * 13 * 1024;
        const int p_begin = offsets[e], p_end = offsets[e + 1];
        for (int p0 = p_begin; p0 < p_end; p0 += tmc) {
            const int me = min(tmc, p_end - p0);
            __syncthreads();
            for (int i = tid; i < me * (K >> 4); i += WPB * 64) {
                const int t = i / (K >> 4), j = i % (K >> 4);
                const float* p = inter + (int64_t)(p0 + t) * K + 16 * j;
                float s = 0.f;
#pragma unroll
                for (int k = 0; k < 16; ++k) s += p[k];
                isum[i] = s;
            }
            __syncthreads();
            float acc[kDecTM];
#pragma unroll
            for (int t = 0; t < kDecTM; ++t) acc[t] = 0.f;
            for (int b = w; b < nb; b += WPB) {
                const uint8_t* tl = tile_ptr<QT>(dm, nb, rg, b) + lane * 16;
                const uint8_t* dp = dm + dpl + (((int64_t)rg * nb + b) * 64 + lane) * 2;
                Down<QT>::block(tl, dp, inter + (int64_t)p0 * K + 256 * b, isum + 16 * b, K, me, acc);
            }
#pragma unroll
            for (int t = 0; t < kDecTM; ++t)
                if (t < me) red[(w * tmc + t) * 64 + lane] = acc[t];
            __syncthreads();
            for (int i = tid; i < me * 64; i += WPB * 64) {
                const int t = i >> 6, r = i & 63;
                float v = 0.f;
#pragma unroll
                for (int ww = 0; ww < WPB; ++ww) v += red[(ww * tmc + t) * 64 + r];
                const int row = 64 * rg + r;
                if (row < N) partial[(int64_t)(p0 + t) * N + row] = topk_w[perm[p0 + t]] * v;
            }
        }
    }
    if (!out) return;
    // deterministic combine by the last block of this row group
    __threadfence();
    __syncthreads();
    if (tid == 0) last = live ? (atomicAdd(&counters[rg], 1) == nact - 1) : 0;
    __syncthreads();
    if (!last) return;
    __threadfence();
    for (int i = tid; i < M * 64; i += WPB * 64) {
        const int t = i >> 6, r = i & 63;
        const int row = 64 * rg + r;
        if (row >= N) continue;
        int pos[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) pos[k] = k < topk ? inv[t * topk + k] : 0x7fffffff;
        for (int x1 = 1; x1 < topk; ++x1) {  // ascending position = ascending expert id
            const int v = pos[x1];
            int y = x1 - 1;
            while (y >= 0 && pos[y] > v) {
                pos[y + 1] = pos[y];
                --y;
            }
            pos[y + 1] = v;
        }
        float acc = 0.f;
        for (int k = 0; k < topk; ++k) acc += partial[(int64_t)pos[k] * N + row];
        if (shared) {
            const float g = shared_logit ? 1.0f / (1.0f + expf(-shared_logit[t])) : 1.0f;
            acc += shared[(int64_t)t * N + row] * g;
        }
        out[(int64_t)t * N + row] = acc;
    }
    __syncthreads();
    if (tid == 0) counters[rg] = 0;
}

// ============================================================================ route
// Blocks of 4 waves; wave = one router row (expert, or the shared-expert gate vector as
// row E) for all M <= 8 tokens, in the fixed order of the CPU oracle.  The last block
// to finish then does top-k + softmax per token and the stable dispatch of the M*K
// pairs, writes the identity dispatch of the shared expert, and resets the counter.
template <int R>
__global__ __launch_bounds__(256) void route_small_kernel(
    const uint16_t* __restrict__ x, const float* __restrict__ W, const float* __restrict__ bias,
    const float* __restrict__ sh_w, int M, int H, int E, int K, int norm, float* __restrict__ logits,
    float* __restrict__ s_logit, int32_t* __restrict__ idx_out, float* __restrict__ w_out,
    int32_t* __restrict__ offsets, int32_t* __restrict__ perm, int32_t* __restrict__ inv,
    int32_t* __restrict__ active, int32_t* __restrict__ n_active, int32_t* __restrict__ s_disp,
    float* __restrict__ s_w, int32_t* __restrict__ counter) {
    constexpr int TM = kDecTM;
    __shared__ int s_idx[TM * 16];
    __shared__ float s_wt[TM * 16];
    __shared__ uint32_t used[16];
    __shared__ int last;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int rows = E + (sh_w ? 1 : 0);
    const int e = blockIdx.x * 4 + wv;
    if (e < rows) {
        const float* wr = e < E ? W + (int64_t)e * H : sh_w;
        float acc[TM];
#pragma unroll
        for (int i = 0; i < TM; ++i) acc[i] = 0.f;
        const int C = H >> 3;
        for (int c = lane; c < C; c += 64) {
            const float4 w0 = *(const float4*)(wr + 8 * c);
            const float4 w1 = *(const float4*)(wr + 8 * c + 4);
            const float wv8[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                if (i < M) {
                    const uint4 v = *(const uint4*)(x + (int64_t)i * H + 8 * c);
                    const uint32_t x4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        acc[i] = __builtin_fmaf(lo_half(x4[k]), wv8[2 * k], acc[i]);
                        acc[i] = __builtin_fmaf(hi_half(x4[k]), wv8[2 * k + 1], acc[i]);
                    }
                }
            }
        }
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            if (i < M) {
                float v = group_sum<64>(acc[i]);
                if (lane == 0) {
                    if (e < E) logits[i * E + e] = bias ? v + bias[e] : v;
                    else s_logit[i] = v;
                }
            }
        }
    }
    __threadfence();
    __syncthreads();
    if (tid == 0) last = atomicAdd(counter, 1) == (int)gridDim.x - 1;
    __syncthreads();
    if (!last) return;
    __threadfence();
    if (tid < 16) used[tid] = 0u;
    // top-k per token: one wave per token
    for (int m = wv; m < M; m += 4) {
        const float* l = logits + m * E;
        float v[R];
        bool taken[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int ee = lane + 64 * r;
            v[r] = ee < E ? l[ee] : 0.f;
            taken[r] = ee >= E;
        }
        float top = 0.f, my_v = 0.f;
        int my_id = 0;
        for (int k = 0; k < K; ++k) {
            float bv = -INFINITY;
            int bi = 0x7fffffff;
#pragma unroll
            for (int r = 0; r < R; ++r)
                if (!taken[r] && (bi == 0x7fffffff || v[r] > bv)) {
                    bv = v[r];
                    bi = lane + 64 * r;
                }
#pragma unroll
            for (int s = 32; s >= 1; s >>= 1) {
                const float ov = __shfl_xor(bv, s, 64);
                const int oi = __shfl_xor(bi, s, 64);
                if (oi != 0x7fffffff && (bi == 0x7fffffff || ov > bv || (ov == bv && oi < bi))) {
                    bv = ov;
                    bi = oi;
                }
            }
#pragma unroll
            for (int r = 0; r < R; ++r)
                if (lane + 64 * r == bi) taken[r] = true;
            if (k == 0) top = bv;
            if (lane == k) {
                my_id = bi;
                my_v = bv;
            }
        }
        float den = 0.f;
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (lane + 64 * r < E) den += expf(v[r] - top);
        den = group_sum<64>(den);
        float p = lane < K ? expf(my_v - top) / den : 0.f;
        const float sp = group_sum<64>(p);
        if (norm) p = p / fmaxf(sp, 1e-20f);
        if (lane < K) {
            s_idx[m * K + lane] = my_id;
            s_wt[m * K + lane] = p;
        }
    }
    __syncthreads();
    const int P = M * K;
    for (int f = tid; f < P; f += 256) atomicOr(&used[s_idx[f] >> 5], 1u << (s_idx[f] & 31));
    __syncthreads();
    for (int f = tid; f < P; f += 256) {
        const int ef = s_idx[f];
        int pos = 0;
        for (int j = 0; j < P; ++j) {
            const int ej = s_idx[j];
            pos += (ej < ef) || (ej == ef && j < f);
        }
        perm[pos] = f;
        inv[f] = pos;
        idx_out[f] = ef;
        w_out[f] = s_wt[f];
    }
    for (int ee = tid; ee <= E; ee += 256) {
        int c = 0;
        for (int j = 0; j < P; ++j) c += s_idx[j] < ee;
        offsets[ee] = c;
    }
    for (int ee = tid; ee < E; ee += 256) {
        if ((used[ee >> 5] >> (ee & 31)) & 1u) {
            int rank = __popc(used[ee >> 5] & ((1u << (ee & 31)) - 1u));
            for (int q = 0; q < (ee >> 5); ++q) rank += __popc(used[q]);
            active[rank] = ee;
        }
    }
    if (tid == 0) {
        int tot = 0;
        for (int q = 0; q < 16; ++q) tot += __popc(used[q]);
        *n_active = tot;
    }
    if (s_disp) {  // shared expert: offsets {0, M}, perm = identity, active {0}, n_active 1, w = 1
        if (tid == 0) {
            s_disp[0] = 0;
            s_disp[1] = M;
            s_disp[2] = 0;
            s_disp[3] = 1;
        }
        if (tid < M) {
            s_disp[4 + tid] = tid;
            s_w[tid] = 1.0f;
        }
    }
    __syncthreads();
    if (tid == 0) *counter = 0;
}

// ============================================================================ launchers
static int pick_wpb(int nb) {
    for (int w = 8; w >= 1; --w)
        if (nb % w == 0) return w;
    return 1;
}

static int gateup_tmc(int K) {
    const int per = K * 2 + (K / 16) * 4;  // bytes of LDS per staged token
    int t = (60 * 1024) / per;
    return t < 1 ? 1 : (t > kDecTM ? kDecTM : t);
}

static int down_tmc(int K, int wpb) {
    const int per = (K / 16) * 4 + wpb * 64 * 4;
    int t = (60 * 1024) / per;
    return t < 1 ? 1 : (t > kDecTM ? kDecTM : t);
}

template <int QT>
static void dec_gateup_q(const Mats& g, const Mats& u, const uint16_t* x, int topk, const int32_t* offsets,
                         const int32_t* perm, const int32_t* active, const int32_t* n_active, int max_active,
                         float* inter, hipStream_t st) {
    const int nb = g.K >> 8, wpb = pick_wpb(nb), tmc = gateup_tmc(g.K);
    const size_t lds = (size_t)tmc * g.K * 2 + (size_t)tmc * (g.K / 16) * 4;
    const size_t red = (size_t)wpb * tmc * 2 * 64 * 4;
    const size_t sh = lds > red ? lds : red;
    const dim3 grid(row_groups(g.N), max_active);
#define PG_DGU(W)                                                                                                \
    hipLaunchKernelGGL((dec_gateup_kernel<QT, W>), grid, dim3(64 * W), sh, st, g.base, u.base, g.stride, u.stride, \
                       g.N, g.K, tmc, x, topk, offsets, perm, active, n_active, inter)
    switch (wpb) {
    case 8: PG_DGU(8); break;
    case 7: PG_DGU(7); break;
    case 6: PG_DGU(6); break;
    case 5: PG_DGU(5); break;
    case 4: PG_DGU(4); break;
    case 3: PG_DGU(3); break;
    case 2: PG_DGU(2); break;
    default: PG_DGU(1); break;
    }
#undef PG_DGU
}

template <int QT>
static void dec_down_q(const Mats& d, const float* inter, const int32_t* offsets, const int32_t* perm,
                       const int32_t* active, const int32_t* n_active, int max_active, const float* topk_w,
                       float* partial, int M, int topk, const int32_t* inv, const float* shared,
                       const float* shared_logit, float* out, int32_t* counters, hipStream_t st) {
    const int nb = d.K >> 8, wpb = pick_wpb(nb), tmc = down_tmc(d.K, wpb);
    const size_t sh = (size_t)tmc * (d.K / 16) * 4 + (size_t)wpb * tmc * 64 * 4;
    const dim3 grid(row_groups(d.N), max_active);
#define PG_DDN(W)                                                                                               \
    hipLaunchKernelGGL((dec_down_kernel<QT, W>), grid, dim3(64 * W), sh, st, d.base, d.stride, d.N, d.K, tmc, inter, \
                       offsets, perm, active, n_active, topk_w, partial, M, topk, inv, shared, shared_logit, out,   \
                       counters)
    switch (wpb) {
    case 8: PG_DDN(8); break;
    case 7: PG_DDN(7); break;
    case 6: PG_DDN(6); break;
    case 5: PG_DDN(5); break;
    case 4: PG_DDN(4); break;
    case 3: PG_DDN(3); break;
    case 2: PG_DDN(2); break;
    default: PG_DDN(1); break;
    }
#undef PG_DDN
}

int launch_dec_gateup(const Mats& g, const Mats& u, const uint16_t* x, int topk, const int32_t* offsets,
                      const int32_t* perm, const int32_t* active, const int32_t* n_active, int max_active,
                      float* inter, hipStream_t st) {
    switch (g.qtype) {
    case PGMOE_Q4_K: dec_gateup_q<PGMOE_Q4_K>(g, u, x, topk, offsets, perm, active, n_active, max_active, inter, st); break;
    case PGMOE_Q6_K: dec_gateup_q<PGMOE_Q6_K>(g, u, x, topk, offsets, perm, active, n_active, max_active, inter, st); break;
    case PGMOE_Q8_0: dec_gateup_q<PGMOE_Q8_0>(g, u, x, topk, offsets, perm, active, n_active, max_active, inter, st); break;
    }
    return check_launch("dec_gateup");
}

int launch_dec_down(const Mats& d, const float* inter, const int32_t* offsets, const int32_t* perm,
                    const int32_t* active, const int32_t* n_active, int max_active, const float* topk_w,
                    float* partial, int M, int topk, const int32_t* inv, const float* shared,
                    const float* shared_logit, float* out, int32_t* counters, hipStream_t st) {
    switch (d.qtype) {
    case PGMOE_Q4_K: dec_down_q<PGMOE_Q4_K>(d, inter, offsets, perm, active, n_active, max_active, topk_w, partial, M, topk, inv, shared, shared_logit, out, counters, st); break;
    case PGMOE_Q6_K: dec_down_q<PGMOE_Q6_K>(d, inter, offsets, perm, active, n_active, max_active, topk_w, partial, M, topk, inv, shared, shared_logit, out, counters, st); break;
    case PGMOE_Q8_0: dec_down_q<PGMOE_Q8_0>(d, inter, offsets, perm, active, n_active, max_active, topk_w, partial, M, topk, inv, shared, shared_logit, out, counters, st); break;
    }
    return check_launch("dec_down");
}

int launch_route_small(const uint16_t* x, const float* W, const float* bias, const float* sh_w, int M, int H, int E,
                       int K, int norm, float* logits, float* s_logit, int32_t* idx, float* w, int32_t* offsets,
                       int32_t* perm, int32_t* inv, int32_t* active, int32_t* n_active, int32_t* s_disp, float* s_w,
                       int32_t* counter, hipStream_t st) {
    if (M < 1 || M > kDecTM) return fail(PGMOE_E_INVALID, "route_small handles 1..%d tokens", kDecTM);
    if (K > 16 || E > 512) return fail(PGMOE_E_UNSUPPORTED, "route_small: top_k <= 16 and E <= 512");
    const int rows = E + (sh_w ? 1 : 0);
    const dim3 grid(div_up(rows, 4)), block(256);
#define PG_RS(RR)                                                                                                 \
    hipLaunchKernelGGL((route_small_kernel<RR>), grid, block, 0, st, x, W, bias, sh_w, M, H, E, K, norm, logits,  \
                       s_logit, idx, w, offsets, perm, inv, active, n_active, s_disp, s_w, counter)
    if (E <= 64) PG_RS(1);
    else if (E <= 128) PG_RS(2);
    else if (E <= 256) PG_RS(4);
    else PG_RS(8);
#undef PG_RS
    return check_launch("route_small");
}

int decode_tokens_max() { return kDecTM; }

}  // namespace pgmoe
