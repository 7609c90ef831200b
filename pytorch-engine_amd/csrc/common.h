// Shared device/host helpers for the pgmoe HIP kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "pgmoe.h"

namespace pgmoe {

typedef _Float16 half_t;
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// ---------------------------------------------------------------- host-side status
void set_error(const char* fmt, ...);
int fail(int code, const char* fmt, ...);
int check_launch(const char* what);

// ---------------------------------------------------------------- small device helpers
__device__ __forceinline__ float h2f(uint16_t b) {
    return (float)__builtin_bit_cast(half_t, b);
}

__device__ __forceinline__ float lo_half(uint32_t v) { return h2f((uint16_t)(v & 0xffffu)); }
__device__ __forceinline__ float hi_half(uint32_t v) { return h2f((uint16_t)(v >> 16)); }

// Sum over an aligned group of `G` lanes (G a power of two <= 64); every lane of the
// group ends with the same value (pairing (l, l^G/2), (l, l^G/4), ..., (l, l^1)).
template <int G>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int s = G / 2; s >= 1; s >>= 1) v += __shfl_xor(v, s, kWave);
    return v;
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }

// ---------------------------------------------------------------- quant groups
// Every supported format is processed in "units" of 64 weights of one row, each made of
// four groups of 16 weights sharing one affine scale: w = a*q - b.  Unit u of a row
// covers row elements  unit_col(u, g) + [0, 16)  for g = 0..3:
//   Q4_K: block u/4, 32-byte qs chunk c = u%4: groups at 64c + {0,16,32,48}
//         (low nibbles -> sub-block 2c, high nibbles -> sub-block 2c+1)
//   Q6_K: block u/4, (h, half) = ((u%4)>>1, u&1): groups s at 128h + 16half + 32s
//   Q8_0: blocks 2u, 2u+1: groups at 64u' + {0,16,32,48} (g<2 -> block 2u)
template <int QT> struct Fmt;

template <> struct Fmt<PGMOE_Q4_K> {
    __device__ static __forceinline__ int col(int u, int g) { return 64 * u + 16 * g; }
    // q[16] (integers 0..15 as float), scale a, offset b for group g of unit u of `row`.
    __device__ static __forceinline__ void group(const uint8_t* mat, int K, int N, int row, int u, int g,
                                                 float q[16], float& a, float& b) {
        const int nb = K >> 8;
        const uint8_t* blk = mat + ((int64_t)row * nb + (u >> 2)) * 144;
        const int c = u & 3;
        const uint4 hdr = *(const uint4*)blk;
        const uint4 qv = *(const uint4*)(blk + 16 + 32 * c + 16 * (g & 1));
        const int s = 2 * c + (g >> 1);
        const uint32_t D = hdr.y, Mb = hdr.z, MD = hdr.w;  // scale bytes 0-3, 4-7, 8-11
        int sc, mn;
        if (s < 4) {
            sc = (D >> (8 * s)) & 63;
            mn = (Mb >> (8 * s)) & 63;
        } else {
            const int j = s - 4;
            const uint32_t md = (MD >> (8 * j)) & 0xff;
            sc = (md & 0x0f) | (((D >> (8 * j)) >> 2) & 0x30);
            mn = (md >> 4) | (((Mb >> (8 * j)) >> 2) & 0x30);
        }
        a = lo_half(hdr.x) * (float)sc;
        b = hi_half(hdr.x) * (float)mn;
        const int sh = 4 * (g >> 1);
        const uint32_t w[4] = {qv.x, qv.y, qv.z, qv.w};
#pragma unroll
        for (int i = 0; i < 16; ++i) q[i] = (float)((w[i >> 2] >> (8 * (i & 3) + sh)) & 0xf);
    }
};

template <> struct Fmt<PGMOE_Q6_K> {
    __device__ static __forceinline__ int col(int u, int g) {
        const int un = u & 3;
        return 256 * (u >> 2) + 128 * (un >> 1) + 16 * (un & 1) + 32 * g;
    }
    __device__ static __forceinline__ void group(const uint8_t* mat, int K, int N, int row, int u, int g,
                                                 float q[16], float& a, float& b) {
        const int nb = K >> 8;
        const int64_t blk = (int64_t)row * nb + (u >> 2);
        const int64_t unit = blk * 4 + (u & 3);
        const uint8_t* body = mat + unit * 48;
        const uint4 lo = *(const uint4*)(body + 16 * (g & 1));  // ql chunk A (s even) or B (s odd)
        const uint4 hi = *(const uint4*)(body + 32);            // qh chunk
        const uint32_t scw = *(const uint32_t*)(mat + (int64_t)N * nb * 192 + unit * 4);
        const uint16_t db = *(const uint16_t*)(mat + (int64_t)N * nb * 208 + blk * 2);
        const int sc = (int)(int8_t)((scw >> (8 * g)) & 0xff);
        a = h2f(db) * (float)sc;
        b = 32.0f * a;
        const int lsh = 4 * (g >> 1), hsh = 2 * g;
        const uint32_t lw[4] = {lo.x, lo.y, lo.z, lo.w};
        const uint32_t hw[4] = {hi.x, hi.y, hi.z, hi.w};
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int sft = 8 * (i & 3);
            const int v = ((lw[i >> 2] >> (sft + lsh)) & 0xf) | (((hw[i >> 2] >> (sft + hsh)) & 3) << 4);
            q[i] = (float)v;
        }
    }
};

template <> struct Fmt<PGMOE_Q8_0> {
    __device__ static __forceinline__ int col(int u, int g) { return 64 * u + 16 * g; }
    __device__ static __forceinline__ void group(const uint8_t* mat, int K, int N, int row, int u, int g,
                                                 float q[16], float& a, float& b) {
        const uint4 qv = *(const uint4*)(mat + (int64_t)row * K + 64 * u + 16 * g);
        const uint16_t db = *(const uint16_t*)(mat + (int64_t)N * K + ((int64_t)row * (K >> 5) + 2 * u + (g >> 1)) * 2);
        a = h2f(db);
        b = 0.0f;
        const uint32_t w[4] = {qv.x, qv.y, qv.z, qv.w};
#pragma unroll
        for (int i = 0; i < 16; ++i) q[i] = (float)(int8_t)((w[i >> 2] >> (8 * (i & 3))) & 0xff);
    }
};

// ---------------------------------------------------------------- launch helpers
inline int div_up(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Host-side description of one set of expert matrices, validated.
struct Mats {
    int qtype, N, K, n_mats;
    const uint8_t* base;
    int64_t stride;
};
int check_weights(const pgmoe_weights* w, const char* what, Mats* out);

}  // namespace pgmoe
