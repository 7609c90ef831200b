// Shared device/host helpers for the pgmoe HIP kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "pgmoe.h"

// Phase timestamps for profiling builds only: a build that defines PG_TRACE (relocatable
// device code) also defines `__device__ unsigned long long pg_trace[]`.  A kernel declares
// its marks with PG_DECL, PG_MARK(kern, point) keeps wall_clock64() (100 MHz) in a register,
// and PG_FLUSH(kern) at the kernel's end has thread 0 of each block store them at
// [kern][block][point] (stores at the marks themselves would lengthen the waits that
// follow them).  Without PG_TRACE the macros compile to nothing.
#ifdef PG_TRACE
extern __device__ unsigned long long pg_trace[];
#define PG_DECL unsigned long long pg_t[8] = {0, 0, 0, 0, 0, 0, 0, 0}
#define PG_MARK(kern, pt) (pg_t[(pt)] = wall_clock64())
#define PG_SET(pt, v) (pg_t[(pt)] = (v))
#define PG_FLUSH(kern)                                                                                      \
    do {                                                                                                    \
        const unsigned pg_b = blockIdx.y * gridDim.x + blockIdx.x;                                          \
        if (threadIdx.x == 0 && pg_b < 8192)                                                                \
            for (int pg_i = 0; pg_i < 8; ++pg_i)                                                            \
                if (pg_t[pg_i]) pg_trace[((kern) * 8192 + pg_b) * 8 + pg_i] = pg_t[pg_i];                  \
    } while (0)
#else
#define PG_DECL
#define PG_MARK(kern, pt) ((void)0)
#define PG_SET(pt, v) ((void)0)
#define PG_FLUSH(kern) ((void)0)
#endif

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

// Value of lane (l ^ S) for S in {1, 2, 4, 8, 16, 32}, by VALU lane moves rather than the
// LDS crossbar (ds_bpermute, about a hundred cycles a step): DPP quad_perm [1,0,3,2] and
// [2,3,0,1] for 1 and 2; DPP row_ror:8 (lane (l - 8) mod 16 of its row) for 8; row_ror:4 /
// row_ror:12 chosen by lane bit 2 for 4; v_permlane16_swap / v_permlane32_swap (gfx950:
// swap the odd rows / the upper half of one register with the even rows / lower half of
// another) for 16 and 32.  Every lane of the wave must be active (a DPP read of an inactive
// lane yields 0), and every lane must call it (no divergent call sites).
template <int S>
__device__ __forceinline__ uint32_t xor_lane_u(uint32_t v) {
    static_assert(S == 1 || S == 2 || S == 4 || S == 8 || S == 16 || S == 32, "lane xor distance");
    const int lane = __lane_id();
    if constexpr (S == 32) {
        const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        return lane < 32 ? r[1] : r[0];
    } else if constexpr (S == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        return (lane & 16) ? r[0] : r[1];
    } else if constexpr (S == 8) {
        return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x128, 0xf, 0xf, false);
    } else if constexpr (S == 4) {
        // both reads in every lane (as operands of a conditional they would run under a
        // partial EXEC mask and read inactive lanes)
        const uint32_t a = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x124, 0xf, 0xf, false);
        const uint32_t b = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x12c, 0xf, 0xf, false);
        return (lane & 4) ? a : b;
    } else if constexpr (S == 2) {
        return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4e, 0xf, 0xf, false);
    } else {
        return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xb1, 0xf, 0xf, false);
    }
}
template <int S>
__device__ __forceinline__ float xor_lane(float v) {
    return __builtin_bit_cast(float, xor_lane_u<S>(__builtin_bit_cast(uint32_t, v)));
}
template <int S>
__device__ __forceinline__ int xor_lane(int v) {
    return (int)xor_lane_u<S>((uint32_t)v);
}

// Sum over an aligned group of `G` lanes (G a power of two <= 64); every lane of the
// group ends with the same value (pairing (l, l^G/2), (l, l^G/4), ..., (l, l^1)).  Whole
// waves only (xor_lane).
template <int G, int S = G / 2>
__device__ __forceinline__ float group_sum(float v) {
    if constexpr (S >= 1) {
        v += xor_lane<S>(v);
        return group_sum<G, S / 2>(v);
    } else {
        return v;
    }
}

// Maximum over the 64 lanes (every lane ends with it).
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, xor_lane<32>(v));
    v = fmaxf(v, xor_lane<16>(v));
    v = fmaxf(v, xor_lane<8>(v));
    v = fmaxf(v, xor_lane<4>(v));
    v = fmaxf(v, xor_lane<2>(v));
    return fmaxf(v, xor_lane<1>(v));
}

// group_sum<64> of N values at once (N a power of two <= 64), as a reduce-scatter: at
// stride s each lane keeps the half of its values whose index bit matches its own lane
// bit and receives its partner's partial of that half, so lane l ends holding the total of
// value (l mod N), after N - 1 exchanges instead of 6 N.  Every level adds the same two
// partial sums as group_sum<64> (IEEE addition commutes), so the totals have its bits.
template <int N, int S = 32>
__device__ __forceinline__ float scatter_sum64(float (&v)[N], int lane) {
    if constexpr (S >= 1) {
        if constexpr (S >= N) {  // more lanes than values: plain xor step on all of them
#pragma unroll
            for (int i = 0; i < N; ++i) v[i] += xor_lane<S>(v[i]);
        } else {
            // selects by mask: a select between two array elements would become a select
            // of addresses and push the array to scratch memory
            const uint32_t up = (lane & S) ? 0xffffffffu : 0u;
#pragma unroll
            for (int i = 0; i < S; ++i) {
                const uint32_t lo = __builtin_bit_cast(uint32_t, v[i]), hi = __builtin_bit_cast(uint32_t, v[S + i]);
                const float send = __builtin_bit_cast(float, (lo & up) | (hi & ~up));
                const float keep = __builtin_bit_cast(float, (hi & up) | (lo & ~up));
                v[i] = keep + xor_lane<S>(send);
            }
        }
        return scatter_sum64<N, S / 2>(v, lane);
    } else {
        return v[0];
    }
}

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

__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }
// GELU, tanh approximation: 0.5 g (1 + tanh(z)), z = sqrt(2/pi) (g + 0.044715 g^3), with
// tanh(z) = 1 - 2 / (1 + e^(2z)) (saturates to +-1 for large |z|).
__device__ __forceinline__ float gelu_tanh(float g) {
    const float z = 0.7978845608028654f * (g + 0.044715f * g * g * g);
    return 0.5f * g * (2.0f - 2.0f / (1.0f + expf(2.0f * z)));
}
// The gate activation PGMOE_ACT_* of a gated FFN.
__device__ __forceinline__ float gate_act(int act, float g) { return act ? gelu_tanh(g) : silu(g); }

// Direct global -> LDS copy (global_load_lds_dwordx4): lane l's 16 bytes at g land at
// lds + 16 * l, so one wave fills 1 KB of LDS and holds no registers for the data.  `lds`
// must be the same for every lane of the wave.  The copy is counted by vmcnt: wait_dma()
// before the barrier that hands the LDS to other waves.
__device__ __forceinline__ void dma16(const void* g, void* lds) {
    __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
}
__device__ __forceinline__ void wait_dma() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Zero words [0, n) of p with relaxed agent-scope atomic stores, one word per thread of
// the grid (the decode router's ready-tagged logits, cleared by the forward's last kernel).
__device__ __forceinline__ void clear_words(uint64_t* p, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    const int step = gridDim.x * blockDim.x;
    if (p)
        for (int j = i; j < n; j += step) __hip_atomic_store(p + j, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------- router tile
// Router logits of one wave: TM tokens (m0 ..; rows past M repeat row M-1) x TE expert
// rows (e0 ..; row E is extra_w, the shared expert's gate vector, when given; rows past
// it repeat the last).  Lane l is "slot" l: it owns the 8-wide chunks c = l, l+64,
// l+128, ... of the row and runs one fmaf chain over them in ascending order; the 64
// slot sums are then combined by the xor tree (l, l^32), (l, l^16), ..., (l, l^1), and
// every lane ends with every total.  The caller adds the bias last.  The CPU oracle
// (or_router_logits) performs the same operations in the same order.  Chunks are
// processed PF at a time with every load of the group issued before the first FMA (the
// FMA order per slot is unchanged).
template <int TM, int TE, int PF = (TM * TE <= 8 ? 4 : 2)>
__device__ __forceinline__ void router_tile(const uint16_t* __restrict__ x, const float* __restrict__ W,
                                            const float* __restrict__ extra_w, int M, int H, int E, int m0,
                                            int e0, int lane, float (&acc)[TM][TE]) {
    const int rows = E + (extra_w ? 1 : 0);
    const int C = H >> 3;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TE; ++j) acc[i][j] = 0.0f;
    for (int c0 = lane; c0 < C; c0 += 64 * PF) {
        uint4 xq[PF][TM];
        float4 wq[PF][TE][2];
#pragma unroll
        for (int q = 0; q < PF; ++q) {
            const int c = c0 + 64 * q;
            if (c < C) {
#pragma unroll
                for (int i = 0; i < TM; ++i) {
                    const int m = m0 + i < M ? m0 + i : M - 1;
                    xq[q][i] = *(const uint4*)(x + (int64_t)m * H + 8 * c);
                }
#pragma unroll
                for (int j = 0; j < TE; ++j) {
                    const int e = e0 + j < rows ? e0 + j : rows - 1;
                    const float* wr = e < E ? W + (int64_t)e * H : extra_w;
                    wq[q][j][0] = *(const float4*)(wr + 8 * c);
                    wq[q][j][1] = *(const float4*)(wr + 8 * c + 4);
                }
            }
        }
#pragma unroll
        for (int q = 0; q < PF; ++q) {
            if (c0 + 64 * q < C) {
#pragma unroll
                for (int i = 0; i < TM; ++i) {
                    const uint32_t w4[4] = {xq[q][i].x, xq[q][i].y, xq[q][i].z, xq[q][i].w};
                    float xv[8];
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        xv[2 * k] = lo_half(w4[k]);
                        xv[2 * k + 1] = hi_half(w4[k]);
                    }
#pragma unroll
                    for (int j = 0; j < TE; ++j) {
                        const float wv[8] = {wq[q][j][0].x, wq[q][j][0].y, wq[q][j][0].z, wq[q][j][0].w,
                                             wq[q][j][1].x, wq[q][j][1].y, wq[q][j][1].z, wq[q][j][1].w};
#pragma unroll
                        for (int k = 0; k < 8; ++k) acc[i][j] = __builtin_fmaf(xv[k], wv[k], acc[i][j]);
                    }
                }
            }
        }
    }
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TE; ++j) acc[i][j] = group_sum<64>(acc[i][j]);
}

// ---------------------------------------------------------------- device weight layout
// Every matrix [N rows, K cols] (K a multiple of 256) is stored as tiles of 64 rows x one
// 256-weight super-block.  A tile holds CH 16-byte chunks per row, chunk-major:
//     tile(rg, b) = base + (rg * nb + b) * CH * 1024,   chunk c of row r at + c*1024 + r*16
// so the 64 lanes of a wavefront reading chunk c of 64 consecutive rows touch 1 KB of
// contiguous memory.  Chunk contents (same bits as the GGUF block):
//   Q4_1 (CH 10): c0 = fp16 d of the 8 Q4_1 blocks, c1 = their fp16 m;  c2..c9 = the codes
//                 in the Q4_K arrangement (c2..c9 as Q4_K's c1..c8); value d q + m
//   Q4_K (CH 9):  c0 = d, dmin, 12 scale bytes;  c1..c8 = qs[16(c-1) .. +16]
//   Q5_K (CH 11): c0..c8 as Q4_K;  c9, c10 = the fifth bits per 64-weight quarter p:
//                 word t (t = 0, 1) at chunk 9 + (p >> 1), byte 8(p & 1) + 4t, bit
//                 8(l & 3) + (l >> 2) = fifth bit of element 64p + 32t + l (GGUF: bit
//                 2p + t of qh[l]); (w >> k) & 0x01010101 gives elements 4k .. 4k+3
//   Q6_K (CH 13): c0..c7 = ql[16c ..];  c8..c11 = qh[16(c-8) ..];  c12 = sc[16];
//                 fp16 d in a plane after all tiles: d(rg, b, r) at
//                 base + ng*nb*13*1024 + ((rg*nb + b)*64 + r)*2
//   Q8_0 (CH 17): c0..c15 = qs of the 8 Q8_0 blocks in order (16 weights per chunk);
//                 c16 = their 8 fp16 d
//   F16  (CH 32): c = weights 8c .. 8c+7 of the super-block (fp16)
// N is padded to a multiple of 64 (padding rows are zero and never stored to outputs).
template <int QT> struct Tile;
template <> struct Tile<PGMOE_Q4_1> { static constexpr int CH = 10; };
template <> struct Tile<PGMOE_Q4_K> { static constexpr int CH = 9; };
template <> struct Tile<PGMOE_Q5_K> { static constexpr int CH = 11; };
template <> struct Tile<PGMOE_Q6_K> { static constexpr int CH = 13; };
template <> struct Tile<PGMOE_Q8_0> { static constexpr int CH = 17; };
template <> struct Tile<PGMOE_F16> { static constexpr int CH = 32; };

__host__ __device__ inline int row_groups(int N) { return (N + 63) >> 6; }

template <int QT>
__device__ __forceinline__ const uint8_t* tile_ptr(const uint8_t* mat, int nb, int rg, int b) {
    return mat + ((int64_t)rg * nb + b) * (Tile<QT>::CH * 1024);
}

// ---------------------------------------------------------------- quant groups
// The MFMA GEMM stages weights in units of 64 consecutive weights of one row (four
// groups of 16 sharing an affine scale, w = a*q - b).  Unit u covers row elements
//   col(u, g) + [0, 16) for g = 0..3:
//   Q4_1, Q4_K, Q5_K: block u/4, qs bytes [32c, 32c+32) with c = u%4: groups at 64c + {0,16,32,48}
//         (low nibbles -> sub-block 2c, high nibbles -> sub-block 2c+1)
//   Q6_K: block u/4, (h, half) = ((u%4)>>1, u&1): groups s at 128h + 16half + 32s
//   Q8_0: block u/4, Q8_0 blocks 2(u%4), 2(u%4)+1: groups at 64(u%4) + 16g
template <int QT> struct Fmt {
    __device__ static __forceinline__ int col(int u, int g) { return 64 * u + 16 * g; }
};
template <> struct Fmt<PGMOE_Q6_K> {
    __device__ static __forceinline__ int col(int u, int g) {
        const int un = u & 3;
        return 256 * (u >> 2) + 128 * (un >> 1) + 16 * (un & 1) + 32 * g;
    }
};

// ---------------------------------------------------------------- launch helpers
inline int div_up(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Host-side description of one set of expert matrices, validated.
// K-quant (scale, min) of sub-block s without branches: both
// encodings are decoded and s picks one (Q4_K scale bytes: D = 0-3, Mb = 4-7, MD = 8-11).
__device__ __forceinline__ void kscale_sel(uint32_t D, uint32_t Mb, uint32_t MD, int s, int& sc, int& mn) {
    const int j = 8 * (s & 3);
    const int sl = (D >> j) & 63, ml = (Mb >> j) & 63;
    const uint32_t md = (MD >> j) & 0xff;
    const int sh = (md & 0x0f) | ((D >> (j + 2)) & 0x30), mh = (md >> 4) | ((Mb >> (j + 2)) & 0x30);
    sc = s < 4 ? sl : sh;
    mn = s < 4 ? ml : mh;
}

struct Mats {
    int qtype, N, K, n_mats;
    const uint8_t* base;
    int64_t stride;
    const uint8_t* scales;  // scale plane (K-quants; may be null outside the MFMA products)
};
int check_weights(const pgmoe_weights* w, const char* what, Mats* out);

}  // namespace pgmoe
