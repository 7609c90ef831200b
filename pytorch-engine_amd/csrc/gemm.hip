// Prefill (M > 8) grouped expert products on the MFMA cores.
//
// A tile is 256 sorted pairs of one expert x 256 output columns.  The block is 8 waves
// (two per SIMD), each owning 128 rows x 64 columns as 4 x 2 v_mfma_f32_32x32x16_f16
// tiles (128 fp32 accumulators per lane).  The K loop steps one 64-weight unit at a
// time through two LDS stages: while the MFMAs read unit u from one stage, the block
// writes unit u + 1 into the other (fp16 activations, and weights dequantised as
// w = a*q - b in fp32 with one rounding to fp16), and the raw bytes of unit u + 2 are
// already on their way into a second register set.  One barrier per unit.
//   gate/up: A = x rows gathered through perm (fp16), B = 128 gate rows + 128 up rows of
//            the same intermediate indices, arranged so every wave holds matching gate
//            and up columns; epilogue = SwiGLU in fp32 -> inter [P][I].
//   down   : A = a16 [P][I] (the row-scaled fp16 SwiGLU rows), B = 256 down rows;
//            epilogue = partial[p][h] = w_p * rs_p * acc.
// Tiles: the dispatch's tile_off counts 256-row tiles per expert; the last tile of an
// expert holds the remainder (1..256 rows, waves past it skip their MFMAs).  Block ids
// are ordered so the N tiles of one M tile run back to back on one XCD (blocks go to the
// 8 XCDs round-robin), so its gathered A rows are shared through that XCD's L2.
// Reference: GGUFQuantMoEExperts.forward_expert (quant_kernels.py:1990-2011) ->
// exec_w4a16_matmul / exec_w8a16_matmul (:1165-1420) and model.py:916-919.
#include "common.h"
#include "launch.h"

namespace pgmoe {

constexpr int kGM = 256;      // pair rows per tile
constexpr int kGN = 256;      // B rows (output columns) per tile
constexpr int kGP = 64 + 8;   // LDS pitch in halves (16-byte pad against bank conflicts)
constexpr int kGThreads = 512;
constexpr int kXcd = 8;

typedef _Float16 gh8 __attribute__((ext_vector_type(8)));
typedef uint32_t gu4 __attribute__((ext_vector_type(4)));
typedef float gf16 __attribute__((ext_vector_type(16)));

// ---------------------------------------------------------------- raw weight half rows
// Groups h and h + 2 (h = 0 or 1) of one row in one 64-weight unit (see Fmt<QT>): the
// groups that share their quant bytes (Q4_K: one qs chunk, low / high nibbles; Q6_K: one
// ql chunk, low / high nibbles, plus the qh chunk; Q8_0: two chunks).  Loaded a step ahead,
// decoded to 2 x 16 fp16 values with Fmt<QT>::group's arithmetic (fp32 math, one rounding).
template <int QT> struct GHalf;
template <> struct GHalf<PGMOE_Q4_K> { uint4 hdr, q; };
template <> struct GHalf<PGMOE_Q6_K> { uint4 lo, hi; uint2 scw; uint32_t db; };
template <> struct GHalf<PGMOE_Q8_0> { uint4 q0, q1; uint32_t dw; };

template <int QT>
__device__ __forceinline__ void gload(const uint8_t* mat, int nb, int N, int row, int u, int h, GHalf<QT>& r);

template <>
__device__ __forceinline__ void gload<PGMOE_Q4_K>(const uint8_t* mat, int nb, int N, int row, int u, int h,
                                                   GHalf<PGMOE_Q4_K>& r) {
    const uint8_t* t = tile_ptr<PGMOE_Q4_K>(mat, nb, row >> 6, u >> 2) + (row & 63) * 16;
    r.hdr = *(const uint4*)t;
    r.q = *(const uint4*)(t + (1 + 2 * (u & 3) + h) * 1024);
}

template <>
__device__ __forceinline__ void gload<PGMOE_Q6_K>(const uint8_t* mat, int nb, int N, int row, int u, int h,
                                                   GHalf<PGMOE_Q6_K>& r) {
    const int rg = row >> 6, rr = row & 63, blk = u >> 2, h6 = (u & 3) >> 1, half = u & 1;
    const uint8_t* t = tile_ptr<PGMOE_Q6_K>(mat, nb, rg, blk) + rr * 16;
    r.lo = *(const uint4*)(t + (4 * h6 + 2 * h + half) * 1024);  // ql[64h6 + 32h + 16half ..]
    r.hi = *(const uint4*)(t + (8 + 2 * h6 + half) * 1024);      // qh[32h6 + 16half ..]
    r.scw = *(const uint2*)(t + 12 * 1024 + 8 * h6);             // scales 8h6 .. 8h6+7
    const int64_t dplane = (int64_t)row_groups(N) * nb * 13 * 1024;
    r.db = *(const uint16_t*)(mat + dplane + (((int64_t)rg * nb + blk) * 64 + rr) * 2);
}

template <>
__device__ __forceinline__ void gload<PGMOE_Q8_0>(const uint8_t* mat, int nb, int N, int row, int u, int h,
                                                   GHalf<PGMOE_Q8_0>& r) {
    const uint8_t* t = tile_ptr<PGMOE_Q8_0>(mat, nb, row >> 6, u >> 2) + (row & 63) * 16;
    r.q0 = *(const uint4*)(t + (4 * (u & 3) + h) * 1024);
    r.q1 = *(const uint4*)(t + (4 * (u & 3) + h + 2) * 1024);
    r.dw = *(const uint32_t*)(t + 16 * 1024 + 4 * (u & 3));
}

__device__ __forceinline__ uint32_t pack_h2(float a, float b) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)a) |
           ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)b) << 16);
}

// 4 bytes of codes v (one code per byte) -> w = a*code + nb as two fp16 pairs
__device__ __forceinline__ void dq4(uint32_t v, float a, float nb, uint32_t* o) {
    o[0] = pack_h2(__builtin_fmaf(a, (float)(v & 0xff), nb), __builtin_fmaf(a, (float)((v >> 8) & 0xff), nb));
    o[1] = pack_h2(__builtin_fmaf(a, (float)((v >> 16) & 0xff), nb), __builtin_fmaf(a, (float)(v >> 24), nb));
}

// Group g = h + 2*gg (gg = 0 or 1) of the half row -> 8 packed fp16 pairs.
template <int QT>
__device__ __forceinline__ void gdecode(const GHalf<QT>& r, int u, int h, int gg, uint32_t out[8]);

template <>
__device__ __forceinline__ void gdecode<PGMOE_Q4_K>(const GHalf<PGMOE_Q4_K>& r, int u, int h, int gg,
                                                     uint32_t out[8]) {
    const int s = 2 * (u & 3) + gg;  // group h + 2gg: sub-block 2(u%4) + gg, nibble gg
    const uint32_t D = r.hdr.y, Mb = r.hdr.z, MD = r.hdr.w;
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
    const float a = lo_half(r.hdr.x) * (float)sc;
    const float nb = -(hi_half(r.hdr.x) * (float)mn);
    const int sh = 4 * gg;
    const uint32_t w[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) dq4((w[k] >> sh) & 0x0f0f0f0fu, a, nb, out + 2 * k);
}

template <>
__device__ __forceinline__ void gdecode<PGMOE_Q6_K>(const GHalf<PGMOE_Q6_K>& r, int u, int h, int gg,
                                                     uint32_t out[8]) {
    const int g = h + 2 * gg, half = u & 1;
    const int sb = 2 * g + half;  // scale byte within the 8 loaded (8h6 + sb)
    const uint32_t sw = sb < 4 ? r.scw.x : r.scw.y;
    const int sc = (int)(int8_t)((sw >> (8 * (sb & 3))) & 0xff);
    const float a = h2f((uint16_t)r.db) * (float)sc;
    const float nb = -32.0f * a;
    const int lsh = 4 * gg, hsh = 2 * g;
    const uint32_t lw[4] = {r.lo.x, r.lo.y, r.lo.z, r.lo.w};
    const uint32_t hw[4] = {r.hi.x, r.hi.y, r.hi.z, r.hi.w};
#pragma unroll
    for (int k = 0; k < 4; ++k)
        dq4(((lw[k] >> lsh) & 0x0f0f0f0fu) | (((hw[k] >> hsh) & 0x03030303u) << 4), a, nb, out + 2 * k);
}

template <>
__device__ __forceinline__ void gdecode<PGMOE_Q8_0>(const GHalf<PGMOE_Q8_0>& r, int u, int h, int gg,
                                                     uint32_t out[8]) {
    const int g = h + 2 * gg;
    const float a = (g < 2) ? lo_half(r.dw) : hi_half(r.dw);
    const uint4 qv = gg ? r.q1 : r.q0;
    const uint32_t w[4] = {qv.x, qv.y, qv.z, qv.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t v = w[k];
        out[2 * k] = pack_h2(a * (float)(int8_t)(v & 0xff), a * (float)(int8_t)((v >> 8) & 0xff));
        out[2 * k + 1] = pack_h2(a * (float)(int8_t)((v >> 16) & 0xff), a * (float)(int8_t)(v >> 24));
    }
}

// ---------------------------------------------------------------- tile mapping
// Block id -> (M tile, N tile): XCD x = id % 8 takes M tiles x, x+8, ... and runs all N
// tiles of one M tile consecutively.  Returns false for ids past the last M tile.
__device__ __forceinline__ bool gemm_tile_of(int id, int n_ntiles, int n_mtiles, int& mt, int& nt) {
    const int x = id % kXcd, local = id / kXcd;
    nt = local % n_ntiles;
    mt = (local / n_ntiles) * kXcd + x;
    return mt < n_mtiles;
}

__device__ __forceinline__ int gemm_tile_expert(const int32_t* tile_off, int E, int tile) {
    int lo = 0, hi = E - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (tile_off[mid] <= tile) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

// ---------------------------------------------------------------- the kernel
// k columns [ko0, ko0 + 32) of the 64-wide unit: 2 slices of 16, each 8
// v_mfma_f32_32x32x16_f16 over the wave's 4 x 2 tiles of 32 x 32 (the f16 MFMA with the
// full matrix-core rate on gfx950; 16x16x32 runs at half).  Operand layout: lane l holds
// A[l%32][8(l/32) .. +8] and B[8(l/32) .. +8][l%32]; register v of D is
// D[8(v/4) + 4(l/32) + v%4][l%32].
// NI = the wave's 32-row slices that hold pairs (1..4); the others are skipped.
template <int NI>
__device__ __forceinline__ void gemm_half(const _Float16* As, const _Float16* Bs, int wm, int wn, int lane, int ko0,
                                          gf16 (&acc)[4][2]) {
#pragma unroll
    for (int ks = 0; ks < 32; ks += 16) {
        const int ko = ko0 + ks + 8 * (lane >> 5);
        gh8 af[NI];
#pragma unroll
        for (int i = 0; i < NI; ++i) af[i] = *(const gh8*)&As[(128 * wm + 32 * i + (lane & 31)) * kGP + ko];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const gh8 bf = *(const gh8*)&Bs[(64 * wn + 32 * j + (lane & 31)) * kGP + ko];
#pragma unroll
            for (int i = 0; i < NI; ++i)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf, acc[i][j], 0, 0, 0);
        }
    }
}

__device__ __forceinline__ void gemm_unit(const _Float16* As, const _Float16* Bs, int wm, int wn, int lane, int ni,
                                          gf16 (&acc)[4][2]) {
    switch (ni) {
    case 4:
        gemm_half<4>(As, Bs, wm, wn, lane, 0, acc);
        gemm_half<4>(As, Bs, wm, wn, lane, 32, acc);
        break;
    case 3:
        gemm_half<3>(As, Bs, wm, wn, lane, 0, acc);
        gemm_half<3>(As, Bs, wm, wn, lane, 32, acc);
        break;
    case 2:
        gemm_half<2>(As, Bs, wm, wn, lane, 0, acc);
        gemm_half<2>(As, Bs, wm, wn, lane, 32, acc);
        break;
    case 1:
        gemm_half<1>(As, Bs, wm, wn, lane, 0, acc);
        gemm_half<1>(As, Bs, wm, wn, lane, 32, acc);
        break;
    default: break;
    }
}

template <int QT, bool GATEUP>
__global__ __launch_bounds__(kGThreads) void gemm_kernel(
    const uint8_t* __restrict__ w0, const uint8_t* __restrict__ w1, int64_t wstride0, int64_t wstride1,
    int N, int K, const uint16_t* __restrict__ act, int topk, int E, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ perm, const int32_t* __restrict__ tile_off, int n_ntiles,
    const float* __restrict__ rs, const float* __restrict__ topk_w, float* __restrict__ out) {
    // two LDS stages: the next unit is staged into one while the other feeds the MFMAs
    __shared__ __attribute__((aligned(16))) _Float16 A0[kGM * kGP];
    __shared__ __attribute__((aligned(16))) _Float16 B0[kGN * kGP];
    __shared__ __attribute__((aligned(16))) _Float16 A1[kGM * kGP];
    __shared__ __attribute__((aligned(16))) _Float16 B1[kGN * kGP];
    __shared__ int rowsrc[kGM];
    int mt, nt;
    PG_MARK(GATEUP ? 4 : 5, 0);
    if (!gemm_tile_of(blockIdx.x, n_ntiles, tile_off[E], mt, nt)) return;
    const int e = gemm_tile_expert(tile_off, E, mt);
    const int m0 = offsets[e] + (mt - tile_off[e]) * kGM;
    const int mrows = min(kGM, offsets[e + 1] - m0);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // wave tile: rows 128 wm .., B rows 64 wn .. (waves w and w + 4 share a SIMD)
    const int wm = wave >> 2, wn = wave & 3;
    const int units = K >> 6;
    // A source rows: gate/up gathers token rows of x, down reads its own pair rows.  Rows
    // past the tile's pairs repeat its last pair: they only feed accumulator rows that
    // are never stored.
    if (tid < kGM) {
        const int p = m0 + min(tid, mrows - 1);
        rowsrc[tid] = GATEUP ? perm[p] / topk : p;
    }
    __syncthreads();

    // staging: thread t moves A chunks (rows t/8 + 64q, 16-byte chunk t%8) and groups
    // h, h + 2 (h = t%2) of B row t/2
    const int ar = tid >> 3, ac = tid & 7;
    const int br = tid >> 1, bh = tid & 1;
    const int nb = K >> 8;
    int asrc[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) asrc[q] = rowsrc[ar + 64 * q];
    // B rows: gate/up tile rows, per wave column wn: 32 gate then 32 up rows of the
    // intermediate indices nt*128 + 32wn + ..; down: output rows nt*256 + r.  Rows past N
    // repeat row N-1: they only feed columns that are never stored.
    const uint8_t* bmat;
    int brow;
    if (GATEUP) {
        const bool up = (br >> 5) & 1;
        bmat = up ? w1 + (int64_t)e * wstride1 : w0 + (int64_t)e * wstride0;
        brow = nt * (kGN / 2) + 32 * (br >> 6) + (br & 31);
    } else {
        bmat = w0 + (int64_t)e * wstride0;
        brow = nt * kGN + br;
    }
    brow = min(brow, N - 1);

    gf16 acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

    const bool active = 128 * wm < mrows;
    const int ni = active ? min(4, (mrows - 128 * wm + 31) >> 5) : 0;  // 32-row slices with pairs
    const bool store_first = wave >= 4;
    // Two register sets of raw staging data and two LDS stages.  The loads are
    // unconditional (every index is valid), so every step issues the same instructions and
    // the waits for the previous step's loads stay exact; the last steps load a repeated
    // unit that is never stored.
    gu4 a0[4], a1[4];
    GHalf<QT> b0, b1;
#define PG_GLOAD(AR, BR, UU)                                                              \
    do {                                                                                  \
        const int pg_u = (UU);                                                            \
        const int pg_col = Fmt<QT>::col(pg_u, ac >> 1) + 8 * (ac & 1);                    \
        AR[0] = *(const gu4*)(act + (int64_t)asrc[0] * K + pg_col);                      \
        AR[1] = *(const gu4*)(act + (int64_t)asrc[1] * K + pg_col);                      \
        AR[2] = *(const gu4*)(act + (int64_t)asrc[2] * K + pg_col);                      \
        AR[3] = *(const gu4*)(act + (int64_t)asrc[3] * K + pg_col);                      \
        gload<QT>(bmat, nb, N, brow, pg_u, bh, BR);                                       \
    } while (0)
#define PG_GSTORE(AR, BR, UU, AS, BS)                                                     \
    do {                                                                                  \
        *(gu4*)&AS[(ar + 0) * kGP + 8 * ac] = AR[0];                                     \
        *(gu4*)&AS[(ar + 64) * kGP + 8 * ac] = AR[1];                                    \
        *(gu4*)&AS[(ar + 128) * kGP + 8 * ac] = AR[2];                                   \
        *(gu4*)&AS[(ar + 192) * kGP + 8 * ac] = AR[3];                                   \
        _Pragma("unroll") for (int gg = 0; gg < 2; ++gg) {                                \
            uint32_t hv[8];                                                               \
            gdecode<QT>(BR, (UU), bh, gg, hv);                                            \
            uint4* pg_d = (uint4*)&BS[br * kGP + 16 * (bh + 2 * gg)];                     \
            pg_d[0] = make_uint4(hv[0], hv[1], hv[2], hv[3]);                             \
            pg_d[1] = make_uint4(hv[4], hv[5], hv[6], hv[7]);                             \
        }                                                                                 \
    } while (0)
    PG_GLOAD(a0, b0, 0);
    PG_GLOAD(a1, b1, min(1, units - 1));
    PG_GSTORE(a0, b0, 0, A0, B0);
    __syncthreads();
    // Step u: issue the loads of unit u + 2 into the free register set, run the MFMAs of
    // unit u (stage u & 1) and write unit u + 1 (loaded a step earlier) into the other
    // stage; one barrier.  The two waves of a SIMD do the write at opposite ends of their
    // MFMAs (waves 0-3 compute first, waves 4-7 write first), so one wave's dequantisation
    // runs while the other keeps the matrix core busy.  The last steps re-store a unit that
    // is never read.
#define PG_GSTEP(AC, BC, AN, BN, ARN, BRN, ARF, BRF, UNEXT, ULOAD)                        \
    do {                                                                                  \
        PG_GLOAD(ARF, BRF, (ULOAD));                                                      \
        if (store_first) PG_GSTORE(ARN, BRN, (UNEXT), AN, BN);                            \
        gemm_unit(AC, BC, wm, wn, lane, ni, acc);                                         \
        if (!store_first) PG_GSTORE(ARN, BRN, (UNEXT), AN, BN);                           \
        __syncthreads();                                                                  \
    } while (0)
    for (int u = 0; u < units; u += 2) {
        if (u == 4) PG_MARK(GATEUP ? 4 : 5, 1);
        PG_GSTEP(A0, B0, A1, B1, a1, b1, a0, b0, min(u + 1, units - 1), min(u + 2, units - 1));
        if (u == 4) PG_MARK(GATEUP ? 4 : 5, 2);
        if (u + 1 >= units) break;
        PG_GSTEP(A1, B1, A0, B0, a0, b0, a1, b1, min(u + 2, units - 1), min(u + 3, units - 1));
        if (u == 4) PG_MARK(GATEUP ? 4 : 5, 3);
    }
#undef PG_GSTEP
#undef PG_GLOAD
#undef PG_GSTORE
    PG_MARK(GATEUP ? 4 : 5, 4);
    if (!active) return;
    // epilogue: register v of tile (i, j) is row 32i + 8(v/4) + 4(l/32) + v%4, column
    // 32j + l%32 of the wave tile
    if (GATEUP) {
        // wave columns: tile 0 gate indices nt*128 + 32wn + l%32, tile 1 the matching up
        const int col = nt * (kGN / 2) + 32 * wn + (lane & 31);
        if (col < N) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int r = 128 * wm + 32 * i + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
                    if (r < mrows) out[(int64_t)(m0 + r) * N + col] = silu(acc[i][0][v]) * acc[i][1][v];
                }
        }
    } else {
        const int c0 = nt * kGN + 64 * wn + (lane & 31);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int r = 128 * wm + 32 * i + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
                if (r >= mrows) continue;
                const int p = m0 + r;
                const float sc = rs[p] * topk_w[perm[p]];
                float* orow = out + (int64_t)p * N;
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int col = c0 + 32 * j;
                    if (col < N) orow[col] = acc[i][j][v] * sc;
                }
            }
    }
}

int gemm_tile_pairs() { return kGM; }

// Upper bound of 256-row tiles for P pairs over at most E experts, rounded up to whole
// XCD groups.
static int gemm_max_mtiles(int64_t P, int E) {
    const int t = div_up(P, kGM) + (int)(P < E ? P : E);
    return div_up(t, kXcd) * kXcd;
}

int launch_gemm_gateup(const Mats& g, const Mats& u, const uint16_t* x, int M, int topk, const int32_t* offsets,
                       const int32_t* perm, const int32_t* tile_off, float* inter, hipStream_t st) {
    const int64_t P = (int64_t)M * topk;
    if (P == 0) return PGMOE_OK;
    const int E = g.n_mats;
    const int nnt = div_up(g.N, kGN / 2);
    const dim3 grid(gemm_max_mtiles(P, E) * nnt), block(kGThreads);
#define PG_GU(QT)                                                                                               \
    PG_LAUNCH((gemm_kernel<QT, true>), grid, block, 0, st, g.base, u.base, g.stride, u.stride, g.N, g.K, x, topk, \
              E, offsets, perm, tile_off, nnt, (const float*)nullptr, (const float*)nullptr, inter)
    switch (g.qtype) {
    case PGMOE_Q4_K: PG_GU(PGMOE_Q4_K); break;
    case PGMOE_Q6_K: PG_GU(PGMOE_Q6_K); break;
    case PGMOE_Q8_0: PG_GU(PGMOE_Q8_0); break;
    default: return fail(PGMOE_E_UNSUPPORTED, "gemm gate/up: qtype %d", g.qtype);
    }
#undef PG_GU
    return check_launch("gemm_gateup");
}

int launch_gemm_down(const Mats& d, const uint16_t* a16, const float* rs, int M, int topk, const int32_t* offsets,
                     const int32_t* perm, const int32_t* tile_off, const float* topk_w, float* partial,
                     hipStream_t st) {
    const int64_t P = (int64_t)M * topk;
    if (P == 0) return PGMOE_OK;
    const int E = d.n_mats;
    const int nnt = div_up(d.N, kGN);
    const dim3 grid(gemm_max_mtiles(P, E) * nnt), block(kGThreads);
#define PG_DN(QT)                                                                                               \
    PG_LAUNCH((gemm_kernel<QT, false>), grid, block, 0, st, d.base, d.base, d.stride, d.stride, d.N, d.K, a16,   \
              topk, E, offsets, perm, tile_off, nnt, rs, topk_w, partial)
    switch (d.qtype) {
    case PGMOE_Q4_K: PG_DN(PGMOE_Q4_K); break;
    case PGMOE_Q6_K: PG_DN(PGMOE_Q6_K); break;
    case PGMOE_Q8_0: PG_DN(PGMOE_Q8_0); break;
    default: return fail(PGMOE_E_UNSUPPORTED, "gemm down: qtype %d", d.qtype);
    }
#undef PG_DN
    return check_launch("gemm_down");
}

}  // namespace pgmoe
