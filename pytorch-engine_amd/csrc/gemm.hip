// Prefill (M > 8) grouped expert products on the MFMA cores.
//
// A tile is 256 sorted pairs of one expert x 256 output columns.  The gate/up block is 8
// waves (two per SIMD; each owns 128 rows x 64 columns, so each B column is decoded by the
// two waves of its column), the down block 8 waves (two per SIMD; each all 256 rows x 32
// columns, every B column decoded once), as 4 x 2 or 8 x 1 v_mfma_f32_32x32x16_f16 tiles
// per wave (other layouts are build-time choices: CT column tiles, WM waves along M).  The K loop steps one 64-weight unit at a time
// through a ring of three LDS stages (two for fp16 weights) filled by direct HBM -> LDS
// copies three (two) units ahead: the fp16 activation rows (16-byte slots XOR-swizzled by row) and the raw GGUF
// bytes of the 256 weight rows (whole 1 KB chunks of the 64-row tile layout, with their
// scale chunks).  Each wave decodes its own B fragments from the raw bytes in registers
// (w = a * code + c in fp32, one rounding to fp16) one k16 group ahead of the MFMAs that
// use them, across unit boundaries.  One barrier per unit.
//   gate/up: A = x rows gathered through perm (fp16), B = 128 gate rows + 128 up rows of
//            the same intermediate indices, arranged so every wave holds matching gate
//            and up columns; epilogue = SwiGLU in fp32 -> inter [P][I].
//   down   : A = a16 [P][I] (the row-scaled fp16 SwiGLU rows), B = 256 down rows;
//            epilogue = partial[p][h] = w_p * rs_p * acc.
// Tiles: the dispatch's tile_off counts 256-row tiles per expert; the last tile of an
// expert holds the remainder (1..256 rows; 32-row slices past it skip their MFMAs and,
// with 4 waves, their activation copies).  With the dispatch's tile map the M tiles run
// every full tile first, then the partial ones by rows, most first: the long tiles do not
// land at the end of the launch (a Zipf routing scatters the large experts over the ids).  Block ids are ordered so the N tiles of one M
// tile run back to back on one XCD (blocks go to the 8 XCDs round-robin), so its
// gathered A rows are shared through that XCD's L2.
// Reference: GGUFQuantMoEExperts.forward_expert (quant_kernels.py:1990-2011) ->
// exec_w4a16_matmul / exec_w8a16_matmul (:1165-1420) and model.py:916-919.
#include <algorithm>
#include <atomic>
#include <type_traits>

#include "common.h"
#include "launch.h"

namespace pgmoe {

constexpr int kGM = 256;      // pair rows per tile
constexpr int kGN = 256;      // B rows (output columns) per tile
constexpr int kXcd = 8;

typedef _Float16 gh8 __attribute__((ext_vector_type(8)));
typedef uint32_t gu4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float gf16 __attribute__((ext_vector_type(16)));
typedef float gf4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------- staged weight bytes
// Per 64-weight unit u (see Fmt<QT>) a tile stages, for each of its four 64-row groups,
// CH chunks of quant bytes plus one scale chunk (whole 1 KB chunks):
//   Q4_K: qs chunks 1 + 2c, 2 + 2c (c = u % 4); scales: chunk u of the row group's scale
//         plane ({a, c} of sub-blocks 2c, 2c + 1 in fp32, decoded at load time)
//   Q5_K: as Q4_K, plus the fifth-bit chunk 9 + (c >> 1) (the unit's words at bytes 8(c & 1))
//   Q4_1: code chunks 2 + 2c, 3 + 2c; scales: chunk u of the scale plane ({a, c} of blocks
//         2c, 2c + 1), as Q4_K
//   Q6_K: ql chunks 4h + half, 4h + 2 + half, qh chunk 8 + 2h + half ((h, half) =
//         ((u % 4) >> 1, u & 1)); scales: chunk u of the scale plane (a of its four
//         16-weight sub-blocks)
//   Q8_0: chunks 4c .. 4c + 3 (the qs of Q8_0 blocks 2c, 2c + 1); scales: tile chunk 16
//   F16:  chunks 8c .. 8c + 7 (the weights); no scales
// Group g of the unit (k = 16g .. 16g + 15) reads, for the 8 weights 8h .. 8h + 7 of a lane
// half h, bytes 8h .. 8h + 7 of one staged chunk:
//   Q4_K: chunk g & 1, nibble g >> 1;  Q5_K: the same, and fifth-bit word g >> 1 (bits
//   4(g & 1) + 2h, + 1);  Q6_K: ql chunk g & 1 (nibble g >> 1) and the qh
//   chunk (bits 2g, 2g + 1);  Q8_0: chunk g;  F16: all 16 bytes of chunk 2g + h.
template <int QT> struct GStage;
template <> struct GStage<PGMOE_Q4_K> {
    static constexpr int CH = 2, HC = -1;  // HC: tile chunk of the scales (-1: scale plane)
    static constexpr int NS = 3;           // LDS stages of the ring
    __device__ static __forceinline__ int chunk(int u, int cc) { return 1 + 2 * (u & 3) + cc; }
};
template <> struct GStage<PGMOE_Q4_1> {
    static constexpr int CH = 2, HC = -1, NS = 3;
    __device__ static __forceinline__ int chunk(int u, int cc) { return 2 + 2 * (u & 3) + cc; }
};
template <> struct GStage<PGMOE_Q5_K> {
    static constexpr int CH = 3, HC = -1, NS = 3;
    __device__ static __forceinline__ int chunk(int u, int cc) { return cc < 2 ? 1 + 2 * (u & 3) + cc : 9 + ((u & 3) >> 1); }
};
template <> struct GStage<PGMOE_Q6_K> {
    static constexpr int CH = 3, HC = -1, NS = 3;
    __device__ static __forceinline__ int chunk(int u, int cc) {
        const int h = (u & 3) >> 1, half = u & 1;
        return cc == 0 ? 4 * h + half : cc == 1 ? 4 * h + 2 + half : 8 + 2 * h + half;
    }
};
template <> struct GStage<PGMOE_Q8_0> {
    static constexpr int CH = 4, HC = 16, NS = 3;
    __device__ static __forceinline__ int chunk(int u, int cc) { return 4 * (u & 3) + cc; }
};
// F16: the unit's 64 weights of a row are 8 chunks, 4 row groups x 8 KB a stage beside the
// 32 KB of A, so the ring has two stages (three would exceed the 160 KB of LDS); the
// "scale" slot repeats chunk 0 and is never read.
template <> struct GStage<PGMOE_F16> {
    static constexpr int CH = 8, HC = 0, NS = 2;
    __device__ static __forceinline__ int chunk(int u, int cc) { return 8 * (u & 3) + cc; }
};

// LDS stage: A [256 rows][128 bytes] (16-byte slot s of row r holds k chunk s ^ key(r),
// key(r) = (r & 7) ^ ((r >> 3) & 1): the 16 rows a 256-byte LDS pass reads then fall on 16
// different 16-byte bank groups),
// then B: row group bg, chunk cc (cc = CH: scales) at kGA + (bg * (CH + 1) + cc) * 1024.
constexpr int kGA = kGM * 128;
// CT = 32-column B tiles per wave, WM = waves along M: the block's 256 x 256 tile is cut
// into WM x (8 / CT) wave tiles of 256 / WM rows x 32 CT columns.  WM = 2, CT = 2: 8 waves,
// two per SIMD, each B column decoded by both waves of its column; WM = 1, CT = 2: 4 waves,
// one per SIMD, every B column decoded once (256 accumulators per lane, in AGPRs).
template <int QT, int CT, int WM>
struct GLay {
    static constexpr int CH = GStage<QT>::CH;
    static constexpr int NW = WM * 8 / CT;                          // waves
    static constexpr int WN = 8 / CT;                               // waves along N
    static constexpr int RS = 8 / WM;                               // 32-row slices per wave
    static constexpr int SLOTS = 4 * (CH + 1);                      // 1 KB copies for B
    static constexpr int AQ = 32 / NW;                              // A copies per wave
    static constexpr int BQ = (SLOTS + NW - 1) / NW;                // B copies per wave
    static constexpr int STAGE = kGA + SLOTS * 1024;
    static constexpr int VM = AQ + BQ;                              // copies per wave per unit
};

// HBM -> LDS copy of 16 bytes per lane (lane l to lds + 16 l), written as inline asm so
// the compiler neither adds waits for it before unrelated LDS reads nor counts it in its
// own vmcnt bookkeeping; the kernel waits for the copies itself (vm_wait) before the
// barrier that publishes a stage.  lds is the wave-uniform LDS byte address.
__device__ __forceinline__ void g2l(const void* g, uint32_t lds) {
    uint32_t keep;  // m0 is reserved to the compiler: restore it around the copy
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %1, off\n\ts_mov_b32 m0, %0"
                 : "=&s"(keep)
                 : "v"(g), "s"(lds)
                 : "memory");
}
template <int N>
__device__ __forceinline__ void vm_wait() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

typedef _Float16 gh2 __attribute__((ext_vector_type(2)));

// w = a * code + c2 as fp16 for 8 codes given as fp16 (1024 + code) pairs (c2 = c - 1024a
// folded by the caller: one fp32 FMA per weight, one rounding to fp16).
__device__ __forceinline__ gh8 deq8(const uint32_t (&m)[4], float a, float c) {
    gh8 r;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const gh2 h = __builtin_bit_cast(gh2, m[k]);
        r[2 * k] = (_Float16)__builtin_fmaf((float)h.x, a, c);
        r[2 * k + 1] = (_Float16)__builtin_fmaf((float)h.y, a, c);
    }
    return r;
}

// SiLU with the hardware exp2 and reciprocal (about 1 ulp each; the MFMA path's inputs
// are fp16 already).
__device__ __forceinline__ float silu_fast(float g) {
    return g * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-1.4426950408889634f * g));
}
// GELU (tanh approximation) with the same hardware exp2 / reciprocal:
// 0.5 g (1 + tanh(z)) = g - g / (1 + e^(2z)), z = sqrt(2/pi) (g + 0.044715 g^3).
__device__ __forceinline__ float gelu_fast(float g) {
    const float z = 0.7978845608028654f * (g + 0.044715f * g * g * g);
    return g - g * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(2.8853900817779268f * z));
}
__device__ __forceinline__ float act_fast(int act, float g) { return act ? gelu_fast(g) : silu_fast(g); }

__device__ __forceinline__ void magic8(uint32_t lo, uint32_t hi, uint32_t (&m)[4]) {
    m[0] = __builtin_amdgcn_perm(0x64646464u, lo, 0x04010400u);
    m[1] = __builtin_amdgcn_perm(0x64646464u, lo, 0x04030402u);
    m[2] = __builtin_amdgcn_perm(0x64646464u, hi, 0x04010400u);
    m[3] = __builtin_amdgcn_perm(0x64646464u, hi, 0x04030402u);
}

// One B column (row of W) of one unit in a lane: its staged bytes and scales, decoded per
// group into the MFMA B operand (8 fp16 weights k = 16g + 8h .. +8).
template <int QT> struct GCol;

template <> struct GCol<PGMOE_Q4_K> {
    u32x2 q[2];
    gf4 sv;            // scale plane: {a, c} of sub-block 2(u%4), then of 2(u%4) + 1
    float a[2], c[2];  // sub-blocks 2(u%4) (groups 0, 1), 2(u%4) + 1 (groups 2, 3)
    __device__ __forceinline__ void fetch(const uint8_t* B, int bg, int rig, int h, int u) {
        const uint8_t* base = B + bg * 3 * 1024 + rig * 16;
        q[0] = *(const u32x2*)(base + 8 * h);
        q[1] = *(const u32x2*)(base + 1024 + 8 * h);
        sv = *(const gf4*)(base + 2 * 1024);
    }
    __device__ __forceinline__ void prep(int u) {
        a[0] = sv.x;
        c[0] = sv.y;
        a[1] = sv.z;
        c[1] = sv.w;
    }
    __device__ __forceinline__ gh8 group(int g) const {
        const u32x2 s = q[g & 1];
        const int sh = 4 * (g >> 1);
        uint32_t m[4];
        magic8((s.x >> sh) & 0x0f0f0f0fu, (s.y >> sh) & 0x0f0f0f0fu, m);
        return deq8(m, a[g >> 1], c[g >> 1]);
    }
};

// Q4_1: the staged bytes and plane of Q4_K (codes in the same arrangement, {a, c} per block).
template <> struct GCol<PGMOE_Q4_1> : GCol<PGMOE_Q4_K> {};

template <> struct GCol<PGMOE_Q5_K> {
    u32x2 q[2], hw;    // qs chunks (bytes 8h .. 8h+7), the unit's two fifth-bit words
    gf4 sv;            // scale plane, as Q4_K
    float a[2], c[2];
    int hs;            // 2h: the lane half's first element quad within a 16-element group
    __device__ __forceinline__ void fetch(const uint8_t* B, int bg, int rig, int h, int u) {
        const uint8_t* base = B + bg * 4 * 1024 + rig * 16;
        q[0] = *(const u32x2*)(base + 8 * h);
        q[1] = *(const u32x2*)(base + 1024 + 8 * h);
        hw = *(const u32x2*)(base + 2 * 1024 + 8 * (u & 1));
        sv = *(const gf4*)(base + 3 * 1024);
        hs = 2 * h;
    }
    __device__ __forceinline__ void prep(int u) {
        a[0] = sv.x;
        c[0] = sv.y;
        a[1] = sv.z;
        c[1] = sv.w;
    }
    __device__ __forceinline__ gh8 group(int g) const {
        // elements 16(g & 1) + 8h + [0, 8) of sub-block 2(u%4) + (g >> 1): quads 4(g & 1) + 2h, + 1
        const u32x2 s = q[g & 1];
        const uint32_t w = (g >> 1) ? hw.y : hw.x;
        const int sh = 4 * (g >> 1), hb = 4 * (g & 1) + hs;
        const uint32_t c0 = ((s.x >> sh) & 0x0f0f0f0fu) | (((w >> hb) & 0x01010101u) << 4);
        const uint32_t c1 = ((s.y >> sh) & 0x0f0f0f0fu) | (((w >> (hb + 1)) & 0x01010101u) << 4);
        uint32_t m[4];
        magic8(c0, c1, m);
        return deq8(m, a[g >> 1], c[g >> 1]);
    }
};

template <> struct GCol<PGMOE_Q6_K> {
    u32x2 q[3];
    gf4 sv;  // scale plane: a of the unit's four sub-blocks, in group order
    float a[4];
    __device__ __forceinline__ void fetch(const uint8_t* B, int bg, int rig, int h, int u) {
        const uint8_t* base = B + bg * 4 * 1024 + rig * 16;
        q[0] = *(const u32x2*)(base + 8 * h);
        q[1] = *(const u32x2*)(base + 1024 + 8 * h);
        q[2] = *(const u32x2*)(base + 2 * 1024 + 8 * h);
        sv = *(const gf4*)(base + 3 * 1024);
    }
    __device__ __forceinline__ void prep(int u) {
        a[0] = sv.x;
        a[1] = sv.y;
        a[2] = sv.z;
        a[3] = sv.w;
    }
    __device__ __forceinline__ gh8 group(int g) const {
        const u32x2 l = q[g & 1], hq = q[2];
        const int sh = 4 * (g >> 1), hs = 2 * g;
        const uint32_t c0 = ((l.x >> sh) & 0x0f0f0f0fu) | (((hq.x >> hs) & 0x03030303u) << 4);
        const uint32_t c1 = ((l.y >> sh) & 0x0f0f0f0fu) | (((hq.y >> hs) & 0x03030303u) << 4);
        uint32_t m[4];
        magic8(c0, c1, m);
        return deq8(m, a[g], -1056.0f * a[g]);  // (1024 + q6) a - 1056 a = (q6 - 32) a
    }
};

template <> struct GCol<PGMOE_Q8_0> {
    u32x2 q[4];
    uint32_t dw;  // fp16 scales of Q8_0 blocks 2(u%4) (groups 0, 1), 2(u%4) + 1 (groups 2, 3)
    float d[2];
    __device__ __forceinline__ void fetch(const uint8_t* B, int bg, int rig, int h, int u) {
        const uint8_t* base = B + bg * 5 * 1024 + rig * 16;
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) q[cc] = *(const u32x2*)(base + cc * 1024 + 8 * h);
        dw = *(const uint32_t*)(base + 4 * 1024 + 4 * (u & 3));
    }
    __device__ __forceinline__ void prep(int u) {
        d[0] = lo_half(dw);
        d[1] = hi_half(dw);
    }
    __device__ __forceinline__ gh8 group(int g) const {
        const u32x2 s = q[g];
        uint32_t m[4];
        magic8(s.x ^ 0x80808080u, s.y ^ 0x80808080u, m);  // fp16 1152 + q
        return deq8(m, d[g >> 1], -1152.0f * d[g >> 1]);
    }
};

template <> struct GCol<PGMOE_F16> {
    gu4 c[4];  // group g: weights 16g + 8h .. +8 of the unit (chunk 2g + h)
    __device__ __forceinline__ void fetch(const uint8_t* B, int bg, int rig, int h, int u) {
        const uint8_t* base = B + bg * 9 * 1024 + rig * 16;
#pragma unroll
        for (int g = 0; g < 4; ++g) c[g] = *(const gu4*)(base + (2 * g + h) * 1024);
    }
    __device__ __forceinline__ void prep(int u) {}
    __device__ __forceinline__ gh8 group(int g) const { return __builtin_bit_cast(gh8, c[g]); }
};

// ---------------------------------------------------------------- tile mapping
// Block id -> (M tile, N tile).  Each M tile's N tiles form `runs` runs of consecutive N
// tiles; run u = (M tile u / runs, run u % runs) goes to XCD u % 8 (blocks go to the 8 XCDs
// round-robin), which runs its N tiles back to back, sharing the tile's gathered A rows
// through its L2.  runs = 1 from 32 M tiles on (M tile x on XCD x % 8); below 8 M tiles
// 8 / n_mtiles, so that no XCD is left without tiles; from 8 to 31, 8 / gcd(n_mtiles, 8)
// when that divides the N tiles, so that every XCD gets as many runs.  Returns false for
// ids past the last tile.  (The grid holds a multiple of 8 M tiles' blocks.)
__device__ __forceinline__ bool gemm_tile_of(int id, int n_ntiles, int n_mtiles, int& mt, int& nt) {
    if (n_mtiles <= 0) return false;
    const int x = id % kXcd, local = id / kXcd;
    int runs = 1;
    if (n_mtiles < kXcd) {
        runs = kXcd / n_mtiles;
    } else if (n_mtiles < 4 * kXcd) {
        const int r = kXcd / min(n_mtiles & -n_mtiles, kXcd);  // 8 / gcd(n_mtiles, 8)
        if (n_ntiles % r == 0) runs = r;
    }
    const int per = (n_ntiles + runs - 1) / runs;  // N tiles per run
    const int k = local / per, t = local - k * per;
    const int u = x + kXcd * k;
    mt = u / runs;
    nt = (u - mt * runs) * per + t;
    return mt < n_mtiles && nt < n_ntiles;
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

// ---------------------------------------------------------------- the unit loop
// Wave (wm, wn): rows 32 RS wm + 32 i (i < NI, the 32-row slices holding pairs), CT
// column tiles j.  Group g = k16 slice g of a unit: A fragment lane l = row l % 32, k chunk
// 2g + l / 32 (slot (2g + l/32) ^ key(row)); B fragment = the lane's column's group g,
// weights 8(l/32) .. +8.  Register v of D is D[8(v/4) + 4(l/32) + v%4][l%32].
// The groups of all units form one stream: the A fragments and B decode of group q + 1 are
// issued between the MFMAs of group q (a wave issues in order; each MFMA runs while the
// next few VALU / LDS instructions issue).  The one barrier of a unit comes before its last
// group's MFMAs: every read of the unit's stage has then been issued and waited for, so the
// barrier both publishes the next unit's stage (its copies waited for by vm_wait) and
// frees this one, which takes the copies of unit u + NS.  The next unit's scales and its
// first group are decoded under the last group's MFMAs.
// AC = A copies per wave per unit (the copies of empty 32-row slices are skipped when the
// wave copies whole slices), BQ = B copies: a wave has AC + BQ copies in flight per unit.
template <int QT, int NI, int CT, int RS, int AC, int BQ, int STAGE, class CopyF, int NS = GStage<QT>::NS>
__device__ __forceinline__ void gemm_loop(const uint8_t* smem, int units, const int (&bg)[CT], const int (&rig)[CT],
                                          int wm, int lane, gf16 (&acc)[RS][CT], CopyF& copy_unit) {
    constexpr int VM = AC + BQ;
    constexpr int NA = NI > 0 ? NI : 1;
    // VALU instructions (B decode) placed after each MFMA: about 16 CT + 16 per group
    constexpr int VPM = (16 * CT + 16 + CT * NA - 1) / (CT * NA);
    const int h = lane >> 5;
    // row r = 32 RS wm + 32 i + l%32 has key(r) = (l & 7) ^ ((l >> 3) & 1): one address per
    // group, the 32-row slices at immediate offsets 4096 i
    const int aoff = (32 * RS * wm + (lane & 31)) * 128;
    GCol<QT> col[CT];
    gh8 af[2][NA], bf[2][CT];
    auto cols = [&](const uint8_t* S, int u) {  // every LDS read of the columns, then the scales
#pragma unroll
        for (int j = 0; j < CT; ++j) col[j].fetch(S + kGA, bg[j], rig[j], h, u);
#pragma unroll
        for (int j = 0; j < CT; ++j) col[j].prep(u);
    };
    auto frag = [&](const uint8_t* S, int g, gh8 (&a)[NA], gh8 (&b)[CT]) {
        const uint8_t* p = S + aoff + 16 * ((2 * g + h) ^ (lane & 7) ^ ((lane >> 3) & 1));
#pragma unroll
        for (int i = 0; i < NI; ++i) a[i] = *(const gh8*)(p + 4096 * i);
#pragma unroll
        for (int j = 0; j < CT; ++j) b[j] = col[j].group(g);
    };
    const std::integral_constant<int, AC> ac;
#pragma unroll
    for (int s = 0; s < NS; ++s) copy_unit(ac, s, s);
    vm_wait<(NS - 1) * VM>();  // this wave's copies of unit 0 landed
    lds_barrier();             // and every wave's
    if constexpr (NI > 0) {
        cols(smem, 0);
        frag(smem, 0, af[0], bf[0]);
    }
    for (int u = 0, st = 0; u < units; ++u) {
        const int sn = st == NS - 1 ? 0 : st + 1;
        const uint8_t* S = smem + st * STAGE;
        const uint8_t* Sn = smem + sn * STAGE;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            if (g == 3) {
                vm_wait<(NS - 2) * VM>();
                lds_barrier();
                copy_unit(ac, u + NS, st);
            }
            if constexpr (NI > 0) {
                if (g < 3) {
                    frag(S, g + 1, af[(g + 1) & 1], bf[(g + 1) & 1]);
                } else {  // the next unit (past the last one: unused reads of a stale stage)
                    cols(Sn, u + 1);
                    frag(Sn, 0, af[0], bf[0]);
                }
#pragma unroll
                for (int i = 0; i < NI; ++i)
#pragma unroll
                    for (int j = 0; j < CT; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[g & 1][i], bf[g & 1][j], acc[i][j], 0, 0, 0);
#pragma unroll
                for (int k = 0; k < CT * NI; ++k) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
                    if (k < NI) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // 1 LDS read
                    __builtin_amdgcn_sched_group_barrier(0x002, VPM, 0);  // VALU
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        st = sn;
    }
}

// ---------------------------------------------------------------- the kernel
template <int QT, bool GATEUP, int CT, int WM>
__global__ __launch_bounds__(64 * (WM * 8 / CT)) void gemm_kernel(
    const uint8_t* __restrict__ w0, const uint8_t* __restrict__ w1, int64_t wstride0, int64_t wstride1,
    int N, int K, const uint16_t* __restrict__ act, int topk, int E, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ perm, const int32_t* __restrict__ tile_off, const int32_t* __restrict__ tile_map,
    int n_ntiles, const float* __restrict__ rs, const float* __restrict__ topk_w, float* __restrict__ out,
    const uint8_t* __restrict__ s0, const uint8_t* __restrict__ s1, int ksplit, int kper, float* __restrict__ raw,
    int gate_act) {
    using L = GLay<QT, CT, WM>;
    constexpr int NW = L::NW, WN = L::WN, RS = L::RS, WR = 32 * RS;  // WR rows per wave
    static_assert(!GATEUP || CT >= 2, "gate/up: each wave holds gate and matching up columns");
    static_assert(L::AQ * WN * WM == 32, "the waves' A copies cover the 32 row octets once");
    constexpr int CH = L::CH;
    __shared__ __attribute__((aligned(1024))) uint8_t smem[GStage<QT>::NS * L::STAGE];
    __shared__ int rowsrc[kGM];
    __shared__ float rowscale[kGM];  // down: rs[p] * topk_w[perm[p]] of every tile row
    int mt, nt;
    PG_DECL;
    PG_MARK(GATEUP ? 4 : 5, 0);
    PG_SET(6, 1u + (uint32_t)__builtin_amdgcn_s_getreg((31 << 11) | 4));  // HW_ID (CU, SIMD, wave)
    PG_SET(7, 1u + (uint32_t)__builtin_amdgcn_s_getreg((15 << 11) | 20));  // XCC_ID
    // split K (ksplit > 1): block = (tile, split ks); split ks takes super-blocks
    // [ks kper, (ks + 1) kper) and writes raw accumulators, reduced by gemm_split_reduce_kernel
    const int ks = ksplit > 1 ? (int)(blockIdx.x % ksplit) : 0;
    if (!gemm_tile_of(ksplit > 1 ? blockIdx.x / ksplit : blockIdx.x, n_ntiles, tile_off[E], mt, nt)) return;
    int e, m0;
    if (tile_map) {  // the dispatch's tile order: full tiles first, then the partial ones
        const int tm = tile_map[mt];
        e = tm & ((1 << kTileMapShift) - 1);
        m0 = offsets[e] + (tm >> kTileMapShift) * kGM;
    } else {
        e = gemm_tile_expert(tile_off, E, mt);
        m0 = offsets[e] + (mt - tile_off[e]) * kGM;
    }
    const int mrows = min(kGM, offsets[e + 1] - m0);
    PG_SET(2, 1u + (uint32_t)mrows);  // profiling builds: the tile's rows
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;  // waves w and w + WN: same columns
    const int nb = K >> 8;
    const int u0 = 4 * ks * kper;                       // first unit of this block's K range
    const int units = 4 * (min(nb, (ks + 1) * kper) - ks * kper);  // its units (>= 4)
    // A source rows: gate/up gathers token rows of x, down reads its own pair rows.  Rows
    // past the tile's pairs repeat its last pair: they only feed accumulator rows that
    // are never stored.
    if (tid < kGM) {
        const int p = m0 + min(tid, mrows - 1);
        rowsrc[tid] = GATEUP ? perm[p] / topk : p;
        if (!GATEUP) rowscale[tid] = rs[p] * topk_w[perm[p]];
    }
    __syncthreads();

    // ---- copy plan.  A: wave (wm, wn) copies rows 8i .. 8i+7 for the row octets
    // i = (32 / WM) wm + wn + WN q (q < AQ), all within its own 256 / WM rows; lane l takes
    // row 8i + l/8, slot l%8 = k chunk (l%8) ^ (l/8) ^ (i & 1), and i & 1 = wn & 1 for every
    // copy of the wave (WN and 32 / WM are even).  With WN = 4 copy q is octet wn of the
    // wave's slice q, so a wave copies only its slices with pairs.
    const int aoct = (32 / WM) * wm + wn;
    const int akc = (lane & 7) ^ (lane >> 3) ^ (wn & 1);
    const uint16_t* arow[L::AQ];
#pragma unroll
    for (int q = 0; q < L::AQ; ++q) arow[q] = act + (int64_t)rowsrc[8 * (aoct + WN * q) + (lane >> 3)] * K;
    // B row groups bg: gate/up: 0, 1 = gate rows nt*128 + 64bg, 2, 3 = the same up rows;
    // down: rows nt*256 + 64bg.  Groups past N repeat the last one (their columns are
    // never stored).
    const int ngr = row_groups(N);
    auto bmat = [&](int bg) -> const uint8_t* {
        return GATEUP ? (bg < 2 ? w0 + (int64_t)e * wstride0 : w1 + (int64_t)e * wstride1) : w0 + (int64_t)e * wstride0;
    };
    auto brg = [&](int bg) { return min(GATEUP ? 2 * nt + (bg & 1) : 4 * nt + bg, ngr - 1); };
    // scale plane of the row group (K-quants): nb * 4 chunks, chunk u for unit u
    const int64_t pstride = (int64_t)ngr * nb * 4096;
    auto bplane = [&](int bg) -> const uint8_t* {
        const uint8_t* pm = GATEUP ? (bg < 2 ? s0 : s1) : s0;
        return pm + (int64_t)e * pstride + (int64_t)brg(bg) * nb * 4096;
    };
    // B copy slots of this wave: s = wave + NW q; slot s: row group s / (CH + 1), chunk
    // s % (CH + 1) (CH = the scales: a tile chunk, or the scale plane); slots past SLOTS
    // repeat slot s - SLOTS (same source, same place).
    const uint8_t* bsrc[L::BQ];
    int bkind[L::BQ], bcc[L::BQ];
    uint32_t bdst[L::BQ];
#pragma unroll
    for (int q = 0; q < L::BQ; ++q) {
        int s = wave + NW * q;
        if (s >= L::SLOTS) s -= L::SLOTS;
        bdst[q] = s * 1024;
        const int bg = s / (CH + 1), cc = s % (CH + 1);
        bcc[q] = cc;
        if (cc == CH && GStage<QT>::HC < 0) {  // kind 1: scale plane chunk u
            bkind[q] = 1;
            bsrc[q] = bplane(bg) + lane * 16;
        } else {  // kind 0: tile chunk of super-block u / 4
            bkind[q] = 0;
            bsrc[q] = bmat(bg) + (int64_t)brg(bg) * nb * (Tile<QT>::CH * 1024) + lane * 16;
        }
    }
    const uint32_t sbase = lds_addr(smem);
    // Issue every copy of unit u into stage st (u clamped: the last steps repeat it).
    auto copy_unit = [&](auto ac, int u, int st) {  // ac: A copies (integral_constant)
        static_assert(decltype(ac)::value <= L::AQ, "more A copies than the wave's row octets");
        u = u0 + min(u, units - 1);  // relative unit -> absolute (past the range: repeat the last)
        const uint32_t S = sbase + st * L::STAGE;
#pragma unroll
        for (int q = 0; q < decltype(ac)::value; ++q)
            g2l(arow[q] + Fmt<QT>::col(u, akc >> 1) + 8 * (akc & 1), S + (aoct + WN * q) * 1024);
#pragma unroll
        for (int q = 0; q < L::BQ; ++q) {
            const uint8_t* src;
            if (bkind[q] == 0) {
                const int ch = bcc[q] == CH ? GStage<QT>::HC : GStage<QT>::chunk(u, bcc[q]);
                src = bsrc[q] + (int64_t)(u >> 2) * (Tile<QT>::CH * 1024) + ch * 1024;
            } else {
                src = bsrc[q] + (int64_t)u * 1024;
            }
            g2l(src, S + kGA + bdst[q]);
        }
    };

    gf16 acc[RS][CT];
#pragma unroll
    for (int i = 0; i < RS; ++i)
#pragma unroll
        for (int j = 0; j < CT; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;
    const bool active = WR * wm < mrows;
    const int ni = active ? min(RS, (mrows - WR * wm + 31) >> 5) : 0;  // 32-row slices with pairs
    // the lane's CT B columns (j): gate/up: j < CT/2 gate tile column c = 16 CT wn + 32j +
    // l%32 (rows nt*128 + c), j >= CT/2 the same up columns; down: tile column
    // c = 32 CT wn + 32j + l%32 (rows nt*256 + c).  Row group c / 64 (+ 2 for up), row c % 64.
    int bgj[CT], rigj[CT];
#pragma unroll
    for (int j = 0; j < CT; ++j) {
        const int jj = GATEUP ? j % (CT / 2) : j;
        const int c = (GATEUP ? 16 : 32) * CT * wn + 32 * jj + (lane & 31);
        bgj[j] = (c >> 6) + (GATEUP && j >= CT / 2 ? 2 : 0);
        rigj[j] = c & 63;
    }

    // ---- pipeline: NS stages (three; two for F16); unit u + NS is copied into unit u's
    // stage once every wave is done with it (see gemm_loop).  The loop is instantiated per NI (a whole copy each)
    // so the register allocation of one copy never has to merge the others'.
    PG_MARK(GATEUP ? 4 : 5, 1);
    // With 4 waves along N (CT = 2), wave (wm, wn) copies row octet wn of each of its 32-row
    // slices q, so the slices without pairs (q >= ni) are not copied at all.  With 8 waves
    // along N and one along M (the down product), copy q of wave w is octet w % 4 of slice
    // 2q + w / 4, so ceil(ni / 2) copies a wave cover the slices with pairs (for odd ni the
    // waves w >= 4 also copy slice ni, whose rows repeat the tile's last pair: unused, and
    // in bounds).  Other layouts copy every slice.
#define PG_GLOOP(NI_) \
    gemm_loop<QT, NI_, CT, RS, (WN == 4) ? NI_ : (WN == 8 && WM == 1) ? (NI_ + 1) / 2 : L::AQ, L::BQ, L::STAGE>( \
        smem, units, bgj, rigj, wm, \
                                                                                     lane, acc, copy_unit);
    switch (ni) {
    case 8: if constexpr (RS == 8) { PG_GLOOP(8) } break;
    case 7: if constexpr (RS == 8) { PG_GLOOP(7) } break;
    case 6: if constexpr (RS == 8) { PG_GLOOP(6) } break;
    case 5: if constexpr (RS == 8) { PG_GLOOP(5) } break;
    case 4: PG_GLOOP(4) break;
    case 3: PG_GLOOP(3) break;
    case 2: PG_GLOOP(2) break;
    case 1: PG_GLOOP(1) break;
    default: PG_GLOOP(0) break;
    }
#undef PG_GLOOP
    vm_wait<0>();  // the clamped copies past the last unit land before the block ends
    PG_MARK(GATEUP ? 4 : 5, 4);
    if (!active) return;
    if (ksplit > 1) {  // raw sums of this K range: [ks][p][c], gate/up c < 2N (up at N + c), down c < N
        const int NC = GATEUP ? 2 * N : N;
        float* rb = raw + (int64_t)ks * offsets[E] * NC;
#pragma unroll
        for (int j = 0; j < CT; ++j) {
            const int jj = GATEUP ? j % (CT / 2) : j;
            const int c = GATEUP ? nt * (kGN / 2) + 16 * CT * wn + 32 * jj + (lane & 31)
                                 : nt * kGN + 32 * CT * wn + 32 * j + (lane & 31);
            if (c >= N) continue;
            const int cc = GATEUP && j >= CT / 2 ? N + c : c;
#pragma unroll
            for (int i = 0; i < RS; ++i)
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int r = WR * wm + 32 * i + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
                    if (r < mrows) rb[(int64_t)(m0 + r) * NC + cc] = acc[i][j][v];
                }
        }
        return;
    }
    // epilogue: register v of tile (i, j) is row 32i + 8(v/4) + 4(l/32) + v%4, column
    // 32j + l%32 of the wave tile.  Nontemporal stores: the rows are read once, by the next
    // kernel, and must not evict the tiles' reused lines from the L2.
    if (GATEUP) {
        // wave columns: tiles j < CT/2 gate indices nt*128 + 16 CT wn + 32j + l%32, tile
        // j + CT/2 the matching up
#pragma unroll
        for (int j = 0; j < CT / 2; ++j) {
            const int col = nt * (kGN / 2) + 16 * CT * wn + 32 * j + (lane & 31);
            if (col < N) {
#pragma unroll
                for (int i = 0; i < RS; ++i)
#pragma unroll
                    for (int v = 0; v < 16; ++v) {
                        const int r = WR * wm + 32 * i + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
                        if (r < mrows)
                            __builtin_nontemporal_store(act_fast(gate_act, acc[i][j][v]) * acc[i][j + CT / 2][v],
                                                        &out[(int64_t)(m0 + r) * N + col]);
                    }
            }
        }
    } else if constexpr (WM == 1) {
        // Down, staged: the ring's LDS is free once every wave has left the loop.  Each half
        // of the tile's rows (128) goes through LDS as scaled fp32 rows of 256 columns and
        // then out as whole rows, 16 bytes a lane: a quarter of the store instructions of the
        // accumulator layout (4 bytes a lane, two 128-byte row pieces an instruction), which
        // is what bounds a CU's epilogue (the tile's 256 KB of partial rows).  Rows r and
        // r + 4 of a staged half are 4 LD floats apart: LD = 264 puts them on the two
        // halves of the LDS banks.
        constexpr int LD = kGN + 8;
        static_assert(128 * LD * 4 <= GStage<QT>::NS * L::STAGE, "a staged half fits the ring's LDS");
        float* stg = reinterpret_cast<float*>(smem);
        const int col = nt * kGN + 4 * lane;  // the lane's four columns of a row
        const bool vec = (N & 3) == 0;        // rows start 16-byte aligned
        __syncthreads();                      // every wave's copies landed and reads of the ring done
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            if (128 * half >= mrows) break;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if (128 * half + 32 * i >= mrows) break;
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int rr = 32 * i + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
                    const float sc = rowscale[128 * half + rr];
#pragma unroll
                    for (int j = 0; j < CT; ++j)
                        stg[rr * LD + 32 * CT * wn + 32 * j + (lane & 31)] = acc[4 * half + i][j][v] * sc;
                }
            }
            __syncthreads();
            for (int rr = wave; rr < 128; rr += NW) {
                const int r = 128 * half + rr;
                if (r >= mrows) break;
                const gf4 val = *reinterpret_cast<const gf4*>(&stg[rr * LD + 4 * lane]);
                float* dst = out + (int64_t)(m0 + r) * N + col;
                if (vec && col + 3 < N) {
                    __builtin_nontemporal_store(val, reinterpret_cast<gf4*>(dst));
                } else {
#pragma unroll
                    for (int c = 0; c < 4; ++c)
                        if (col + c < N) dst[c] = val[c];
                }
            }
            __syncthreads();  // the next half overwrites the staging
        }
    } else {
        const int c0 = nt * kGN + 32 * CT * wn + (lane & 31);
#pragma unroll
        for (int i = 0; i < RS; ++i)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int r = WR * wm + 32 * i + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
                if (r >= mrows) continue;
                const int p = m0 + r;
                const float sc = rowscale[r];
                float* orow = out + (int64_t)p * N;
#pragma unroll
                for (int j = 0; j < CT; ++j) {
                    const int col = c0 + 32 * j;
                    if (col < N) __builtin_nontemporal_store(acc[i][j][v] * sc, &orow[col]);
                }
            }
    }
    PG_MARK(GATEUP ? 4 : 5, 5);
    PG_FLUSH(GATEUP ? 4 : 5);
}

// The epilogue of a split-K product over every sorted pair p < P: the S raw partial sums
// of each output added in split order, then gate/up: inter[p][c] = silu(g) * u; down:
// partial[p][c] = rs[p] * topk_w[perm[p]] * acc (the unsplit kernel's epilogues).
// Four columns a thread (N % 4 == 0), every split's words loaded before the sums (at
// most kMaxSplitLoads splits in flight, then the next group), so the same additions in
// the same order run at streaming rate.  Measured (Qwen2 shared expert's down product,
// M = 512): one column a thread 17.3 us, four 13.2 us.
constexpr int kMaxSplitLoads = 8;
template <bool GATEUP>
__global__ __launch_bounds__(256) void gemm_split_reduce_kernel(const float* __restrict__ raw, int S, int64_t P,
                                                                int N, const float* __restrict__ rs,
                                                                const float* __restrict__ topk_w,
                                                                const int32_t* __restrict__ perm,
                                                                float* __restrict__ out, int act) {
    const int N4 = N >> 2;
    const int64_t n4 = P * N4;
    const int NC = GATEUP ? 2 * N : N;
    const int64_t sstride = P * NC;  // floats between splits
    auto ld4 = [](const float* q) {
        const floatx4 v = __builtin_nontemporal_load((const floatx4*)q);
        return make_float4(v.x, v.y, v.z, v.w);
    };
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t p = i / N4;
        const int c = 4 * (int)(i - p * N4);
        const float* r = raw + p * NC + c;
        float4 a = ld4(r), b = GATEUP ? ld4(r + N) : make_float4(0.f, 0.f, 0.f, 0.f);
        for (int k0 = 1; k0 < S; k0 += kMaxSplitLoads) {
            float4 va[kMaxSplitLoads], vb[kMaxSplitLoads];
#pragma unroll
            for (int j = 0; j < kMaxSplitLoads; ++j)
                if (k0 + j < S) {
                    va[j] = ld4(r + (k0 + j) * sstride);
                    if (GATEUP) vb[j] = ld4(r + (k0 + j) * sstride + N);
                }
#pragma unroll
            for (int j = 0; j < kMaxSplitLoads; ++j)
                if (k0 + j < S) {
                    a.x = a.x + va[j].x;
                    a.y = a.y + va[j].y;
                    a.z = a.z + va[j].z;
                    a.w = a.w + va[j].w;
                    if (GATEUP) {
                        b.x = b.x + vb[j].x;
                        b.y = b.y + vb[j].y;
                        b.z = b.z + vb[j].z;
                        b.w = b.w + vb[j].w;
                    }
                }
        }
        float4 o;
        if constexpr (GATEUP) {
            o = make_float4(act_fast(act, a.x) * b.x, act_fast(act, a.y) * b.y, act_fast(act, a.z) * b.z,
                            act_fast(act, a.w) * b.w);
        } else {
            const float f = rs[p] * topk_w[perm[p]];
            o = make_float4(f * a.x, f * a.y, f * a.z, f * a.w);
        }
        *(float4*)(out + p * N + c) = o;
    }
}

int gemm_tile_pairs() { return kGM; }

// Compute units of the current device (cached per device; an atomic, as host threads may
// launch concurrently).
static int device_cus() {
    static std::atomic<int> cached[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int n = cached[dev].load(std::memory_order_relaxed);
    if (!n) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cached[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

// K splits of a grouped product whose tiles would not fill the chip: tiles (an estimate:
// exact for one expert, P / 256 plus half the possible remainder tiles otherwise) times N
// tiles below one workgroup per CU (a workgroup's LDS fills a CU) gets the smallest split
// count that reaches it, cut at super-block boundaries (kper super-blocks per split, every
// split non-empty).
GemmSplit gemm_split(int64_t P, int E, int N, int K, bool gateup) {
    GemmSplit sp{1, K >> 8};
    if (P <= 0) return sp;
    const int64_t tiles = div_up(P, kGM) + (E > 1 ? (P < E ? P : E) / 2 : 0);
    const int64_t blocks = tiles * div_up(N, gateup ? kGN / 2 : kGN);
    const int64_t want = device_cus();
    if (blocks >= want) return sp;
    const int nb = K >> 8;
    int s = (int)div_up(want, blocks);
    s = s < nb ? s : nb;
    s = s < 32 ? s : 32;
    if (s <= 1) return sp;
    sp.kper = div_up(nb, s);
    sp.ksplit = div_up(nb, sp.kper);
    return sp;
}

size_t gemm_split_bytes(int64_t P, int E, int N, int K, bool gateup) {
    const GemmSplit sp = gemm_split(P, E, N, K, gateup);
    return sp.ksplit > 1 ? (size_t)sp.ksplit * P * (gateup ? 2 * N : N) * 4 : 0;
}

// The most split scratch any P' <= P pairs take.  gemm_split_bytes is not monotone in P
// (one more M tile can lower the split count), so a workspace sized for P must hold the
// largest of them to serve every smaller batch.  The split count never grows with P' (the
// tile estimate never shrinks), so for each count s > 1 the largest P' still splitting at
// least s ways is found by bisection, and the maximum lies at one of those P'.
size_t gemm_split_bytes_upto(int64_t P, int E, int N, int K, bool gateup) {
    size_t best = gemm_split_bytes(P, E, N, K, gateup);
    if (P <= 0) return best;
    const int s1 = gemm_split(1, E, N, K, gateup).ksplit;
    for (int s = 2; s <= s1; ++s) {
        int64_t lo = 1, hi = P;  // largest P' in [1, P] with ksplit(P') >= s (ksplit(1) >= s)
        if (gemm_split(hi, E, N, K, gateup).ksplit >= s) {
            lo = hi;
        } else {
            while (hi - lo > 1) {
                const int64_t mid = lo + (hi - lo) / 2;
                if (gemm_split(mid, E, N, K, gateup).ksplit >= s) lo = mid;
                else hi = mid;
            }
        }
        best = std::max(best, gemm_split_bytes(lo, E, N, K, gateup));
    }
    return best;
}

static int launch_split_reduce(bool gateup, const float* raw, int S, int64_t P, int N, const float* rs,
                               const float* topk_w, const int32_t* perm, float* out, hipStream_t st, int act) {
    const int64_t n = P * (N / 4);  // four columns a thread
    const int blocks = (int)(div_up(n, 256) < 16384 ? div_up(n, 256) : 16384);
    if (N % 4) return fail(PGMOE_E_UNSUPPORTED, "split reduce: N %d is not a multiple of 4", N);
    if (gateup)
        PG_LAUNCH(gemm_split_reduce_kernel<true>, dim3(blocks), dim3(256), 0, st, raw, S, P, N, rs, topk_w, perm, out,
                  act);
    else
        PG_LAUNCH(gemm_split_reduce_kernel<false>, dim3(blocks), dim3(256), 0, st, raw, S, P, N, rs, topk_w, perm, out,
                  act);
    return check_launch("gemm split reduce");
}

// Wave layout of each product (build-time choices): CT column tiles per wave, WM waves
// along M.  gate/up: 8 waves of 128 rows x 64 columns (CT = 2, WM = 2; two waves a SIMD,
// each B column decoded by the two waves of its column).  With one wave a SIMD (WM = 1,
// 256 rows x 64 columns, every B column decoded once) the matrix cores co-execute with
// VALU for only a fifth of their busy cycles (SQ_VALU_MFMA_COEXEC_CYCLES / _BUSY_CYCLES,
// Mixtral's all-full-tile gate/up): the second wave's decode fills part of that.  Measured
// (same box, two A/B pairs): Qwen3 Zipf M = 4096 gate/up 311 / 309 -> 299 / 298 us, Qwen2
// shared gate/up 232 -> 212-218 us, Mixtral M = 2048 unchanged (1055 us).  Down: 8 waves
// of 256 rows x 32 columns (CT = 1, WM = 1: each B column decoded once, two waves a SIMD):
// Q6_K 229 -> 225 us, Mixtral's Q4_K 770 -> 712 us against 8 waves of 128 x 64 (CT = 2,
// WM = 2, every B column decoded by two waves).
#ifndef PG_GU_CT
#define PG_GU_CT 2
#endif
#ifndef PG_DN_CT
#define PG_DN_CT 1
#endif
#ifndef PG_GU_WM
#define PG_GU_WM 2
#endif
#ifndef PG_DN_WM
#define PG_DN_WM 1
#endif

// Upper bound of 256-row tiles for P pairs over at most E experts, rounded up to whole
// XCD groups.
static int gemm_max_mtiles(int64_t P, int E) {
    const int t = div_up(P, kGM) + (int)(P < E ? P : E);
    return div_up(t, kXcd) * kXcd;
}

int launch_gemm_gateup(const Mats& g, const Mats& u, const uint16_t* x, int M, int topk, const int32_t* offsets,
                       const int32_t* perm, const int32_t* tile_off, float* inter, hipStream_t st, float* raw,
                       int act, const int32_t* tile_map) {
    const int64_t P = (int64_t)M * topk;
    if (P == 0) return PGMOE_OK;
    const int E = g.n_mats;
    if (g.qtype != PGMOE_Q8_0 && g.qtype != PGMOE_F16 && (!g.scales || !u.scales))
        return fail(PGMOE_E_INVALID, "gemm gate/up: K-quant weights need their scale plane (pgmoe_build_scale_plane)");
    const int nnt = div_up(g.N, kGN / 2);
    const GemmSplit sp = raw ? gemm_split(P, E, g.N, g.K, true) : GemmSplit{1, g.K >> 8};
    const dim3 grid(gemm_max_mtiles(P, E) * nnt * sp.ksplit);
#define PG_GU(QT)                                                                                               \
    PG_LAUNCH((gemm_kernel<QT, true, PG_GU_CT, PG_GU_WM>), grid, dim3(64 * GLay<QT, PG_GU_CT, PG_GU_WM>::NW), 0, st, g.base, u.base, g.stride, u.stride, g.N, g.K, x, topk, \
              E, offsets, perm, tile_off, tile_map, nnt, (const float*)nullptr, (const float*)nullptr, inter, g.scales, u.scales, \
              sp.ksplit, sp.kper, raw, act)
    switch (g.qtype) {
    case PGMOE_Q4_1: PG_GU(PGMOE_Q4_1); break;
    case PGMOE_Q4_K: PG_GU(PGMOE_Q4_K); break;
    case PGMOE_Q5_K: PG_GU(PGMOE_Q5_K); break;
    case PGMOE_Q6_K: PG_GU(PGMOE_Q6_K); break;
    case PGMOE_Q8_0: PG_GU(PGMOE_Q8_0); break;
    case PGMOE_F16: PG_GU(PGMOE_F16); break;
    default: return fail(PGMOE_E_UNSUPPORTED, "gemm gate/up: qtype %d", g.qtype);
    }
#undef PG_GU
    int rc = check_launch("gemm_gateup");
    if (rc || sp.ksplit == 1) return rc;
    return launch_split_reduce(true, raw, sp.ksplit, P, g.N, nullptr, nullptr, nullptr, inter, st, act);
}

int launch_gemm_down(const Mats& d, const uint16_t* a16, const float* rs, int M, int topk, const int32_t* offsets,
                     const int32_t* perm, const int32_t* tile_off, const float* topk_w, float* partial,
                     hipStream_t st, float* raw, const int32_t* tile_map) {
    const int64_t P = (int64_t)M * topk;
    if (P == 0) return PGMOE_OK;
    const int E = d.n_mats;
    if (d.qtype != PGMOE_Q8_0 && d.qtype != PGMOE_F16 && !d.scales)
        return fail(PGMOE_E_INVALID, "gemm down: K-quant weights need their scale plane (pgmoe_build_scale_plane)");
    const int nnt = div_up(d.N, kGN);
    const GemmSplit sp = raw ? gemm_split(P, E, d.N, d.K, false) : GemmSplit{1, d.K >> 8};
    const dim3 grid(gemm_max_mtiles(P, E) * nnt * sp.ksplit);
#define PG_DN(QT)                                                                                               \
    PG_LAUNCH((gemm_kernel<QT, false, PG_DN_CT, PG_DN_WM>), grid, dim3(64 * GLay<QT, PG_DN_CT, PG_DN_WM>::NW), 0, st, d.base, d.base, d.stride, d.stride, d.N, d.K, a16,   \
              topk, E, offsets, perm, tile_off, tile_map, nnt, rs, topk_w, partial, d.scales, d.scales, sp.ksplit, sp.kper, raw, \
              PGMOE_ACT_SILU)
    switch (d.qtype) {
    case PGMOE_Q4_1: PG_DN(PGMOE_Q4_1); break;
    case PGMOE_Q4_K: PG_DN(PGMOE_Q4_K); break;
    case PGMOE_Q5_K: PG_DN(PGMOE_Q5_K); break;
    case PGMOE_Q6_K: PG_DN(PGMOE_Q6_K); break;
    case PGMOE_Q8_0: PG_DN(PGMOE_Q8_0); break;
    case PGMOE_F16: PG_DN(PGMOE_F16); break;
    default: return fail(PGMOE_E_UNSUPPORTED, "gemm down: qtype %d", d.qtype);
    }
#undef PG_DN
    int rc = check_launch("gemm_down");
    if (rc || sp.ksplit == 1) return rc;
    return launch_split_reduce(false, raw, sp.ksplit, P, d.N, rs, topk_w, perm, partial, st, PGMOE_ACT_SILU);
}

}  // namespace pgmoe
