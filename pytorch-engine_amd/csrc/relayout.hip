// Load-time GGUF -> device layout conversion (same bits, 64-row interleaved tiles).
// Replaces the reference's CPU numpy repack (quant_kernels.py:854-1036), which
// re-quantises into W4/W8 arrays; here the GGUF bits are kept and only moved.
#include "common.h"
#include "launch.h"

namespace pgmoe {

template <int QT> struct Gguf;
template <> struct Gguf<PGMOE_Q4_K> { static constexpr int per = 256, bytes = 144; };
template <> struct Gguf<PGMOE_Q5_K> { static constexpr int per = 256, bytes = 176; };
template <> struct Gguf<PGMOE_Q6_K> { static constexpr int per = 256, bytes = 210; };
template <> struct Gguf<PGMOE_Q8_0> { static constexpr int per = 32, bytes = 34; };
template <> struct Gguf<PGMOE_Q4_0> { static constexpr int per = 32, bytes = 18; };
template <> struct Gguf<PGMOE_Q4_1> { static constexpr int per = 32, bytes = 20; };
template <> struct Gguf<PGMOE_Q5_0> { static constexpr int per = 32, bytes = 22; };
template <> struct Gguf<PGMOE_F16> { static constexpr int per = 256, bytes = 512; };  // a row's 256 fp16

// 16 bytes from s (A-byte aligned: 16 for blocks of a multiple of 16 bytes, 2 for Q6_K's
// 210 and Q8_0's 34) to d (16-byte aligned): one 16-byte store, the loads as wide as A allows.
template <int A>
__device__ __forceinline__ void copy16(uint8_t* d, const uint8_t* s) {
    uint4 v;
    if constexpr (A >= 16) {
        v = *(const uint4*)s;
    } else {
        static_assert(A == 2, "2- or 16-byte aligned sources");
        const uint16_t* p = (const uint16_t*)s;
        v = make_uint4(p[0] | ((uint32_t)p[1] << 16), p[2] | ((uint32_t)p[3] << 16), p[4] | ((uint32_t)p[5] << 16),
                       p[6] | ((uint32_t)p[7] << 16));
    }
    *(uint4*)d = v;
}

__device__ __forceinline__ void zero16(uint8_t* d) { *(uint4*)d = make_uint4(0, 0, 0, 0); }

// 16 bytes built in registers to d (16-byte aligned), one store.
__device__ __forceinline__ void store16(uint8_t* d, const uint8_t (&v)[16]) {
    uint32_t w[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
        w[k] = v[4 * k] | ((uint32_t)v[4 * k + 1] << 8) | ((uint32_t)v[4 * k + 2] << 16) | ((uint32_t)v[4 * k + 3] << 24);
    *(uint4*)d = make_uint4(w[0], w[1], w[2], w[3]);
}

// One thread per (matrix, padded row, 256-weight block) of the device matrix [N, 256 nb]
// (rows padded to 64).  Thread order: the row fastest, so the 64 threads of a wave fill one
// 64-row tile and each 16-byte chunk slot of the tile is one contiguous 1 KB store; for
// Q4_K the block fastest instead (a wave reads 64 consecutive 144-byte blocks of a row),
// which measured faster for its small blocks (113 MB: 93 against 108 us; Q8_0 624 MB 595 ->
// 487 us, Q6_K 165 MB 187 -> 176 us, F16 50 MB 56 -> 42 us with the row fastest).  The source matrix is [Ns, kbs blocks of the format] (Ns <= N;
// K-quants: kbs = nb; 32-weight formats: kbs <= 8 nb, any count): rows past Ns and 32-weight
// blocks past kbs are written as zeros, whose value is exactly 0 in every format.  Q5_0
// sources are written as Q8_0 tiles: d * (q - 16) (5-bit q) is the Q8_0 value d * qs with
// qs = q - 16 (same d, same 32-weight blocks).  Q4_0 sources are written as Q4_1 tiles:
// d * (q - 8) = d q + m with m = -8d (exact in fp16 for |d| < 8188).  Every value is kept
// exactly.
template <int QT>
__global__ void relayout_kernel(const uint8_t* __restrict__ src, int64_t n_mats, int Ns, int kbs, int N, int nb,
                                uint8_t* __restrict__ dst, int64_t dst_stride) {
    const int ng = row_groups(N);
    const int64_t per_mat = (int64_t)ng * 64 * nb;
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= per_mat * n_mats) return;
    const int64_t mat = gid / per_mat;
    const int64_t rem = gid % per_mat;
    int row, b;
    if constexpr (QT == PGMOE_Q4_K) {
        row = (int)(rem / nb);
        b = (int)(rem % nb);
    } else {
        const int tb = (int)(rem >> 6);  // tile rg * nb + b
        const int rg0 = tb / nb;
        b = tb - rg0 * nb;
        row = rg0 * 64 + (int)(rem & 63);
    }
    const int rg = row >> 6, r = row & 63;
    constexpr int DT = QT == PGMOE_Q5_0 ? PGMOE_Q8_0 : QT == PGMOE_Q4_0 ? PGMOE_Q4_1 : QT;  // device layout
    constexpr int CH = Tile<DT>::CH;
    uint8_t* md = dst + mat * dst_stride;
    uint8_t* t = md + ((int64_t)rg * nb + b) * (CH * 1024) + r * 16;
    const bool real = row < Ns;
    // GGUF bytes of this (row, 256-weight block): 32-weight blocks j of it are real while
    // 8b + j < kbs (K-quants: one block, b < kbs = nb)
    constexpr int BYT = Gguf<QT>::bytes, PER = Gguf<QT>::per;
    constexpr int sb = BYT * (256 / PER);
    const int64_t srow = (int64_t)kbs * BYT;  // source bytes per row
    const uint8_t* s = src + (mat * Ns + (real ? row : 0)) * srow + (int64_t)b * sb;
    auto realj = [&](int j) { return real && (PER == 256 || 8 * b + j < kbs); };
    if (QT == PGMOE_Q5_K) {  // GGUF: d, dmin, scales (0-15), qh (16-47), qs (48-175)
        for (int c = 0; c < 9; ++c) {
            if (real) copy16<16>(t + c * 1024, s + (c == 0 ? 0 : 48 + 16 * (c - 1)));
            else zero16(t + c * 1024);
        }
        // fifth bits regrouped: word (p, tt) bit 8(l & 3) + (l >> 2) = bit 2p + tt of qh[l]
        uint32_t w[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) w[i] = 0;
        if (real) {
            for (int l = 0; l < 32; ++l) {
                const uint32_t hb = s[16 + l];
#pragma unroll
                for (int i = 0; i < 8; ++i) w[i] |= ((hb >> i) & 1u) << (8 * (l & 3) + (l >> 2));
            }
        }
        for (int i = 0; i < 8; ++i) {  // word i = (p, tt) = (i >> 1, i & 1)
            uint8_t* d = t + (9 + (i >> 2)) * 1024 + 4 * (i & 3);
            d[0] = (uint8_t)w[i];
            d[1] = (uint8_t)(w[i] >> 8);
            d[2] = (uint8_t)(w[i] >> 16);
            d[3] = (uint8_t)(w[i] >> 24);
        }
    } else if (QT == PGMOE_Q4_K || QT == PGMOE_Q6_K || QT == PGMOE_F16) {
        for (int c = 0; c < CH; ++c) {
            if (real) copy16<QT == PGMOE_Q6_K ? 2 : 16>(t + c * 1024, s + 16 * c);
            else zero16(t + c * 1024);
        }
        if (QT == PGMOE_Q6_K) {
            uint8_t* d = md + (int64_t)ng * nb * CH * 1024 + (((int64_t)rg * nb + b) * 64 + r) * 2;
            d[0] = real ? s[208] : 0;
            d[1] = real ? s[209] : 0;
        }
    } else if (QT == PGMOE_Q5_0) {  // eight 22-byte blocks per 256 weights -> Q8_0 tiles
        for (int j = 0; j < 8; ++j) {
            const bool rj = realj(j);
            const uint8_t* bj = s + 22 * j;
            const uint32_t qh = rj ? (uint32_t)bj[2] | ((uint32_t)bj[3] << 8) | ((uint32_t)bj[4] << 16) |
                                         ((uint32_t)bj[5] << 24)
                                   : 0xffffffffu;  // padding: q = 16 -> 0
            uint8_t lo[16], hi[16];
#pragma unroll
            for (int l = 0; l < 16; ++l) {
                const int q = rj ? bj[6 + l] : 0;
                lo[l] = (uint8_t)(int8_t)(((q & 15) | (int)(((qh >> l) & 1) << 4)) - 16);
                hi[l] = (uint8_t)(int8_t)(((q >> 4) | (int)(((qh >> (16 + l)) & 1) << 4)) - 16);
            }
            store16(t + (2 * j) * 1024, lo);
            store16(t + (2 * j + 1) * 1024, hi);
            t[16 * 1024 + 2 * j] = rj ? bj[0] : 0;
            t[16 * 1024 + 2 * j + 1] = rj ? bj[1] : 0;
        }
    } else if (QT == PGMOE_Q4_0 || QT == PGMOE_Q4_1) {  // eight 18 / 20-byte blocks -> Q4_1 tiles
        constexpr int BB = Gguf<QT>::bytes, QO = QT == PGMOE_Q4_0 ? 2 : 4;  // block bytes, qs offset
        // codes of element l of block j: low nibble of qs[l] (l < 16), high nibble of qs[l - 16]
        auto code = [&](int j, int l) -> uint32_t {
            if (!realj(j)) return 0u;
            const uint8_t bt = s[BB * j + QO + (l & 15)];
            return l < 16 ? (bt & 15u) : (uint32_t)(bt >> 4);
        };
        for (int j = 0; j < 8; ++j) {
            uint16_t d = 0, m = 0;  // padding: d = m = 0
            if (realj(j)) {
                d = (uint16_t)s[BB * j] | ((uint16_t)s[BB * j + 1] << 8);
                if (QT == PGMOE_Q4_1)
                    m = (uint16_t)s[BB * j + 2] | ((uint16_t)s[BB * j + 3] << 8);
                else
                    m = __builtin_bit_cast(uint16_t, (half_t)(-8.0f * h2f(d)));
            }
            t[2 * j] = (uint8_t)d;
            t[2 * j + 1] = (uint8_t)(d >> 8);
            t[1024 + 2 * j] = (uint8_t)m;
            t[1024 + 2 * j + 1] = (uint8_t)(m >> 8);
        }
        for (int c = 0; c < 8; ++c) {  // Q4_K arrangement: byte 32J + l = element 64J + l | element 64J + 32 + l
            uint8_t v[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int k = 16 * c + i, J = k >> 5, l = k & 31;
                v[i] = (uint8_t)(code(2 * J, l) | (code(2 * J + 1, l) << 4));
            }
            store16(t + (2 + c) * 1024, v);
        }
    } else {  // Q8_0: eight 34-byte blocks per 256 weights
        for (int j = 0; j < 8; ++j) {
            const uint8_t* bj = s + 34 * j;
            if (realj(j)) {
                copy16<2>(t + (2 * j) * 1024, bj + 2);
                copy16<2>(t + (2 * j + 1) * 1024, bj + 18);
                t[16 * 1024 + 2 * j] = bj[0];
                t[16 * 1024 + 2 * j + 1] = bj[1];
            } else {
                zero16(t + (2 * j) * 1024);
                zero16(t + (2 * j + 1) * 1024);
                t[16 * 1024 + 2 * j] = 0;
                t[16 * 1024 + 2 * j + 1] = 0;
            }
        }
    }
}

// Scale plane: one thread per (matrix, 64-row group, super-block, 64-weight unit c, row):
// the unit's sub-block scales decoded from the tile bytes exactly as the MFMA products
// would decode them (same expressions, fp32), stored as one float4 per row.
template <int QT>
__global__ void scale_plane_kernel(const uint8_t* __restrict__ src, int64_t n_mats, int N, int nb,
                                   int64_t src_stride, uint8_t* __restrict__ dst, int64_t dst_stride) {
    const int ng = row_groups(N);
    const int64_t per_mat = (int64_t)ng * nb * 4 * 64;
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= per_mat * n_mats) return;
    const int64_t mat = gid / per_mat;
    const int64_t rem = gid % per_mat;  // ((rg * nb + b) * 4 + c) * 64 + r
    const int r = (int)(rem & 63), c = (int)((rem >> 6) & 3);
    const int64_t tb = rem >> 8;  // rg * nb + b
    const uint8_t* md = src + mat * src_stride;
    float4 v;
    if (QT == PGMOE_Q4_1) {  // fp16 d in chunk 0, m in chunk 1
        const uint8_t* tt = md + tb * (10 * 1024) + r * 16;
        const uint32_t dw = *(const uint32_t*)(tt + 4 * c), mw = *(const uint32_t*)(tt + 1024 + 4 * c);
        const float a0 = lo_half(dw), a1 = hi_half(dw);
        v = make_float4(a0, lo_half(mw) - 1024.0f * a0, a1, hi_half(mw) - 1024.0f * a1);
    } else if (QT == PGMOE_Q4_K || QT == PGMOE_Q5_K) {
        const uint4 hd = *(const uint4*)(md + tb * (Tile<QT>::CH * 1024) + r * 16);
        const float d = lo_half(hd.x), dm = hi_half(hd.x);
        float a[2], cc[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            int sc, mn;
            kscale_sel(hd.y, hd.z, hd.w, 2 * c + t, sc, mn);
            a[t] = d * (float)sc;
            cc[t] = -(dm * (float)mn) - 1024.0f * a[t];
        }
        v = make_float4(a[0], cc[0], a[1], cc[1]);
    } else {  // Q6_K: int8 scales in chunk 12, fp16 d in the plane after the tiles
        const uint8_t* sc = md + tb * (13 * 1024) + 12 * 1024 + r * 16;
        const uint16_t db = *(const uint16_t*)(md + (int64_t)ng * nb * 13 * 1024 + (tb * 64 + r) * 2);
        const float d = h2f(db);
        const int h = c >> 1, half = c & 1;
        float a[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) a[g] = d * (float)(int8_t)sc[8 * h + 2 * g + half];
        v = make_float4(a[0], a[1], a[2], a[3]);
    }
    *(float4*)(dst + mat * dst_stride + rem * 16) = v;
}

int64_t scale_plane_bytes(int qtype, int64_t rows, int64_t cols) {
    if (qtype == PGMOE_Q4_0 || qtype == PGMOE_Q5_0 || layout_bytes(qtype, rows, cols) < 0)
        return -1;  // Q4_0 / Q5_0: source formats (their device layouts are Q4_1 / Q8_0)
    if (qtype == PGMOE_Q8_0 || qtype == PGMOE_F16) return 0;  // scales in the tiles, or none
    return (int64_t)row_groups((int)rows) * (cols / 256) * 4 * 1024;
}

int launch_scale_plane(int qtype, const uint8_t* src, int64_t n_mats, int64_t rows, int64_t cols,
                       int64_t src_stride, uint8_t* dst, hipStream_t st) {
    const int nb = (int)(cols / 256);
    const int64_t n = n_mats * (int64_t)row_groups((int)rows) * nb * 4 * 64;
    const int64_t dst_stride = scale_plane_bytes(qtype, rows, cols);
    if (n == 0) return PGMOE_OK;
    const dim3 grid((unsigned)((n + 255) / 256));
    switch (qtype) {
    case PGMOE_Q4_1:
        PG_LAUNCH(scale_plane_kernel<PGMOE_Q4_1>, grid, dim3(256), 0, st, src, n_mats, (int)rows, nb, src_stride,
                  dst, dst_stride);
        break;
    case PGMOE_Q4_K:
        PG_LAUNCH(scale_plane_kernel<PGMOE_Q4_K>, grid, dim3(256), 0, st, src, n_mats, (int)rows, nb, src_stride,
                  dst, dst_stride);
        break;
    case PGMOE_Q5_K:
        PG_LAUNCH(scale_plane_kernel<PGMOE_Q5_K>, grid, dim3(256), 0, st, src, n_mats, (int)rows, nb, src_stride,
                  dst, dst_stride);
        break;
    case PGMOE_Q6_K:
        PG_LAUNCH(scale_plane_kernel<PGMOE_Q6_K>, grid, dim3(256), 0, st, src, n_mats, (int)rows, nb, src_stride,
                  dst, dst_stride);
        break;
    default:
        return fail(PGMOE_E_UNSUPPORTED, "scale plane: qtype %d has none", qtype);
    }
    return check_launch("scale_plane");
}

int64_t layout_bytes(int qtype, int64_t rows, int64_t cols) {
    if (cols % 256 || rows < 1) return -1;
    const int64_t ng = (rows + 63) / 64, nb = cols / 256;
    switch (qtype) {
    case PGMOE_Q4_K: return ng * nb * 9 * 1024;
    case PGMOE_Q5_K: return ng * nb * 11 * 1024;
    case PGMOE_Q6_K: return ng * nb * (13 * 1024 + 128);
    case PGMOE_Q4_0:  // stored as Q4_1
    case PGMOE_Q4_1: return ng * nb * 10 * 1024;
    case PGMOE_Q8_0:
    case PGMOE_Q5_0: return ng * nb * 17 * 1024;  // Q5_0 is stored as Q8_0
    case PGMOE_F16: return ng * nb * 32 * 1024;
    default: return -1;
    }
}

int launch_relayout(int qtype, const uint8_t* src, int64_t n_mats, int64_t rows, int64_t cols, int64_t rows_out,
                    int64_t cols_out, uint8_t* dst, int64_t dst_stride, hipStream_t st) {
    const int nb = (int)(cols_out / 256);
    int per = 256;  // weights per GGUF block
    if (qtype == PGMOE_Q8_0 || qtype == PGMOE_Q4_0 || qtype == PGMOE_Q4_1 || qtype == PGMOE_Q5_0) per = 32;
    const int kbs = (int)(cols / per);
    const int64_t n = n_mats * (int64_t)row_groups((int)rows_out) * 64 * nb;
    if (n == 0) return PGMOE_OK;
    const int threads = 256;
    const dim3 grid((unsigned)((n + threads - 1) / threads));
    const int Ns = (int)rows, N = (int)rows_out;
    switch (qtype) {
    case PGMOE_Q4_K:
        PG_LAUNCH(relayout_kernel<PGMOE_Q4_K>, grid, dim3(threads), 0, st, src, n_mats, Ns, kbs, N, nb, dst, dst_stride);
        break;
    case PGMOE_Q5_K:
        PG_LAUNCH(relayout_kernel<PGMOE_Q5_K>, grid, dim3(threads), 0, st, src, n_mats, Ns, kbs, N, nb, dst, dst_stride);
        break;
    case PGMOE_Q6_K:
        PG_LAUNCH(relayout_kernel<PGMOE_Q6_K>, grid, dim3(threads), 0, st, src, n_mats, Ns, kbs, N, nb, dst, dst_stride);
        break;
    case PGMOE_Q8_0:
        PG_LAUNCH(relayout_kernel<PGMOE_Q8_0>, grid, dim3(threads), 0, st, src, n_mats, Ns, kbs, N, nb, dst, dst_stride);
        break;
    case PGMOE_Q4_0:
        PG_LAUNCH(relayout_kernel<PGMOE_Q4_0>, grid, dim3(threads), 0, st, src, n_mats, Ns, kbs, N, nb, dst, dst_stride);
        break;
    case PGMOE_Q4_1:
        PG_LAUNCH(relayout_kernel<PGMOE_Q4_1>, grid, dim3(threads), 0, st, src, n_mats, Ns, kbs, N, nb, dst, dst_stride);
        break;
    case PGMOE_Q5_0:
        PG_LAUNCH(relayout_kernel<PGMOE_Q5_0>, grid, dim3(threads), 0, st, src, n_mats, Ns, kbs, N, nb, dst, dst_stride);
        break;
    case PGMOE_F16:
        PG_LAUNCH(relayout_kernel<PGMOE_F16>, grid, dim3(threads), 0, st, src, n_mats, Ns, kbs, N, nb, dst, dst_stride);
        break;
    default:
        return fail(PGMOE_E_UNSUPPORTED, "relayout: qtype %d", qtype);
    }
    return check_launch("relayout");
}

}  // namespace pgmoe
