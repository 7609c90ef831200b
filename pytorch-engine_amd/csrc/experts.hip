// R4-R7: grouped expert products over the dispatched (sorted) token-expert pairs.
//   prefill (M > 8): LDS-staged dequant-to-fp16 tiles feeding v_mfma_f32_16x16x32_f16
//   (the decode GEMVs live in decode.hip)
// Reference: GGUFQuantMoEExperts.forward_expert (quant_kernels.py:1990-2011) ->
// exec_w4a16_matmul / exec_w8a16_matmul (:1165-1420), exec_fused_act_mul_rowscale
// (:1423-1475), and the per-expert loop of model.py:911-922.
#include "common.h"
#include "launch.h"

namespace pgmoe {

constexpr int kBM = 64;  // pair rows per GEMM tile

// --------------------------------------------------------------------------- GEMM
// Tile lookup: tile_off is the exclusive scan of per-expert tile counts; the expert of
// `tile` is the largest e with tile_off[e] <= tile (experts without rows own no tile).
__device__ __forceinline__ int tile_expert(const int32_t* tile_off, int E, int tile) {
    int lo = 0, hi = E - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (tile_off[mid] <= tile) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

// Dequantise group g of unit u of `row` to 16 fp16 values in LDS (zeros past N).
template <int QT>
__device__ __forceinline__ void stage_weights(const uint8_t* m, int K, int N, int row, int u, int g, half_t* dst) {
    half_t hv[16];
    if (row < N) {
        float q[16], av, bv;
        Fmt<QT>::group(m, K, N, row, u, g, q, av, bv);
#pragma unroll
        for (int i = 0; i < 16; ++i) hv[i] = (half_t)(av * q[i] - bv);
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) hv[i] = (half_t)0.0f;
    }
    *(half8*)dst = *(const half8*)&hv[0];
    *(half8*)(dst + 8) = *(const half8*)&hv[8];
}

// The K loop runs over 64-weight units; unit u's tile column j is row element
// Fmt<QT>::col(u, j/16) + j%16 for both operands, so the product is exact for any
// unit-internal ordering.  MFMA fragment layout (16x16x32 f16): lane l holds
// A[l%16][8(l/16) .. +8] and B[8(l/16) .. +8][l%16]; D[4(l/16) + j][l%16] in acc[j].
constexpr int kLdsPitch = 64 + 8;  // halves per LDS row (pad against bank conflicts)

template <int QT>
__global__ __launch_bounds__(256) void gemm_gateup_kernel(const uint8_t* __restrict__ gbase,
                                                          const uint8_t* __restrict__ ubase, int64_t gstride,
                                                          int64_t ustride, int N, int K,
                                                          const uint16_t* __restrict__ x, int topk, int E,
                                                          const int32_t* __restrict__ offsets,
                                                          const int32_t* __restrict__ perm,
                                                          const int32_t* __restrict__ tile_off,
                                                          float* __restrict__ inter) {
    __shared__ __attribute__((aligned(16))) half_t As[kBM * kLdsPitch];
    __shared__ __attribute__((aligned(16))) half_t Bs[64 * kLdsPitch];  // rows 0-31 gate, 32-63 up
    __shared__ int tok_s[kBM];
    const int tile = blockIdx.x;
    if (tile >= tile_off[E]) return;
    const int e = tile_expert(tile_off, E, tile);
    const int m0 = offsets[e] + (tile - tile_off[e]) * kBM;
    const int mrows = min(kBM, offsets[e + 1] - m0);
    const int i0 = blockIdx.y * 32;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    if (tid < kBM) tok_s[tid] = tid < mrows ? perm[m0 + tid] / topk : -1;
    __syncthreads();
    const uint8_t* gm = gbase + (int64_t)e * gstride;
    const uint8_t* um = ubase + (int64_t)e * ustride;
    floatx4 accg[2], accu[2];
#pragma unroll
    for (int mi = 0; mi < 2; ++mi) {
        accg[mi] = floatx4{0.f, 0.f, 0.f, 0.f};
        accu[mi] = floatx4{0.f, 0.f, 0.f, 0.f};
    }
    const int sr = tid >> 2, sg = tid & 3;  // staging: row and group of this thread
    const int tk = tok_s[sr];
    const int units = K >> 6;
    for (int u = 0; u < units; ++u) {
        {
            const int col = Fmt<QT>::col(u, sg);
            uint4 v0 = make_uint4(0, 0, 0, 0), v1 = v0;
            if (tk >= 0) {
                const uint4* p = (const uint4*)(x + (int64_t)tk * K + col);
                v0 = p[0];
                v1 = p[1];
            }
            *(uint4*)&As[sr * kLdsPitch + 16 * sg] = v0;
            *(uint4*)&As[sr * kLdsPitch + 16 * sg + 8] = v1;
        }
        stage_weights<QT>(sr < 32 ? gm : um, K, N, i0 + (sr & 31), u, sg, &Bs[sr * kLdsPitch + 16 * sg]);
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < 64; kk += 32) {
            const int ko = kk + 8 * (lane >> 4);
            const half8 bg = *(const half8*)&Bs[(16 * wn + (lane & 15)) * kLdsPitch + ko];
            const half8 bu = *(const half8*)&Bs[(32 + 16 * wn + (lane & 15)) * kLdsPitch + ko];
#pragma unroll
            for (int mi = 0; mi < 2; ++mi) {
                const half8 af = *(const half8*)&As[(32 * wm + 16 * mi + (lane & 15)) * kLdsPitch + ko];
                accg[mi] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bg, accg[mi], 0, 0, 0);
                accu[mi] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bu, accu[mi], 0, 0, 0);
            }
        }
        __syncthreads();
    }
    const int col = i0 + 16 * wn + (lane & 15);
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int r = 32 * wm + 16 * mi + 4 * (lane >> 4) + j;
            if (r < mrows && col < N) inter[(int64_t)(m0 + r) * N + col] = silu(accg[mi][j]) * accu[mi][j];
        }
}

// partial[p, h] = rs[p] * w[perm[p]] * (a16_p . d_h); a16 = fp16(inter / rs).
template <int QT>
__global__ __launch_bounds__(256) void gemm_down_kernel(const uint8_t* __restrict__ dbase, int64_t dstride,
                                                        int N, int K, const uint16_t* __restrict__ a16,
                                                        const float* __restrict__ rs, int E,
                                                        const int32_t* __restrict__ offsets,
                                                        const int32_t* __restrict__ perm,
                                                        const int32_t* __restrict__ tile_off,
                                                        const float* __restrict__ topk_w,
                                                        float* __restrict__ partial) {
    __shared__ __attribute__((aligned(16))) half_t As[kBM * kLdsPitch];
    __shared__ __attribute__((aligned(16))) half_t Bs[64 * kLdsPitch];
    const int tile = blockIdx.x;
    if (tile >= tile_off[E]) return;
    const int e = tile_expert(tile_off, E, tile);
    const int m0 = offsets[e] + (tile - tile_off[e]) * kBM;
    const int mrows = min(kBM, offsets[e + 1] - m0);
    const int h0 = blockIdx.y * 64;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const uint8_t* dm = dbase + (int64_t)e * dstride;
    floatx4 acc[2][2];
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) acc[mi][ni] = floatx4{0.f, 0.f, 0.f, 0.f};
    const int sr = tid >> 2, sg = tid & 3;
    const bool arow = sr < mrows;
    const int units = K >> 6;
    for (int u = 0; u < units; ++u) {
        {
            const int col = Fmt<QT>::col(u, sg);
            uint4 v0 = make_uint4(0, 0, 0, 0), v1 = v0;
            if (arow) {
                const uint4* p = (const uint4*)(a16 + (int64_t)(m0 + sr) * K + col);
                v0 = p[0];
                v1 = p[1];
            }
            *(uint4*)&As[sr * kLdsPitch + 16 * sg] = v0;
            *(uint4*)&As[sr * kLdsPitch + 16 * sg + 8] = v1;
        }
        stage_weights<QT>(dm, K, N, h0 + sr, u, sg, &Bs[sr * kLdsPitch + 16 * sg]);
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < 64; kk += 32) {
            const int ko = kk + 8 * (lane >> 4);
            half8 bf[2];
#pragma unroll
            for (int ni = 0; ni < 2; ++ni) bf[ni] = *(const half8*)&Bs[(32 * wn + 16 * ni + (lane & 15)) * kLdsPitch + ko];
#pragma unroll
            for (int mi = 0; mi < 2; ++mi) {
                const half8 af = *(const half8*)&As[(32 * wm + 16 * mi + (lane & 15)) * kLdsPitch + ko];
#pragma unroll
                for (int ni = 0; ni < 2; ++ni)
                    acc[mi][ni] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[ni], acc[mi][ni], 0, 0, 0);
            }
        }
        __syncthreads();
    }
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int r = 32 * wm + 16 * mi + 4 * (lane >> 4) + j;
            if (r >= mrows) continue;
            const int p = m0 + r;
            const float sc = rs[p] * topk_w[perm[p]];
#pragma unroll
            for (int ni = 0; ni < 2; ++ni) {
                const int h = h0 + 32 * wn + 16 * ni + (lane & 15);
                if (h < N) partial[(int64_t)p * N + h] = acc[mi][ni][j] * sc;
            }
        }
}

// exec_fused_act_mul_rowscale's second half on an fp32 inter row: rs = max(max|v|/16384, 1),
// a16 = fp16(v / rs)  (quant_kernels.py:1467-1475).  One block per row.
__global__ __launch_bounds__(256) void rowscale_kernel(const float* __restrict__ inter, int I,
                                                       uint16_t* __restrict__ a16, float* __restrict__ rs) {
    __shared__ float red[4];
    const int64_t p = blockIdx.x;
    const float* row = inter + p * I;
    float mx = 0.0f;
    for (int i = threadIdx.x; i < I; i += 256) mx = fmaxf(mx, fabsf(row[i]));
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) mx = fmaxf(mx, __shfl_xor(mx, s, 64));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float s = fmaxf(mx * (1.0f / 16384.0f), 1.0f);
    if (threadIdx.x == 0) rs[p] = s;
    for (int i = threadIdx.x; i < I; i += 256)
        a16[p * I + i] = __builtin_bit_cast(uint16_t, (half_t)(row[i] / s));
}

// out[t, h] = sum of the token's K pair rows in ascending sorted position (= ascending
// expert id), then + shared[t, h] * sigmoid(shared_logit[t]).  Block = (token, 256 columns).
__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ partial,
                                                      const int32_t* __restrict__ inv, int K, int H,
                                                      const float* __restrict__ shared,
                                                      const float* __restrict__ shared_logit,
                                                      float* __restrict__ out) {
    const int t = blockIdx.x;
    const int h = blockIdx.y * 256 + threadIdx.x;
    int pos[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) pos[k] = k < K ? inv[(int64_t)t * K + k] : 0x7fffffff;
    // insertion sort (K <= 16)
    for (int a = 1; a < K; ++a) {
        const int v = pos[a];
        int b = a - 1;
        while (b >= 0 && pos[b] > v) {
            pos[b + 1] = pos[b];
            --b;
        }
        pos[b + 1] = v;
    }
    float gate = 1.0f;
    if (shared_logit) gate = 1.0f / (1.0f + expf(-shared_logit[t]));
    if (h < H) {
        float acc = 0.0f;
        for (int k = 0; k < K; ++k) acc += partial[(int64_t)pos[k] * H + h];
        if (shared) acc += shared[(int64_t)t * H + h] * gate;
        out[(int64_t)t * H + h] = acc;
    }
}

// --------------------------------------------------------------------------- launchers
int launch_gateup(const Mats& g, const Mats& u, const uint16_t* x, int M, int topk, const int32_t* offsets,
                  const int32_t* perm, const int32_t* active, const int32_t* n_active, const int32_t* tile_off,
                  int mode, float* inter, hipStream_t st) {
    const int64_t P = (int64_t)M * topk;
    if (P == 0) return PGMOE_OK;
    const int E = g.n_mats;
    if (mode == 0)
        return launch_dec_gateup(g, u, x, nullptr, topk, M, offsets, perm, active, n_active, (int)(P < E ? P : E),
                                 inter, nullptr, st);
    const int max_tiles = div_up(P, kBM) + (int)(P < E ? P : E);
    const dim3 grid(max_tiles, div_up(g.N, 32)), block(256);
    switch (g.qtype) {
    case PGMOE_Q4_K: PG_LAUNCH((gemm_gateup_kernel<PGMOE_Q4_K>), grid, block, 0, st, g.base, u.base, g.stride, u.stride, g.N, g.K, x, topk, E, offsets, perm, tile_off, inter); break;
    case PGMOE_Q6_K: PG_LAUNCH((gemm_gateup_kernel<PGMOE_Q6_K>), grid, block, 0, st, g.base, u.base, g.stride, u.stride, g.N, g.K, x, topk, E, offsets, perm, tile_off, inter); break;
    case PGMOE_Q8_0: PG_LAUNCH((gemm_gateup_kernel<PGMOE_Q8_0>), grid, block, 0, st, g.base, u.base, g.stride, u.stride, g.N, g.K, x, topk, E, offsets, perm, tile_off, inter); break;
    }
    return check_launch("gemm_gateup");
}

int launch_down(const Mats& d, const float* inter, int M, int topk, const int32_t* offsets, const int32_t* perm,
                const int32_t* active, const int32_t* n_active, const int32_t* tile_off, const float* topk_w,
                int mode, uint16_t* a16, float* rs, float* partial, hipStream_t st) {
    const int64_t P = (int64_t)M * topk;
    if (P == 0) return PGMOE_OK;
    const int E = d.n_mats;
    if (mode == 0)
        return launch_dec_down(d, inter, nullptr, M, offsets, perm, active, n_active, (int)(P < E ? P : E), topk_w,
                               partial, st);
    if (!a16 || !rs) return fail(PGMOE_E_INVALID, "GEMM mode needs a16 and rs scratch");
    PG_LAUNCH(rowscale_kernel, dim3((unsigned)P), dim3(256), 0, st, inter, d.K, a16, rs);
    int rc = check_launch("rowscale");
    if (rc) return rc;
    const int max_tiles = div_up(P, kBM) + (int)(P < E ? P : E);
    const dim3 grid(max_tiles, div_up(d.N, 64)), block(256);
    switch (d.qtype) {
    case PGMOE_Q4_K: PG_LAUNCH((gemm_down_kernel<PGMOE_Q4_K>), grid, block, 0, st, d.base, d.stride, d.N, d.K, a16, rs, E, offsets, perm, tile_off, topk_w, partial); break;
    case PGMOE_Q6_K: PG_LAUNCH((gemm_down_kernel<PGMOE_Q6_K>), grid, block, 0, st, d.base, d.stride, d.N, d.K, a16, rs, E, offsets, perm, tile_off, topk_w, partial); break;
    case PGMOE_Q8_0: PG_LAUNCH((gemm_down_kernel<PGMOE_Q8_0>), grid, block, 0, st, d.base, d.stride, d.N, d.K, a16, rs, E, offsets, perm, tile_off, topk_w, partial); break;
    }
    return check_launch("gemm_down");
}

int launch_combine(const float* partial, const int32_t* inv, int M, int K, int H, const float* shared,
                   const float* shared_logit, float* out, hipStream_t st) {
    if (M <= 0) return PGMOE_OK;
    if (K > 16) return fail(PGMOE_E_UNSUPPORTED, "combine supports top_k <= 16");
    PG_LAUNCH(combine_kernel, dim3(M, div_up(H, 256)), dim3(256), 0, st, partial, inv, K, H, shared,
                       shared_logit, out);
    return check_launch("combine");
}

int gemm_tile_rows() { return kBM; }

}  // namespace pgmoe
