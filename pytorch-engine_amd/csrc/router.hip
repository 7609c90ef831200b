// R1 + R2: router logits in a fixed reduction order, then softmax / top-k / renorm.
// Reference: pygguf_engine/model.py:902-907.
#include "common.h"
#include "launch.h"

namespace pgmoe {

// logits[m, e] = sum_h f32(x[m, h]) * W[e, h] (+ bias[e]).
// One wavefront per (TM tokens, TE experts) tile.  Lane l is "slot" l: it owns the 8-wide
// chunks c = l, l+64, l+128, ... of the row and runs one fmaf chain over them in
// ascending order; the 64 slot sums are then combined by the xor tree
// (l, l^32), (l, l^16), ..., (l, l^1); the bias is added last.  The CPU oracle
// (or_router_logits) performs the same operations in the same order, so both produce
// identical bits.
// An optional extra row (the shared expert's sigmoid-gate vector) is treated as expert E
// and written to extra_out[m] instead of logits.
// xsum (optional side output for the decode expert kernels): 16-element sums of every x
// row, computed by the blocks past the first rblocks (which hold the router waves).
template <int TM, int TE>
__global__ __launch_bounds__(256) void router_logits_kernel(const uint16_t* __restrict__ x,
                                                            const float* __restrict__ W,
                                                            const float* __restrict__ bias, int M, int H,
                                                            int E, float* __restrict__ logits,
                                                            const float* __restrict__ extra_w,
                                                            float* __restrict__ extra_out,
                                                            float* __restrict__ xsum, int rblocks) {
    PG_DECL;
    PG_MARK(0, 0);
    if ((int)blockIdx.x >= rblocks) {
        const int i = (blockIdx.x - rblocks) * blockDim.x + threadIdx.x;
        if (xsum && i < M * (H >> 4)) {
            const uint16_t* p = x + (int64_t)(i / (H >> 4)) * H + 16 * (i % (H >> 4));
            const uint4 a = *(const uint4*)p, b = *(const uint4*)(p + 8);
            const uint32_t v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
            float s = 0.f;
#pragma unroll
            for (int k = 0; k < 8; ++k) s += lo_half(v[k]) + hi_half(v[k]);
            xsum[i] = s;
        }
        return;
    }
    const int lane = threadIdx.x & 63;
    const int wave = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int rows = E + (extra_w ? 1 : 0);
    const int n_etiles = (rows + TE - 1) / TE;
    const int mt = wave / n_etiles, et = wave % n_etiles;
    const int m0 = mt * TM, e0 = et * TE;
    if (m0 >= M) return;
    float acc[TM][TE];
    router_tile<TM, TE>(x, W, extra_w, M, H, E, m0, e0, lane, acc);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TE; ++j) {
            float v = acc[i][j];
            const int m = m0 + i, e = e0 + j;
            if (lane == 0 && m < M && e < E) {
                if (bias) v = v + bias[e];
                logits[(int64_t)m * E + e] = v;
            } else if (lane == 0 && m < M && e == E && extra_w) {
                extra_out[m] = v;
            }
        }
    PG_MARK(0, 1);
    PG_FLUSH(0);
}

// Prefill logits (M > 8, no extra row): the same arithmetic as router_logits_kernel, tiled
// for reuse.  A block of 4 waves owns 16 tokens x 16 experts; wave w holds tokens
// 8 (w >> 1) .. +7 and experts 8 (w & 1) .. +7 (64 accumulators per lane).  The h axis is
// walked in rounds of 512 (round i = chunks 64i .. 64i+63): the block copies those x (fp16)
// and W (fp32) columns straight from HBM into LDS, and lane l extends, for each of its
// 8 x 8 (token, expert) pairs, the fmaf chain of slot l by chunk 64i + l (elements 0..7
// in order).  The slot sums then meet by the same xor tree (32, 16, ..., 1) and the bias
// is added last, so every logit has the bits of router_logits_kernel and of the CPU
// oracle.  48 KB of LDS and ~110 VGPRs: three blocks share a CU, so one block's copies
// overlap the others' FMAs.
constexpr int kRgT = 16, kRgE = 16, kRgH = 512;

__global__ __launch_bounds__(256) void router_gemm_kernel(const uint16_t* __restrict__ x, const float* __restrict__ W,
                                                          const float* __restrict__ bias, int M, int H, int E,
                                                          float* __restrict__ logits) {
    __shared__ __attribute__((aligned(16))) uint16_t xs[kRgT * kRgH];  // 16 KB
    __shared__ __attribute__((aligned(16))) float ws[kRgE * kRgH];     // 32 KB
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: row bases stay scalar
    const int m0 = blockIdx.x * kRgT, e0 = blockIdx.y * kRgE;
    const int wt = wave >> 1, we = wave & 1;
    float acc[8][8];
#pragma unroll
    for (int t = 0; t < 8; ++t)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[t][j] = 0.0f;
    for (int h0 = 0; h0 < H; h0 += kRgH) {
        __syncthreads();
        // stage by direct HBM -> LDS copies, 1 KB per wave instruction: x rows (16 x 1 KB)
        // and W rows (16 x 2 KB); wave w copies x rows w + 4q and W half-rows w + 4q
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int t = wave + 4 * q;
            dma16(x + (int64_t)min(m0 + t, M - 1) * H + h0 + 8 * lane, &xs[t * kRgH]);
        }
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const int hr = wave + 4 * q, r = hr >> 1, half = hr & 1;
            dma16(W + (int64_t)min(e0 + r, E - 1) * H + h0 + 256 * half + 4 * lane, &ws[r * kRgH + 256 * half]);
        }
        wait_dma();
        __syncthreads();
        float xv[8][8];
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const uint4 q = *(const uint4*)&xs[(8 * wt + t) * kRgH + 8 * lane];
            const uint32_t w4[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                xv[t][2 * k] = lo_half(w4[k]);
                xv[t][2 * k + 1] = hi_half(w4[k]);
            }
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float4 wa = *(const float4*)&ws[(8 * we + j) * kRgH + 8 * lane];
            const float4 wb = *(const float4*)&ws[(8 * we + j) * kRgH + 8 * lane + 4];
            const float wv[8] = {wa.x, wa.y, wa.z, wa.w, wb.x, wb.y, wb.z, wb.w};
#pragma unroll
            for (int t = 0; t < 8; ++t)
#pragma unroll
                for (int k = 0; k < 8; ++k) acc[t][j] = __builtin_fmaf(xv[t][k], wv[k], acc[t][j]);
        }
    }
    // slot sums -> logits: the xor tree as a reduce-scatter leaves pair l = (t, j) = (l / 8,
    // l % 8) of the wave's 64 in lane l
    float flat[64];
#pragma unroll
    for (int t = 0; t < 8; ++t)
#pragma unroll
        for (int j = 0; j < 8; ++j) flat[t * 8 + j] = acc[t][j];
    float mine = scatter_sum64<64>(flat, lane);
    const int m = m0 + 8 * wt + (lane >> 3), e = e0 + 8 * we + (lane & 7);
    if (m < M && e < E) {
        if (bias) mine = mine + bias[e];
        logits[(int64_t)m * E + e] = mine;
    }
}

// Per token: top-K experts by (logit desc, id asc); w = softmax prob (max-subtracted,
// denominator over all E); optional renorm w / max(sum w, 1e-20).  G lanes per token (16 or
// 32: four or two tokens a wave, for E <= 128 and K <= 16; else 64), lane g holding experts
// g + G r.
// Selection on logits equals selection on softmax probabilities (monotone map).  Each of
// the K rounds takes every lane's best untaken expert, then the group's best by xor
// exchanges within the group (DPP / permlane: groups never read each other's lanes).
template <int R, int G>  // logits held per lane: E <= G * R
__global__ __launch_bounds__(256) void topk_kernel(const float* __restrict__ logits, int M, int E, int K,
                                                   int norm, int32_t* __restrict__ idx,
                                                   float* __restrict__ w) {
    static_assert(G == 16 || G == 32 || G == 64, "lanes per token");
    const int g = threadIdx.x & (G - 1);
    const int m = blockIdx.x * (256 / G) + threadIdx.x / G;
    if (G == 64 && m >= M) return;
    const float* l = logits + (int64_t)min(m, M - 1) * E;  // a group past M repeats the last token, unstored
    float v[R];
    bool taken[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int e = g + G * r;
        v[r] = e < E ? l[e] : 0.0f;
        taken[r] = e >= E;
    }
    float top_logit = 0.0f, sum_sel = 0.0f;
    float my_w = 0.0f;
    int my_id = -1;
    for (int k = 0; k < K; ++k) {
        // lane-local best among untaken, lower id first on ties
        float bv = -INFINITY;
        int bi = 0x7fffffff;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int e = g + G * r;
            if (!taken[r] && (bi == 0x7fffffff || v[r] > bv)) {
                bv = v[r];
                bi = e;
            }
        }
        auto merge = [&](float ov, int oi) {
            if (oi != 0x7fffffff && (bi == 0x7fffffff || ov > bv || (ov == bv && oi < bi))) {
                bv = ov;
                bi = oi;
            }
        };
        if constexpr (G == 64) merge(xor_lane<32>(bv), xor_lane<32>(bi));
        if constexpr (G >= 32) merge(xor_lane<16>(bv), xor_lane<16>(bi));
        merge(xor_lane<8>(bv), xor_lane<8>(bi));
        merge(xor_lane<4>(bv), xor_lane<4>(bi));
        merge(xor_lane<2>(bv), xor_lane<2>(bi));
        merge(xor_lane<1>(bv), xor_lane<1>(bi));
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (g + G * r == bi) taken[r] = true;
        if (k == 0) top_logit = bv;
        if (g == k) {
            my_id = bi;
            my_w = bv;  // logit for now
        }
    }
    // softmax denominator over all experts
    float den = 0.0f;
#pragma unroll
    for (int r = 0; r < R; ++r)
        if (g + G * r < E) den += expf(v[r] - top_logit);
    den = group_sum<G>(den);
    float p = g < K ? expf(my_w - top_logit) / den : 0.0f;
    sum_sel = group_sum<G>(p);
    if (norm) p = p / fmaxf(sum_sel, 1e-20f);
    if (g < K && m < M) {
        idx[(int64_t)m * K + g] = my_id;
        w[(int64_t)m * K + g] = p;
    }
}

int launch_router_logits(const uint16_t* x, const float* W, const float* bias, int M, int H, int E,
                         float* logits, hipStream_t st, const float* extra_w, float* extra_out, float* xsum) {
    if (M <= 0) return PGMOE_OK;
    const int rows = E + (extra_w ? 1 : 0);
    // decode (M <= 8): one single-wave block per (all tokens, one expert), so the router
    // read spreads over as many CUs as there are experts; prefill: 4-wave blocks
    const int threads = M <= 8 ? 64 : 256;
    const int xblocks = xsum ? div_up(M * (H >> 4), threads) : 0;
#define PG_ROUTER(TM_, TE_)                                                                                   \
    do {                                                                                                      \
        const int rb = div_up(div_up(M, TM_) * div_up(rows, TE_), threads >> 6);                             \
        PG_LAUNCH((router_logits_kernel<TM_, TE_>), dim3(rb + xblocks), dim3(threads), 0, st, x, W, bias, \
                           M, H, E, logits, extra_w, extra_out, xsum, rb);                                    \
    } while (0)
    if (M == 1)
        PG_ROUTER(1, 1);
    else if (M == 2)
        PG_ROUTER(2, 1);
    else if (M <= 4)
        PG_ROUTER(4, 1);
    else if (M <= 8)
        PG_ROUTER(8, 1);
    else if (!extra_w && !xsum && E >= 16 && H % kRgH == 0 && div_up(M, kRgT) * div_up(E, kRgE) >= 1024) {
        PG_LAUNCH(router_gemm_kernel, dim3(div_up(M, kRgT), div_up(E, kRgE)), dim3(256), 0, st, x, W, bias, M, H, E,
                  logits);
    } else {
        // (the LDS-tiled GEMM only from 1024 blocks: at Qwen2's M = 512 it ran 128, 18.9 us;
        // 4 x 2 tiles 17.0 us)
        // tiles of 8 tokens x 4 rows while that still makes 2048 waves; else smaller ones (the
        // shared expert's one gate row, Mixtral's 8 experts), which change no logit (each
        // (token, row) pair is summed in the same order in every tile shape).  Measured: Qwen2's
        // shared gate at M = 512 15.3 -> 4.0 us, Mixtral's router at M = 2048 18.4 -> 11.5 us.
        auto waves = [&](int tm, int te) { return (long)div_up(M, tm) * div_up(rows, te); };
        if (waves(8, 4) >= 2048)
            PG_ROUTER(8, 4);
        else if (waves(4, 2) >= 2048)
            PG_ROUTER(4, 2);
        else
            PG_ROUTER(1, 1);
    }
#undef PG_ROUTER
    return check_launch("router_logits");
}

int launch_topk(const float* logits, int M, int E, int K, int norm, int32_t* idx, float* w, hipStream_t st) {
    if (M <= 0) return PGMOE_OK;
    const dim3 block(256);
    if (E > 1024) return fail(PGMOE_E_UNSUPPORTED, "top-k supports at most 1024 experts (got %d)", E);
    if (E <= 128 && K <= 16) {
        // four tokens a wave up to 32 experts, then two (Qwen3's E = 128 at M = 4096: 9.2 us
        // one token a wave, 7.5 four, 6.7 two)
        const dim3 g16(div_up(M, 16)), g32(div_up(M, 8));
        if (E <= 16)
            PG_LAUNCH((topk_kernel<1, 16>), g16, block, 0, st, logits, M, E, K, norm, idx, w);
        else if (E <= 32)
            PG_LAUNCH((topk_kernel<2, 16>), g16, block, 0, st, logits, M, E, K, norm, idx, w);
        else if (E <= 64)
            PG_LAUNCH((topk_kernel<2, 32>), g32, block, 0, st, logits, M, E, K, norm, idx, w);
        else
            PG_LAUNCH((topk_kernel<4, 32>), g32, block, 0, st, logits, M, E, K, norm, idx, w);
    } else {
        const dim3 grid(div_up(M, 4));
        if (E <= 64)
            PG_LAUNCH((topk_kernel<1, 64>), grid, block, 0, st, logits, M, E, K, norm, idx, w);
        else if (E <= 128)
            PG_LAUNCH((topk_kernel<2, 64>), grid, block, 0, st, logits, M, E, K, norm, idx, w);
        else if (E <= 256)
            PG_LAUNCH((topk_kernel<4, 64>), grid, block, 0, st, logits, M, E, K, norm, idx, w);
        else
            PG_LAUNCH((topk_kernel<16, 64>), grid, block, 0, st, logits, M, E, K, norm, idx, w);
    }
    return check_launch("topk");
}

}  // namespace pgmoe
