// R4-R7 launchers for the expert stages over the dispatched (sorted) token-expert pairs,
// the row-scale of the prefill down input, and the deterministic combine.
//   prefill (M > 8): grouped MFMA GEMMs in gemm.hip; decode GEMVs in decode_kernels.h
// Reference: GGUFQuantMoEExperts.forward_expert (quant_kernels.py:1990-2011) ->
// exec_w4a16_matmul / exec_w8a16_matmul (:1165-1420), exec_fused_act_mul_rowscale
// (:1423-1475), and the per-expert loop of model.py:911-922.
#include "common.h"
#include "launch.h"

namespace pgmoe {

// The prefill's streamed rows (SwiGLU rows, fp16 down input, per-pair partials, output)
// are each written once and read once by the next kernel, and do not fit the L2: they move
// with nontemporal loads and stores, so they do not evict the GEMMs' reused activation and
// weight lines.  Measured on the Qwen3 Zipf prefill (M = 4096): combine 63 -> 52 us, down
// GEMM 221 -> 214 us, gate/up 323 -> 317 us, step 712 -> 694 us; Mixtral's row-scale
// (M = 2048) 103 -> 92 us.
typedef float nf4 __attribute__((ext_vector_type(4)));
typedef uint32_t nu2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float4 ld_nt4(const float* p) {
    const nf4 v = __builtin_nontemporal_load((const nf4*)p);
    return make_float4(v.x, v.y, v.z, v.w);
}

// exec_fused_act_mul_rowscale's second half on an fp32 inter row: rs = max(max|v|/16384, 1),
// a16 = fp16(v / rs)  (quant_kernels.py:1467-1475).  One wave per row; rows of up to
// 64 * 4 * NV values are read once into registers, longer rows are read twice.
template <int NV>
__global__ __launch_bounds__(256) void rowscale_kernel(const float* __restrict__ inter, int P, int I,
                                                       uint16_t* __restrict__ a16, float* __restrict__ rs) {
    const int lane = threadIdx.x & 63;
    const int64_t p = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (p >= P) return;
    const float* row = inter + p * I;
    const int n4 = I >> 2;  // float4 words of the row (I % 4 == 0)
    float4 v[NV > 0 ? NV : 1];
    float mx = 0.0f;
    if (NV > 0) {
#pragma unroll
        for (int q = 0; q < NV; ++q) {
            const int i = lane + 64 * q;
            v[q] = i < n4 ? ld_nt4(row + 4 * i) : make_float4(0.f, 0.f, 0.f, 0.f);
            mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[q].x), fabsf(v[q].y)), fmaxf(fabsf(v[q].z), fabsf(v[q].w))));
        }
    } else {
        for (int i = lane; i < n4; i += 64) {
            const float4 u = *(const float4*)(row + 4 * i);
            mx = fmaxf(mx, fmaxf(fmaxf(fabsf(u.x), fabsf(u.y)), fmaxf(fabsf(u.z), fabsf(u.w))));
        }
    }
    mx = wave_max(mx);
    const float sc = fmaxf(mx * (1.0f / 16384.0f), 1.0f);
    if (lane == 0) rs[p] = sc;
    uint16_t* orow = a16 + p * I;
    auto put = [&](int i, float4 u) {
        const uint32_t lo = (uint32_t)__builtin_bit_cast(uint16_t, (half_t)(u.x / sc)) |
                            ((uint32_t)__builtin_bit_cast(uint16_t, (half_t)(u.y / sc)) << 16);
        const uint32_t hi = (uint32_t)__builtin_bit_cast(uint16_t, (half_t)(u.z / sc)) |
                            ((uint32_t)__builtin_bit_cast(uint16_t, (half_t)(u.w / sc)) << 16);
        __builtin_nontemporal_store(nu2{lo, hi}, (nu2*)(orow + 4 * i));
    };
    if (NV > 0) {
#pragma unroll
        for (int q = 0; q < NV; ++q) {
            const int i = lane + 64 * q;
            if (i < n4) put(i, v[q]);
        }
    } else {
        for (int i = lane; i < n4; i += 64) put(i, *(const float4*)(row + 4 * i));
    }
}

// The same for rows longer than 4096 (Mixtral's 14336, Qwen2's shared 20480): one block
// of 4 waves a row, read once into registers (NV float4 words a thread, rows of up to
// 1024 * NV values), the maximum over the block (order-free: the scale is rowscale_kernel's),
// then the fp16 row.  The one-wave form read such rows twice and, at a few hundred rows,
// left most CUs idle.
template <int NV>
__global__ __launch_bounds__(256) void rowscale_block_kernel(const float* __restrict__ inter, int I,
                                                             uint16_t* __restrict__ a16, float* __restrict__ rs) {
    __shared__ float wmx[4];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int64_t p = blockIdx.x;
    const float* row = inter + p * I;
    const int n4 = I >> 2;
    float4 v[NV];
    float mx = 0.0f;
#pragma unroll
    for (int q = 0; q < NV; ++q) {
        const int i = tid + 256 * q;
        v[q] = i < n4 ? ld_nt4(row + 4 * i) : make_float4(0.f, 0.f, 0.f, 0.f);
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[q].x), fabsf(v[q].y)), fmaxf(fabsf(v[q].z), fabsf(v[q].w))));
    }
    mx = wave_max(mx);
    if (lane == 0) wmx[w] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(wmx[0], wmx[1]), fmaxf(wmx[2], wmx[3]));
    const float sc = fmaxf(mx * (1.0f / 16384.0f), 1.0f);
    if (tid == 0) rs[p] = sc;
    uint16_t* orow = a16 + p * I;
#pragma unroll
    for (int q = 0; q < NV; ++q) {
        const int i = tid + 256 * q;
        if (i < n4) {
            const float4 u = v[q];
            const uint32_t lo = (uint32_t)__builtin_bit_cast(uint16_t, (half_t)(u.x / sc)) |
                                ((uint32_t)__builtin_bit_cast(uint16_t, (half_t)(u.y / sc)) << 16);
            const uint32_t hi = (uint32_t)__builtin_bit_cast(uint16_t, (half_t)(u.z / sc)) |
                                ((uint32_t)__builtin_bit_cast(uint16_t, (half_t)(u.w / sc)) << 16);
            __builtin_nontemporal_store(nu2{lo, hi}, (nu2*)(orow + 4 * i));
        }
    }
}

// Ascending order of N ints (N a power of two) by Batcher's odd-even merge sort: a fixed
// network of compare-exchanges on registers (N = 8: 19 of them).
template <int N>
__device__ __forceinline__ void sort_net(int (&a)[N]) {
#pragma unroll
    for (int p = 1; p < N; p += p)
#pragma unroll
        for (int k = p; k > 0; k /= 2)
#pragma unroll
            for (int j = k % p; j + k < N; j += k + k)
#pragma unroll
                for (int i = 0; i < k; ++i)
                    if (i + j + k < N && (i + j) / (p + p) == (i + j + k) / (p + p)) {
                        const int lo = min(a[i + j], a[i + j + k]), hi = max(a[i + j], a[i + j + k]);
                        a[i + j] = lo;
                        a[i + j + k] = hi;
                    }
}

// out[t, h] = sum of the token's K pair rows in ascending sorted position (= ascending
// expert id), then + shared[t, h] * sigmoid(shared_logit[t]).  Thread = 4 columns of one
// token; the K <= KP positions (KP a power of two, the rest padded past every position) are
// ordered (a sorting network for KP <= 4, else a selection), then all K row loads are
// issued before the in-order sum.  A 16 x 16 selection for K = 2 (Mixtral) took the
// combine at M = 2048 to 49 us, the network 19 us.
template <int KP>
__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ partial,
                                                      const int32_t* __restrict__ inv, int K, int H,
                                                      const float* __restrict__ shared,
                                                      const float* __restrict__ shared_logit,
                                                      float* __restrict__ out, uint64_t* __restrict__ clear,
                                                      int n_clear) {
    if (blockIdx.y == 0) clear_words(clear, n_clear);  // decode router logits (grid x = tokens)
    // the last token first: with the grouped GEMMs' tile order the rows of each expert's
    // last tiles were written last, and those hold its highest tokens
    const int t = gridDim.x - 1 - blockIdx.x;
    const int c = blockIdx.y * 256 + threadIdx.x;  // float4 column
    if (4 * c >= H) return;
    int srt[KP];
    if constexpr (KP <= 4) {
#pragma unroll
        for (int k = 0; k < KP; ++k) srt[k] = k < K ? inv[(int64_t)t * K + k] : 0x7fffffff;
        sort_net<KP>(srt);
    } else {
        // a selection (KP x KP on the scalar unit; 16 for every K > 4): at K = 8, where the
        // combine is bound by its row reads, it measured 51.5 us against 53.6 for the
        // network and 53.1 for an 8 x 8 selection (Qwen3 M = 4096, two A/B pairs each)
        int pos[KP];
#pragma unroll
        for (int k = 0; k < KP; ++k) pos[k] = k < K ? inv[(int64_t)t * K + k] : 0x7fffffff;
        int last = -1;
#pragma unroll
        for (int s = 0; s < KP; ++s) {
            int best = 0x7fffffff;
#pragma unroll
            for (int k = 0; k < KP; ++k) best = (pos[k] > last && pos[k] < best) ? pos[k] : best;
            srt[s] = best;
            last = best;
        }
    }
    float4 rows[KP];
#pragma unroll
    for (int s = 0; s < KP; ++s)
        if (s < K) rows[s] = ld_nt4(partial + (int64_t)srt[s] * H + 4 * c);
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int s = 0; s < KP; ++s)
        if (s < K) {
            acc.x += rows[s].x;
            acc.y += rows[s].y;
            acc.z += rows[s].z;
            acc.w += rows[s].w;
        }
    if (shared) {
        const float gate = shared_logit ? 1.0f / (1.0f + expf(-shared_logit[t])) : 1.0f;
        const float4 sv = *(const float4*)(shared + (int64_t)t * H + 4 * c);
        acc.x += sv.x * gate;
        acc.y += sv.y * gate;
        acc.z += sv.z * gate;
        acc.w += sv.w * gate;
    }
    __builtin_nontemporal_store(nf4{acc.x, acc.y, acc.z, acc.w}, (nf4*)(out + (int64_t)t * H + 4 * c));
}

// --------------------------------------------------------------------------- launchers
int launch_gateup(const Mats& g, const Mats& u, const uint16_t* x, int M, int topk, const int32_t* offsets,
                  const int32_t* perm, const int32_t* active, const int32_t* n_active, const int32_t* tile_off,
                  int mode, float* inter, hipStream_t st, float* raw, int act, const int32_t* tile_map) {
    const int64_t P = (int64_t)M * topk;
    if (P == 0) return PGMOE_OK;
    const int E = g.n_mats;
    if (mode == 0)
        return launch_dec_gateup(g, u, x, nullptr, topk, M, offsets, perm, active, n_active, (int)(P < E ? P : E),
                                 inter, nullptr, st, act);
    return launch_gemm_gateup(g, u, x, M, topk, offsets, perm, tile_off, inter, st, raw, act, tile_map);
}

int launch_down(const Mats& d, const float* inter, int M, int topk, const int32_t* offsets, const int32_t* perm,
                const int32_t* active, const int32_t* n_active, const int32_t* tile_off, const float* topk_w,
                int mode, uint16_t* a16, float* rs, float* partial, hipStream_t st, float* raw,
                const int32_t* tile_map) {
    const int64_t P = (int64_t)M * topk;
    if (P == 0) return PGMOE_OK;
    const int E = d.n_mats;
    if (mode == 0)
        return launch_dec_down(d, inter, nullptr, M, offsets, perm, active, n_active, (int)(P < E ? P : E), topk_w,
                               partial, st);
    if (!a16 || !rs) return fail(PGMOE_E_INVALID, "GEMM mode needs a16 and rs scratch");
    const int I = d.K;  // a multiple of 256 (checked with the weights)
    const dim3 rgrid(div_up(P, 4));
    if (I <= 1024)
        PG_LAUNCH(rowscale_kernel<4>, rgrid, dim3(256), 0, st, inter, (int)P, I, a16, rs);
    else if (I <= 4096)
        PG_LAUNCH(rowscale_kernel<16>, rgrid, dim3(256), 0, st, inter, (int)P, I, a16, rs);
    else if (I <= 16384)
        PG_LAUNCH(rowscale_block_kernel<16>, dim3((unsigned)P), dim3(256), 0, st, inter, I, a16, rs);
    else if (I <= 24576)
        PG_LAUNCH(rowscale_block_kernel<24>, dim3((unsigned)P), dim3(256), 0, st, inter, I, a16, rs);
    else
        PG_LAUNCH(rowscale_kernel<0>, rgrid, dim3(256), 0, st, inter, (int)P, I, a16, rs);
    int rc = check_launch("rowscale");
    if (rc) return rc;
    return launch_gemm_down(d, a16, rs, M, topk, offsets, perm, tile_off, topk_w, partial, st, raw, tile_map);
}

int launch_combine(const float* partial, const int32_t* inv, int M, int K, int H, const float* shared,
                   const float* shared_logit, float* out, hipStream_t st, uint64_t* clear,
                   int n_clear) {
    if (M <= 0) return PGMOE_OK;
    if (K > 16) return fail(PGMOE_E_UNSUPPORTED, "combine supports top_k <= 16");
    if (H % 4) return fail(PGMOE_E_UNSUPPORTED, "combine: H %d is not a multiple of 4", H);
    const dim3 grid(M, div_up(H / 4, 256));
    if (K <= 2)
        PG_LAUNCH(combine_kernel<2>, grid, dim3(256), 0, st, partial, inv, K, H, shared, shared_logit, out, clear,
                  n_clear);
    else if (K <= 4)
        PG_LAUNCH(combine_kernel<4>, grid, dim3(256), 0, st, partial, inv, K, H, shared, shared_logit, out, clear,
                  n_clear);
    else
        PG_LAUNCH(combine_kernel<16>, grid, dim3(256), 0, st, partial, inv, K, H, shared, shared_logit, out, clear,
                  n_clear);
    return check_launch("combine");
}

int gemm_tile_rows() { return gemm_tile_pairs(); }

}  // namespace pgmoe
