// R4-R7 launchers for the expert stages over the dispatched (sorted) token-expert pairs,
// the row-scale of the prefill down input, and the deterministic combine.
//   prefill (M > 8): grouped MFMA GEMMs in gemm.hip; decode GEMVs in decode_kernels.h
// Reference: GGUFQuantMoEExperts.forward_expert (quant_kernels.py:1990-2011) ->
// exec_w4a16_matmul / exec_w8a16_matmul (:1165-1420), exec_fused_act_mul_rowscale
// (:1423-1475), and the per-expert loop of model.py:911-922.
#include "common.h"
#include "launch.h"

namespace pgmoe {

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
    return launch_gemm_gateup(g, u, x, M, topk, offsets, perm, tile_off, inter, st);
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
    return launch_gemm_down(d, a16, rs, M, topk, offsets, perm, tile_off, topk_w, partial, st);
}

int launch_combine(const float* partial, const int32_t* inv, int M, int K, int H, const float* shared,
                   const float* shared_logit, float* out, hipStream_t st) {
    if (M <= 0) return PGMOE_OK;
    if (K > 16) return fail(PGMOE_E_UNSUPPORTED, "combine supports top_k <= 16");
    PG_LAUNCH(combine_kernel, dim3(M, div_up(H, 256)), dim3(256), 0, st, partial, inv, K, H, shared,
                       shared_logit, out);
    return check_launch("combine");
}

int gemm_tile_rows() { return gemm_tile_pairs(); }

}  // namespace pgmoe
