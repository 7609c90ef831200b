// Decode-path dispatch by qtype and the one-block top-k / dispatch kernel.
#include "decode_kernels.h"

namespace pgmoe {

// One block: top-k of M <= 8 tokens by (logit desc, id asc) through ranks, softmax
// weights, renorm, the stable dispatch of the M*K pairs and the shared expert's identity
// dispatch.  Reference: model.py:903-914.  No loop here is longer than E/4 iterations.
__global__ __launch_bounds__(256) void topk_dispatch_small_kernel(
    const float* __restrict__ logits, int M, int E, int K, int norm, int32_t* __restrict__ idx_out,
    float* __restrict__ w_out, int32_t* __restrict__ offsets, int32_t* __restrict__ perm,
    int32_t* __restrict__ inv, int32_t* __restrict__ active, int32_t* __restrict__ n_active,
    int32_t* __restrict__ s_disp, float* __restrict__ s_w) {
    __shared__ __attribute__((aligned(16))) float sl[kDecTM * 512];
    __shared__ int s_idx[kDecTM * 16];
    __shared__ float s_val[kDecTM * 16];
    __shared__ float s_wt[kDecTM * 16];
    __shared__ uint32_t pres[kDecTM][16];  // token x expert membership bits
    __shared__ uint32_t used[16];
    __shared__ int cnt[512];
    __shared__ int scan[256];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    for (int i = tid; i < M * E; i += 256) sl[i] = logits[i];
    for (int i = tid; i < 512; i += 256) cnt[i] = 0;
    if (tid < kDecTM * 16) (&pres[0][0])[tid] = 0u;
    __syncthreads();
    // rank of logit (m, e) within its token: #{e' : l_e' > l_e or (l_e' == l_e and e' < e)}
    for (int i = tid; i < M * E; i += 256) {
        const int m = i / E, ee = i % E;
        const float v = sl[i];
        const float* row = sl + m * E;
        int rank = 0, j = 0;
        if ((E & 3) == 0) {
            for (; j < E; j += 4) {
                const float4 u = *(const float4*)(row + j);
                rank += (u.x > v) || (u.x == v && j < ee);
                rank += (u.y > v) || (u.y == v && j + 1 < ee);
                rank += (u.z > v) || (u.z == v && j + 2 < ee);
                rank += (u.w > v) || (u.w == v && j + 3 < ee);
            }
        }
        for (; j < E; ++j) rank += (row[j] > v) || (row[j] == v && j < ee);
        if (rank < K) {
            s_idx[m * K + rank] = ee;
            s_val[m * K + rank] = v;
            atomicOr(&pres[m][ee >> 5], 1u << (ee & 31));
            atomicAdd(&cnt[ee], 1);
        }
    }
    __syncthreads();
    for (int m = wv; m < M; m += 4) {  // softmax over all E, then the selected K
        const float top = s_val[m * K];
        float den = 0.f;
        for (int j = lane; j < E; j += 64) den += expf(sl[m * E + j] - top);
        den = group_sum<64>(den);
        float p = lane < K ? expf(s_val[m * K + lane] - top) / den : 0.f;
        const float sp = group_sum<64>(p);
        if (norm) p = p / fmaxf(sp, 1e-20f);
        if (lane < K) s_wt[m * K + lane] = p;
    }
    if (tid < 16) {
        uint32_t u = 0;
        for (int m = 0; m < M; ++m) u |= pres[m][tid];
        used[tid] = u;
    }
    // exclusive scan of the expert counts (two per thread, E <= 512)
    const int c0 = cnt[2 * tid], c1 = cnt[2 * tid + 1];
    scan[tid] = c0 + c1;
    __syncthreads();
    for (int off = 1; off < 256; off <<= 1) {
        const int add = tid >= off ? scan[tid - off] : 0;
        __syncthreads();
        scan[tid] += add;
        __syncthreads();
    }
    const int base = scan[tid] - c0 - c1;  // exclusive prefix of entry 2*tid
    if (2 * tid < E) offsets[2 * tid] = base;
    if (2 * tid + 1 < E) offsets[2 * tid + 1] = base + c0;
    if (tid == 0) offsets[E] = M * K;
    // reuse cnt as offsets (entries 2*tid and 2*tid + 1 belong to this thread only)
    cnt[2 * tid] = base;
    cnt[2 * tid + 1] = base + c0;
    __syncthreads();
    const int P = M * K;
    for (int f = tid; f < P; f += 256) {
        const int t = f / K, ef = s_idx[f];
        int rank = 0;
        for (int t2 = 0; t2 < t; ++t2) rank += (pres[t2][ef >> 5] >> (ef & 31)) & 1u;
        const int pos = cnt[ef] + rank;
        perm[pos] = f;
        inv[f] = pos;
        idx_out[f] = ef;
        w_out[f] = s_wt[f];
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
    if (s_disp) {  // shared expert: offsets {0, M}, active {0}, n_active 1, perm identity, w 1
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
}


int launch_dec_gateup(const Mats& g, const Mats& u, const uint16_t* x, const float* xsum, int topk, int M,
                      const int32_t* offsets, const int32_t* perm, const int32_t* active, const int32_t* n_active,
                      int max_active, float* inter, float* isum, hipStream_t st) {
    switch (g.qtype) {
    case PGMOE_Q4_K: return dec_gateup_q<PGMOE_Q4_K>(g, u, x, xsum, topk, M, offsets, perm, active, n_active, max_active, inter, isum, st);
    case PGMOE_Q6_K: return dec_gateup_q<PGMOE_Q6_K>(g, u, x, xsum, topk, M, offsets, perm, active, n_active, max_active, inter, isum, st);
    case PGMOE_Q8_0: return dec_gateup_q<PGMOE_Q8_0>(g, u, x, xsum, topk, M, offsets, perm, active, n_active, max_active, inter, isum, st);
    }
    return fail(PGMOE_E_UNSUPPORTED, "decode gate/up: qtype %d", g.qtype);
}

int launch_dec_down(const Mats& d, const float* inter, const float* isum, int M, const int32_t* offsets,
                    const int32_t* perm, const int32_t* active, const int32_t* n_active, int max_active,
                    const float* topk_w, float* partial, hipStream_t st) {
    switch (d.qtype) {
    case PGMOE_Q4_K: return dec_down_q<PGMOE_Q4_K>(d, inter, isum, M, offsets, perm, active, n_active, max_active, topk_w, partial, st);
    case PGMOE_Q6_K: return dec_down_q<PGMOE_Q6_K>(d, inter, isum, M, offsets, perm, active, n_active, max_active, topk_w, partial, st);
    case PGMOE_Q8_0: return dec_down_q<PGMOE_Q8_0>(d, inter, isum, M, offsets, perm, active, n_active, max_active, topk_w, partial, st);
    }
    return fail(PGMOE_E_UNSUPPORTED, "decode down: qtype %d", d.qtype);
}

int launch_topk_dispatch_small(const float* logits, int M, int E, int K, int norm, int32_t* idx, float* w,
                               int32_t* offsets, int32_t* perm, int32_t* inv, int32_t* active, int32_t* n_active,
                               int32_t* s_disp, float* s_w, hipStream_t st) {
    if (M < 1 || M > kDecTM) return fail(PGMOE_E_INVALID, "small top-k handles 1..%d tokens", kDecTM);
    if (K > 16 || E > 512) return fail(PGMOE_E_UNSUPPORTED, "small top-k: top_k <= 16 and E <= 512");
    hipLaunchKernelGGL(topk_dispatch_small_kernel, dim3(1), dim3(256), 0, st, logits, M, E, K, norm, idx, w, offsets,
                       perm, inv, active, n_active, s_disp, s_w);
    return check_launch("topk_dispatch_small");
}

int decode_tokens_max() { return kDecTM; }

}  // namespace pgmoe
