// Decode-path entry points: dispatch by qtype to the per-qtype launchers.
#include <atomic>

#include "decode_kernels.h"

namespace pgmoe {

#define PG_BY_QTYPE(qt, what, call)                                  \
    switch (qt) {                                                    \
    case PGMOE_Q4_1: return call(PGMOE_Q4_1);                        \
    case PGMOE_Q4_K: return call(PGMOE_Q4_K);                        \
    case PGMOE_Q5_K: return call(PGMOE_Q5_K);                        \
    case PGMOE_Q6_K: return call(PGMOE_Q6_K);                        \
    case PGMOE_Q8_0: return call(PGMOE_Q8_0);                        \
    case PGMOE_F16: return call(PGMOE_F16);                          \
    }                                                                \
    return fail(PGMOE_E_UNSUPPORTED, what ": qtype %d", qt);

bool decode_isum_rows8(int qtype, int M) {
    if (M < 1 || M > 2) return false;
    switch (qtype) {
    case PGMOE_Q4_1: return gu_rows8<PGMOE_Q4_1>();
    case PGMOE_Q4_K: return gu_rows8<PGMOE_Q4_K>();
    case PGMOE_Q5_K: return gu_rows8<PGMOE_Q5_K>();
    case PGMOE_Q6_K: return gu_rows8<PGMOE_Q6_K>();
    case PGMOE_Q8_0: return gu_rows8<PGMOE_Q8_0>();
    case PGMOE_F16: return gu_rows8<PGMOE_F16>();
    }
    return false;
}

int launch_dec_gateup(const Mats& g, const Mats& u, const uint16_t* x, const float* xsum, int topk, int M,
                      const int32_t* offsets, const int32_t* perm, const int32_t* active, const int32_t* n_active,
                      int max_active, float* inter, float* isum, hipStream_t st, int act) {
    DecDisp dp{kDispatch, offsets, perm, active, n_active, nullptr, nullptr, nullptr, M, g.n_mats, 0, {}};
    dp.act = act;
#define CALL(QT) dec_gateup_q<QT>(g, u, x, xsum, topk, M, dp, RouterIn{}, max_active, inter, isum, st)
    PG_BY_QTYPE(g.qtype, "decode gate/up", CALL)
#undef CALL
}

int launch_dec_gateup_routed(const Mats& g, const Mats& u, const uint16_t* x, int topk, int M, const float* rw,
                             const float* bias, const float* sgw, float* s_logit, uint64_t* rlog, int32_t* status,
                             float* xsum_out, int E, int norm, int32_t* desc, const DecFlat& flat, int max_active,
                             float* inter, float* isum, hipStream_t st, int act, int32_t* status_host) {
    if (M < 1 || M > kDecTM) return fail(PGMOE_E_INVALID, "routed decode handles 1..%d tokens", kDecTM);
    if (topk > 16 || E > 512 || M * topk > 128)
        return fail(PGMOE_E_UNSUPPORTED, "routed decode: top_k <= 16, E <= 512, M*top_k <= 128");
    DecDisp dp{kRoute, nullptr, nullptr, nullptr, nullptr, rlog, desc, status, M, E, norm,
               {flat.offsets, flat.perm, flat.inv, flat.active, flat.n_active, flat.w}};
    dp.act = act;
    dp.status_host = status_host;
    const RouterIn rt{rw, bias, sgw, s_logit, xsum_out};
#define CALL(QT) dec_gateup_q<QT>(g, u, x, nullptr, topk, M, dp, rt, max_active, inter, isum, st)
    PG_BY_QTYPE(g.qtype, "decode gate/up", CALL)
#undef CALL
}

int launch_dec_linear(const Mats& w, const uint16_t* x, int M, const float* bias, void* out, int out_f16,
                      hipStream_t st) {
    DecDisp dp{kLinear, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, M, 1, 0, {}};
    dp.bias = bias;
    dp.out_f16 = out_f16;
#define CALL(QT) dec_gateup_q<QT>(w, w, x, nullptr, 1, M, dp, RouterIn{}, 1, (float*)out, nullptr, st)
    PG_BY_QTYPE(w.qtype, "decode linear", CALL)
#undef CALL
}

int launch_dec_gateup_ident(const Mats& g, const Mats& u, const uint16_t* x, const float* xsum, int M, float* inter,
                            float* isum, hipStream_t st, int act) {
    DecDisp dp{kIdent, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, M, 1, 0, {}};
    dp.act = act;
#define CALL(QT) dec_gateup_q<QT>(g, u, x, xsum, 1, M, dp, RouterIn{}, 1, inter, isum, st)
    PG_BY_QTYPE(g.qtype, "decode gate/up", CALL)
#undef CALL
}

int launch_dec_down(const Mats& d, const float* inter, const float* isum, int M, const int32_t* offsets,
                    const int32_t* perm, const int32_t* active, const int32_t* n_active, int max_active,
                    const float* topk_w, float* partial, hipStream_t st) {
    const DecDisp dp{kDispatch, offsets, perm, active, n_active, nullptr, nullptr, nullptr, M, d.n_mats, 0, {}};
#define CALL(QT) dec_down_q<QT>(d, inter, isum, M, kDispatch, dp, max_active, topk_w, partial, st)
    PG_BY_QTYPE(d.qtype, "decode down", CALL)
#undef CALL
}

int launch_dec_down_ident(const Mats& d, const float* inter, const float* isum, int M, float* out, hipStream_t st) {
    const DecDisp dp{kIdent, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, M, 1, 0, {}};
#define CALL(QT) dec_down_q<QT>(d, inter, isum, M, kIdent, dp, 1, nullptr, out, st)
    PG_BY_QTYPE(d.qtype, "decode down", CALL)
#undef CALL
}

int launch_dec_down_combine(const Mats& d, const float* inter, const float* isum, int isum8, const int32_t* desc,
                            int M, int K, int max_active, const float* shared, const float* shared_logit, float* out,
                            uint64_t* clear, int n_clear, hipStream_t st) {
    if (M < 1 || M > kDecTM || M * K > 128) return fail(PGMOE_E_INVALID, "down + combine: 1..%d tokens", kDecTM);
#define CALL(QT) dec_down_combine_q<QT>(d, inter, isum, isum8, desc, M, M * K, max_active, shared, shared_logit, out, clear, n_clear, st)
    PG_BY_QTYPE(d.qtype, "decode down + combine", CALL)
#undef CALL
}

bool decode_fused_down(int P, int K) { return P <= 128 && dc_chunk(P, K) >= 1; }

// The device's LDS per block less 16 KB for the decode kernels' static arrays, cached per
// device (hipDeviceAttributeMaxSharedMemoryPerBlock).  The per-device caches here are
// atomics: host threads may launch on one device concurrently (each writes the same value).
size_t dec_lds_limit() {
    static std::atomic<size_t> cached[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 48 * 1024;
    size_t c = cached[dev].load(std::memory_order_relaxed);
    if (!c) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || v <= 0)
            v = 64 * 1024;
        c = (size_t)v - 16 * 1024;
        cached[dev].store(c, std::memory_order_relaxed);
    }
    return c;
}

int resident_blocks(const void* kernel, int threads, size_t lds) {
    return resident_rows(kernel, threads, lds, 1, 1 << 30);
}

int resident_rows(const void* kernel, int threads, size_t lds, int gx, int gy) {
    static std::atomic<int> cus[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return gy;
    int n = cus[dev].load(std::memory_order_relaxed);
    if (!n) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return gy;
        cus[dev].store(n, std::memory_order_relaxed);
    }
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, lds) != hipSuccess || per_cu <= 0)
        return gy;
    const int rows = per_cu * n / gx;
    return rows < 1 ? 1 : rows < gy ? rows : gy;
}

// Routing of a finished forward in sorted pair order (ascending expert, then ascending
// token): one block.  decode: from the routing descriptor the routed gate/up launch
// published (slot a = {expert, first pair, count}, pair p = {token, weight bits});
// prefill: from the top-k and dispatch arrays (pair p = flat id perm[p] = token * K + k).
__global__ __launch_bounds__(256) void route_readback_kernel(int decode, const int32_t* __restrict__ desc,
                                                             const int32_t* __restrict__ idx,
                                                             const float* __restrict__ w,
                                                             const int32_t* __restrict__ offsets_in,
                                                             const int32_t* __restrict__ perm, int M, int K, int E,
                                                             int32_t* __restrict__ offsets,
                                                             int32_t* __restrict__ pair_expert,
                                                             int32_t* __restrict__ pair_token,
                                                             float* __restrict__ pair_w) {
    const int P = M * K;
    if (decode) {
        const int n_act = desc[0];
        for (int e = threadIdx.x; e <= E; e += blockDim.x) {  // pairs of the experts below e
            int o = 0;
            for (int a = 0; a < n_act; ++a)
                if (desc[kDescSlot + 4 * a] < e) o += desc[kDescSlot + 4 * a + 2];
            offsets[e] = o;
        }
        for (int a = 0; a < n_act; ++a) {
            const int e = desc[kDescSlot + 4 * a], pb = desc[kDescSlot + 4 * a + 1];
            const int c = desc[kDescSlot + 4 * a + 2];
            for (int i = threadIdx.x; i < c; i += blockDim.x) {
                const int p = pb + i;
                if (p < P) pair_expert[p] = e;
            }
        }
        for (int p = threadIdx.x; p < P; p += blockDim.x) {
            pair_token[p] = desc[kDescPair + 2 * p];
            pair_w[p] = __builtin_bit_cast(float, desc[kDescPair + 2 * p + 1]);
        }
        return;
    }
    for (int e = threadIdx.x; e <= E; e += blockDim.x) offsets[e] = offsets_in[e];
    for (int p = threadIdx.x; p < P; p += blockDim.x) {
        const int f = perm[p];
        pair_expert[p] = idx[f];
        pair_token[p] = f / K;
        pair_w[p] = w[f];
    }
}

int launch_route_readback(int decode, const int32_t* desc, const int32_t* idx, const float* w,
                          const int32_t* offsets_in, const int32_t* perm, int M, int K, int E, int32_t* offsets,
                          int32_t* pair_expert, int32_t* pair_token, float* pair_w, hipStream_t st) {
    if (decode && (M > kDecTM || M * K > 128)) return fail(PGMOE_E_INVALID, "route readback: decode M=%d", M);
    PG_LAUNCH(route_readback_kernel, dim3(1), dim3(256), 0, st, decode, desc, idx, w, offsets_in, perm, M, K, E,
              offsets, pair_expert, pair_token, pair_w);
    return check_launch("route readback");
}

bool linear_gemv_fits(int M, int K) { return M >= 1 && M <= kDecTM && gu_lds_bytes(M, K) <= dec_lds_limit(); }

int decode_tokens_max() { return kDecTM; }
int decode_desc_words() { return kDescWords; }
int decode_rlog_words(int M, int E) { return kRlogCopies * M * E; }

}  // namespace pgmoe
