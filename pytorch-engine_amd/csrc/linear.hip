// The quantized linear y = x . W^T (+ bias) on the MoE kernels, and the dequantisation of
// selected rows (embedding lookup).
// Reference: GGUFQuantLinear.forward (pygguf_engine/quant_kernels.py:1826-1837: exec_w4a16
// / exec_w8a16_matmul, :1165-1420), FusedLinearPack.forward_single_concat (:1895-1898) and
// GGUFQuantLinear.embed_lookup (:1839-1863).
//   M <= 8 : the decode GEMV in its single-matrix mode (dec_gu_kernel<..., kLinear>), bias
//            and output rounding in its epilogue;
//   M  > 8 : identity dispatch, then the grouped MFMA GEMM (the down product's form, A = x
//            read directly, unit row scales), then a bias / fp16 pass when asked for.
#include "decode_kernels.h"

namespace pgmoe {

// out[i] = src[i] (+ bias[i % N]), fp32 or fp16 (round to nearest even).
__global__ __launch_bounds__(256) void bias_cast_kernel(const float* __restrict__ src, const float* __restrict__ bias,
                                                        int64_t n, int N, void* __restrict__ out, int out_f16) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        float v = src[i];
        if (bias) v = v + bias[i % N];
        if (out_f16)
            ((half_t*)out)[i] = (half_t)v;
        else
            ((float*)out)[i] = v;
    }
}

// Row `rows[i]` of W (N x K in the tile layout), super-block b, decoded to 256 values:
// one thread per (i, b); an id outside [0, N) gives a row of NaN.  Values as the ggml block definitions give them, products in fp32
// (Q4_K, Q5_K: d*sc*q - dmin*m; Q4_1: d*q - (-m); Q6_K: d*sc*(q - 32); Q8_0: d*q; F16: as stored).
template <int QT>
__global__ __launch_bounds__(256) void dequant_rows_kernel(const uint8_t* __restrict__ base, int N, int K,
                                                           const int32_t* __restrict__ rows, int n,
                                                           void* __restrict__ out, int out_f16) {
    const int nb = K >> 8;
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= (int64_t)n * nb) return;
    const int i = (int)(gid / nb), b = (int)(gid % nb);
    const int row = rows[i];
    if ((unsigned)row >= (unsigned)N) {  // an id past the matrix: NaN row, no read
        for (int e = 0; e < 256; ++e) {
            if (out_f16)
                ((half_t*)out)[(int64_t)i * K + 256 * b + e] = (half_t)__builtin_nanf("");
            else
                ((float*)out)[(int64_t)i * K + 256 * b + e] = __builtin_nanf("");
        }
        return;
    }
    // byte k of chunk ch of (row, b) in the tile layout
    const uint8_t* t = tile_ptr<QT>(base, nb, row >> 6, b) + (row & 63) * 16;
    auto byte = [&](int ch, int k) -> uint32_t { return t[ch * 1024 + k]; };
    const int64_t o = (int64_t)i * K + 256 * b;
    auto put = [&](int e, float v) {
        if (out_f16)
            ((half_t*)out)[o + e] = (half_t)v;
        else
            ((float*)out)[o + e] = v;
    };
    if constexpr (QT == PGMOE_Q4_K || QT == PGMOE_Q5_K || QT == PGMOE_Q4_1) {
        // Q4_K / Q5_K: chunk 0 = d, dmin, 12 scale bytes; 1..8: qs; 9, 10: fifth bits
        // Q4_1: chunk 0 = 8 fp16 d, 1 = 8 fp16 m; 2..9: qs (the Q4_K arrangement)
        constexpr int QC = QT == PGMOE_Q4_1 ? 2 : 1;
        const uint4 h = *(const uint4*)t;
        const float d = lo_half(h.x), dmin = hi_half(h.x);
        for (int s = 0; s < 8; ++s) {
            float a, z;
            if constexpr (QT == PGMOE_Q4_1) {
                a = h2f((uint16_t)(byte(0, 2 * s) | (byte(0, 2 * s + 1) << 8)));
                z = -h2f((uint16_t)(byte(1, 2 * s) | (byte(1, 2 * s + 1) << 8)));
            } else {
                int sc, mn;
                kscale(h.y, h.z, h.w, s, sc, mn);
                a = d * (float)sc;
                z = dmin * (float)mn;
            }
            for (int l = 0; l < 32; ++l) {
                const int j = 32 * (s >> 1) + l;  // qs byte
                int q = (byte(QC + (j >> 4), j & 15) >> (4 * (s & 1))) & 15;
                if constexpr (QT == PGMOE_Q5_K)  // fifth-bit word s: chunk 9 + (s >> 2), byte 4(s & 3) + (l & 3)
                    q |= ((byte(9 + (s >> 2), 4 * (s & 3) + (l & 3)) >> (l >> 2)) & 1) << 4;
                put(32 * s + l, a * (float)q - z);
            }
        }
    } else if constexpr (QT == PGMOE_Q6_K) {  // chunks 0..7: ql, 8..11: qh, 12: scales; d in its plane
        const int64_t dpl = (int64_t)row_groups(N) * nb * 13 * 1024;
        const float d = h2f(*(const uint16_t*)(base + dpl + (((int64_t)(row >> 6) * nb + b) * 64 + (row & 63)) * 2));
        for (int hh = 0; hh < 2; ++hh)
            for (int s = 0; s < 4; ++s)
                for (int l = 0; l < 32; ++l) {
                    const int e = 128 * hh + 32 * s + l;
                    const int jl = 64 * hh + 32 * (s & 1) + l, jh = 32 * hh + l;
                    const int lo = (byte(jl >> 4, jl & 15) >> (4 * (s >> 1))) & 15;
                    const int hb = (byte(8 + (jh >> 4), jh & 15) >> (2 * s)) & 3;
                    const float sc = (float)(int8_t)byte(12, e >> 4);
                    put(e, (d * sc) * (float)((lo | (hb << 4)) - 32));
                }
    } else if constexpr (QT == PGMOE_F16) {  // chunk c: weights 8c .. 8c + 7
        for (int e = 0; e < 256; ++e) put(e, h2f((uint16_t)(byte(e >> 3, 2 * (e & 7)) | (byte(e >> 3, 2 * (e & 7) + 1) << 8))));
    } else {  // chunks 2j, 2j + 1: qs of block j; chunk 16: the 8 fp16 d
        for (int j = 0; j < 8; ++j) {
            const float d = h2f(*(const uint16_t*)(t + 16 * 1024 + 2 * j));
            for (int l = 0; l < 32; ++l) put(32 * j + l, d * (float)(int8_t)byte(2 * j + (l >> 4), l & 15));
        }
    }
}

int launch_dequant_rows(const Mats& w, const int32_t* rows, int n, void* out, int out_f16, hipStream_t st) {
    if (n == 0) return PGMOE_OK;
    const int64_t threads = (int64_t)n * (w.K >> 8);
    const dim3 grid((unsigned)div_up(threads, 256));
#define DQ(QT) PG_LAUNCH(dequant_rows_kernel<QT>, grid, dim3(256), 0, st, w.base, w.N, w.K, rows, n, out, out_f16)
    switch (w.qtype) {
    case PGMOE_Q4_1: DQ(PGMOE_Q4_1); break;
    case PGMOE_Q4_K: DQ(PGMOE_Q4_K); break;
    case PGMOE_Q5_K: DQ(PGMOE_Q5_K); break;
    case PGMOE_Q6_K: DQ(PGMOE_Q6_K); break;
    case PGMOE_Q8_0: DQ(PGMOE_Q8_0); break;
    case PGMOE_F16: DQ(PGMOE_F16); break;
    default: return fail(PGMOE_E_UNSUPPORTED, "dequant rows: qtype %d", w.qtype);
    }
#undef DQ
    return check_launch("dequant_rows");
}

// Workspace of the linear for M tokens: nothing on the GEMV path; on the GEMM path the
// identity dispatch and, with a bias or fp16 output, the fp32 product rows.
static bool linear_gemv(int M, int K) { return M <= decode_tokens_max() && linear_gemv_fits(M, K); }

size_t linear_ws_bytes(const Mats& w, int M, bool staged) {
    if (M <= 0 || linear_gemv(M, w.K)) return 0;
    auto al = [](size_t b) { return (b + 255) & ~(size_t)255; };
    size_t n = 4 * al(8) + 3 * al((size_t)M * 4);  // offsets, tile_off, active, nact | perm, inv, unit weights
    if (staged) n += al((size_t)M * w.N * 4);
    return n + al(gemm_split_bytes_upto(M, 1, w.N, w.K, false));  // split-K partial sums (any batch up to M)
}

int launch_linear(const Mats& w, const float* bias, const uint16_t* x, int M, void* out, int out_f16, uint8_t* ws,
                  size_t ws_bytes, hipStream_t st) {
    if (M == 0) return PGMOE_OK;
    if (linear_gemv(M, w.K)) return launch_dec_linear(w, x, M, bias, out, out_f16, st);
    const bool staged = bias || out_f16;
    if (ws_bytes < linear_ws_bytes(w, M, staged))
        return fail(PGMOE_E_WORKSPACE, "linear: workspace %zu bytes, need %zu", ws_bytes, linear_ws_bytes(w, M, staged));
    size_t c = 0;
    auto take = [&](size_t bytes) {
        uint8_t* p = ws + c;
        c += (bytes + 255) & ~(size_t)255;
        return p;
    };
    int32_t* offsets = (int32_t*)take(8);
    int32_t* tile_off = (int32_t*)take(8);
    int32_t* active = (int32_t*)take(8);
    int32_t* nact = (int32_t*)take(8);
    int32_t* perm = (int32_t*)take((size_t)M * 4);
    int32_t* inv = (int32_t*)take((size_t)M * 4);
    float* ones = (float*)take((size_t)M * 4);
    float* prod = staged ? (float*)take((size_t)M * w.N * 4) : (float*)out;
    const size_t rb = gemm_split_bytes(M, 1, w.N, w.K, false);
    float* raw = rb ? (float*)take(rb) : nullptr;
    int rc = launch_identity_dispatch(M, gemm_tile_rows(), offsets, perm, inv, active, nact, tile_off, ones, st);
    if (rc) return rc;
    // the down GEMM's epilogue scales row p by rs[p] * topk_w[perm[p]]: both 1 here
    if ((rc = launch_gemm_down(w, x, ones, M, 1, offsets, perm, tile_off, ones, prod, st, raw))) return rc;
    if (!staged) return PGMOE_OK;
    const int64_t n = (int64_t)M * w.N;
    const int blocks = (int)(div_up(n, 256) < 8192 ? div_up(n, 256) : 8192);
    PG_LAUNCH(bias_cast_kernel, dim3(blocks), dim3(256), 0, st, prod, bias, n, w.N, out, out_f16);
    return check_launch("linear bias / cast");
}

}  // namespace pgmoe
