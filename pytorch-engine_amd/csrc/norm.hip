// Residual add + RMSNorm, the step that produces the MoE block's input (and every other
// norm of the reference's blocks): h = f32(x) + f32(delta), out = (h * r) * w with
// r = 1 / sqrt(sum(h^2) / D + eps).
// Reference: exec_fused_add_rmsnorm (pygguf_engine/quant_kernels.py:1552-1597) and
// exec_fused_rmsnorm (:1510-1549), their Triton kernel _fused_rmsnorm_kernel (:803-837) and
// CPU branch F.rms_norm; called at model.py:1037 (ffn_norm.forward_with_residual, whose
// fp16 output is the MoE block's x) and model.py:1025 (attn_norm).
//
// One 256-thread workgroup per row; HBM-bound (x, delta, h and out streamed once, w from
// cache).  Thread t owns the 4-element chunks t, t + 256, ... of the row.  The sum of
// squares has a fixed order, restated by the CPU oracle (or_add_rmsnorm): each thread adds
// its elements' squares in element order, the 64 lanes of a wave meet by the halving tree
// (l, l + 32), (l, l + 16), ..., (l, l + 1), and the 4 wave sums are added left to right.
// Division and square root are IEEE (correctly rounded), so h and out have the oracle's
// bits.
#include "common.h"
#include "launch.h"

namespace pgmoe {

constexpr int kNormThreads = 256;

__device__ __forceinline__ float4 load4(const void* p, int dt, int64_t i4) {
    if (dt == PGMOE_DT_F32) return ((const float4*)p)[i4];
    const uint2 u = ((const uint2*)p)[i4];
    if (dt == PGMOE_DT_F16)
        return make_float4(lo_half(u.x), hi_half(u.x), lo_half(u.y), hi_half(u.y));
    // bf16: the high half of an fp32
    return make_float4(__builtin_bit_cast(float, u.x << 16), __builtin_bit_cast(float, u.x & 0xffff0000u),
                       __builtin_bit_cast(float, u.y << 16), __builtin_bit_cast(float, u.y & 0xffff0000u));
}

__device__ __forceinline__ void store4(void* p, int dt, int64_t i4, float4 v) {
    if (dt == PGMOE_DT_F32) {
        ((float4*)p)[i4] = v;
        return;
    }
    // fp16, round to nearest even
    const uint32_t lo = (uint32_t)__builtin_bit_cast(uint16_t, (half_t)v.x) |
                        ((uint32_t)__builtin_bit_cast(uint16_t, (half_t)v.y) << 16);
    const uint32_t hi = (uint32_t)__builtin_bit_cast(uint16_t, (half_t)v.z) |
                        ((uint32_t)__builtin_bit_cast(uint16_t, (half_t)v.w) << 16);
    ((uint2*)p)[i4] = make_uint2(lo, hi);
}

__device__ __forceinline__ float4 add4(float4 a, float4 b) {
    return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}

__device__ __forceinline__ float sq4(float acc, float4 h) {
    acc = acc + h.x * h.x;
    acc = acc + h.y * h.y;
    acc = acc + h.z * h.z;
    return acc + h.w * h.w;
}

// VPT > 0: the row's chunks stay in registers (D <= 1024 * VPT); VPT == 0: the row is read
// twice (any D), with the same order of operations.
template <int VPT>
__global__ __launch_bounds__(kNormThreads) void add_rmsnorm_kernel(const void* __restrict__ x, int xdt,
                                                                  const void* __restrict__ delta, int ddt,
                                                                  const float* __restrict__ w, int D, float eps,
                                                                  float* __restrict__ h_out, void* __restrict__ out,
                                                                  int odt) {
    __shared__ float wsum[kNormThreads / 64];
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    const int n4 = D >> 2;
    const int64_t row4 = (int64_t)blockIdx.x * n4;
    auto h_at = [&](int c) {
        float4 h = load4(x, xdt, row4 + c);
        if (delta) h = add4(h, load4(delta, ddt, row4 + c));
        return h;
    };
    float acc = 0.0f;
    float4 hv[VPT > 0 ? VPT : 1];
    if constexpr (VPT > 0) {
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            const int c = t + kNormThreads * j;
            if (c < n4) {
                hv[j] = h_at(c);
                acc = sq4(acc, hv[j]);
                if (h_out) ((float4*)h_out)[row4 + c] = hv[j];
            }
        }
    } else {
        for (int c = t; c < n4; c += kNormThreads) {
            const float4 h = h_at(c);
            acc = sq4(acc, h);
            if (h_out) ((float4*)h_out)[row4 + c] = h;
        }
    }
    acc = group_sum<64>(acc);
    if (lane == 0) wsum[wv] = acc;
    __syncthreads();
    float tot = wsum[0];
#pragma unroll
    for (int i = 1; i < kNormThreads / 64; ++i) tot = tot + wsum[i];
    const float r = 1.0f / sqrtf(tot / (float)D + eps);
    auto put = [&](int c, float4 h) {
        const float4 g = ((const float4*)w)[c];
        store4(out, odt, row4 + c, make_float4((h.x * r) * g.x, (h.y * r) * g.y, (h.z * r) * g.z, (h.w * r) * g.w));
    };
    if constexpr (VPT > 0) {
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
            const int c = t + kNormThreads * j;
            if (c < n4) put(c, hv[j]);
        }
    } else {
        for (int c = t; c < n4; c += kNormThreads) put(c, h_at(c));
    }
}

int launch_add_rmsnorm(const void* x, int xdt, const void* delta, int ddt, const float* w, int R, int D, float eps,
                       float* h_out, void* out, int odt, hipStream_t st) {
    if (R == 0) return PGMOE_OK;
    const int n4 = D >> 2;
    const dim3 grid(R), block(kNormThreads);
#define NORM(V) PG_LAUNCH(add_rmsnorm_kernel<V>, grid, block, 0, st, x, xdt, delta, ddt, w, D, eps, h_out, out, odt)
    if (n4 <= kNormThreads)
        NORM(1);
    else if (n4 <= 2 * kNormThreads)
        NORM(2);
    else if (n4 <= 4 * kNormThreads)
        NORM(4);
    else if (n4 <= 8 * kNormThreads)
        NORM(8);
    else
        NORM(0);
#undef NORM
    return check_launch("add_rmsnorm");
}

}  // namespace pgmoe
