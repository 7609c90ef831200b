// Load-time GGUF -> device layout conversion (same bits, aligned planes).
// Replaces the reference's CPU numpy repack (quant_kernels.py:854-1036), which
// re-quantises into W4/W8 arrays; here the GGUF bits are kept and only moved.
#include "common.h"
#include "launch.h"

namespace pgmoe {

// One thread per Q6_K block (210 B: ql[128] qh[64] sc[16] d[2]).
__global__ void relayout_q6k_kernel(const uint8_t* __restrict__ src, int64_t n_blocks, int64_t blocks_per_mat,
                                    uint8_t* __restrict__ dst, int64_t dst_stride) {
    const int64_t gb = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gb >= n_blocks) return;
    const int64_t mat = gb / blocks_per_mat, b = gb % blocks_per_mat;  // b = row * nb + block
    const uint8_t* s = src + gb * 210;
    uint8_t* d = dst + mat * dst_stride;
    uint8_t* body = d + b * 192;
    uint8_t* scale = d + blocks_per_mat * 192 + b * 16;
    for (int un = 0; un < 4; ++un) {
        const int h = un >> 1, half = un & 1;
        for (int i = 0; i < 16; ++i) {
            body[un * 48 + i] = s[64 * h + 16 * half + i];
            body[un * 48 + 16 + i] = s[64 * h + 32 + 16 * half + i];
            body[un * 48 + 32 + i] = s[128 + 32 * h + 16 * half + i];
        }
        for (int q = 0; q < 4; ++q) scale[un * 4 + q] = s[192 + 8 * h + 2 * q + half];
    }
    uint8_t* dd = d + blocks_per_mat * 208 + b * 2;
    dd[0] = s[208];
    dd[1] = s[209];
}

// One thread per Q8_0 block (34 B: d[2] q[32]).
__global__ void relayout_q8_0_kernel(const uint8_t* __restrict__ src, int64_t n_blocks, int64_t blocks_per_mat,
                                     uint8_t* __restrict__ dst, int64_t dst_stride) {
    const int64_t gb = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gb >= n_blocks) return;
    const int64_t mat = gb / blocks_per_mat, b = gb % blocks_per_mat;
    const uint8_t* s = src + gb * 34;
    uint8_t* d = dst + mat * dst_stride;
    for (int i = 0; i < 32; ++i) d[b * 32 + i] = s[2 + i];
    d[blocks_per_mat * 32 + b * 2] = s[0];
    d[blocks_per_mat * 32 + b * 2 + 1] = s[1];
}

int launch_relayout(int qtype, const uint8_t* src, int64_t n_mats, int64_t rows, int64_t cols, uint8_t* dst,
                    int64_t dst_stride, hipStream_t st) {
    if (qtype == PGMOE_Q4_K) {
        const int64_t mb = rows * (cols / 256) * 144;
        if (dst_stride == mb) {
            if (hipMemcpyAsync(dst, src, mb * n_mats, hipMemcpyDeviceToDevice, st) != hipSuccess)
                return fail(PGMOE_E_HIP, "relayout copy failed");
        } else {
            for (int64_t m = 0; m < n_mats; ++m)
                if (hipMemcpyAsync(dst + m * dst_stride, src + m * mb, mb, hipMemcpyDeviceToDevice, st) != hipSuccess)
                    return fail(PGMOE_E_HIP, "relayout copy failed");
        }
        return PGMOE_OK;
    }
    const int per = qtype == PGMOE_Q6_K ? 256 : 32;
    const int64_t bpm = rows * (cols / per);
    const int64_t nb = bpm * n_mats;
    if (nb == 0) return PGMOE_OK;
    const int threads = 256;
    const int64_t grid = (nb + threads - 1) / threads;
    if (qtype == PGMOE_Q6_K)
        hipLaunchKernelGGL(relayout_q6k_kernel, dim3((unsigned)grid), dim3(threads), 0, st, src, nb, bpm, dst, dst_stride);
    else
        hipLaunchKernelGGL(relayout_q8_0_kernel, dim3((unsigned)grid), dim3(threads), 0, st, src, nb, bpm, dst, dst_stride);
    return check_launch("relayout");
}

}  // namespace pgmoe
