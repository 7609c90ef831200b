// Host-side launchers shared between the translation units of libpgmoe.so.
#pragma once

#include <hip/hip_ext.h>

#include "common.h"

namespace pgmoe {

// Per-launch timing for pgmoe_moe_forward_timed: while armed on this thread, the i-th
// kernel launch records start[i] / stop[i] at the kernel's own begin and end (the events
// hipExtLaunchKernel stamps, the same interval a kernel trace reports).
struct LaunchTiming {
    hipEvent_t* start;
    hipEvent_t* stop;
    const char** names;  // optional: the kernel (as written at its launch) of each launch
    int n, next;
};
LaunchTiming*& launch_timing();  // this thread's armed timing (nullptr when off)

inline void timing_events(hipEvent_t* s, hipEvent_t* e, const char* name) {
    LaunchTiming* t = launch_timing();
    if (t) {
        if (t->next < t->n) {
            *s = t->start ? t->start[t->next] : nullptr;
            *e = t->stop ? t->stop[t->next] : nullptr;
            if (t->names) t->names[t->next] = name;
        }
        ++t->next;
    }
}

// Kernel launch on `st`; records the armed timing events, if any.
#define PG_LAUNCH(kernel, grid, block, shmem, st, ...)                                            \
    do {                                                                                          \
        hipEvent_t pg_ev_s = nullptr, pg_ev_e = nullptr;                                          \
        ::pgmoe::timing_events(&pg_ev_s, &pg_ev_e, #kernel);                                      \
        if (pg_ev_s || pg_ev_e)                                                                   \
            hipExtLaunchKernelGGL(kernel, grid, block, shmem, st, pg_ev_s, pg_ev_e, 0, __VA_ARGS__); \
        else                                                                                      \
            hipLaunchKernelGGL(kernel, grid, block, shmem, st, __VA_ARGS__);                      \
    } while (0)

int launch_router_logits(const uint16_t* x, const float* W, const float* bias, int M, int H, int E,
                         float* logits, hipStream_t st, const float* extra_w = nullptr, float* extra_out = nullptr,
                         float* xsum = nullptr);
int launch_topk(const float* logits, int M, int E, int K, int norm, int32_t* idx, float* w, hipStream_t st);
// counts (optional scratch of dispatch_ws_bytes): several blocks instead of one.
// tile_map (optional, dispatch_tile_map_words ints): the grouped GEMMs' tile order, entry
// i = expert | (tile of the expert << kTileMapShift): every full tile in expert order, then
// each expert's partial last tile, the ones with most rows first.
constexpr int kTileMapShift = 9;  // expert ids < 512
int launch_dispatch(const int32_t* idx, int M, int K, int E, int tile_rows, int32_t* offsets, int32_t* perm,
                    int32_t* inv, int32_t* active, int32_t* n_active, int32_t* tile_off, hipStream_t st,
                    int32_t* counts = nullptr, int32_t* tile_map = nullptr);
size_t dispatch_tile_map_words(int64_t P, int E, int tile_rows);
size_t dispatch_ws_bytes(int64_t P, int E);
int launch_identity_dispatch(int M, int tile_rows, int32_t* offsets, int32_t* perm, int32_t* inv,
                             int32_t* active, int32_t* n_active, int32_t* tile_off, float* w, hipStream_t st);
int launch_gateup(const Mats& g, const Mats& u, const uint16_t* x, int M, int topk, const int32_t* offsets,
                  const int32_t* perm, const int32_t* active, const int32_t* n_active, const int32_t* tile_off,
                  int mode, float* inter, hipStream_t st, float* raw = nullptr, int act = PGMOE_ACT_SILU,
                  const int32_t* tile_map = nullptr);
int launch_down(const Mats& d, const float* inter, int M, int topk, const int32_t* offsets, const int32_t* perm,
                const int32_t* active, const int32_t* n_active, const int32_t* tile_off, const float* topk_w,
                int mode, uint16_t* a16, float* rs, float* partial, hipStream_t st, float* raw = nullptr,
                const int32_t* tile_map = nullptr);
// clear (optional): n_clear words the kernel sets to zero (the decode router's tagged logits).
int launch_combine(const float* partial, const int32_t* inv, int M, int K, int H, const float* shared,
                   const float* shared_logit, float* out, hipStream_t st, uint64_t* clear = nullptr,
                   int n_clear = 0);
// GGUF [n_mats, rows, cols] -> device matrices [rows_out, cols_out] (zero padding past
// rows / cols; cols_out a multiple of 256, cols == cols_out for K-quants).
// Q2_K / Q3_K / IQ4_NL / IQ4_XS / MXFP4 -> Q4_1 GGUF blocks with the reference's W4 values
// (requant.hip); requant_w4_block gives a format's GGUF block (weights, bytes), -1 if none.
int requant_w4_block(int qtype, int* per, int* bytes);
int launch_requant_w4(int qtype, const uint8_t* src, int64_t rows, int cols, uint8_t* dst, hipStream_t st);
// Q5_1 -> fp16 [rows, cols_out] weights with the reference's W8 values (zero past cols).
int launch_requant_w8_f16(int qtype, const uint8_t* src, int64_t rows, int cols, int cols_out, uint8_t* dst,
                          hipStream_t st);
int launch_relayout(int qtype, const uint8_t* src, int64_t n_mats, int64_t rows, int64_t cols, int64_t rows_out,
                    int64_t cols_out, uint8_t* dst, int64_t dst_stride, hipStream_t st);
// Decode expert stages (M <= decode_tokens_max()).
int launch_dec_gateup(const Mats& g, const Mats& u, const uint16_t* x, const float* xsum, int topk, int M,
                      const int32_t* offsets, const int32_t* perm, const int32_t* active, const int32_t* n_active,
                      int max_active, float* inter, float* isum, hipStream_t st, int act = PGMOE_ACT_SILU);
int launch_dec_down(const Mats& d, const float* inter, const float* isum, int M, const int32_t* offsets,
                    const int32_t* perm, const int32_t* active, const int32_t* n_active, int max_active,
                    const float* topk_w, float* partial, hipStream_t st);
// Flat routing outputs of the routed gate/up (all null: only the descriptor is written).
struct DecFlat {
    int32_t *offsets, *perm, *inv, *active, *n_active;
    float* w;
};
// The routed gate/up also computes the router logits (rw [E][H], bias, the shared
// expert's gate row sgw -> s_logit) into `rlog` (decode_rlog_words ready-tagged words, zero on entry;
// the forward's last kernel clears them), and, when xsum_out is set, the 16-element sums
// of x for the shared expert's launches.
// status: the workspace status word a wave whose bounded wait for the logits gave up
// marks (kStatusSpinTimeout), or null; status_host: the caller's host-mapped word it also
// marks, or null.  isum gets 16-row sums [P][N/16], or 8-row sums
// [P][N/8] where decode_isum_rows8(g.qtype, M).
bool decode_isum_rows8(int qtype, int M);
int launch_dec_gateup_routed(const Mats& g, const Mats& u, const uint16_t* x, int topk, int M, const float* rw,
                             const float* bias, const float* sgw, float* s_logit, uint64_t* rlog, int32_t* status,
                             float* xsum_out, int E, int norm, int32_t* desc, const DecFlat& flat, int max_active,
                             float* inter, float* isum, hipStream_t st, int act = PGMOE_ACT_SILU,
                             int32_t* status_host = nullptr);
// Routing a forward produced, read back from its workspace in sorted pair order (decode:
// from the descriptor at desc; prefill: from the flat arrays).  offsets [E+1]; pair_*[P].
int launch_route_readback(int decode, const int32_t* desc, const int32_t* idx, const float* w,
                          const int32_t* offsets_in, const int32_t* perm, int M, int K, int E, int32_t* offsets,
                          int32_t* pair_expert, int32_t* pair_token, float* pair_w, hipStream_t st);
// y[M, N] = x . W^T (+ bias[N]) on the decode GEMV (M <= decode_tokens_max()); out fp32, or
// fp16 with out_f16.
int launch_dec_linear(const Mats& w, const uint16_t* x, int M, const float* bias, void* out, int out_f16,
                      hipStream_t st);
// Whether the decode GEMV can stage M rows of K inputs (the linear's M <= 8 path).
bool linear_gemv_fits(int M, int K);
// The quantized linear (linear.hip): out[M, N] = x . W^T (+ bias), fp32 or fp16; ws of
// linear_ws_bytes(w, M, bias || out_f16) bytes (none on the GEMV path).
size_t linear_ws_bytes(const Mats& w, int M, bool staged);
int launch_linear(const Mats& w, const float* bias, const uint16_t* x, int M, void* out, int out_f16, uint8_t* ws,
                  size_t ws_bytes, hipStream_t st);
// Rows rows[0..n) of w decoded to out [n, K] (fp32, or fp16 with out_f16).
int launch_dequant_rows(const Mats& w, const int32_t* rows, int n, void* out, int out_f16, hipStream_t st);
int launch_dec_gateup_ident(const Mats& g, const Mats& u, const uint16_t* x, const float* xsum, int M, float* inter,
                            float* isum, hipStream_t st, int act = PGMOE_ACT_SILU);
int launch_dec_down_ident(const Mats& d, const float* inter, const float* isum, int M, float* out, hipStream_t st);
// clear (may be null): n_clear words the kernel sets to zero (the decode router's tagged logits).
// desc null: the identity (matrix 0 applied to every token with weight 1; P = M, K = 1).
// isum8: isum holds 8-row sums [P][K/8] (the routed gate/up's where decode_isum_rows8),
// else 16-row sums.
int launch_dec_down_combine(const Mats& d, const float* inter, const float* isum, int isum8, const int32_t* desc,
                            int M, int K, int max_active, const float* shared, const float* shared_logit, float* out,
                            uint64_t* clear, int n_clear, hipStream_t st);
int decode_desc_words();
// 64-bit words of the decode router's ready-tagged logits (all copies) for M tokens.
int decode_rlog_words(int M, int E);
// Whether the fused down + combine kernels take P inter rows of K values (staged in LDS
// whole, or a chunk of super-block columns at a time for rows of up to 32 super-blocks).
bool decode_fused_down(int P, int K);
// Prefill grouped GEMMs (gemm.hip); tile_off counts gemm_tile_pairs()-row tiles.
// raw (optional): scratch of gemm_split_bytes(...) for a split-K run when the tiles would
// not fill the chip; null runs the product unsplit.  tile_map (optional): the dispatch's
// tile order (launch_dispatch); null takes the tiles in expert order.
int launch_gemm_gateup(const Mats& g, const Mats& u, const uint16_t* x, int M, int topk, const int32_t* offsets,
                       const int32_t* perm, const int32_t* tile_off, float* inter, hipStream_t st,
                       float* raw = nullptr, int act = PGMOE_ACT_SILU, const int32_t* tile_map = nullptr);
int launch_gemm_down(const Mats& d, const uint16_t* a16, const float* rs, int M, int topk, const int32_t* offsets,
                     const int32_t* perm, const int32_t* tile_off, const float* topk_w, float* partial,
                     hipStream_t st, float* raw = nullptr, const int32_t* tile_map = nullptr);
// K split of a grouped product: ksplit workgroups per tile, kper super-blocks each.
struct GemmSplit {
    int ksplit, kper;
};
GemmSplit gemm_split(int64_t P, int E, int N, int K, bool gateup);
// Scratch bytes of the raw partial sums of a split product (0 when it runs unsplit).
size_t gemm_split_bytes(int64_t P, int E, int N, int K, bool gateup);
// The largest gemm_split_bytes over every P' <= P (what a workspace that serves any batch up
// to P pairs must hold).
size_t gemm_split_bytes_upto(int64_t P, int E, int N, int K, bool gateup);
int gemm_tile_pairs();
int64_t layout_bytes(int qtype, int64_t rows, int64_t cols);
// Scale plane (relayout.hip): bytes of one matrix's plane (0 for Q8_0, -1 if unsupported)
// and its load-time construction from the device layout.
int64_t scale_plane_bytes(int qtype, int64_t rows, int64_t cols);
int launch_scale_plane(int qtype, const uint8_t* src, int64_t n_mats, int64_t rows, int64_t cols,
                       int64_t src_stride, uint8_t* dst, hipStream_t st);
int gemm_tile_rows();
// Residual add + RMSNorm (norm.hip): dtypes PGMOE_DT_*; delta and h_out may be null.
int launch_add_rmsnorm(const void* x, int xdt, const void* delta, int ddt, const float* w, int R, int D, float eps,
                       float* h_out, void* out, int odt, hipStream_t st);
int decode_tokens_max();

}  // namespace pgmoe
