/*
 * pgmoe -- MI355X (gfx950) quantized mixture-of-experts FFN layer, C ABI.
 *
 * Replaces the hot path of PyGGUF's sparse MoE block, GGUFSparseMoEMLP.forward
 * (pygguf_engine/model.py:898-937), with HIP kernels.  The Python class
 * pgmoe.HipSparseMoEMLP keeps the reference's constructor/forward surface and calls
 * these entry points through ctypes.
 *
 * Conventions for every entry point:
 *   - returns 0 (PGMOE_OK) or a negative PGMOE_E_* status; pgmoe_last_error() holds a
 *     thread-local message for the last failure on the calling thread;
 *   - pointers are device pointers unless stated; sizes are element counts;
 *   - `stream` is a hipStream_t passed as void* (NULL = the default stream); work is
 *     enqueued on it with no host synchronisation and no device allocation;
 *   - activations are IEEE fp16 passed as uint16_t bits; outputs are fp32.
 *
 * Device weight layout (pgmoe_weights.base, matrices mat_stride bytes apart, each
 * exactly as many bytes as the GGUF blocks it holds, rows padded to a multiple of 64 with
 * zero rows, see pgmoe_weight_bytes): a matrix [N rows, K cols] (K a multiple of 256) is
 * stored as tiles of 64 rows x one 256-weight super-block; tile (rg, b) at
 * base + (rg * K/256 + b) * CH * 1024 holds CH 16-byte chunks per row, chunk-major:
 * chunk c of row r at + c*1024 + r*16.  Chunk contents (same bits as the GGUF block):
 *   Q4_1 (type 3, CH 10):  c0 = the fp16 d of the super-block's 8 Q4_1 blocks, c1 = their
 *                          fp16 m; c2..c9 = their 4-bit codes in the Q4_K arrangement
 *                          (byte 32j + l of c2..c9: code of element 64j + l in the low
 *                          nibble, of element 64j + 32 + l in the high one); value d q + m
 *   Q4_K (type 12, CH 9):  c0 = d, dmin, 12 scale bytes;  c1..c8 = qs[16(c-1) .. +16]
 *   Q5_K (type 13, CH 11): c0..c8 as Q4_K (the GGUF block's bytes 0-15 and 48-175);
 *                          c9, c10 = the 256 fifth bits (qh, bytes 16-47) regrouped per
 *                          64-weight quarter p: 8 bytes at chunk 9 + (p >> 1), byte 8(p & 1),
 *                          as two 32-bit words t = 0, 1 whose bit 8(l & 3) + (l >> 2) is
 *                          the fifth bit of element 64p + 32t + l (GGUF: bit 2p + t of qh[l])
 *   Q6_K (type 14, CH 13): c0..c7 = ql[16c ..];  c8..c11 = qh[16(c-8) ..];  c12 = the 16
 *                          int8 scales; the fp16 d in a plane after all tiles:
 *                          d(rg, b, r) at base + ceil(N/64)*(K/256)*13*1024
 *                          + ((rg*(K/256) + b)*64 + r)*2
 *   Q8_0 (type 8, CH 17):  c0..c15 = the qs of the super-block's 8 Q8_0 blocks in order;
 *                          c16 = their 8 fp16 d
 * pgmoe_relayout_weights() converts GGUF bytes already on the device into this layout.
 *
 * Scale plane (pgmoe_weights.scales, K-quants; read only by the mode-1 MFMA products):
 * the sub-block scales of the layout above decoded once at load time, in fp32, one 1 KB
 * chunk per (64-row group rg, super-block b, 64-weight unit c = 0..3), matrices
 * pgmoe_scale_plane_bytes() apart: row r of chunk (rg, b, c) at
 * scales + ((rg*(K/256) + b)*4 + c)*1024 + r*16 holds four floats
 *   Q4_K, Q5_K: {a0, c0, a1, c1} of sub-blocks 2c + t: a = d*sc, c = -(dmin*m) - 1024*a
 *   Q4_1:       {a0, c0, a1, c1} of blocks 2c + t: a = d, c = m - 1024*a
 *   Q6_K: {a0, a1, a2, a3}: a_g = d * scale[8*(c >> 1) + 2g + (c & 1)]
 * (the values a lane computes from the chunk bytes otherwise).  pgmoe_build_scale_plane()
 * writes it from the device layout.
 */
#ifndef PGMOE_H
#define PGMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PGMOE_ABI_VERSION 4

#define PGMOE_OK 0
#define PGMOE_E_INVALID (-1)     /* bad argument, shape or pointer */
#define PGMOE_E_UNSUPPORTED (-2) /* qtype / shape the kernels do not cover */
#define PGMOE_E_WORKSPACE (-3)   /* workspace too small */
#define PGMOE_E_HIP (-4)         /* HIP runtime error (launch or query) */

#define PGMOE_F16 1   /* fp16 weights (GGUF F16; BF16 / F32 tensors rounded to fp16 on the host, as the
                         reference's fp16 expert mode loads them, quant_kernels.py:1962-1964) */
#define PGMOE_Q4_0 2  /* source format only: relaid out as PGMOE_Q4_1 with m = -8d (exact values) */
#define PGMOE_Q4_1 3
#define PGMOE_Q5_0 6  /* source format only: relaid out as PGMOE_Q8_0 (exact values) */
#define PGMOE_Q8_0 8
#define PGMOE_Q4_K 12
#define PGMOE_Q5_K 13
#define PGMOE_Q6_K 14
/* Source formats only, re-quantised at load by pgmoe_requant_w4 into PGMOE_Q4_1 blocks with
 * the values the reference's W4 repack gives them: */
#define PGMOE_Q2_K 10
#define PGMOE_Q3_K 11
#define PGMOE_IQ4_NL 20
#define PGMOE_IQ4_XS 23
#define PGMOE_MXFP4 39
/* Source format only, re-quantised at load by pgmoe_requant_w8_f16 into PGMOE_F16 weights
 * with the values of the reference's W8 repack: */
#define PGMOE_Q5_1 7

/* Gate activation of the gated FFNs: act(gate) * up (exec_fused_act_mul_rowscale,
 * quant_kernels.py:1423-1475).  SiLU g / (1 + e^-g); GELU with the tanh approximation
 * 0.5 g (1 + tanh(sqrt(2/pi) (g + 0.044715 g^3))), the reference's use_gelu for gemma
 * architectures (model.py:868). */
#define PGMOE_ACT_SILU 0
#define PGMOE_ACT_GELU_TANH 1

typedef struct pgmoe_weights {
    int32_t qtype;      /* PGMOE_Q4_1 / PGMOE_Q4_K / PGMOE_Q5_K / PGMOE_Q6_K / PGMOE_Q8_0 / PGMOE_F16 */
    int32_t n_rows;     /* N: output features per matrix */
    int32_t n_cols;     /* K: input features, a multiple of 256 (pgmoe_relayout_weights_padded pads the
                           32-weight formats' rows to one) */
    int32_t n_mats;     /* experts (1 for a shared expert) */
    const void* base;   /* device layout described above, 16-B aligned */
    int64_t mat_stride; /* bytes between consecutive matrices */
    const void* scales; /* K-quants: the scale plane of the n_mats matrices (required by the
                           mode-1 products, unused by mode 0); Q8_0: NULL */
} pgmoe_weights;

typedef struct pgmoe_layer {
    int32_t hidden;     /* H */
    int32_t n_experts;  /* E <= 1024 */
    int32_t top_k;      /* K <= min(E, 16) */
    int32_t norm_topk;  /* renormalise the top-k weights (model.py:906-907) */
    const float* router_w;    /* [E, H] fp32 */
    const float* router_bias; /* [E] fp32 or NULL (harness extension; reference has none) */
    pgmoe_weights gate, up, down; /* [E, I, H], [E, I, H], [E, H, I] */
    int32_t has_shared;
    pgmoe_weights sh_gate, sh_up, sh_down; /* [I_s, H], [I_s, H], [H, I_s] */
    const float* sh_inp_gate; /* [H] fp32 or NULL: sigmoid gate on the shared expert */
    int32_t act;              /* PGMOE_ACT_*: the experts' gate activation (model.py:868) */
    int32_t* status_host;     /* optional host-mapped word (hipHostMalloc'd / pinned host memory
                                 that the device can write), or NULL: a kernel that sets a
                                 PGMOE_STATUS_* bit in the workspace status word also ORs it in
                                 here, so the caller can poll it with a plain host read, without
                                 synchronising the stream; the no-alloc entry point reports
                                 through it too.  The caller clears it. */
} pgmoe_layer;

/* A dense SwiGLU FFN: one matrix triple, no router (GGUFDenseMLP, model.py:778-846). */
typedef struct pgmoe_dense {
    int32_t hidden;               /* H */
    pgmoe_weights gate, up, down; /* [I, H], [I, H], [H, I], n_mats = 1 */
    int32_t act;                  /* PGMOE_ACT_* */
} pgmoe_dense;

int pgmoe_abi_version(void);
const char* pgmoe_last_error(void);

/* Bytes of one matrix in the device layout (== GGUF bytes; Q4_0: the Q4_1 layout it is
 * converted to, Q5_0: the Q8_0 layout); -1 if unsupported. */
int64_t pgmoe_weight_bytes(int32_t qtype, int64_t rows, int64_t cols);

/* GGUF blocks (device, n_mats matrices back to back; src 16-byte aligned, dst 256-byte
 * aligned) -> device layout.
 * Load-time replacement of repack_gguf_to_w4a16 / repack_gguf_to_w8a16
 * (quant_kernels.py:854-1036), keeping the GGUF bits instead of re-quantising.  A Q4_0
 * source is written in the Q4_1 layout with the same d and codes and m = -8d (exact for
 * |d| < 8188; pass the result as PGMOE_Q4_1 weights); a Q5_0 source in the Q8_0 layout
 * with qs = q - 16 and the same d (pass it as PGMOE_Q8_0).  Every value is kept exactly. */
int pgmoe_relayout_weights(int32_t qtype, const void* src, int64_t n_mats, int64_t rows, int64_t cols,
                           void* dst, void* stream);

/* pgmoe_relayout_weights into zero-padded matrices: GGUF blocks of n_mats [rows, cols]
 * matrices -> device matrices [rows_out, cols_out] (rows_out >= rows, cols_out >= cols a
 * multiple of 256, dst matrices pgmoe_weight_bytes(qtype, rows_out, cols_out) bytes apart)
 * whose extra rows and columns hold exact zeros.  The 32-weight formats (Q8_0, Q5_0, Q4_0,
 * Q4_1) take any cols that is a multiple of 32; the K-quants keep cols == cols_out.  For an
 * expert intermediate size I that is not a multiple of 256 (e.g. 1408): gate / up padded to
 * I_out rows and down to I_out columns compute what the unpadded layer does, since the zero
 * rows give SwiGLU values of exactly 0, which meet zero weights.  Load time only; the
 * reference accepts these widths in its W8 / W4 repack (quant_kernels.py:958, :1966-1967). */
int pgmoe_relayout_weights_padded(int32_t qtype, const void* src, int64_t n_mats, int64_t rows, int64_t cols,
                                  int64_t rows_out, int64_t cols_out, void* dst, void* stream);

/* The reference's W4 re-quantisation of Q2_K / Q3_K / IQ4_NL / IQ4_XS / MXFP4 tensors
 * (repack_gguf_to_w4a16's gguf-py branch, quant_kernels.py:906-942, taken for these formats
 * at :1966-1967 and :1812): each 32-weight group of the n_rows x cols matrix at src (GGUF
 * blocks, device, rows back to back) is decoded exactly and quantised again to 4 bits,
 * scale = (max - min) / 15 in fp32, codes round((w - min) / scale) clipped to 0..15, and
 * written to dst as Q4_1 GGUF blocks (n_rows * cols / 32 blocks of 20 bytes, 4-byte aligned
 * dst): d = fp16(scale), m = fp16(min).  Those hold exactly the reference's W4 values
 * (q * scale16 - fp16(-min)); pass dst to pgmoe_relayout_weights(_padded) as PGMOE_Q4_1.
 * cols: a multiple of 32 (IQ4_NL, MXFP4) or 256 (the others).  Load time only. */
int pgmoe_requant_w4(int32_t qtype, const void* src, int64_t n_rows, int64_t cols, void* dst, void* stream);

/* The reference's W8 re-quantisation of Q5_1 tensors (repack_gguf_to_w8a16's gguf-py
 * fallback, quant_kernels.py:1005-1025, taken at :1979 and :1822): each 16-weight group of
 * the n_rows x cols matrix at src (GGUF blocks, device, rows back to back) is decoded
 * exactly, sc = max|w| / 127 in fp32 (1 for an all-zero group), codes round(w / sc) clipped
 * to -127..127, and written to dst as fp16 weights [n_rows, cols_out] (16-byte aligned;
 * columns cols .. cols_out - 1 zero): fp16(fp16(sc) * q), the weight operand the reference's
 * W8 tensor-core GEMM forms (quant_kernels.py:553-620; its GEMV applies fp16(sc) to the
 * int8 dot product instead, 2^-12 relative apart at most).  Pass dst to
 * pgmoe_relayout_weights(_padded) as PGMOE_F16 with cols_out columns.  cols: a multiple of
 * 32; cols_out >= cols, a multiple of 32.  Load time only. */
int pgmoe_requant_w8_f16(int32_t qtype, const void* src, int64_t n_rows, int64_t cols, int64_t cols_out, void* dst,
                         void* stream);

/* Bytes of one matrix's scale plane (0 for Q8_0, which has none; -1 if unsupported).  No
 * counterpart in the reference: it sizes the buffer of pgmoe_build_scale_plane. */
int64_t pgmoe_scale_plane_bytes(int32_t qtype, int64_t rows, int64_t cols);

/* Scale plane of n_mats matrices in the device layout (src, mat_stride bytes apart) ->
 * dst (pgmoe_scale_plane_bytes apart).  Load time, next to pgmoe_relayout_weights; no
 * counterpart in the reference (its repack decodes the scales on the CPU instead,
 * quant_kernels.py:854-904). */
int pgmoe_build_scale_plane(int32_t qtype, const void* src, int64_t n_mats, int64_t rows, int64_t cols,
                            int64_t mat_stride, void* dst, void* stream);

/* Workspace bytes pgmoe_moe_forward needs for M tokens.  Zero the workspace once when it
 * is allocated: for every M it begins with the decode router's ready-tagged logits (the
 * same bytes whatever M is), which decode forwards leave at zero for the next call, so a
 * workspace sized for the largest M may serve calls of any M in turn (calls that share a
 * workspace must not overlap, and a workspace whose forward failed part-way must be
 * zeroed again). */
size_t pgmoe_workspace_bytes(const pgmoe_layer* L, int32_t M);

/* One MoE layer: out[M, H] = GGUFSparseMoEMLP.forward(x[M, H]) (model.py:898-937).
 * Host-sync free and allocation free (graph-capturable with a fixed M). */
int pgmoe_moe_forward(const pgmoe_layer* L, const uint16_t* x, int32_t M, float* out, void* ws,
                      size_t ws_bytes, void* stream);

/* pgmoe_moe_forward without a caller workspace, for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference.  The workspace is a fixed 32 MiB device
 * array inside the library, one per GPU, held until the process ends; the call allocates
 * nothing.  Same kernels and results as pgmoe_moe_forward.  Limits and rules:
 *   - M must fit the 32 MiB (laid out as pgmoe_workspace_bytes with the decode router's
 *     region reserved for 512 experts): every decode M (<= 8) of the BASELINE layers and
 *     small prefill batches; larger M returns PGMOE_E_WORKSPACE;
 *   - every call on a GPU shares that GPU's array: calls that overlap on one GPU (other
 *     streams or threads) race and give wrong results;
 *   - the first call on a device, and the first after a failed call, clears the array's
 *     state words with a kernel and so must not run under graph capture
 *     (PGMOE_E_INVALID otherwise);
 *   - pgmoe_moe_status and pgmoe_moe_routing cannot reach this workspace: a kernel's
 *     status bits reach the caller through pgmoe_layer.status_host when it is set. */
int pgmoe_moe_forward_noalloc(const pgmoe_layer* L, const uint16_t* x, int32_t M, float* out, void* stream);

/* The routing the last pgmoe_moe_forward of M tokens on this workspace produced, read back
 * in sorted pair order (ascending expert id, then ascending token: the order of the
 * reference's expert loop and torch.where, model.py:911-914): offsets[E+1] (pairs of the
 * experts below e), and for each sorted pair p < M*K its expert, token and top-k weight
 * (softmax, renormalised when norm_topk; model.py:903-907).  For M <= 8 this decodes the
 * routing descriptor the routed gate/up launch itself published (the routing the timed
 * decode path computed), for larger M the top-k / dispatch arrays.  Enqueued on stream
 * after the forward; no host sync.  No counterpart in the reference (its routing is
 * Python-visible tensors): it lets tests and benchmarks pin the forward's own routing. */
int pgmoe_moe_routing(const pgmoe_layer* L, int32_t M, const void* ws, size_t ws_bytes, int32_t* offsets,
                      int32_t* pair_expert, int32_t* pair_token, float* pair_w, void* stream);

/* Status word of a MoE workspace: 0, or PGMOE_STATUS_* bits set by kernels of an earlier
 * forward (PGMOE_STATUS_SPIN_TIMEOUT: a decode wave's bounded wait for the router logits
 * gave up, so that forward's output is wrong).  Synchronises `stream`, writes the word to
 * *status (host) and, with clear != 0, resets it.  No counterpart in the reference (its
 * PyTorch path has no device-side waits). */
#define PGMOE_STATUS_SPIN_TIMEOUT 1
int pgmoe_moe_status(const pgmoe_layer* L, void* ws, size_t ws_bytes, int32_t* status, int32_t clear,
                     void* stream);

/* Workspace bytes pgmoe_dense_forward needs for M tokens (0 for invalid arguments).  It
 * holds no state between calls: any workspace of this size serves. */
size_t pgmoe_dense_workspace_bytes(const pgmoe_dense* D, int32_t M);

/* One dense SwiGLU FFN: out[M, H] (fp32) = GGUFDenseMLP.forward(x[M, H]) (model.py:839-846:
 * gate||up GGUF products -> silu(gate) * up -> down).  Host-sync free and allocation free.
 * The reference's GeGLU variant (gemma) has no kernel here. */
int pgmoe_dense_forward(const pgmoe_dense* D, const uint16_t* x, int32_t M, float* out, void* ws, size_t ws_bytes,
                        void* stream);

/* Element types of pgmoe_add_rmsnorm's tensors (ggml type numbers). */
#define PGMOE_DT_F32 0
#define PGMOE_DT_F16 1
#define PGMOE_DT_BF16 30

/* Residual add + RMSNorm over `rows` rows of `dim` elements (dim a multiple of 4):
 *   h[r]   = f32(x[r]) + f32(delta[r])                       (fp32, written when h_out != NULL)
 *   out[r] = (h[r] * (1 / sqrt(sum(h[r]^2) / dim + eps))) * weight    (out_dtype F32 or F16)
 * exec_fused_add_rmsnorm (quant_kernels.py:1552-1597: returns (h, normed)), and with
 * delta == NULL exec_fused_rmsnorm (:1510-1549: h = f32(x)); the pre-FFN norm whose fp16
 * output is the MoE block's input (model.py:1037).  x / delta: F32, F16 or BF16; weight:
 * fp32 [dim].  Bit-identical to the CPU oracle's fixed summation order. */
int pgmoe_add_rmsnorm(const void* x, int32_t x_dtype, const void* delta, int32_t delta_dtype, const float* weight,
                      int32_t rows, int32_t dim, float eps, float* h_out, void* out, int32_t out_dtype, void* stream);

/* Workspace bytes pgmoe_linear_forward needs for M tokens (0: none, or invalid arguments):
 * nothing when it runs the GEMV (M <= 8), the identity dispatch of the GEMM otherwise, plus
 * M x N fp32 product rows when there is a bias or the output is fp16.  No state between
 * calls. */
size_t pgmoe_linear_workspace_bytes(const pgmoe_weights* W, int32_t M, int32_t has_bias, int32_t out_dtype);

/* The quantized linear: out[M, N] = x[M, K] . W^T (+ bias[N]) with W one matrix
 * (n_mats = 1) in the device layout, fp32 accumulate, out PGMOE_DT_F32 or PGMOE_DT_F16
 * (round to nearest even).  GGUFQuantLinear.forward (quant_kernels.py:1826-1837 ->
 * exec_w4a16_matmul / exec_w8a16_matmul, :1165-1420) and
 * FusedLinearPack.forward_single_concat (:1895-1898): attention projections, lm_head, the
 * shared expert's fused gate||up.  M <= 8: wavefront GEMV; else the MFMA GEMM (K-quant
 * weights then need their scale plane).  bias: fp32 [N] or NULL.  Host-sync free. */
int pgmoe_linear_forward(const pgmoe_weights* W, const float* bias, const uint16_t* x, int32_t M, void* out,
                         int32_t out_dtype, void* ws, size_t ws_bytes, void* stream);

/* Rows rows[0..n) of W dequantised: out[n, K] (PGMOE_DT_F32 or PGMOE_DT_F16); values as
 * the ggml block definitions give them with fp32 products; an id outside [0, N) gives a
 * row of NaN (nothing is read for it).  GGUFQuantLinear.embed_lookup
 * (quant_kernels.py:1839-1863): the token-embedding lookup from a quantised table. */
int pgmoe_dequant_rows(const pgmoe_weights* W, const int32_t* rows, int32_t n, void* out, int32_t out_dtype,
                       void* stream);

/* pgmoe_moe_forward with per-kernel timing.  No counterpart in the reference: it is for
 * benchmarks and profilers that want each kernel's duration from the caller's own stream.
 * The i-th kernel the call launches (i < n_events) records start_events[i] when it begins
 * and stop_events[i] when it ends (hipEvent_t handles created by the caller; either array
 * may be NULL), and kernel_names[i] (if that array is not NULL) points to a static string
 * naming the kernel as its launch writes it (e.g. "(gemm_kernel<QT, true, PG_GU_CT,
 * PG_GU_WM>)").  *n_launches (if not NULL) receives the number of kernels launched.
 * Launch order: decode (M <= 8): gate/up (router and routing folded in), [shared gate/up,
 * shared down], down + combine (or down, combine); prefill: router, top-k, dispatch
 * (a counting pass first when it takes several workgroups), gate/up, row-scale, down,
 * [shared: identity dispatch, gate/up, row-scale, down, shared gate], combine; a product
 * split over K when its tiles cannot fill the chip is followed by its reduce kernel. */
int pgmoe_moe_forward_timed(const pgmoe_layer* L, const uint16_t* x, int32_t M, float* out, void* ws,
                            size_t ws_bytes, void* stream, void** start_events, void** stop_events,
                            int32_t n_events, int32_t* n_launches, const char** kernel_names);

/* ---- stages of the forward, exposed for tests and for callers that fuse around them ---- */

/* R1+R2: logits[M, E] = f32(x) . W^T (+ bias) in the fixed order of the CPU oracle,
 * softmax, top-k by (logit desc, id asc), optional renorm (model.py:902-907).
 * logits may be NULL.  topk_idx/topk_w are [M, K]. */
int pgmoe_router_topk(const uint16_t* x, const float* w, const float* bias, int32_t M, int32_t H,
                      int32_t E, int32_t K, int32_t norm_topk, float* logits, int32_t* topk_idx,
                      float* topk_w, void* stream);

/* R3: stable counting sort of the M*K flat pair ids (t*K + k) by expert
 * (topk_indices.unique() / torch.where / index_select, model.py:911-914).
 * offsets[E+1]; perm[M*K] = flat id at each sorted position; inv[M*K] = position of
 * each flat id; active[E] = experts with rows, ascending; n_active[1];
 * tile_off[E+1] = exclusive scan of ceil(count/tile_rows) (tile_rows > 0; the mode-1
 * expert products below take tile_off computed with tile_rows = 256). */
int pgmoe_dispatch(const int32_t* topk_idx, int32_t M, int32_t K, int32_t E, int32_t tile_rows,
                   int32_t* offsets, int32_t* perm, int32_t* inv, int32_t* active, int32_t* n_active,
                   int32_t* tile_off, void* stream);

/* pgmoe_dispatch with caller scratch (ws, at least pgmoe_dispatch_ws_bytes(M, K, E)
 * bytes): the same outputs, bit for bit, from several workgroups (a counting pass, then
 * the scatter) instead of one.  No counterpart in the reference: it is the form the
 * one-call forward uses, exposed so callers with scratch can take it. */
size_t pgmoe_dispatch_ws_bytes(int32_t M, int32_t K, int32_t E);
int pgmoe_dispatch_ws(const int32_t* topk_idx, int32_t M, int32_t K, int32_t E, int32_t tile_rows,
                      int32_t* offsets, int32_t* perm, int32_t* inv, int32_t* active, int32_t* n_active,
                      int32_t* tile_off, void* ws, size_t ws_bytes, void* stream);

/* R4+R5: inter[P, I] = silu(x_p . Wg_e^T) * (x_p . Wu_e^T) for every sorted pair position p,
 * fp32 accumulate and output (gate/up_exps.forward_expert + exec_fused_act_mul_rowscale,
 * model.py:916-918).  mode 0 = wavefront GEMV (M <= 8), 1 = MFMA grouped GEMM over
 * 256-pair tiles (tile_off from pgmoe_dispatch with tile_rows = 256). */
int pgmoe_expert_gateup(const pgmoe_weights* gate, const pgmoe_weights* up, const uint16_t* x,
                        int32_t M, int32_t K, const int32_t* offsets, const int32_t* perm,
                        const int32_t* active, const int32_t* n_active, const int32_t* tile_off,
                        int32_t mode, float* inter, void* stream);

/* R6: partial[P, H] = w_p * (inter_p . Wd_e^T) (down_exps.forward_expert(...) * row_scale
 * * topk weight, model.py:919-921).  mode 1 first rescales inter to fp16 per row exactly
 * as exec_fused_act_mul_rowscale does (a16/rs are scratch [P, I] fp16 and [P] fp32;
 * may be NULL in mode 0). */
int pgmoe_expert_down(const pgmoe_weights* down, const float* inter, int32_t M, int32_t K,
                      const int32_t* offsets, const int32_t* perm, const int32_t* active,
                      const int32_t* n_active, const int32_t* tile_off, const float* topk_w,
                      int32_t mode, uint16_t* a16, float* rs, float* partial, void* stream);

/* R7(+R8): out[t, :] = sum over the token's K pairs in ascending expert id of
 * partial[inv[t*K+k], :] (index_add_, model.py:921-922), plus
 * shared[t, :] * sigmoid(shared_logit[t]) when shared != NULL (model.py:931-935;
 * shared_logit NULL = gate 1). */
int pgmoe_combine(const float* partial, const int32_t* inv, int32_t M, int32_t K, int32_t H,
                  const float* shared, const float* shared_logit, float* out, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* PGMOE_H */
