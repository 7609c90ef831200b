// extern "C" entry points of libpgmoe.so (declared in include/pgmoe.h).
#include <stdarg.h>
#include <stdio.h>

#include <algorithm>
#include <mutex>

#include "common.h"
#include "launch.h"

namespace pgmoe {

static thread_local char g_err[512] = "";

LaunchTiming*& launch_timing() {
    static thread_local LaunchTiming* t = nullptr;
    return t;
}

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

int check_launch(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(PGMOE_E_HIP, "%s launch failed: %s", what, hipGetErrorString(e));
    return PGMOE_OK;
}

int check_weights(const pgmoe_weights* w, const char* what, Mats* out) {
    if (!w) return fail(PGMOE_E_INVALID, "%s: NULL weights", what);
    if (w->qtype != PGMOE_Q4_1 && w->qtype != PGMOE_Q4_K && w->qtype != PGMOE_Q5_K && w->qtype != PGMOE_Q6_K &&
        w->qtype != PGMOE_Q8_0 && w->qtype != PGMOE_F16)
        return fail(PGMOE_E_UNSUPPORTED,
                    "%s: qtype %d not supported (F16=1, Q4_1=3, Q4_K=12, Q5_K=13, Q6_K=14, Q8_0=8; Q4_0 weights are "
                    "relaid out as Q4_1, Q5_0 as Q8_0)", what,
                    w->qtype);
    if (w->n_rows <= 0 || w->n_cols <= 0 || w->n_mats <= 0)
        return fail(PGMOE_E_INVALID, "%s: bad shape [%d, %d, %d]", what, w->n_mats, w->n_rows, w->n_cols);
    const int64_t need = layout_bytes(w->qtype, w->n_rows, w->n_cols);
    if (need < 0)
        return fail(PGMOE_E_UNSUPPORTED, "%s: %d input features is not a multiple of 256", what, w->n_cols);
    if (!w->base || ((uintptr_t)w->base & 15))
        return fail(PGMOE_E_INVALID, "%s: base must be a 16-byte aligned device pointer", what);
    if (w->n_mats > 1 && (w->mat_stride < need || (w->mat_stride & 15)))
        return fail(PGMOE_E_INVALID, "%s: mat_stride %lld below %lld bytes or not 16-byte aligned", what,
                    (long long)w->mat_stride, (long long)need);
    out->qtype = w->qtype;
    out->N = w->n_rows;
    out->K = w->n_cols;
    out->n_mats = w->n_mats;
    out->base = (const uint8_t*)w->base;
    out->stride = w->mat_stride;
    out->scales = (const uint8_t*)w->scales;
    if (out->scales && ((uintptr_t)out->scales & 15))
        return fail(PGMOE_E_INVALID, "%s: scales must be 16-byte aligned", what);
    return PGMOE_OK;
}

static int check_pair(const Mats& g, const Mats& u, const char* what) {
    if (g.qtype != u.qtype || g.N != u.N || g.K != u.K || g.n_mats != u.n_mats)
        return fail(PGMOE_E_UNSUPPORTED, "%s: gate and up must share qtype and shape", what);
    return PGMOE_OK;
}

// ---------------------------------------------------------------- workspace layout
struct Layout {
    size_t rlog, status, desc, xsum, isum, s_isum;
    size_t logits, idx, w, offsets, perm, inv, active, nact, tile_off, tile_map, dcounts, inter, a16, rs, partial, raw;
    size_t s_offsets, s_perm, s_inv, s_active, s_nact, s_tile_off, s_w, s_logit, s_inter, s_a16, s_rs, s_partial;
    size_t total;
};

static size_t take(size_t& cur, size_t bytes) {
    const size_t at = cur;
    cur += (bytes + 255) & ~(size_t)255;
    return at;
}

// rlog_experts: the expert count the decode router's tagged-logit region is sized for
// (the layer's own E; the allocation-free entry point reserves it for kMaxRlogExperts so
// that layers of different E sharing its scratch all find the region at the same place).
static Layout layout_for(const pgmoe_layer* L, int M, int rlog_experts = 0) {
    Layout o{};
    const size_t E = L->n_experts, K = L->top_k, H = L->hidden, I = L->gate.n_rows;
    const size_t P = (size_t)M * K;
    const bool gemm = M > decode_tokens_max();
    size_t c = 0;
    // first, laid out the same for every M: the decode router's ready-tagged logits.  They
    // persist between calls (zero when the workspace is first allocated, and each decode
    // forward leaves them at zero), so a workspace shared by calls of different M must
    // find them at the same offset, where no other call writes
    o.rlog = take(c, (size_t)decode_rlog_words(decode_tokens_max(), rlog_experts > 0 ? rlog_experts : (int)E) * 8);
    // then the status word (also at the same offset for every M, zero until a wave's
    // bounded wait gives up; pgmoe_moe_status reads and clears it)
    o.status = take(c, 4);
    o.desc = take(c, gemm ? 0 : (size_t)decode_desc_words() * 4);
    o.xsum = take(c, gemm ? 0 : (size_t)M * (H / 16) * 4);
    o.isum = take(c, gemm ? 0 : P * (I / 8) * 4);  // 16-row sums, or 8-row sums at one token
    o.s_isum = take(c, (gemm || !L->has_shared) ? 0 : (size_t)M * (L->sh_gate.n_rows / 16) * 4);
    o.logits = take(c, gemm ? (size_t)M * E * 4 : 0);
    o.idx = take(c, P * 4);
    o.w = take(c, P * 4);
    o.offsets = take(c, (E + 1) * 4);
    o.perm = take(c, P * 4);
    o.inv = take(c, P * 4);
    o.active = take(c, E * 4);
    o.nact = take(c, 4);
    o.tile_off = take(c, (E + 1) * 4);
    o.tile_map = take(c, gemm ? dispatch_tile_map_words((int64_t)P, (int)E, gemm_tile_rows()) * 4 : 0);
    o.dcounts = take(c, gemm ? dispatch_ws_bytes((int64_t)P, (int)E) : 0);  // multi-block dispatch scratch
    o.inter = take(c, P * I * 4);
    o.a16 = take(c, gemm ? P * I * 2 : 0);
    o.rs = take(c, gemm ? P * 4 : 0);
    // the fused decode down kernel combines in place; otherwise per-pair partial rows
    o.partial = take(c, (gemm || !decode_fused_down((int)P, (int)I)) ? P * H * 4 : 0);
    if (gemm) {  // split-K scratch, shared by the products in turn (stream-ordered); sized for
                 // the largest any smaller batch takes, so that the total never falls as M grows
        size_t r = gemm_split_bytes_upto((int64_t)P, (int)E, (int)I, (int)H, true);
        r = std::max(r, gemm_split_bytes_upto((int64_t)P, (int)E, (int)H, (int)I, false));
        if (L->has_shared) {
            const int Is = L->sh_gate.n_rows;
            r = std::max(r, gemm_split_bytes_upto(M, 1, Is, (int)H, true));
            r = std::max(r, gemm_split_bytes_upto(M, 1, (int)H, Is, false));
        }
        o.raw = take(c, r);
    }
    if (L->has_shared) {
        const size_t Is = L->sh_gate.n_rows;
        o.s_offsets = take(c, 2 * 4);
        o.s_perm = take(c, (size_t)M * 4);
        o.s_inv = take(c, (size_t)M * 4);
        o.s_active = take(c, 4);
        o.s_nact = take(c, 4);
        o.s_tile_off = take(c, 2 * 4);
        o.s_w = take(c, (size_t)M * 4);
        o.s_logit = take(c, (size_t)M * 4);
        o.s_inter = take(c, (size_t)M * Is * 4);
        o.s_a16 = take(c, gemm ? (size_t)M * Is * 2 : 0);
        o.s_rs = take(c, gemm ? (size_t)M * 4 : 0);
        o.s_partial = take(c, (size_t)M * H * 4);
    }
    o.total = c;
    return o;
}

struct LayerMats {
    Mats gate, up, down, sg, su, sd;
};

static int check_layer(const pgmoe_layer* L, LayerMats* lm) {
    if (!L) return fail(PGMOE_E_INVALID, "NULL layer");
    if (L->hidden <= 0 || L->hidden % 256 || L->hidden > 65536)
        return fail(PGMOE_E_UNSUPPORTED, "hidden size %d must be a positive multiple of 256 (<= 65536)", L->hidden);
    if (L->n_experts < 1 || L->n_experts > 512)
        return fail(PGMOE_E_UNSUPPORTED, "n_experts %d outside [1, 512]", L->n_experts);
    if (L->top_k < 1 || L->top_k > L->n_experts || L->top_k > 16)
        return fail(PGMOE_E_UNSUPPORTED, "top_k %d outside [1, min(E, 16)]", L->top_k);
    if (!L->router_w) return fail(PGMOE_E_INVALID, "NULL router weight");
    if (L->act != PGMOE_ACT_SILU && L->act != PGMOE_ACT_GELU_TANH)
        return fail(PGMOE_E_UNSUPPORTED, "activation %d (SiLU = 0, GELU-tanh = 1)", L->act);
    int rc;
    if ((rc = check_weights(&L->gate, "gate", &lm->gate)) || (rc = check_weights(&L->up, "up", &lm->up)) ||
        (rc = check_weights(&L->down, "down", &lm->down)) || (rc = check_pair(lm->gate, lm->up, "experts")))
        return rc;
    const Mats& g = lm->gate;
    const Mats& d = lm->down;
    if (g.n_mats != L->n_experts || d.n_mats != L->n_experts || g.K != L->hidden || d.N != L->hidden || d.K != g.N)
        return fail(PGMOE_E_INVALID, "expert shapes do not match E=%d H=%d (gate [%d,%d,%d], down [%d,%d,%d])",
                    L->n_experts, L->hidden, g.n_mats, g.N, g.K, d.n_mats, d.N, d.K);
    if (L->has_shared) {
        if ((rc = check_weights(&L->sh_gate, "shared gate", &lm->sg)) ||
            (rc = check_weights(&L->sh_up, "shared up", &lm->su)) ||
            (rc = check_weights(&L->sh_down, "shared down", &lm->sd)) || (rc = check_pair(lm->sg, lm->su, "shared")))
            return rc;
        if (lm->sg.K != L->hidden || lm->sd.N != L->hidden || lm->sd.K != lm->sg.N)
            return fail(PGMOE_E_INVALID, "shared expert shapes do not match hidden size %d", L->hidden);
    }
    return PGMOE_OK;
}

// ---------------------------------------------------------------- dense SwiGLU MLP
// The same kernels with one matrix triple applied to every token with weight 1 (the
// shared expert's launches without a router).
struct DenseLayout {
    size_t offsets, perm, inv, active, nact, tile_off, w, inter, isum, a16, rs, raw, total;
};

static DenseLayout dense_layout(int M, int I, int H) {
    DenseLayout o{};
    const bool gemm = M > decode_tokens_max();
    size_t c = 0;
    o.offsets = take(c, gemm ? 2 * 4 : 0);
    o.perm = take(c, gemm ? (size_t)M * 4 : 0);
    o.inv = take(c, gemm ? (size_t)M * 4 : 0);
    o.active = take(c, gemm ? 4 : 0);
    o.nact = take(c, gemm ? 4 : 0);
    o.tile_off = take(c, gemm ? 2 * 4 : 0);
    o.w = take(c, gemm ? (size_t)M * 4 : 0);
    o.inter = take(c, (size_t)M * I * 4);
    o.isum = take(c, gemm ? 0 : (size_t)M * (I / 16) * 4);
    o.a16 = take(c, gemm ? (size_t)M * I * 2 : 0);
    o.rs = take(c, gemm ? (size_t)M * 4 : 0);
    o.raw = take(c, gemm ? std::max(gemm_split_bytes_upto(M, 1, I, H, true), gemm_split_bytes_upto(M, 1, H, I, false))
                         : 0);
    o.total = c;
    return o;
}

static int check_dense(const pgmoe_dense* D, Mats* g, Mats* u, Mats* d) {
    if (!D) return fail(PGMOE_E_INVALID, "NULL dense layer");
    if (D->hidden <= 0 || D->hidden % 256 || D->hidden > 65536)
        return fail(PGMOE_E_UNSUPPORTED, "hidden size %d must be a positive multiple of 256 (<= 65536)", D->hidden);
    if (D->act != PGMOE_ACT_SILU && D->act != PGMOE_ACT_GELU_TANH)
        return fail(PGMOE_E_UNSUPPORTED, "activation %d (SiLU = 0, GELU-tanh = 1)", D->act);
    int rc;
    if ((rc = check_weights(&D->gate, "dense gate", g)) || (rc = check_weights(&D->up, "dense up", u)) ||
        (rc = check_weights(&D->down, "dense down", d)) || (rc = check_pair(*g, *u, "dense")))
        return rc;
    if (g->n_mats != 1 || d->n_mats != 1 || g->K != D->hidden || d->N != D->hidden || d->K != g->N)
        return fail(PGMOE_E_INVALID, "dense shapes do not match H=%d (gate [%d,%d,%d], down [%d,%d,%d])", D->hidden,
                    g->n_mats, g->N, g->K, d->n_mats, d->N, d->K);
    return PGMOE_OK;
}

}  // namespace pgmoe

using namespace pgmoe;

extern "C" {

size_t pgmoe_dense_workspace_bytes(const pgmoe_dense* D, int32_t M) {
    Mats g, u, d;
    if (M < 0 || check_dense(D, &g, &u, &d)) return 0;
    return dense_layout(M, g.N, D->hidden).total;
}

int pgmoe_dense_forward(const pgmoe_dense* D, const uint16_t* x, int32_t M, float* out, void* ws, size_t ws_bytes,
                        void* stream) {
    Mats g, u, d;
    int rc = check_dense(D, &g, &u, &d);
    if (rc) return rc;
    if (M < 0) return fail(PGMOE_E_INVALID, "negative token count");
    if (M == 0) return PGMOE_OK;
    if (!x || !out || !ws) return fail(PGMOE_E_INVALID, "dense_forward: NULL pointer");
    if ((uintptr_t)ws & 255) return fail(PGMOE_E_INVALID, "workspace must be 256-byte aligned");
    const DenseLayout o = dense_layout(M, g.N, D->hidden);
    if (ws_bytes < o.total) return fail(PGMOE_E_WORKSPACE, "workspace %zu bytes, need %zu", ws_bytes, o.total);
    uint8_t* b = (uint8_t*)ws;
#define WS(T, f) reinterpret_cast<T*>(b + o.f)
    const hipStream_t st = as_stream(stream);
    if (M <= decode_tokens_max()) {  // gate/up + SwiGLU, then down straight into out
        if ((rc = launch_dec_gateup_ident(g, u, x, nullptr, M, WS(float, inter), WS(float, isum), st, D->act)))
            return rc;
        // the 8-row, 16-wave down blocks when the SwiGLU rows fit in LDS, else the per-expert one
        if (decode_fused_down(M, g.N))
            return launch_dec_down_combine(d, WS(float, inter), WS(float, isum), 0, nullptr, M, 1, 1, nullptr, nullptr,
                                           out, nullptr, 0, st);
        return launch_dec_down_ident(d, WS(float, inter), WS(float, isum), M, out, st);
    }
    const int BM = gemm_tile_rows();
    if ((rc = launch_identity_dispatch(M, BM, WS(int32_t, offsets), WS(int32_t, perm), WS(int32_t, inv),
                                       WS(int32_t, active), WS(int32_t, nact), WS(int32_t, tile_off), WS(float, w),
                                       st)))
        return rc;
    if ((rc = launch_gateup(g, u, x, M, 1, WS(int32_t, offsets), WS(int32_t, perm), WS(int32_t, active),
                            WS(int32_t, nact), WS(int32_t, tile_off), 1, WS(float, inter), st, WS(float, raw),
                            D->act)))
        return rc;
    // identity order: sorted pair p is token p, so the down rows are the output rows
    return launch_down(d, WS(float, inter), M, 1, WS(int32_t, offsets), WS(int32_t, perm), WS(int32_t, active),
                       WS(int32_t, nact), WS(int32_t, tile_off), WS(float, w), 1, WS(uint16_t, a16), WS(float, rs),
                       out, st, WS(float, raw));
#undef WS
}

int pgmoe_abi_version(void) { return PGMOE_ABI_VERSION; }

const char* pgmoe_last_error(void) { return g_err; }

int64_t pgmoe_weight_bytes(int32_t qtype, int64_t rows, int64_t cols) {
    const int64_t b = layout_bytes(qtype, rows, cols);
    return b < 0 ? -1 : (b + 255) & ~(int64_t)255;
}

int pgmoe_relayout_weights(int32_t qtype, const void* src, int64_t n_mats, int64_t rows, int64_t cols, void* dst,
                           void* stream) {
    if (layout_bytes(qtype, rows, cols) < 0)
        return fail(PGMOE_E_UNSUPPORTED, "relayout: qtype %d with %lld columns", qtype, (long long)cols);
    if (!src || !dst || n_mats < 1 || rows < 1) return fail(PGMOE_E_INVALID, "relayout: bad arguments");
    if ((uintptr_t)dst & 255) return fail(PGMOE_E_INVALID, "relayout: dst must be 256-byte aligned");
    if ((uintptr_t)src & 15) return fail(PGMOE_E_INVALID, "relayout: src must be 16-byte aligned");
    return launch_relayout(qtype, (const uint8_t*)src, n_mats, rows, cols, rows, cols, (uint8_t*)dst,
                           pgmoe_weight_bytes(qtype, rows, cols), as_stream(stream));
}

int pgmoe_relayout_weights_padded(int32_t qtype, const void* src, int64_t n_mats, int64_t rows, int64_t cols,
                                  int64_t rows_out, int64_t cols_out, void* dst, void* stream) {
    if (layout_bytes(qtype, rows_out, cols_out) < 0)
        return fail(PGMOE_E_UNSUPPORTED, "relayout: qtype %d with %lld output columns (a multiple of 256)", qtype,
                    (long long)cols_out);
    const bool w32 = qtype == PGMOE_Q8_0 || qtype == PGMOE_Q4_0 || qtype == PGMOE_Q4_1 || qtype == PGMOE_Q5_0;
    if (!src || !dst || n_mats < 1 || rows < 1 || rows > rows_out || cols < 1 || cols > cols_out)
        return fail(PGMOE_E_INVALID, "relayout: bad arguments (rows %lld of %lld, cols %lld of %lld)", (long long)rows,
                    (long long)rows_out, (long long)cols, (long long)cols_out);
    if (w32 ? cols % 32 : cols != cols_out)
        return fail(PGMOE_E_UNSUPPORTED, "relayout: qtype %d with %lld source columns padded to %lld", qtype,
                    (long long)cols, (long long)cols_out);
    if ((uintptr_t)dst & 255) return fail(PGMOE_E_INVALID, "relayout: dst must be 256-byte aligned");
    if ((uintptr_t)src & 15) return fail(PGMOE_E_INVALID, "relayout: src must be 16-byte aligned");
    return launch_relayout(qtype, (const uint8_t*)src, n_mats, rows, cols, rows_out, cols_out, (uint8_t*)dst,
                           pgmoe_weight_bytes(qtype, rows_out, cols_out), as_stream(stream));
}

int pgmoe_requant_w4(int32_t qtype, const void* src, int64_t n_rows, int64_t cols, void* dst, void* stream) {
    int per = 0, bytes = 0;
    if (requant_w4_block(qtype, &per, &bytes))
        return fail(PGMOE_E_UNSUPPORTED, "requant: qtype %d is not re-quantised (Q2_K=10, Q3_K=11, IQ4_NL=20, "
                    "IQ4_XS=23, MXFP4=39)", qtype);
    if (!src || !dst || n_rows < 1 || cols < 1 || cols > (1 << 30))
        return fail(PGMOE_E_INVALID, "requant: bad arguments");
    if (cols % per) return fail(PGMOE_E_UNSUPPORTED, "requant: %lld columns are not whole %d-weight blocks",
                                (long long)cols, per);
    if ((uintptr_t)dst & 3) return fail(PGMOE_E_INVALID, "requant: dst must be 4-byte aligned");
    if (n_rows > (((int64_t)1 << 38) / (cols / 32))) return fail(PGMOE_E_INVALID, "requant: matrix too large");
    return launch_requant_w4(qtype, (const uint8_t*)src, n_rows, (int)cols, (uint8_t*)dst, as_stream(stream));
}

int pgmoe_requant_w8_f16(int32_t qtype, const void* src, int64_t n_rows, int64_t cols, int64_t cols_out, void* dst,
                         void* stream) {
    if (qtype != PGMOE_Q5_1)
        return fail(PGMOE_E_UNSUPPORTED, "requant w8: qtype %d is not re-quantised (Q5_1=7)", qtype);
    if (!src || !dst || n_rows < 1 || cols < 1 || cols_out < cols || cols_out > (1 << 30) || cols_out % 32)
        return fail(PGMOE_E_INVALID, "requant w8: bad arguments");
    if (cols % 32) return fail(PGMOE_E_UNSUPPORTED, "requant w8: %lld columns are not whole 32-weight blocks",
                               (long long)cols);
    if ((uintptr_t)dst & 15) return fail(PGMOE_E_INVALID, "requant w8: dst must be 16-byte aligned");
    if (n_rows > (((int64_t)1 << 38) / (cols_out / 32))) return fail(PGMOE_E_INVALID, "requant w8: matrix too large");
    return launch_requant_w8_f16(qtype, (const uint8_t*)src, n_rows, (int)cols, (int)cols_out, (uint8_t*)dst,
                                 as_stream(stream));
}

int64_t pgmoe_scale_plane_bytes(int32_t qtype, int64_t rows, int64_t cols) {
    return scale_plane_bytes(qtype, rows, cols);
}

int pgmoe_build_scale_plane(int32_t qtype, const void* src, int64_t n_mats, int64_t rows, int64_t cols,
                            int64_t mat_stride, void* dst, void* stream) {
    const int64_t pb = scale_plane_bytes(qtype, rows, cols);
    if (pb <= 0) return fail(PGMOE_E_UNSUPPORTED, "scale plane: qtype %d with %lld columns", qtype, (long long)cols);
    if (!src || !dst || n_mats < 1 || rows < 1 || ((uintptr_t)src & 15) || ((uintptr_t)dst & 15))
        return fail(PGMOE_E_INVALID, "scale plane: bad arguments");
    if (n_mats > 1 && mat_stride < layout_bytes(qtype, rows, cols))
        return fail(PGMOE_E_INVALID, "scale plane: mat_stride %lld below the matrix bytes", (long long)mat_stride);
    return launch_scale_plane(qtype, (const uint8_t*)src, n_mats, rows, cols, mat_stride, (uint8_t*)dst,
                              as_stream(stream));
}

size_t pgmoe_workspace_bytes(const pgmoe_layer* L, int32_t M) {
    LayerMats lm;
    if (M < 0 || check_layer(L, &lm)) return 0;
    return layout_for(L, M).total;
}

int pgmoe_router_topk(const uint16_t* x, const float* w, const float* bias, int32_t M, int32_t H, int32_t E,
                      int32_t K, int32_t norm_topk, float* logits, int32_t* topk_idx, float* topk_w, void* stream) {
    if (M < 0 || H <= 0 || H % 8 || E < 1 || E > 1024 || K < 1 || K > E || K > 64)
        return fail(PGMOE_E_INVALID, "router_topk: bad sizes M=%d H=%d E=%d K=%d", M, H, E, K);
    if (M == 0) return PGMOE_OK;
    if (!x || !w || !logits || !topk_idx || !topk_w) return fail(PGMOE_E_INVALID, "router_topk: NULL pointer");
    const hipStream_t st = as_stream(stream);
    int rc = launch_router_logits(x, w, bias, M, H, E, logits, st);
    if (rc) return rc;
    return launch_topk(logits, M, E, K, norm_topk, topk_idx, topk_w, st);
}

int pgmoe_dispatch(const int32_t* topk_idx, int32_t M, int32_t K, int32_t E, int32_t tile_rows, int32_t* offsets,
                   int32_t* perm, int32_t* inv, int32_t* active, int32_t* n_active, int32_t* tile_off,
                   void* stream) {
    if (M < 0 || K < 1 || E < 1 || E > 512 || tile_rows < 1)
        return fail(PGMOE_E_INVALID, "dispatch: bad sizes M=%d K=%d E=%d tile_rows=%d", M, K, E, tile_rows);
    if (!offsets || !perm || !inv || !active || !n_active || !tile_off || (M > 0 && !topk_idx))
        return fail(PGMOE_E_INVALID, "dispatch: NULL pointer");
    return launch_dispatch(topk_idx, M, K, E, tile_rows, offsets, perm, inv, active, n_active, tile_off,
                           as_stream(stream));
}

size_t pgmoe_dispatch_ws_bytes(int32_t M, int32_t K, int32_t E) {
    if (M < 0 || K < 1 || E < 1 || E > 512) return 0;
    return dispatch_ws_bytes((int64_t)M * K, E);
}

int pgmoe_dispatch_ws(const int32_t* topk_idx, int32_t M, int32_t K, int32_t E, int32_t tile_rows, int32_t* offsets,
                      int32_t* perm, int32_t* inv, int32_t* active, int32_t* n_active, int32_t* tile_off, void* ws,
                      size_t ws_bytes, void* stream) {
    if (M < 0 || K < 1 || E < 1 || E > 512 || tile_rows < 1)
        return fail(PGMOE_E_INVALID, "dispatch: bad sizes M=%d K=%d E=%d tile_rows=%d", M, K, E, tile_rows);
    if (!offsets || !perm || !inv || !active || !n_active || !tile_off || !ws || (M > 0 && !topk_idx))
        return fail(PGMOE_E_INVALID, "dispatch: NULL pointer");
    if (ws_bytes < dispatch_ws_bytes((int64_t)M * K, E))
        return fail(PGMOE_E_WORKSPACE, "dispatch: scratch %zu bytes, need %zu", ws_bytes,
                    dispatch_ws_bytes((int64_t)M * K, E));
    return launch_dispatch(topk_idx, M, K, E, tile_rows, offsets, perm, inv, active, n_active, tile_off,
                           as_stream(stream), (int32_t*)ws);
}

int pgmoe_expert_gateup(const pgmoe_weights* gate, const pgmoe_weights* up, const uint16_t* x, int32_t M,
                        int32_t K, const int32_t* offsets, const int32_t* perm, const int32_t* active,
                        const int32_t* n_active, const int32_t* tile_off, int32_t mode, float* inter,
                        void* stream) {
    Mats g, u;
    int rc;
    if ((rc = check_weights(gate, "gate", &g)) || (rc = check_weights(up, "up", &u)) ||
        (rc = check_pair(g, u, "gate/up")))
        return rc;
    if (M < 0 || K < 1 || (mode != 0 && mode != 1)) return fail(PGMOE_E_INVALID, "gateup: bad M/K/mode");
    return launch_gateup(g, u, x, M, K, offsets, perm, active, n_active, tile_off, mode, inter, as_stream(stream));
}

int pgmoe_expert_down(const pgmoe_weights* down, const float* inter, int32_t M, int32_t K, const int32_t* offsets,
                      const int32_t* perm, const int32_t* active, const int32_t* n_active, const int32_t* tile_off,
                      const float* topk_w, int32_t mode, uint16_t* a16, float* rs, float* partial, void* stream) {
    Mats d;
    int rc;
    if ((rc = check_weights(down, "down", &d))) return rc;
    if (M < 0 || K < 1 || (mode != 0 && mode != 1)) return fail(PGMOE_E_INVALID, "down: bad M/K/mode");
    return launch_down(d, inter, M, K, offsets, perm, active, n_active, tile_off, topk_w, mode, a16, rs, partial,
                       as_stream(stream));
}

int pgmoe_combine(const float* partial, const int32_t* inv, int32_t M, int32_t K, int32_t H, const float* shared,
                  const float* shared_logit, float* out, void* stream) {
    if (M < 0 || K < 1 || H < 1) return fail(PGMOE_E_INVALID, "combine: bad sizes");
    return launch_combine(partial, inv, M, K, H, shared, shared_logit, out, as_stream(stream));
}

}  // extern "C"

namespace pgmoe {

// The layer's kernels on a validated layer and workspace b laid out as o.
static int moe_forward_impl(const pgmoe_layer* L, const LayerMats& lm, const Layout& o, uint8_t* b,
                            const uint16_t* x, int M, float* out, hipStream_t st) {
    int rc;
#define WS(T, f) reinterpret_cast<T*>(b + o.f)
    const int E = L->n_experts, K = L->top_k, H = L->hidden;
    const int mode = M > decode_tokens_max() ? 1 : 0;
    const int BM = gemm_tile_rows();
    if (mode == 0) {
        // decode: gate/up with the router and the routing folded in -> [shared gate/up ->
        // shared down] -> down + combine
        const float* sgw = L->has_shared ? L->sh_inp_gate : nullptr;
        const int max_active = M * K < E ? M * K : E;
        const bool fused = decode_fused_down(M * K, lm.down.K);
        DecFlat flat{};
        if (!fused)
            flat = DecFlat{WS(int32_t, offsets), WS(int32_t, perm), WS(int32_t, inv), WS(int32_t, active),
                           WS(int32_t, nact), WS(float, w)};
        if ((rc = launch_dec_gateup_routed(lm.gate, lm.up, x, K, M, L->router_w, L->router_bias, sgw,
                                           sgw ? WS(float, s_logit) : nullptr, WS(uint64_t, rlog),
                                           WS(int32_t, status), L->has_shared ? WS(float, xsum) : nullptr, E,
                                           L->norm_topk, WS(int32_t, desc), flat, max_active, WS(float, inter),
                                           WS(float, isum), st, L->act, L->status_host)))
            return rc;
        const float* shared = nullptr;
        const float* shared_logit = nullptr;
        if (L->has_shared) {
            if ((rc = launch_dec_gateup_ident(lm.sg, lm.su, x, WS(float, xsum), M, WS(float, s_inter),
                                              WS(float, s_isum), st, L->act)))
                return rc;
            if (decode_fused_down(M, lm.sd.K))
                rc = launch_dec_down_combine(lm.sd, WS(float, s_inter), WS(float, s_isum), 0, nullptr, M, 1, 1, nullptr,
                                             nullptr, WS(float, s_partial), nullptr, 0, st);
            else
                rc = launch_dec_down_ident(lm.sd, WS(float, s_inter), WS(float, s_isum), M, WS(float, s_partial), st);
            if (rc) return rc;
            shared = WS(float, s_partial);
            if (sgw) shared_logit = WS(float, s_logit);
        }
        if (fused)
            return launch_dec_down_combine(lm.down, WS(float, inter), WS(float, isum),
                                           decode_isum_rows8(lm.gate.qtype, M), WS(int32_t, desc), M, K,
                                           max_active, shared, shared_logit, out, WS(uint64_t, rlog), decode_rlog_words(M, E), st);
        // (one token, or 8-row sums from the gate/up: the down kernel forms its 16-row sums
        // itself from the staged rows)
        const bool own_sums = M == 1 || decode_isum_rows8(lm.gate.qtype, M);
        if ((rc = launch_dec_down(lm.down, WS(float, inter), own_sums ? nullptr : WS(float, isum), M, WS(int32_t, offsets),
                                  WS(int32_t, perm), WS(int32_t, active), WS(int32_t, nact), max_active, WS(float, w),
                                  WS(float, partial), st)))
            return rc;
        return launch_combine(WS(float, partial), WS(int32_t, inv), M, K, H, shared, shared_logit, out, st,
                              WS(uint64_t, rlog), decode_rlog_words(M, E));
    }
    if ((rc = launch_router_logits(x, L->router_w, L->router_bias, M, H, E, WS(float, logits), st))) return rc;
    if ((rc = launch_topk(WS(float, logits), M, E, K, L->norm_topk, WS(int32_t, idx), WS(float, w), st))) return rc;
    if ((rc = launch_dispatch(WS(int32_t, idx), M, K, E, BM, WS(int32_t, offsets), WS(int32_t, perm),
                              WS(int32_t, inv), WS(int32_t, active), WS(int32_t, nact), WS(int32_t, tile_off), st,
                              WS(int32_t, dcounts), WS(int32_t, tile_map))))
        return rc;
    if ((rc = launch_gateup(lm.gate, lm.up, x, M, K, WS(int32_t, offsets), WS(int32_t, perm), WS(int32_t, active),
                            WS(int32_t, nact), WS(int32_t, tile_off), mode, WS(float, inter), st, WS(float, raw),
                            L->act, WS(int32_t, tile_map))))
        return rc;
    if ((rc = launch_down(lm.down, WS(float, inter), M, K, WS(int32_t, offsets), WS(int32_t, perm),
                          WS(int32_t, active), WS(int32_t, nact), WS(int32_t, tile_off), WS(float, w), mode,
                          WS(uint16_t, a16), WS(float, rs), WS(float, partial), st, WS(float, raw),
                          WS(int32_t, tile_map))))
        return rc;
    const float* shared = nullptr;
    const float* shared_logit = nullptr;
    if (L->has_shared) {
        if ((rc = launch_identity_dispatch(M, BM, WS(int32_t, s_offsets), WS(int32_t, s_perm), WS(int32_t, s_inv),
                                           WS(int32_t, s_active), WS(int32_t, s_nact), WS(int32_t, s_tile_off),
                                           WS(float, s_w), st)))
            return rc;
        if ((rc = launch_gateup(lm.sg, lm.su, x, M, 1, WS(int32_t, s_offsets), WS(int32_t, s_perm),
                                WS(int32_t, s_active), WS(int32_t, s_nact), WS(int32_t, s_tile_off), mode,
                                WS(float, s_inter), st, WS(float, raw), L->act)))
            return rc;
        if ((rc = launch_down(lm.sd, WS(float, s_inter), M, 1, WS(int32_t, s_offsets), WS(int32_t, s_perm),
                              WS(int32_t, s_active), WS(int32_t, s_nact), WS(int32_t, s_tile_off), WS(float, s_w),
                              mode, WS(uint16_t, s_a16), WS(float, s_rs), WS(float, s_partial), st, WS(float, raw))))
            return rc;
        shared = WS(float, s_partial);
        if (L->sh_inp_gate) {
            if ((rc = launch_router_logits(x, L->sh_inp_gate, nullptr, M, H, 1, WS(float, s_logit), st))) return rc;
            shared_logit = WS(float, s_logit);
        }
    }
    return launch_combine(WS(float, partial), WS(int32_t, inv), M, K, H, shared, shared_logit, out, st);
#undef WS
}

}  // namespace pgmoe

extern "C" {

int pgmoe_moe_forward(const pgmoe_layer* L, const uint16_t* x, int32_t M, float* out, void* ws, size_t ws_bytes,
                      void* stream) {
    LayerMats lm;
    int rc = check_layer(L, &lm);
    if (rc) return rc;
    if (M < 0) return fail(PGMOE_E_INVALID, "negative token count");
    if (M == 0) return PGMOE_OK;
    if (!x || !out || !ws) return fail(PGMOE_E_INVALID, "moe_forward: NULL pointer");
    if ((uintptr_t)ws & 255) return fail(PGMOE_E_INVALID, "workspace must be 256-byte aligned");
    const Layout o = layout_for(L, M);
    if (ws_bytes < o.total)
        return fail(PGMOE_E_WORKSPACE, "workspace %zu bytes, need %zu", ws_bytes, o.total);
    return moe_forward_impl(L, lm, o, (uint8_t*)ws, x, M, out, as_stream(stream));
}

size_t pgmoe_linear_workspace_bytes(const pgmoe_weights* W, int32_t M, int32_t has_bias, int32_t out_dtype) {
    Mats w;
    if (M < 0 || check_weights(W, "linear", &w) || w.n_mats != 1) return 0;
    return linear_ws_bytes(w, M, has_bias || out_dtype == PGMOE_DT_F16);
}

int pgmoe_linear_forward(const pgmoe_weights* W, const float* bias, const uint16_t* x, int32_t M, void* out,
                         int32_t out_dtype, void* ws, size_t ws_bytes, void* stream) {
    Mats w;
    int rc = check_weights(W, "linear", &w);
    if (rc) return rc;
    if (w.n_mats != 1) return fail(PGMOE_E_INVALID, "linear: one matrix (n_mats = 1), got %d", w.n_mats);
    if (M < 0) return fail(PGMOE_E_INVALID, "negative token count");
    if (out_dtype != PGMOE_DT_F32 && out_dtype != PGMOE_DT_F16)
        return fail(PGMOE_E_UNSUPPORTED, "linear: output dtype %d (F32=0, F16=1)", out_dtype);
    if (M == 0) return PGMOE_OK;
    if (!x || !out) return fail(PGMOE_E_INVALID, "linear: NULL pointer");
    if (((uintptr_t)x & 15) || ((uintptr_t)ws & 255) || ((uintptr_t)out & 3))
        return fail(PGMOE_E_INVALID, "linear: x must be 16-byte, ws 256-byte, out 4-byte aligned");
    if (w.qtype != PGMOE_Q8_0 && w.qtype != PGMOE_F16 && !w.scales && !linear_gemv_fits(M, w.K))
        return fail(PGMOE_E_INVALID, "linear: K-quant weights need their scale plane for %d tokens", M);
    return launch_linear(w, bias, x, M, out, out_dtype == PGMOE_DT_F16, (uint8_t*)ws, ws_bytes, as_stream(stream));
}

int pgmoe_dequant_rows(const pgmoe_weights* W, const int32_t* rows, int32_t n, void* out, int32_t out_dtype,
                       void* stream) {
    Mats w;
    int rc = check_weights(W, "dequant rows", &w);
    if (rc) return rc;
    if (w.n_mats != 1) return fail(PGMOE_E_INVALID, "dequant rows: one matrix (n_mats = 1), got %d", w.n_mats);
    if (n < 0 || (out_dtype != PGMOE_DT_F32 && out_dtype != PGMOE_DT_F16))
        return fail(PGMOE_E_INVALID, "dequant rows: n %d, output dtype %d", n, out_dtype);
    if (n == 0) return PGMOE_OK;
    if (!rows || !out) return fail(PGMOE_E_INVALID, "dequant rows: NULL pointer");
    return launch_dequant_rows(w, rows, n, out, out_dtype == PGMOE_DT_F16, as_stream(stream));
}

int pgmoe_add_rmsnorm(const void* x, int32_t x_dtype, const void* delta, int32_t delta_dtype, const float* weight,
                      int32_t rows, int32_t dim, float eps, float* h_out, void* out, int32_t out_dtype, void* stream) {
    auto dt_ok = [](int d) { return d == PGMOE_DT_F32 || d == PGMOE_DT_F16 || d == PGMOE_DT_BF16; };
    if (rows < 0 || dim <= 0 || dim % 4) return fail(PGMOE_E_INVALID, "add_rmsnorm: rows %d, dim %d (a multiple of 4)", rows, dim);
    if (!dt_ok(x_dtype) || (delta && !dt_ok(delta_dtype)) || (out_dtype != PGMOE_DT_F32 && out_dtype != PGMOE_DT_F16))
        return fail(PGMOE_E_UNSUPPORTED, "add_rmsnorm: dtypes x %d, delta %d, out %d (F32=0, F16=1, BF16=30; out F32/F16)",
                    x_dtype, delta_dtype, out_dtype);
    if (!(eps >= 0.0f)) return fail(PGMOE_E_INVALID, "add_rmsnorm: eps must be >= 0");
    if (rows == 0) return PGMOE_OK;
    if (!x || !weight || !out) return fail(PGMOE_E_INVALID, "add_rmsnorm: NULL pointer");
    const uintptr_t al = (uintptr_t)x | (uintptr_t)weight | (uintptr_t)out | (uintptr_t)delta | (uintptr_t)h_out;
    if (al & 7) return fail(PGMOE_E_INVALID, "add_rmsnorm: pointers must be 8-byte aligned");
    if ((((uintptr_t)weight | (uintptr_t)h_out) & 15) || (x_dtype == PGMOE_DT_F32 && ((uintptr_t)x & 15)) ||
        (delta && delta_dtype == PGMOE_DT_F32 && ((uintptr_t)delta & 15)) ||
        (out_dtype == PGMOE_DT_F32 && ((uintptr_t)out & 15)))
        return fail(PGMOE_E_INVALID, "add_rmsnorm: fp32 tensors must be 16-byte aligned");
    return launch_add_rmsnorm(x, x_dtype, delta, delta_dtype, weight, rows, dim, eps, h_out, out, out_dtype,
                              as_stream(stream));
}

int pgmoe_moe_routing(const pgmoe_layer* L, int32_t M, const void* ws, size_t ws_bytes, int32_t* offsets,
                      int32_t* pair_expert, int32_t* pair_token, float* pair_w, void* stream) {
    LayerMats lm;
    int rc = check_layer(L, &lm);
    if (rc) return rc;
    if (M < 0) return fail(PGMOE_E_INVALID, "negative token count");
    if (!ws || !offsets || (M > 0 && (!pair_expert || !pair_token || !pair_w)))
        return fail(PGMOE_E_INVALID, "moe_routing: NULL pointer");
    if ((uintptr_t)ws & 255) return fail(PGMOE_E_INVALID, "workspace must be 256-byte aligned");
    const Layout o = layout_for(L, M);
    if (ws_bytes < o.total) return fail(PGMOE_E_WORKSPACE, "workspace %zu bytes, need %zu", ws_bytes, o.total);
    const uint8_t* b = (const uint8_t*)ws;
#define WS(T, f) reinterpret_cast<const T*>(b + o.f)
    const hipStream_t st = as_stream(stream);
    if (M == 0) {
        if (hipMemsetAsync(offsets, 0, sizeof(int32_t) * (L->n_experts + 1), st) != hipSuccess)
            return fail(PGMOE_E_HIP, "moe_routing: memset failed");
        return PGMOE_OK;
    }
    const int decode = M <= decode_tokens_max() ? 1 : 0;
    return launch_route_readback(decode, WS(int32_t, desc), WS(int32_t, idx), WS(float, w), WS(int32_t, offsets),
                                 WS(int32_t, perm), M, L->top_k, L->n_experts, offsets, pair_expert, pair_token,
                                 pair_w, st);
#undef WS
}

int pgmoe_moe_status(const pgmoe_layer* L, void* ws, size_t ws_bytes, int32_t* status, int32_t clear,
                     void* stream) {
    LayerMats lm;
    int rc = check_layer(L, &lm);
    if (rc) return rc;
    if (!ws || !status) return fail(PGMOE_E_INVALID, "moe_status: NULL pointer");
    if ((uintptr_t)ws & 255) return fail(PGMOE_E_INVALID, "workspace must be 256-byte aligned");
    const Layout o = layout_for(L, 1);  // the status word sits at the same offset for every M
    if (ws_bytes < o.status + 4) return fail(PGMOE_E_WORKSPACE, "workspace %zu bytes too small", ws_bytes);
    const hipStream_t st = as_stream(stream);
    int32_t* word = reinterpret_cast<int32_t*>((uint8_t*)ws + o.status);
    int32_t v = 0;
    if (hipMemcpyAsync(&v, word, 4, hipMemcpyDeviceToHost, st) != hipSuccess || hipStreamSynchronize(st) != hipSuccess)
        return fail(PGMOE_E_HIP, "moe_status: reading the status word failed");
    if (clear && v) {
        if (hipMemsetAsync(word, 0, 4, st) != hipSuccess || hipStreamSynchronize(st) != hipSuccess)
            return fail(PGMOE_E_HIP, "moe_status: clearing the status word failed");
    }
    *status = v;
    return PGMOE_OK;
}

int pgmoe_moe_forward_timed(const pgmoe_layer* L, const uint16_t* x, int32_t M, float* out, void* ws,
                            size_t ws_bytes, void* stream, void** start_events, void** stop_events, int32_t n_events,
                            int32_t* n_launches, const char** kernel_names) {
    if (n_events < 0) return fail(PGMOE_E_INVALID, "negative event count");
    LaunchTiming t{(hipEvent_t*)start_events, (hipEvent_t*)stop_events, kernel_names, n_events, 0};
    launch_timing() = &t;
    const int rc = pgmoe_moe_forward(L, x, M, out, ws, ws_bytes, stream);
    launch_timing() = nullptr;
    if (n_launches) *n_launches = t.next;
    return rc;
}

}  // extern "C"

// ---------------------------------------------------------------- allocation-free forward
// pgmoe_moe_forward_noalloc keeps its workspace in `scratch`, a file-scope device array of
// which every GPU holds its own copy.  Host code never uses the array's name as an
// address (on the host it is only a stand-in for the symbol): once per device, with that
// device current, hipGetSymbolAddress gives the device address, kept in g_noalloc[dev].
namespace pgmoe {

constexpr size_t kNoAllocScratchBytes = (size_t)32 << 20;
constexpr int kMaxRlogExperts = 512;  // check_layer's bound on n_experts
constexpr int kMaxDevices = 64;

static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

struct NoAllocState {
    uint8_t* ptr;      // device address of this device's scratch (null until resolved)
    bool need_clear;   // the state words (tagged logits, status) must be zeroed before use
};
static NoAllocState g_noalloc[kMaxDevices];
static std::mutex g_noalloc_mu;

__global__ __launch_bounds__(256) void zero_kernel(uint4* __restrict__ p, int64_t n16) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += (int64_t)gridDim.x * blockDim.x)
        p[i] = make_uint4(0u, 0u, 0u, 0u);
}

}  // namespace pgmoe

extern "C" {

int pgmoe_moe_forward_noalloc(const pgmoe_layer* L, const uint16_t* x, int32_t M, float* out, void* stream) {
    LayerMats lm;
    int rc = check_layer(L, &lm);
    if (rc) return rc;
    if (M < 0) return fail(PGMOE_E_INVALID, "negative token count");
    if (M == 0) return PGMOE_OK;
    if (!x || !out) return fail(PGMOE_E_INVALID, "moe_forward_noalloc: NULL pointer");
    const Layout o = layout_for(L, M, kMaxRlogExperts);
    if (o.total > kNoAllocScratchBytes)
        return fail(PGMOE_E_WORKSPACE,
                    "moe_forward_noalloc: %d tokens need %zu bytes of scratch, above its fixed %zu bytes "
                    "(use pgmoe_moe_forward with a caller workspace)",
                    M, o.total, kNoAllocScratchBytes);
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
        return fail(PGMOE_E_HIP, "moe_forward_noalloc: no usable current device");
    const hipStream_t st = as_stream(stream);
    uint8_t* b;
    {
        std::lock_guard<std::mutex> lock(g_noalloc_mu);
        NoAllocState& S = g_noalloc[dev];
        if (!S.ptr) {
            void* p = nullptr;
            const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            if (e != hipSuccess || !p)
                return fail(PGMOE_E_HIP, "moe_forward_noalloc: hipGetSymbolAddress failed: %s", hipGetErrorString(e));
            S.ptr = (uint8_t*)p;
            S.need_clear = true;
        }
        if (S.need_clear) {
            // tagged logits + status word; later forwards leave them at zero themselves.  A
            // captured clear would only run when its graph replays, so it must be eager.
            hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
            if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone)
                return fail(PGMOE_E_INVALID, "moe_forward_noalloc: the first call on a device (and the first after "
                                             "a failed call) must run outside graph capture, to clear its scratch");
            const int64_t n16 = (int64_t)(o.status + 256) / 16;
            hipLaunchKernelGGL(zero_kernel, dim3(64), dim3(256), 0, st, (uint4*)S.ptr, n16);
            if ((rc = check_launch("noalloc scratch clear"))) return rc;
            S.need_clear = false;
        }
        b = S.ptr;
    }
    rc = moe_forward_impl(L, lm, o, b, x, M, out, st);
    if (rc) {  // a forward stopped part-way may leave tagged words set
        std::lock_guard<std::mutex> lock(g_noalloc_mu);
        g_noalloc[dev].need_clear = true;
    }
    return rc;
}

}  // extern "C"
