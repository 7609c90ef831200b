/*
 * pgmoe CPU oracle -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's quantized MoE FFN path
 * (pygguf_engine/model.py:898-937 and the helpers it calls in
 * pygguf_engine/quant_kernels.py).  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load this library, and only as the checker.
 * The product path (pgmoe, libpgmoe.so) never calls it.
 *
 * Parity pins (see tests/test_oracle_*.py):
 *   or_dequant_rows      golden vectors written by the reference's own repack
 *                        (quant_kernels.py:854-1036) + closed-form special cases;
 *                        Q5_K: equals Q4_K on the same header/qs with qh = 0, one
 *                        qh bit adds exactly 16*d*sc at its element, and the numpy
 *                        restatement of the reference's Q5_K repack (torch_port);
 *                        Q4_1: equals Q4_0 when m = -8d, closed form on exact
 *                        values, and the restated W4 repack of Q4_0 / Q4_1;
 *                        F16 (the fp16 expert mode): numpy's IEEE binary16
 *                        conversion of every bit pattern
 *   or_router_logits     textbook dot product (checked against float64 numpy to
 *                        fp32 rounding), fixed reduction order mirrored by the
 *                        GPU router kernel bit for bit
 *   or_topk              brute force on tiny inputs, tie rule (value desc, id asc)
 *   or_dispatch          stable argsort (numpy), invariants
 *   or_moe_forward_tokens golden vectors from the reference block forward
 *                        (model.py:898-937) + one-hot / linearity / zero cases
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define QT_F16 1  /* fp16 weights: the reference's fp16 expert mode (quant_kernels.py:1962-1964) */
#define QT_Q4_0 2
#define QT_Q4_1 3
#define QT_Q5_0 6
#define QT_Q8_0 8
#define QT_Q4_K 12
#define QT_Q5_K 13
#define QT_Q6_K 14

/* ---------------- IEEE half <-> float (exact / round-to-nearest-even) ---------- */
float or_half_to_float(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: value = man * 2^-24 */
            float v = (float)man * 5.9604644775390625e-08f;
            memcpy(&bits, &v, 4);
            bits |= sign;
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t or_float_to_half(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) /* inf / nan */
        return sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u);
    if (ax >= 0x477ff000u) /* rounds to >= 65520 -> inf */
        return sign | 0x7c00u;
    if (ax < 0x38800000u) { /* below the smallest normal half: subnormal or zero */
        if (ax < 0x33000000u) return sign; /* < 2^-25 rounds to 0 */
        uint32_t man = (ax & 0x7fffffu) | 0x800000u;
        int e = (int)(ax >> 23); /* biased float exponent */
        int shift = 126 - e;     /* value = man * 2^(e-150); half subnormal unit 2^-24 */
        uint32_t q = man >> (shift);
        uint32_t rem = man & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return sign | (uint16_t)q;
    }
    uint32_t e = (ax >> 23) - 112u;
    uint32_t man = ax & 0x7fffffu;
    uint32_t q = (e << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    return sign | (uint16_t)q;
}

static inline float rnd16(float v) { return or_half_to_float(or_float_to_half(v)); }

static inline uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* ---------------- GGUF block decode ------------------------------------------- */
/* convention 0 ("ggml-exact"): sub-scale products in fp32.
 * convention 1 ("pygguf-repack"): sub-scale products rounded to fp16 as the
 * reference's load-time repack does (quant_kernels.py:896-897, :981). */

/* Q4_K: [d f16][dmin f16][12 scale bytes][128 qs]; 8 sub-blocks of 32.
 * 6-bit (sc, m) unpack as quant_kernels.py:844-851. */
static void q4k_scale_min(const uint8_t* s12, int j, int* sc, int* m) {
    const uint8_t* D = s12;       /* bytes 0..3 */
    const uint8_t* Mb = s12 + 4;  /* bytes 4..7 */
    const uint8_t* MD = s12 + 8;  /* bytes 8..11 */
    if (j < 4) {
        *sc = D[j] & 63;
        *m = Mb[j] & 63;
    } else {
        *sc = (MD[j - 4] & 0x0F) | ((D[j - 4] >> 2) & 0x30);
        *m = (MD[j - 4] >> 4) | ((Mb[j - 4] >> 2) & 0x30);
    }
}

static void decode_q4k_block(const uint8_t* b, int conv, float* out) {
    float d = or_half_to_float(rd16(b));
    float dmin = or_half_to_float(rd16(b + 2));
    const uint8_t* qs = b + 16;
    for (int s = 0; s < 8; ++s) {
        int sc, m;
        q4k_scale_min(b + 4, s, &sc, &m);
        float a = d * (float)sc, z = dmin * (float)m;
        if (conv) { a = rnd16(a); z = rnd16(z); }
        int c = s >> 1, hi = s & 1;
        for (int l = 0; l < 32; ++l) {
            int q = (qs[32 * c + l] >> (4 * hi)) & 0xF;
            out[32 * s + l] = a * (float)q - z;
        }
    }
}

/* Q5_K: [d f16][dmin f16][12 scale bytes][qh 32][qs 128]; element n = 32s + l of
 * sub-block s = 2c + t: q = ((qs[32c + l] >> 4t) & 15) | (((qh[l] >> s) & 1) << 4), value
 * (d*sc_s) q - dmin*m_s (ggml dequantize_row_q5_K; the reference's W8 repack of Q5_K,
 * quant_kernels.py:984-1004, with conv = 1: both products rounded to fp16). */
static void decode_q5k_block(const uint8_t* b, int conv, float* out) {
    float d = or_half_to_float(rd16(b));
    float dmin = or_half_to_float(rd16(b + 2));
    const uint8_t* qh = b + 16;
    const uint8_t* qs = b + 48;
    for (int s = 0; s < 8; ++s) {
        int sc, m;
        q4k_scale_min(b + 4, s, &sc, &m);
        float a = d * (float)sc, z = dmin * (float)m;
        if (conv) { a = rnd16(a); z = rnd16(z); }
        int c = s >> 1, hi = s & 1;
        for (int l = 0; l < 32; ++l) {
            int q = ((qs[32 * c + l] >> (4 * hi)) & 0xF) | (((qh[l] >> s) & 1) << 4);
            out[32 * s + l] = a * (float)q - z;
        }
    }
}

/* Q6_K: [ql 128][qh 64][sc int8 16][d f16]; element n = 128h + 32s + l
 * (quant_kernels.py:968-982). */
static void decode_q6k_block(const uint8_t* b, int conv, float* out) {
    const uint8_t* ql = b;
    const uint8_t* qh = b + 128;
    const int8_t* sc = (const int8_t*)(b + 192);
    float d = or_half_to_float(rd16(b + 208));
    for (int h = 0; h < 2; ++h)
        for (int s = 0; s < 4; ++s)
            for (int l = 0; l < 32; ++l) {
                int n = 128 * h + 32 * s + l;
                int lo = (ql[64 * h + 32 * (s & 1) + l] >> (4 * (s >> 1))) & 0xF;
                int hb = (qh[32 * h + l] >> (2 * s)) & 3;
                int q = (lo | (hb << 4)) - 32;
                float a = d * (float)sc[n >> 4];
                if (conv) a = rnd16(a);
                out[n] = a * (float)q;
            }
}

/* Q8_0: [d f16][int8 x32] */
static void decode_q8_0_block(const uint8_t* b, float* out) {
    float d = or_half_to_float(rd16(b));
    const int8_t* q = (const int8_t*)(b + 2);
    for (int l = 0; l < 32; ++l) out[l] = d * (float)q[l];
}

/* Q4_0: [d f16][16 bytes: weight l in the low nibble of byte l, weight 16 + l in the
 * high nibble]; value d * (nibble - 8) (ggml dequantize_row_q4_0). */
static void decode_q4_0_block(const uint8_t* b, float* out) {
    float d = or_half_to_float(rd16(b));
    for (int l = 0; l < 16; ++l) {
        out[l] = d * (float)((int)(b[2 + l] & 15) - 8);
        out[16 + l] = d * (float)((int)(b[2 + l] >> 4) - 8);
    }
}

/* Q4_1: [d f16][m f16][16 bytes: weight l in the low nibble of byte l, weight 16 + l in
 * the high nibble]; value d * q + m (ggml dequantize_row_q4_1; the reference's W4 repack,
 * quant_kernels.py:870-875: scale d, zero -m). */
static void decode_q4_1_block(const uint8_t* b, float* out) {
    float d = or_half_to_float(rd16(b));
    float m = or_half_to_float(rd16(b + 2));
    for (int l = 0; l < 16; ++l) {
        out[l] = d * (float)(b[4 + l] & 15) + m;
        out[16 + l] = d * (float)(b[4 + l] >> 4) + m;
    }
}

/* Q5_0: [d f16][qh u32 LE: bit l = 5th bit of weight l][16 bytes: weight l in the low
 * nibble of byte l, weight 16 + l in the high nibble]; value d * (q - 16)
 * (ggml dequantize_row_q5_0). */
static void decode_q5_0_block(const uint8_t* b, float* out) {
    float d = or_half_to_float(rd16(b));
    uint32_t qh = (uint32_t)b[2] | ((uint32_t)b[3] << 8) | ((uint32_t)b[4] << 16) | ((uint32_t)b[5] << 24);
    for (int l = 0; l < 16; ++l) {
        out[l] = d * (float)((int)((b[6 + l] & 15) | (((qh >> l) & 1) << 4)) - 16);
        out[16 + l] = d * (float)((int)((b[6 + l] >> 4) | (((qh >> (16 + l)) & 1) << 4)) - 16);
    }
}

int or_block_geometry(int qtype, int* per_block, int* block_bytes) {
    switch (qtype) {
    case QT_Q4_0: *per_block = 32; *block_bytes = 18; return 0;
    case QT_Q4_1: *per_block = 32; *block_bytes = 20; return 0;
    case QT_Q5_0: *per_block = 32; *block_bytes = 22; return 0;
    case QT_Q4_K: *per_block = 256; *block_bytes = 144; return 0;
    case QT_Q5_K: *per_block = 256; *block_bytes = 176; return 0;
    case QT_Q6_K: *per_block = 256; *block_bytes = 210; return 0;
    case QT_Q8_0: *per_block = 32; *block_bytes = 34; return 0;
    case QT_F16: *per_block = 1; *block_bytes = 2; return 0;
    default: return -1;
    }
}

/* Decode `rows` rows of `cols` weights each (rows are whole block runs). */
int or_dequant_rows(int qtype, int conv, const uint8_t* blocks, int64_t rows, int64_t cols, float* out) {
    int pb, bb;
    if (or_block_geometry(qtype, &pb, &bb) || cols % pb) return -1;
    int64_t nblk = rows * (cols / pb);
    for (int64_t i = 0; i < nblk; ++i) {
        const uint8_t* b = blocks + i * bb;
        float* o = out + i * pb;
        if (qtype == QT_Q4_K) decode_q4k_block(b, conv, o);
        else if (qtype == QT_Q5_K) decode_q5k_block(b, conv, o);
        else if (qtype == QT_Q6_K) decode_q6k_block(b, conv, o);
        else if (qtype == QT_Q4_0) decode_q4_0_block(b, o);
        else if (qtype == QT_Q4_1) decode_q4_1_block(b, o);
        else if (qtype == QT_Q5_0) decode_q5_0_block(b, o);
        else if (qtype == QT_F16) o[0] = or_half_to_float(rd16(b));
        else decode_q8_0_block(b, o);
    }
    return 0;
}

/* ---------------- R1 router logits: fixed reduction order --------------------- */
/* logits[m,e] = sum_h f32(x[m,h]) * W[e,h] (+ bias[e]).  Order (mirrored by the GPU
 * kernel): the row is cut into 8-wide chunks c; slot s = c mod 64 owns chunks
 * s, s+64, ...; each slot runs one fmaf chain over its chunks in ascending order and
 * over the 8 elements in order; the 64 slot sums are then combined by the pairwise
 * tree (s, s+32), (s, s+16), ..., (s, s+1); the bias is added last.
 * Reference: model.py:902 (F.linear(x.float(), W)); bias is a harness extension. */
int or_router_logits(const uint16_t* x, const float* W, const float* bias, int M, int H, int E,
                     float* logits) {
    if (H % 8) return -1;
    int C = H / 8;
    for (int m = 0; m < M; ++m) {
        const uint16_t* xr = x + (int64_t)m * H;
        for (int e = 0; e < E; ++e) {
            const float* wr = W + (int64_t)e * H;
            float p[64];
            for (int s = 0; s < 64; ++s) {
                float acc = 0.0f;
                for (int c = s; c < C; c += 64)
                    for (int i = 0; i < 8; ++i)
                        acc = fmaf(or_half_to_float(xr[8 * c + i]), wr[8 * c + i], acc);
                p[s] = acc;
            }
            for (int stride = 32; stride >= 1; stride >>= 1)
                for (int s = 0; s < stride; ++s) p[s] = p[s] + p[s + stride];
            float v = p[0];
            if (bias) v = v + bias[e];
            logits[(int64_t)m * E + e] = v;
        }
    }
    return 0;
}

/* ---------------- R2 softmax + top-k + renorm --------------------------------- */
/* Selection on logits (softmax is monotone) by (logit desc, expert id asc).
 * Weights: p = exp(l - max) / sum_e exp(l_e - max); if norm: w = p / max(sum_k p, 1e-20)
 * (model.py:903-907). */
int or_topk(const float* logits, int M, int E, int K, int norm, int32_t* idx, float* w) {
    if (K < 1 || K > E || K > 64) return -1;
    for (int m = 0; m < M; ++m) {
        const float* l = logits + (int64_t)m * E;
        int32_t* oi = idx + (int64_t)m * K;
        float* ow = w + (int64_t)m * K;
        unsigned char taken[4096];
        if (E > 4096) return -1;
        memset(taken, 0, (size_t)E);
        for (int k = 0; k < K; ++k) {
            int best = -1;
            for (int e = 0; e < E; ++e) {
                if (taken[e]) continue;
                if (best < 0 || l[e] > l[best]) best = e; /* strict: lower id wins ties */
            }
            taken[best] = 1;
            oi[k] = best;
        }
        float mx = l[oi[0]];
        float den = 0.0f;
        for (int e = 0; e < E; ++e) den += expf(l[e] - mx);
        float sp = 0.0f;
        for (int k = 0; k < K; ++k) {
            ow[k] = expf(l[oi[k]] - mx) / den;
            sp += ow[k];
        }
        if (norm) {
            float dd = sp > 1e-20f ? sp : 1e-20f;
            for (int k = 0; k < K; ++k) ow[k] = ow[k] / dd;
        }
    }
    return 0;
}

/* ---------------- R3 dispatch: stable counting sort ----------------------------- */
/* Flat pair id f = t*K + k.  offsets = exclusive scan of per-expert counts;
 * perm[pos] = f in ascending f within each expert (= torch.where row-major order,
 * model.py:911-914); inv[f] = pos. */
int or_dispatch(const int32_t* idx, int M, int K, int E, int32_t* offsets, int32_t* perm, int32_t* inv) {
    int64_t P = (int64_t)M * K;
    int32_t* cur = (int32_t*)calloc((size_t)E + 1, sizeof(int32_t));
    if (!cur) return -2;
    for (int64_t f = 0; f < P; ++f) {
        if (idx[f] < 0 || idx[f] >= E) { free(cur); return -1; }
        cur[idx[f] + 1]++;
    }
    for (int e = 0; e < E; ++e) cur[e + 1] += cur[e];
    memcpy(offsets, cur, sizeof(int32_t) * ((size_t)E + 1));
    for (int64_t f = 0; f < P; ++f) {
        int32_t pos = cur[idx[f]]++;
        perm[pos] = (int32_t)f;
        if (inv) inv[f] = pos;
    }
    free(cur);
    return 0;
}

/* ---------------- R4-R8 expert products, SwiGLU, combine ----------------------- */
typedef struct {
    int qtype;
    int n_rows, n_cols; /* per matrix: [n_rows, n_cols] = [N, K] */
    const uint8_t* data; /* GGUF blocks, matrices back to back */
} or_weights;

static int64_t mat_bytes(const or_weights* w) {
    int pb, bb;
    or_block_geometry(w->qtype, &pb, &bb);
    return (int64_t)w->n_rows * (w->n_cols / pb) * bb;
}

static int64_t row_bytes(const or_weights* w) {
    int pb, bb;
    or_block_geometry(w->qtype, &pb, &bb);
    return (int64_t)(w->n_cols / pb) * bb;
}

static double silu_d(double g) { return g / (1.0 + exp(-g)); }

/* GELU, tanh approximation (F.gelu(approximate="tanh"), the reference's use_gelu branch,
 * quant_kernels.py:1471, kernel :752-756). */
double or_gelu_tanh(double g) {
    return 0.5 * g * (1.0 + tanh(0.7978845608028654 * (g + 0.044715 * g * g * g)));
}

static double act_d(int act, double g) { return act ? or_gelu_tanh(g) : silu_d(g); }

/* y[t][n] = sum_k W[mat][n][k] * xin[t][k] for a set of T input vectors (double). */
static int matvecs(const or_weights* w, int mat, int conv, const double* xin, int T, double* y) {
    float* row = (float*)malloc(sizeof(float) * (size_t)w->n_cols);
    if (!row) return -2;
    const uint8_t* base = w->data + (int64_t)mat * mat_bytes(w);
    int64_t rb = row_bytes(w);
    for (int n = 0; n < w->n_rows; ++n) {
        or_dequant_rows(w->qtype, conv, base + n * rb, 1, w->n_cols, row);
        for (int t = 0; t < T; ++t) {
            const double* xv = xin + (int64_t)t * w->n_cols;
            double acc = 0.0;
            for (int k = 0; k < w->n_cols; ++k) acc += (double)row[k] * xv[k];
            y[(int64_t)t * w->n_rows + n] = acc;
        }
    }
    free(row);
    return 0;
}

/* Gated expert on T inputs: out[t][:] = down(act(gate x) * (up x)), act = SiLU (0) or the
 * tanh GELU (1), all in double
 * (the "fp32-intermediate" variant of model.py:916-919 with the fp16 casts removed). */
static int expert_ffn(const or_weights* g, const or_weights* u, const or_weights* d, int mat, int conv, int act,
                      const double* xin, int T, double* out) {
    int I = g->n_rows;
    double* gv = (double*)malloc(sizeof(double) * (size_t)T * I);
    double* uv = (double*)malloc(sizeof(double) * (size_t)T * I);
    int rc = -2;
    if (!gv || !uv) goto done;
    if ((rc = matvecs(g, mat, conv, xin, T, gv))) goto done;
    if ((rc = matvecs(u, mat, conv, xin, T, uv))) goto done;
    for (int64_t i = 0; i < (int64_t)T * I; ++i) gv[i] = act_d(act, gv[i]) * uv[i];
    rc = matvecs(d, mat, conv, gv, T, out);
done:
    free(gv);
    free(uv);
    return rc;
}

/* Full layer for a subset of tokens, given routing (idx, w) for all M tokens.
 * out[j][h] for tokens[j]; routed experts combined in ascending expert id
 * (model.py:911-922), then the sigmoid-gated shared expert added (model.py:924-935).
 * act: the gate activation of every expert (0 SiLU, 1 GELU-tanh for gemma, model.py:868).
 * shared_* may be NULL.  Accumulation in double. */
int or_moe_forward_tokens(int H, int E, int K, int conv, int act,
                          const or_weights* gate, const or_weights* up, const or_weights* down,
                          const or_weights* sh_gate, const or_weights* sh_up, const or_weights* sh_down,
                          const float* sh_inp_gate,
                          const uint16_t* x, const int32_t* idx, const float* w,
                          const int32_t* tokens, int n_tokens, double* out) {
    double* xt = (double*)malloc(sizeof(double) * (size_t)n_tokens * H);
    double* tmp = (double*)malloc(sizeof(double) * (size_t)n_tokens * H);
    double* xsel = (double*)malloc(sizeof(double) * (size_t)n_tokens * H);
    int* sel = (int*)malloc(sizeof(int) * (size_t)n_tokens + 1);
    double* contrib = (double*)malloc(sizeof(double) * ((size_t)n_tokens * K * H + 1)); /* K = 0: dense */
    int rc = -2;
    if (!xt || !tmp || !xsel || !sel || !contrib) goto done;
    for (int j = 0; j < n_tokens; ++j)
        for (int h = 0; h < H; ++h)
            xt[(int64_t)j * H + h] = or_half_to_float(x[(int64_t)tokens[j] * H + h]);
    /* contrib[j][k] = w[t,k] * expert_{idx[t,k]}(x_t), computed expert by expert */
    for (int e = 0; e < E; ++e) {
        int T = 0;
        for (int j = 0; j < n_tokens; ++j)
            for (int k = 0; k < K; ++k)
                if (idx[(int64_t)tokens[j] * K + k] == e) {
                    sel[T] = j * K + k;
                    memcpy(xsel + (int64_t)T * H, xt + (int64_t)j * H, sizeof(double) * H);
                    ++T;
                }
        if (!T) continue;
        if ((rc = expert_ffn(gate, up, down, e, conv, act, xsel, T, tmp))) goto done;
        for (int s = 0; s < T; ++s) {
            int j = sel[s] / K, k = sel[s] % K;
            double wk = (double)w[(int64_t)tokens[j] * K + k];
            for (int h = 0; h < H; ++h)
                contrib[((int64_t)j * K + k) * H + h] = wk * tmp[(int64_t)s * H + h];
        }
    }
    for (int j = 0; j < n_tokens; ++j) {
        const int32_t* ik = idx + (int64_t)tokens[j] * K;
        /* ascending expert order for this token */
        int order[64];
        for (int k = 0; k < K; ++k) order[k] = k;
        for (int a = 1; a < K; ++a)
            for (int b = a; b > 0 && ik[order[b]] < ik[order[b - 1]]; --b) {
                int t = order[b]; order[b] = order[b - 1]; order[b - 1] = t;
            }
        for (int h = 0; h < H; ++h) {
            double acc = 0.0;
            for (int k = 0; k < K; ++k) acc += contrib[((int64_t)j * K + order[k]) * H + h];
            out[(int64_t)j * H + h] = acc;
        }
    }
    if (sh_gate && sh_up && sh_down) {
        if ((rc = expert_ffn(sh_gate, sh_up, sh_down, 0, conv, act, xt, n_tokens, tmp))) goto done;
        for (int j = 0; j < n_tokens; ++j) {
            double gsc = 1.0;
            if (sh_inp_gate) {
                double z = 0.0;
                for (int h = 0; h < H; ++h) z += xt[(int64_t)j * H + h] * (double)sh_inp_gate[h];
                gsc = 1.0 / (1.0 + exp(-z));
            }
            for (int h = 0; h < H; ++h) out[(int64_t)j * H + h] += tmp[(int64_t)j * H + h] * gsc;
        }
    }
    rc = 0;
done:
    free(xt); free(tmp); free(xsel); free(sel); free(contrib);
    return rc;
}

/* R5 alone: reference activation + dynamic row-scale (quant_kernels.py:1467-1475):
 * inter = silu(g)*u (fp32), rs = max(max|inter|/16384, 1), down_in = fp16(inter/rs). */
void or_act_rowscale(const float* g, const float* u, int M, int I, uint16_t* down_in, float* rs) {
    for (int m = 0; m < M; ++m) {
        float mx = 0.0f;
        for (int i = 0; i < I; ++i) {
            float gg = g[(int64_t)m * I + i];
            float v = (gg / (1.0f + expf(-gg))) * u[(int64_t)m * I + i];
            float a = fabsf(v);
            if (a > mx) mx = a;
        }
        float s = mx / 16384.0f;
        if (s < 1.0f) s = 1.0f;
        rs[m] = s;
        for (int i = 0; i < I; ++i) {
            float gg = g[(int64_t)m * I + i];
            float v = (gg / (1.0f + expf(-gg))) * u[(int64_t)m * I + i];
            down_in[(int64_t)m * I + i] = or_float_to_half(v / s);
        }
    }
}

/* ---------------- residual add + RMSNorm (the MoE block's input) --------------- */
/* exec_fused_add_rmsnorm (quant_kernels.py:1552-1597; CPU branch: h = x.float() +
 * delta.float(), normed = F.rms_norm(h, (D,), w, eps).to(out_dtype)) and, with delta NULL,
 * exec_fused_rmsnorm (:1510-1549).  dtypes: 0 F32, 1 F16, 30 BF16 (inputs), 0 / 1 (out).
 * The sum of squares follows the GPU kernel's fixed order: 256 slots t, slot t owning the
 * 4-element chunks t, t + 256, ... and adding their squares in element order; slots
 * 64w .. 64w + 63 meet by the halving tree (s, s + 32), ..., (s, s + 1); the four group
 * sums are added left to right.  r = 1 / sqrt(sum / D + eps); out = (h * r) * w. */
static float ld_elem(const void* p, int dt, int64_t i) {
    if (dt == 0) return ((const float*)p)[i];
    uint16_t b = ((const uint16_t*)p)[i];
    if (dt == 1) return or_half_to_float(b);
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

int or_add_rmsnorm(const void* x, int xdt, const void* delta, int ddt, const float* w, int R, int D, float eps,
                   float* h_out, void* out, int odt) {
    if (D <= 0 || D % 4) return -1;
    float* h = (float*)malloc(sizeof(float) * (size_t)D);
    if (!h) return -2;
    const int n4 = D / 4;
    for (int r = 0; r < R; ++r) {
        const int64_t base = (int64_t)r * D;
        for (int i = 0; i < D; ++i) {
            float v = ld_elem(x, xdt, base + i);
            if (delta) v = v + ld_elem(delta, ddt, base + i);
            h[i] = v;
            if (h_out) h_out[base + i] = v;
        }
        float slot[256];
        for (int t = 0; t < 256; ++t) {
            float acc = 0.0f;
            for (int c = t; c < n4; c += 256)
                for (int i = 0; i < 4; ++i) acc = acc + h[4 * c + i] * h[4 * c + i];
            slot[t] = acc;
        }
        float tot = 0.0f;
        for (int wv = 0; wv < 4; ++wv) {
            float* p = slot + 64 * wv;
            for (int stride = 32; stride >= 1; stride >>= 1)
                for (int s = 0; s < stride; ++s) p[s] = p[s] + p[s + stride];
            tot = wv == 0 ? p[0] : tot + p[0];
        }
        const float rr = 1.0f / sqrtf(tot / (float)D + eps);
        for (int i = 0; i < D; ++i) {
            const float v = (h[i] * rr) * w[i];
            if (odt == 0) ((float*)out)[base + i] = v;
            else ((uint16_t*)out)[base + i] = or_float_to_half(v);
        }
    }
    free(h);
    return 0;
}
