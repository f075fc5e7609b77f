/*
 * TEST INFRASTRUCTURE ONLY — the parity oracle (see wm_oracle.h).
 *
 * Build: gcc -O2 -ffp-contract=off (no -march=native, no -ffast-math), so that
 * every f32 operation is evaluated exactly as the reference's Rust code does:
 * one IEEE rounding per `+`/`*`/`/`, never fused, in source order.  Rust's
 * f32::{exp,powf,sin,cos,round,sqrt} lower to the platform libm, so this file
 * calls the same glibc functions.
 *
 * Reductions the reference evaluates sequentially are evaluated sequentially
 * here, in the same order; integer reductions (the i8 x ternary dot) are
 * order-free and may be evaluated in any order.
 */
#include "wm_oracle.h"

#include <emmintrin.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#define QK_I2S 128
#define I2S_BLOCK_BYTES 32
#define Q6K_VALUES 256
#define Q6K_BYTES 210

/* ------------------------------------------------------------------------ */
/* scalar helpers                                                           */
/* ------------------------------------------------------------------------ */

/* src/model/primitives.rs:61-88 — exact IEEE binary16 -> binary32. */
float or_f16_to_f32(uint16_t bits) {
    uint32_t sign = (bits >> 15) & 1u, exp = (bits >> 10) & 0x1Fu, man = bits & 0x3FFu;
    uint32_t out;
    float f;
    if (exp == 0) {
        if (man == 0) {
            out = sign << 31;
            memcpy(&f, &out, 4);
            return f;
        }
        /* subnormal: man * 2^-24 (both factors exact, product exact) */
        float m = (float)man;
        float val = m * (1.0f / (float)(1u << 24));
        return sign ? -val : val;
    }
    if (exp == 0x1F) {
        out = (sign << 31) | (0xFFu << 23) | (man << 13);
        memcpy(&f, &out, 4);
        return f;
    }
    out = (sign << 31) | ((exp + (127 - 15)) << 23) | (man << 13);
    memcpy(&f, &out, 4);
    return f;
}

/* src/model/bitlinear.rs:43-50: 00 -> -1, 01 -> 0, 10 -> +1, 11 -> 0 */
static inline int8_t ternary(uint8_t code) {
    switch (code & 3u) {
    case 0: return -1;
    case 2: return 1;
    default: return 0;
    }
}

int8_t or_ternary_from_code(uint8_t code) { return ternary(code); }

/* unpack_block (src/model/bitlinear_sse2.rs:183-193) through a 256-entry
 * table of the four ternary values a byte holds. */
static int8_t g_unpack_lut[256][4];
static pthread_once_t g_lut_once = PTHREAD_ONCE_INIT;
static void init_lut(void) {
    for (int b = 0; b < 256; b++)
        for (int q = 0; q < 4; q++) g_unpack_lut[b][q] = ternary((uint8_t)(b >> (6 - 2 * q)));
}

float or_expf(float x) { return expf(x); }

/* Rust `(v).round().clamp(-127.0, 127.0) as i8`: round half away from zero,
 * clamp that lets NaN through, saturating cast that maps NaN to 0. */
static int8_t rust_round_clamp_i8(float v) {
    float r = roundf(v);
    if (r < -127.0f) r = -127.0f;
    if (r > 127.0f) r = 127.0f;
    if (r != r) return 0;
    return (int8_t)r;
}

/* ------------------------------------------------------------------------ */
/* BitLinear I2_S                                                           */
/* ------------------------------------------------------------------------ */

/* src/model/bitlinear_sse2.rs:285-304 */
float or_quantize_input_absmax_i8(const float *x, size_t n, int8_t *out) {
    float max_abs = 0.0f;
    for (size_t i = 0; i < n; i++) {
        float a = fabsf(x[i]);
        if (a > max_abs) max_abs = a;
    }
    if (max_abs == 0.0f) {
        memset(out, 0, n);
        return 1.0f;
    }
    float inv_scale = 127.0f / max_abs;
    for (size_t i = 0; i < n; i++) out[i] = rust_round_clamp_i8(x[i] * inv_scale);
    return max_abs / 127.0f;
}

/* src/gguf/tensor.rs:278-309 */
int or_i2s_scale(const uint8_t *scale_block, size_t len, float *out) {
    if (!scale_block || len < 4) return -2;
    float s;
    memcpy(&s, scale_block, 4);
    if (!isfinite(s)) return -3;
    *out = s;
    return 0;
}

/* Shape rules of src/model/bitlinear.rs:150-199 / bitlinear_sse2.rs:129-177.
 * The SSE2 entry accepts data.len() >= expected (:166), the scalar one needs
 * equality (:194). */
static int i2s_validate(size_t packed_len, size_t in_dim, size_t out_dim, int exact_len) {
    if (in_dim == 0 || in_dim % QK_I2S) return -2;
    size_t expected = (in_dim / 4) * out_dim;
    if (exact_len ? packed_len != expected : packed_len < expected) return -2;
    return 0;
}

/* src/model/bitlinear.rs:247-299 */
int or_i2s_unpack_row(const uint8_t *packed, size_t in_dim, size_t out_dim, size_t row,
                      int8_t *out) {
    if (row >= out_dim || in_dim == 0 || in_dim % QK_I2S) return -2;
    const uint8_t *r = packed + row * (in_dim / 4);
    for (size_t bk = 0; bk < in_dim / QK_I2S; bk++) {
        for (size_t gp = 0; gp < I2S_BLOCK_BYTES; gp++) {
            uint8_t b = r[bk * I2S_BLOCK_BYTES + gp];
            int8_t *o = out + bk * QK_I2S + gp;
            o[0] = ternary(b >> 6);
            o[32] = ternary(b >> 4);
            o[64] = ternary(b >> 2);
            o[96] = ternary(b);
        }
    }
    return 0;
}

/* One 128-value block: i8 ternary x i8 activation -> i32, the SSE2 select /
 * sign-extend / madd sequence of bitlinear_sse2.rs:353-386 (an integer sum,
 * so its value does not depend on the lane order). */
static int32_t dot_block_sse2(const int8_t *w, const int8_t *a) {
    const __m128i ones = _mm_set1_epi8(1), neg_ones = _mm_set1_epi8(-1);
    const __m128i zero = _mm_setzero_si128(), ones16 = _mm_set1_epi16(1);
    __m128i acc = _mm_setzero_si128();
    for (int i = 0; i < QK_I2S; i += 16) {
        __m128i wv = _mm_loadu_si128((const __m128i *)(w + i));
        __m128i xv = _mm_loadu_si128((const __m128i *)(a + i));
        __m128i pos = _mm_cmpeq_epi8(wv, ones), neg = _mm_cmpeq_epi8(wv, neg_ones);
        __m128i prod = _mm_or_si128(_mm_and_si128(xv, pos),
                                    _mm_and_si128(_mm_sub_epi8(zero, xv), neg));
        __m128i lo = _mm_srai_epi16(_mm_unpacklo_epi8(prod, prod), 8);
        __m128i hi = _mm_srai_epi16(_mm_unpackhi_epi8(prod, prod), 8);
        acc = _mm_add_epi32(acc, _mm_madd_epi16(lo, ones16));
        acc = _mm_add_epi32(acc, _mm_madd_epi16(hi, ones16));
    }
    int32_t l[4];
    _mm_storeu_si128((__m128i *)l, acc);
    return l[0] + l[1] + l[2] + l[3];
}

/* src/model/bitlinear_sse2.rs:313-342 */
int or_bitlinear_i2s_matvec_f32_sse2_i8(const uint8_t *packed, size_t packed_len,
                                        float w_scale, size_t in_dim, size_t out_dim,
                                        const float *x, float *y, int8_t *dbg_act,
                                        float *dbg_act_scale, int32_t *dbg_acc) {
    int rc = i2s_validate(packed_len, in_dim, out_dim, 0);
    if (rc) return rc;
    if (!isfinite(w_scale)) return -3;
    int8_t *act = (int8_t *)malloc(in_dim);
    if (!act) return -4;
    float input_scale = or_quantize_input_absmax_i8(x, in_dim, act);
    float combined = w_scale * input_scale;
    size_t bpr = in_dim / 4;
    int8_t unpacked[QK_I2S];
    pthread_once(&g_lut_once, init_lut);
    for (size_t j = 0; j < out_dim; j++) {
        int32_t dot = 0;
        for (size_t bk = 0; bk < in_dim / QK_I2S; bk++) {
            const uint8_t *blk = packed + j * bpr + bk * I2S_BLOCK_BYTES;
            for (int gp = 0; gp < I2S_BLOCK_BYTES; gp++) {
                const int8_t *t = g_unpack_lut[blk[gp]];
                unpacked[gp] = t[0];
                unpacked[gp + 32] = t[1];
                unpacked[gp + 64] = t[2];
                unpacked[gp + 96] = t[3];
            }
            dot += dot_block_sse2(unpacked, act + bk * QK_I2S);
        }
        if (dbg_acc) dbg_acc[j] = dot;
        y[j] = combined * (float)dot;
    }
    if (dbg_act) memcpy(dbg_act, act, in_dim);
    if (dbg_act_scale) *dbg_act_scale = input_scale;
    free(act);
    return 0;
}

/* src/model/bitlinear.rs:146-233 */
int or_bitlinear_i2s_matvec_f32_scalar(const uint8_t *packed, size_t packed_len,
                                       float w_scale, size_t in_dim, size_t out_dim,
                                       const float *x, float *y) {
    int rc = i2s_validate(packed_len, in_dim, out_dim, 1);
    if (rc) return rc;
    if (!isfinite(w_scale)) return -3;
    size_t bpr = in_dim / 4;
    for (size_t j = 0; j < out_dim; j++) {
        float pos = 0.0f, neg = 0.0f;
        for (size_t bk = 0; bk < in_dim / QK_I2S; bk++) {
            const uint8_t *blk = packed + j * bpr + bk * I2S_BLOCK_BYTES;
            const float *xb = x + bk * QK_I2S;
            for (int gp = 0; gp < I2S_BLOCK_BYTES; gp++) {
                uint8_t b = blk[gp];
                for (int q = 0; q < 4; q++) {
                    uint8_t c = (b >> (6 - 2 * q)) & 3u;
                    float v = xb[gp + 32 * q];
                    if (c == 0) neg += v;
                    else if (c == 2) pos += v;
                }
            }
        }
        y[j] = w_scale * (pos - neg);
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Q6_K                                                                     */
/* ------------------------------------------------------------------------ */

/* The four 6-bit quants that share byte l of a half-block, minus 32
 * (src/model/q6_k.rs:37-40). */
static void q6k_quad(const uint8_t *ql, const uint8_t *qh, int l, int q[4]) {
    q[0] = (int)((ql[l] & 0x0F) | ((qh[l] & 3) << 4)) - 32;
    q[1] = (int)((ql[l + 32] & 0x0F) | (((qh[l] >> 2) & 3) << 4)) - 32;
    q[2] = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
    q[3] = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
}

static uint16_t le16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* src/model/q6_k.rs:25-69 */
int or_q6k_dequantize_row(const uint8_t *row, size_t row_len, float *out, size_t n) {
    if (n % Q6K_VALUES || row_len != n / Q6K_VALUES * Q6K_BYTES) return -2;
    for (size_t b = 0; b < n / Q6K_VALUES; b++) {
        const uint8_t *blk = row + b * Q6K_BYTES;
        float d = or_f16_to_f32(le16(blk + 208));
        for (int h = 0; h < 2; h++) {
            const uint8_t *ql = blk + h * 64, *qh = blk + 128 + h * 32;
            const int8_t *sc = (const int8_t *)(blk + 192 + h * 8);
            float *o = out + b * Q6K_VALUES + h * 128;
            for (int l = 0; l < 32; l++) {
                int q[4];
                q6k_quad(ql, qh, l, q);
                int s = l / 16;
                for (int k = 0; k < 4; k++) o[l + 32 * k] = d * (float)sc[s + 2 * k] * (float)q[k];
            }
        }
    }
    return 0;
}

/* src/model/q6_k.rs:84-96: one f32 accumulator in for_each_weight order. */
float or_q6k_dot_row_scalar(const uint8_t *row, const float *x, size_t n) {
    float sum = 0.0f;
    for (size_t b = 0; b < n / Q6K_VALUES; b++) {
        const uint8_t *blk = row + b * Q6K_BYTES;
        float d = or_f16_to_f32(le16(blk + 208));
        for (int h = 0; h < 2; h++) {
            const uint8_t *ql = blk + h * 64, *qh = blk + 128 + h * 32;
            const int8_t *sc = (const int8_t *)(blk + 192 + h * 8);
            const float *xb = x + b * Q6K_VALUES + h * 128;
            for (int l = 0; l < 32; l++) {
                int q[4];
                q6k_quad(ql, qh, l, q);
                int s = l / 16;
                for (int k = 0; k < 4; k++) {
                    float w = d * (float)sc[s + 2 * k] * (float)q[k];
                    sum += w * xb[l + 32 * k];
                }
            }
        }
    }
    return sum;
}

/* src/model/q6_k_sse2.rs:46-116.  Accumulator k (quarter of a half-block)
 * lane l receives ((q * (d*sc)) * x) for the values with l == index % 4, in
 * (block, half, band, chunk) order; the 16 partial sums are combined as
 * v = (a0 + a1) + (a2 + a3) per lane, then (v0 + v3) + (v1 + v2). */
float or_q6k_dot_row_sse2(const uint8_t *row, const float *x, size_t n) {
    __m128 acc[4] = {_mm_setzero_ps(), _mm_setzero_ps(), _mm_setzero_ps(), _mm_setzero_ps()};
    for (size_t b = 0; b < n / Q6K_VALUES; b++) {
        const uint8_t *blk = row + b * Q6K_BYTES;
        float d = or_f16_to_f32(le16(blk + 208));
        for (int h = 0; h < 2; h++) {
            const uint8_t *ql = blk + h * 64, *qh = blk + 128 + h * 32;
            const int8_t *sc = (const int8_t *)(blk + 192 + h * 8);
            const float *xb = x + b * Q6K_VALUES + h * 128;
            for (int band = 0; band < 2; band++) {
                __m128 scale[4];
                for (int k = 0; k < 4; k++) scale[k] = _mm_set1_ps(d * (float)sc[band + 2 * k]);
                for (int chunk = 0; chunk < 4; chunk++) {
                    int l = band * 16 + chunk * 4;
                    int q[4][4];
                    for (int lane = 0; lane < 4; lane++) {
                        int qq[4];
                        q6k_quad(ql, qh, l + lane, qq);
                        for (int k = 0; k < 4; k++) q[k][lane] = qq[k];
                    }
                    for (int k = 0; k < 4; k++) {
                        __m128 qf = _mm_cvtepi32_ps(_mm_setr_epi32(q[k][0], q[k][1], q[k][2], q[k][3]));
                        __m128 xv = _mm_loadu_ps(xb + l + 32 * k);
                        acc[k] = _mm_add_ps(acc[k], _mm_mul_ps(_mm_mul_ps(qf, scale[k]), xv));
                    }
                }
            }
        }
    }
    __m128 v = _mm_add_ps(_mm_add_ps(acc[0], acc[1]), _mm_add_ps(acc[2], acc[3]));
    __m128 rev = _mm_shuffle_ps(v, v, 0x1B);
    __m128 pairs = _mm_add_ps(v, rev);
    __m128 high = _mm_movehl_ps(pairs, pairs);
    return _mm_cvtss_f32(_mm_add_ss(pairs, high));
}

typedef struct {
    const uint8_t *embd;
    size_t n_embd, row_bytes, begin, end;
    const float *hidden;
    float *logits;
} logits_job;

static void *logits_worker(void *p) {
    logits_job *j = (logits_job *)p;
    for (size_t v = j->begin; v < j->end; v++)
        j->logits[v] = or_q6k_dot_row_sse2(j->embd + v * j->row_bytes, j->hidden, j->n_embd);
    return NULL;
}

/* src/model/lm_head.rs:29-108: every row is an independent q6_k::dot_row,
 * so splitting rows across threads does not change any value. */
int or_compute_logits_q6k(const uint8_t *embd, size_t n_embd, size_t vocab,
                          const float *hidden, float *logits, int threads) {
    if (n_embd == 0 || n_embd % Q6K_VALUES) return -2;
    size_t rb = n_embd / Q6K_VALUES * Q6K_BYTES;
    if (threads < 1) threads = 1;
    if ((size_t)threads > vocab) threads = vocab ? (int)vocab : 1;
    pthread_t tid[256];
    logits_job jobs[256];
    if (threads > 256) threads = 256;
    for (int t = 0; t < threads; t++) {
        jobs[t] = (logits_job){embd, n_embd, rb, vocab * t / threads, vocab * (t + 1) / threads,
                               hidden, logits};
        if (t) pthread_create(&tid[t], NULL, logits_worker, &jobs[t]);
    }
    logits_worker(&jobs[0]);
    for (int t = 1; t < threads; t++) pthread_join(tid[t], NULL);
    return 0;
}

/* src/model/lm_head.rs:161-174: first index of the maximum, strict `>`. */
int64_t or_argmax(const float *logits, size_t n) {
    if (n == 0) return -1;
    size_t best = 0;
    float bv = logits[0];
    for (size_t i = 1; i < n; i++)
        if (logits[i] > bv) {
            bv = logits[i];
            best = i;
        }
    return (int64_t)best;
}

/* ------------------------------------------------------------------------ */
/* f32 primitives                                                           */
/* ------------------------------------------------------------------------ */

/* src/model/primitives.rs:227-255 */
void or_rms_norm(const float *x, const float *w, size_t n, float eps, float *out) {
    if (n == 0) return;
    float sum_sq = 0.0f;
    for (size_t i = 0; i < n; i++) sum_sq += x[i] * x[i];
    float mean = sum_sq / (float)n;
    float rsqrt = 1.0f / sqrtf(mean + eps);
    for (size_t i = 0; i < n; i++) out[i] = x[i] * rsqrt * w[i];
}

/* src/model/primitives.rs:285-345, RopeType::Neox arm (:326-341). */
void or_rope_neox(float *x, size_t head_dim, size_t n_rot, uint32_t pos, float freq_base) {
    (void)head_dim;
    size_t half = n_rot / 2;
    float p = (float)pos, n_rot_f = (float)n_rot;
    for (size_t j = 0; j < half; j++) {
        float exponent = -2.0f * (float)j / n_rot_f;
        float theta = p * powf(freq_base, exponent);
        float s = sinf(theta), c = cosf(theta);
        float a = x[j], b = x[j + half];
        x[j] = a * c - b * s;
        x[j + half] = a * s + b * c;
    }
}

/* src/model/attention.rs:45-73 */
void or_softmax_inplace(float *x, size_t n) {
    if (n == 0) return;
    float max = -INFINITY;
    for (size_t i = 0; i < n; i++)
        if (x[i] > max) max = x[i];
    if (!isfinite(max)) {
        for (size_t i = 0; i < n; i++) x[i] = 0.0f;
        return;
    }
    float sum = 0.0f;
    for (size_t i = 0; i < n; i++) {
        x[i] = expf(x[i] - max);
        sum += x[i];
    }
    if (sum > 0.0f) {
        float inv = 1.0f / sum;
        for (size_t i = 0; i < n; i++) x[i] *= inv;
    }
}

/* src/model/ffn.rs:37-42 then :52-65 */
void or_relu_square_mul(const float *gate, const float *up, size_t n, float *out) {
    for (size_t i = 0; i < n; i++) {
        float r = gate[i] > 0.0f ? gate[i] : 0.0f;
        out[i] = (r * r) * up[i];
    }
}

/* src/model/kv_cache.rs:245-259.  f32::max ignores a NaN operand, so NaN
 * entries never raise absmax. */
float or_kv_quantise(const float *x, size_t n, int8_t *q) {
    float absmax = 0.0f;
    for (size_t i = 0; i < n; i++) {
        float a = fabsf(x[i]);
        absmax = (a != a) ? absmax : (a > absmax ? a : absmax);
    }
    if (absmax == 0.0f || !isfinite(absmax)) {
        memset(q, 0, n);
        return 0.0f;
    }
    float scale = absmax / 127.0f;
    float inv = 127.0f / absmax;
    for (size_t i = 0; i < n; i++) q[i] = rust_round_clamp_i8(x[i] * inv);
    return scale;
}

/* ------------------------------------------------------------------------ */
/* model                                                                    */
/* ------------------------------------------------------------------------ */

typedef struct {
    const uint8_t *w;
    float scale;
} or_lin;

typedef struct {
    or_lin q, k, v, o, gate, up, down;
    const float *attn_norm, *attn_sub_norm, *ffn_norm, *ffn_sub_norm;
} or_layer;

struct or_model {
    uint32_t n_layers, n_embd, n_ff, n_heads, n_kv_heads, head_dim, vocab, kv_dim;
    float eps, rope_base;
    or_layer *layers;
    const uint8_t *token_embd;
    const float *output_norm;
    int threads;
    /* ForwardWorkspace (src/model/cached_forward.rs:61-79) */
    float *hidden, *x_norm, *q, *k, *v, *attn_out, *scores, *sub, *wo, *xf, *gate, *up,
        *fused, *fused_norm, *down, *kd, *vd;
    size_t scores_cap, kd_cap;
};

struct or_kv {
    uint32_t n_layers, kv_dim, max_seq, pos;
    int8_t *k, *v;
    float *ks, *vs;
};

or_model *or_model_create(uint32_t n_layers, uint32_t n_embd, uint32_t n_ff, uint32_t n_heads,
                          uint32_t n_kv_heads, uint32_t head_dim, uint32_t vocab, float eps,
                          float rope_base) {
    if (!n_layers || !n_embd || !n_heads || !n_kv_heads || n_heads % n_kv_heads ||
        n_heads * head_dim != n_embd)
        return NULL;
    or_model *m = (or_model *)calloc(1, sizeof(*m));
    m->n_layers = n_layers; m->n_embd = n_embd; m->n_ff = n_ff; m->n_heads = n_heads;
    m->n_kv_heads = n_kv_heads; m->head_dim = head_dim; m->vocab = vocab; m->eps = eps;
    m->rope_base = rope_base; m->kv_dim = n_kv_heads * head_dim; m->threads = 1;
    m->layers = (or_layer *)calloc(n_layers, sizeof(or_layer));
    float **bufs[] = {&m->hidden, &m->x_norm, &m->q, &m->attn_out, &m->sub, &m->wo, &m->xf, &m->down};
    for (size_t i = 0; i < sizeof(bufs) / sizeof(bufs[0]); i++) *bufs[i] = (float *)calloc(n_embd, 4);
    m->k = (float *)calloc(m->kv_dim, 4);
    m->v = (float *)calloc(m->kv_dim, 4);
    float **ff[] = {&m->gate, &m->up, &m->fused, &m->fused_norm};
    for (size_t i = 0; i < 4; i++) *ff[i] = (float *)calloc(n_ff, 4);
    return m;
}

void or_model_destroy(or_model *m) {
    if (!m) return;
    float *b[] = {m->hidden, m->x_norm, m->q, m->k, m->v, m->attn_out, m->scores, m->sub, m->wo,
                  m->xf, m->gate, m->up, m->fused, m->fused_norm, m->down, m->kd, m->vd};
    for (size_t i = 0; i < sizeof(b) / sizeof(b[0]); i++) free(b[i]);
    free(m->layers);
    free(m);
}

int or_model_set_layer(or_model *m, uint32_t l, const uint8_t *q, float qs, const uint8_t *k,
                       float ks, const uint8_t *v, float vs, const uint8_t *o, float os,
                       const uint8_t *gate, float gs, const uint8_t *up, float us,
                       const uint8_t *down, float ds, const float *attn_norm,
                       const float *attn_sub_norm, const float *ffn_norm,
                       const float *ffn_sub_norm) {
    if (!m || l >= m->n_layers) return -2;
    or_layer *L = &m->layers[l];
    L->q = (or_lin){q, qs}; L->k = (or_lin){k, ks}; L->v = (or_lin){v, vs};
    L->o = (or_lin){o, os}; L->gate = (or_lin){gate, gs}; L->up = (or_lin){up, us};
    L->down = (or_lin){down, ds};
    L->attn_norm = attn_norm; L->attn_sub_norm = attn_sub_norm;
    L->ffn_norm = ffn_norm; L->ffn_sub_norm = ffn_sub_norm;
    return 0;
}

int or_model_set_output(or_model *m, const uint8_t *token_embd, const float *output_norm) {
    if (!m) return -2;
    m->token_embd = token_embd;
    m->output_norm = output_norm;
    return 0;
}

void or_model_set_threads(or_model *m, int threads) { m->threads = threads < 1 ? 1 : threads; }

or_kv *or_kv_create(uint32_t n_layers, uint32_t kv_dim, uint32_t max_seq) {
    or_kv *kv = (or_kv *)calloc(1, sizeof(*kv));
    kv->n_layers = n_layers; kv->kv_dim = kv_dim; kv->max_seq = max_seq; kv->pos = 0;
    size_t nq = (size_t)n_layers * max_seq * kv_dim;
    kv->k = (int8_t *)calloc(nq, 1);
    kv->v = (int8_t *)calloc(nq, 1);
    kv->ks = (float *)calloc((size_t)n_layers * max_seq, 4);
    kv->vs = (float *)calloc((size_t)n_layers * max_seq, 4);
    if (!kv->k || !kv->v || !kv->ks || !kv->vs) {
        or_kv_destroy(kv);
        return NULL;
    }
    return kv;
}

void or_kv_destroy(or_kv *kv) {
    if (!kv) return;
    free(kv->k); free(kv->v); free(kv->ks); free(kv->vs); free(kv);
}

uint32_t or_kv_position(const or_kv *kv) { return kv->pos; }

/* src/model/kv_cache.rs:141-149 */
void or_kv_rollback(or_kv *kv, uint32_t position) {
    if (position < kv->pos) kv->pos = position;
}

/* src/model/kv_cache.rs:154-185 applied to every layer for the next
 * position: k and v hold n_layers x kv_dim values (layer-major). */
int or_kv_append_position(or_kv *kv, const float *k, const float *v) {
    if (kv->pos >= kv->max_seq) return -5;
    for (uint32_t l = 0; l < kv->n_layers; l++) {
        size_t off = ((size_t)l * kv->max_seq + kv->pos) * kv->kv_dim;
        size_t so = (size_t)l * kv->max_seq + kv->pos;
        kv->ks[so] = or_kv_quantise(k + (size_t)l * kv->kv_dim, kv->kv_dim, kv->k + off);
        kv->vs[so] = or_kv_quantise(v + (size_t)l * kv->kv_dim, kv->kv_dim, kv->v + off);
    }
    kv->pos++;
    return 0;
}

int or_kv_read_raw(const or_kv *kv, uint32_t layer, int8_t *k, float *ks, int8_t *v, float *vs,
                   uint32_t n_pos) {
    if (layer >= kv->n_layers || n_pos > kv->max_seq) return -2;
    size_t off = (size_t)layer * kv->max_seq * kv->kv_dim, so = (size_t)layer * kv->max_seq;
    if (k) memcpy(k, kv->k + off, (size_t)n_pos * kv->kv_dim);
    if (v) memcpy(v, kv->v + off, (size_t)n_pos * kv->kv_dim);
    if (ks) memcpy(ks, kv->ks + so, (size_t)n_pos * 4);
    if (vs) memcpy(vs, kv->vs + so, (size_t)n_pos * 4);
    return 0;
}

static int linear(const or_lin *w, size_t in_dim, size_t out_dim, const float *x, float *y) {
    return or_bitlinear_i2s_matvec_f32_sse2_i8(w->w, (in_dim / 4) * out_dim, w->scale, in_dim,
                                               out_dim, x, y, NULL, NULL, NULL);
}

/* src/model/cached_forward.rs:417-449: attention of one query vector over
 * n_past dequantised K/V rows (row p = kv_dim values, kv head j at
 * j*head_dim), out[n_heads*head_dim]; scores is n_past floats of scratch. */
void or_sdpa(const float *q, const float *kd, const float *vd, uint32_t n_past, uint32_t n_heads,
             uint32_t n_kv_heads, uint32_t head_dim, float *out, float *scores) {
    const size_t hd = head_dim, kvd = (size_t)n_kv_heads * head_dim;
    const float scale = 1.0f / sqrtf((float)hd); /* primitives.rs:354 */
    const uint32_t group = n_heads / n_kv_heads;
    memset(out, 0, (size_t)n_heads * hd * 4);
    for (uint32_t h = 0; h < n_heads; h++) {
        const uint32_t kvh = h / group; /* primitives.rs:377 */
        const float *qh = q + h * hd;
        for (uint32_t p = 0; p < n_past; p++) {
            const float *kh = kd + p * kvd + kvh * hd;
            float s = 0.0f;
            for (size_t i = 0; i < hd; i++) s += qh[i] * kh[i];
            scores[p] = s * scale;
        }
        or_softmax_inplace(scores, n_past);
        float *oh = out + h * hd;
        for (uint32_t p = 0; p < n_past; p++) {
            const float *vh = vd + p * kvd + kvh * hd;
            const float w = scores[p];
            for (size_t d = 0; d < hd; d++) oh[d] += w * vh[d];
        }
    }
}

/* The attention of forward_one_layer on the window that KVCache::read_into
 * dequantises (src/model/kv_cache.rs:192-219: q as f32 * scale). */
static void sdpa(or_model *m, const or_kv *kv, uint32_t layer, uint32_t n_past) {
    size_t kvd = m->kv_dim;
    size_t need = (size_t)n_past * kvd;
    if (m->kd_cap < need) {
        free(m->kd); free(m->vd);
        m->kd = (float *)malloc(need * 4);
        m->vd = (float *)malloc(need * 4);
        m->kd_cap = need;
    }
    if (m->scores_cap < n_past) {
        free(m->scores);
        m->scores = (float *)malloc((size_t)n_past * 4);
        m->scores_cap = n_past;
    }
    size_t off = (size_t)layer * kv->max_seq * kvd, so = (size_t)layer * kv->max_seq;
    for (uint32_t p = 0; p < n_past; p++) {
        float sk = kv->ks[so + p], sv = kv->vs[so + p];
        for (size_t d = 0; d < kvd; d++) {
            m->kd[p * kvd + d] = (float)kv->k[off + p * kvd + d] * sk;
            m->vd[p * kvd + d] = (float)kv->v[off + p * kvd + d] * sv;
        }
    }
    or_sdpa(m->q, m->kd, m->vd, n_past, m->n_heads, m->n_kv_heads, m->head_dim, m->attn_out,
            m->scores);
}

static int finite_all(const float *x, size_t n) {
    for (size_t i = 0; i < n; i++)
        if (!isfinite(x[i])) return 0;
    return 1;
}

/* single_token_attention_position_zero (src/model/attention.rs:135-194):
 * one position, K and V as computed (f32, not through the cache): per head
 * s = dot_f32(q_h, k_kvh) * scale (left to right), softmax_inplace([s])
 * (1 for a finite s, else 0), out_h[i] = w * v_kvh[i]. */
static void attention_position_zero(or_model *m) {
    const size_t hd = m->head_dim;
    const float scale = 1.0f / sqrtf((float)hd);
    const uint32_t group = m->n_heads / m->n_kv_heads;
    for (uint32_t h = 0; h < m->n_heads; h++) {
        const uint32_t kvh = h / group;
        const float *qh = m->q + h * hd, *kh = m->k + kvh * hd, *vh = m->v + kvh * hd;
        float s = 0.0f;
        for (size_t i = 0; i < hd; i++) s += qh[i] * kh[i];
        float w = s * scale;
        or_softmax_inplace(&w, 1);
        for (size_t i = 0; i < hd; i++) m->attn_out[h * hd + i] = w * vh[i];
    }
}

/* ffn_block_forward (src/model/ffn.rs:73-136): ffn_norm, the gate and up
 * BitLinears, relu_square of gate then elementwise_mul with up, ffn_sub_norm
 * (width n_ff) and the down BitLinear into out; no residual add.  The
 * model's layer runs this same function (apply_ffn_block,
 * src/model/cached_forward.rs:451-502, the same sequence).  xf (E), g, u,
 * fused, fused_norm (F each) are scratch. */
static int ffn_block(const or_lin *gate, const or_lin *up, const or_lin *down, const float *norm_w,
                     const float *sub_norm_w, size_t E, size_t F, float eps, const float *x,
                     float *xf, float *g, float *u, float *fused, float *fused_norm, float *out) {
    int rc;
    or_rms_norm(x, norm_w, E, eps, xf);
    if ((rc = linear(gate, E, F, xf, g))) return rc;
    if ((rc = linear(up, E, F, xf, u))) return rc;
    or_relu_square_mul(g, u, F, fused);
    or_rms_norm(fused, sub_norm_w, F, eps, fused_norm);
    return linear(down, F, E, fused_norm, out);
}

int or_ffn_block_forward(const float *x, size_t n_embd, size_t n_ff, const float *ffn_norm_w,
                         const uint8_t *gate, float gate_scale, const uint8_t *up, float up_scale,
                         const uint8_t *down, float down_scale, const float *ffn_sub_norm_w,
                         float eps, float *out) {
    if (!x || !ffn_norm_w || !gate || !up || !down || !ffn_sub_norm_w || !out) return -2;
    const or_lin lg = {gate, gate_scale}, lu = {up, up_scale}, ld = {down, down_scale};
    float *buf = (float *)malloc((n_embd + 4 * n_ff) * sizeof(float));
    if (!buf) return -5;
    int rc = ffn_block(&lg, &lu, &ld, ffn_norm_w, ffn_sub_norm_w, n_embd, n_ff, eps, x, buf,
                       buf + n_embd, buf + n_embd + n_ff, buf + n_embd + 2 * n_ff,
                       buf + n_embd + 3 * n_ff, out);
    free(buf);
    return rc;
}

/* src/model/cached_forward.rs:308-415 + apply_ffn_block :451-502; with kv
 * NULL, transformer_block_forward_position_zero (src/model/block.rs:38-105):
 * the same layer at position 0 with attention_position_zero and no cache */
static int forward_one_layer(or_model *m, or_kv *kv, uint32_t l, uint32_t pos) {
    or_layer *L = &m->layers[l];
    size_t E = m->n_embd, F = m->n_ff, KV = m->kv_dim;
    int rc;
    or_rms_norm(m->hidden, L->attn_norm, E, m->eps, m->x_norm);
    if ((rc = linear(&L->q, E, E, m->x_norm, m->q))) return rc;
    if ((rc = linear(&L->k, E, KV, m->x_norm, m->k))) return rc;
    if ((rc = linear(&L->v, E, KV, m->x_norm, m->v))) return rc;
    for (uint32_t h = 0; h < m->n_heads; h++)
        or_rope_neox(m->q + h * m->head_dim, m->head_dim, m->head_dim, pos, m->rope_base);
    for (uint32_t h = 0; h < m->n_kv_heads; h++)
        or_rope_neox(m->k + h * m->head_dim, m->head_dim, m->head_dim, pos, m->rope_base);
    if (kv) {
        /* append at this position, layer l */
        if (kv->pos != pos) return -2;
        if (pos >= kv->max_seq) return -5;
        size_t off = ((size_t)l * kv->max_seq + pos) * KV, so = (size_t)l * kv->max_seq + pos;
        kv->ks[so] = or_kv_quantise(m->k, KV, kv->k + off);
        kv->vs[so] = or_kv_quantise(m->v, KV, kv->v + off);
        sdpa(m, kv, l, pos + 1);
    } else {
        attention_position_zero(m);
    }
    or_rms_norm(m->attn_out, L->attn_sub_norm, E, m->eps, m->sub);
    if ((rc = linear(&L->o, E, E, m->sub, m->wo))) return rc;
    for (size_t d = 0; d < E; d++) m->hidden[d] += m->wo[d];
    if ((rc = ffn_block(&L->gate, &L->up, &L->down, L->ffn_norm, L->ffn_sub_norm, E, F, m->eps,
                        m->hidden, m->xf, m->gate, m->up, m->fused, m->fused_norm, m->down)))
        return rc;
    for (size_t d = 0; d < E; d++) m->hidden[d] += m->down[d];
    if (!finite_all(m->hidden, E)) return -3; /* cached_forward.rs:511-521 */
    return 0;
}

/* src/model/cached_forward.rs:206-261 */
int or_forward_with_cache(or_model *m, or_kv *kv, uint32_t token, uint32_t pos,
                          float *out_hidden, float *layer_trace) {
    if (!m || !kv || !m->token_embd || !m->output_norm) return -2;
    if (kv->kv_dim != m->kv_dim || kv->n_layers != m->n_layers) return -2;
    if (kv->pos != pos || token >= m->vocab) return -2;
    uint32_t checkpoint = kv->pos;
    size_t rb = m->n_embd / Q6K_VALUES * Q6K_BYTES;
    int rc = or_q6k_dequantize_row(m->token_embd + (size_t)token * rb, rb, m->hidden, m->n_embd);
    for (uint32_t l = 0; !rc && l < m->n_layers; l++) {
        rc = forward_one_layer(m, kv, l, pos);
        if (!rc && layer_trace) memcpy(layer_trace + (size_t)l * m->n_embd, m->hidden, m->n_embd * 4);
    }
    if (rc) {
        kv->pos = checkpoint; /* rollback */
        return rc;
    }
    kv->pos = pos + 1;
    or_rms_norm(m->hidden, m->output_norm, m->n_embd, m->eps, out_hidden);
    return 0;
}

/* forward_single_token_position_zero (src/model/forward.rs:29-69): the
 * token at position 0 with no cache; a non-finite hidden after any layer
 * fails the call (-3). */
int or_forward_single_token_position_zero(or_model *m, uint32_t token, float *out_hidden,
                                          float *layer_trace) {
    if (!m || !m->token_embd || !m->output_norm || token >= m->vocab) return -2;
    size_t rb = m->n_embd / Q6K_VALUES * Q6K_BYTES;
    int rc = or_q6k_dequantize_row(m->token_embd + (size_t)token * rb, rb, m->hidden, m->n_embd);
    for (uint32_t l = 0; !rc && l < m->n_layers; l++) {
        rc = forward_one_layer(m, NULL, l, 0);
        if (!rc && layer_trace) memcpy(layer_trace + (size_t)l * m->n_embd, m->hidden, m->n_embd * 4);
    }
    if (rc) return rc;
    or_rms_norm(m->hidden, m->output_norm, m->n_embd, m->eps, out_hidden);
    return 0;
}

int or_logits_argmax(or_model *m, const float *hidden, float *logits, uint32_t *next) {
    int rc = or_compute_logits_q6k(m->token_embd, m->n_embd, m->vocab, hidden, logits, m->threads);
    if (rc) return rc;
    int64_t a = or_argmax(logits, m->vocab);
    if (a < 0) return -2;
    *next = (uint32_t)a;
    return 0;
}

/* src/model/generate.rs:111-189, on a cache already holding kv->pos
 * positions (the prompt continues from there). */
int or_greedy_generate(or_model *m, or_kv *kv, const uint32_t *prompt, uint32_t n_prompt,
                       uint32_t max_new, int64_t eos, uint32_t *out_ids, uint32_t *n_out,
                       float *logits_trace) {
    if (!n_prompt) return -2;
    float *hidden = (float *)malloc((size_t)m->n_embd * 4);
    float *logits = (float *)malloc((size_t)m->vocab * 4);
    int rc = 0;
    *n_out = 0;
    for (uint32_t i = 0; i < n_prompt && !rc; i++)
        rc = or_forward_with_cache(m, kv, prompt[i], kv->pos, hidden, NULL);
    for (uint32_t step = 0; step < max_new && !rc; step++) {
        uint32_t next;
        if ((rc = or_logits_argmax(m, hidden, logits, &next))) break;
        if (logits_trace) memcpy(logits_trace + (size_t)step * m->vocab, logits, (size_t)m->vocab * 4);
        if (eos >= 0 && (int64_t)next == eos) break;
        out_ids[(*n_out)++] = next;
        if (step + 1 < max_new) rc = or_forward_with_cache(m, kv, next, kv->pos, hidden, NULL);
    }
    free(hidden);
    free(logits);
    return rc;
}

/* ------------------------------------------------------------------------ */
/* sampler (src/model/sampler.rs)                                           */
/* ------------------------------------------------------------------------ */

/* XorShift64::new (sampler.rs:18-25) */
uint64_t or_xorshift64_seed(uint64_t seed) { return seed ? seed : 0xdeadbeefcafebabeull; }

/* XorShift64::next_u64 (sampler.rs:26-33): shifts 13, 7, 17 */
uint64_t or_xorshift64_next(uint64_t *state) {
    uint64_t x = *state;
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    *state = x;
    return x;
}

/* XorShift64::next_unit (sampler.rs:34-37): high 24 bits / 2^24 */
float or_xorshift64_next_unit(uint64_t *state) {
    return (float)(or_xorshift64_next(state) >> 40) / (float)(1ull << 24);
}

/* SamplingParams::is_greedy (sampler.rs:71-78) */
int or_sampling_is_greedy(const or_sampling_params *p) {
    return fabsf(p->temperature) < 1e-9f && !p->has_top_k && !p->has_top_p &&
           !p->has_repetition_penalty;
}

/* Sampler::apply_repetition_penalty (sampler.rs:151-164): each distinct
 * history id below n once, in history order. */
void or_apply_repetition_penalty(float *logits, size_t n, const uint32_t *history,
                                 size_t n_history, float r) {
    if (r <= 0.0f || fabsf(r - 1.0f) < 1e-9f) return;
    for (size_t h = 0; h < n_history; h++) {
        uint32_t id = history[h];
        if (id >= n) continue;
        int seen = 0;
        for (size_t j = 0; j < h && !seen; j++) seen = history[j] == id;
        if (seen) continue;
        float l = logits[id];
        logits[id] = l > 0.0f ? l / r : l * r;
    }
}

/* Sampler::apply_temperature (sampler.rs:166-176) */
void or_apply_temperature(float *logits, size_t n, float t) {
    if (t <= 0.0f || fabsf(t - 1.0f) < 1e-9f) return;
    float inv = 1.0f / t;
    for (size_t i = 0; i < n; i++) logits[i] *= inv;
}

static int desc_float(const void *a, const void *b) {
    float x = *(const float *)a, y = *(const float *)b;
    if (isnan(x) || isnan(y)) return isnan(x) - isnan(y); /* NaN last (order open in the reference) */
    return (x < y) - (x > y);
}

/* apply_top_k (sampler.rs:201-223): the k-th largest value is the
 * threshold; everything strictly below it becomes -inf. */
void or_apply_top_k(float *logits, size_t n, uint64_t k) {
    if (k > n) k = n;
    if (k == 0) {
        for (size_t i = 0; i < n; i++) logits[i] = -INFINITY;
        return;
    }
    if (k == n) return;
    float *v = (float *)malloc(n * sizeof(float));
    memcpy(v, logits, n * sizeof(float));
    qsort(v, n, sizeof(float), desc_float);
    float thr = v[k - 1];
    free(v);
    for (size_t i = 0; i < n; i++)
        if (logits[i] < thr) logits[i] = -INFINITY;
}

/* softmax_to_probs (sampler.rs:225-252) */
void or_softmax_to_probs(const float *logits, size_t n, float *out) {
    if (!n) return;
    float max = -INFINITY;
    for (size_t i = 0; i < n; i++)
        if (logits[i] > max) max = logits[i];
    if (!isfinite(max)) {
        for (size_t i = 0; i < n; i++) out[i] = 0.0f;
        return;
    }
    float sum = 0.0f;
    for (size_t i = 0; i < n; i++) {
        float e = expf(logits[i] - max);
        sum += e;
        out[i] = e;
    }
    if (sum > 0.0f) {
        float inv = 1.0f / sum;
        for (size_t i = 0; i < n; i++) out[i] *= inv;
    }
}

typedef struct { float v; uint32_t i; } prob_idx;
static int desc_prob(const void *a, const void *b) {
    const prob_idx *x = (const prob_idx *)a, *y = (const prob_idx *)b;
    if (x->v != y->v) return x->v < y->v ? 1 : -1;
    return (x->i > y->i) - (x->i < y->i);
}

/* apply_top_p (sampler.rs:254-311); equal probabilities in index order. */
void or_apply_top_p(float *probs, size_t n, float p) {
    if (!n) return;
    if (p <= 0.0f) {
        size_t am = 0;
        float av = probs[0];
        for (size_t i = 1; i < n; i++)
            if (probs[i] > av) {
                av = probs[i];
                am = i;
            }
        for (size_t i = 0; i < n; i++) probs[i] = i == am ? 1.0f : 0.0f;
        return;
    }
    if (p >= 1.0f) return;
    prob_idx *o = (prob_idx *)malloc(n * sizeof(prob_idx));
    unsigned char *keep = (unsigned char *)calloc(n, 1);
    for (size_t i = 0; i < n; i++) {
        o[i].v = probs[i];
        o[i].i = (uint32_t)i;
    }
    qsort(o, n, sizeof(prob_idx), desc_prob);
    float acc = 0.0f;
    for (size_t s = 0; s < n; s++) {
        acc += o[s].v;
        keep[o[s].i] = 1;
        if (acc >= p) break;
    }
    float sum = 0.0f;
    for (size_t i = 0; i < n; i++) {
        if (!keep[i]) probs[i] = 0.0f;
        sum += probs[i];
    }
    if (sum > 0.0f) {
        float inv = 1.0f / sum;
        for (size_t i = 0; i < n; i++) probs[i] *= inv;
    }
    free(o);
    free(keep);
}

/* Sampler::sample (sampler.rs:133-149) + multinomial (:178-196) */
int or_sample(const or_sampling_params *p, uint64_t *state, const uint32_t *history,
              size_t n_history, const float *logits, size_t n, uint32_t *out, float *total_out) {
    if (or_sampling_is_greedy(p)) {
        int64_t a = or_argmax(logits, n);
        if (a < 0) return -1;
        *out = (uint32_t)a;
        return 0;
    }
    if (!n) { /* multinomial over no probabilities: total 0 */
        if (total_out) *total_out = 0.0f;
        return -2;
    }
    float *buf = (float *)malloc(n * sizeof(float));
    float *probs = (float *)malloc(n * sizeof(float));
    memcpy(buf, logits, n * sizeof(float));
    if (p->has_repetition_penalty)
        or_apply_repetition_penalty(buf, n, history, n_history, p->repetition_penalty);
    or_apply_temperature(buf, n, p->temperature);
    int rc = 0;
    /* top-k sorts only when 0 < k < n (sampler.rs:202-212); a NaN among the
     * values it sorts leaves the k-th largest open (the comparator is then
     * no order), so that case is refused, as NaN under top-p is */
    if (p->has_top_k && p->top_k > 0 && p->top_k < n)
        for (size_t i = 0; i < n && !rc; i++)
            if (isnan(buf[i])) rc = -3;
    if (p->has_top_k && !rc) or_apply_top_k(buf, n, p->top_k);
    if (!rc) or_softmax_to_probs(buf, n, probs);
    if (p->has_top_p && !rc) {
        if (p->top_p > 0.0f && p->top_p < 1.0f)
            for (size_t i = 0; i < n && !rc; i++)
                if (isnan(probs[i])) rc = -3;
        if (!rc) or_apply_top_p(probs, n, p->top_p);
    }
    if (!rc) {
        float total = 0.0f;
        for (size_t i = 0; i < n; i++) total += probs[i];
        if (total_out) *total_out = total;
        if (total <= 0.0f || !isfinite(total)) {
            rc = -2;
        } else {
            float r = or_xorshift64_next_unit(state) * total;
            float acc = 0.0f;
            size_t pick = n - 1;
            for (size_t i = 0; i < n; i++) {
                acc += probs[i];
                if (r <= acc) {
                    pick = i;
                    break;
                }
            }
            *out = (uint32_t)pick;
        }
    }
    free(buf);
    free(probs);
    return rc;
}
