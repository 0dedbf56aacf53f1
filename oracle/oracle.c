/*
 * oracle.c — TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Plain C restatement of the reference's CPU algorithms for the hot path.
 * Built with -ffp-contract=off so every multiply and add rounds separately,
 * as Zig's default (strict) float mode does.
 *
 * Summation order notes (the reference's exact order is not observable
 * without building it; see the pin tests for how each function is checked):
 *   - SIMD loops in the reference use @Vector(vec_len, f32) accumulators;
 *     vec_len = 16 is used here (AVX-512 suggestVectorLength(f32)), and
 *     @reduce(.Add) is restated as an ordered lane sum.
 *   - BLAS-backed f32 GEMMs (attention QK^T, P*V) are restated as ordered
 *     dot products; their exact order is not pinned by any reference test.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define VL 16 /* simd.suggestVectorLength(f32) on an AVX-512 host */

/* ------------------------------------------------------------------ */
/* f16 <-> f32 (Zig @floatCast: IEEE round-to-nearest-even)            */
/* ------------------------------------------------------------------ */
uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu)); /* NaN */
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to inf */
    if (ax >= 0x38800000u) { /* normal f16 */
        uint32_t e = (ax >> 23) - 127 + 15;
        uint32_t m = ax & 0x7fffffu;
        uint32_t h = (e << 10) | (m >> 13);
        uint32_t r = m & 0x1fffu;
        if (r > 0x1000u || (r == 0x1000u && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    if (ax <= 0x33000000u) return (uint16_t)sign; /* <= 2^-25 rounds to zero */
    uint32_t E = ax >> 23;
    uint32_t m = (ax & 0x7fffffu) | 0x800000u;
    uint32_t shift = 126 - E; /* 14..24 */
    uint32_t h = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    uint32_t x;
    if (e == 0) {
        if (m == 0) {
            x = sign;
        } else { /* subnormal: normalise */
            int sh = 0;
            while (!(m & 0x400u)) { m <<= 1; sh++; }
            m &= 0x3ffu;
            x = sign | ((uint32_t)(127 - 15 + 1 - sh) << 23) | (m << 13);
        }
    } else if (e == 31) {
        x = sign | 0x7f800000u | (m << 13);
    } else {
        x = sign | ((e - 15 + 127) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

/* ------------------------------------------------------------------ */
/* A1 quantizer: quantize_arctic_xs.zig:94-115                        */
/* ------------------------------------------------------------------ */
void orc_quantize_rows(const float *w, int64_t rows, int64_t cols, int8_t *q, uint16_t *scale) {
    for (int64_t r = 0; r < rows; r++) {
        const float *row = w + r * cols;
        float max_abs = 0.0f; /* :153-159 */
        for (int64_t c = 0; c < cols; c++) {
            float a = fabsf(row[c]);
            if (a > max_abs) max_abs = a;
        }
        float s_f32 = (max_abs == 0.0f) ? 1.0f : max_abs / 127.0f; /* :161 */
        uint16_t s_f16 = orc_f32_to_f16(s_f32);                      /* :162 */
        scale[r] = s_f16;
        float inv_s = 1.0f / orc_f16_to_f32(s_f16); /* :165 */
        for (int64_t c = 0; c < cols; c++) {        /* :166-172 */
            float qf = roundf(row[c] * inv_s);        /* @round: half away from zero */
            /* @intFromFloat then clamp; a zero f16 scale (max_abs < ~3.8e-6)
             * makes qf +-inf or NaN, where the reference is undefined (a
             * safety panic): saturate to +-127, NaN (0 * inf) to 0 */
            int32_t qi = isnan(qf) ? 0 : qf >= 127.0f ? 127 : qf <= -127.0f ? -127 : (int32_t)qf;
            q[r * cols + c] = (int8_t)qi;
        }
    }
}

/* ordered sum of the VL lane accumulators (@reduce(.Add) in strict mode) */
static inline float lane_sum(const float *acc) {
    float s = acc[0];
    for (int l = 1; l < VL; l++) s += acc[l];
    return s;
}

/* ------------------------------------------------------------------ */
/* A5 int8 linear: matmul_w8a32.zig:14-57                              */
/* ------------------------------------------------------------------ */
void orc_matmul_w8a32(const float *a, const int8_t *wq, const uint16_t *scale, const float *bias,
                      float *c, int64_t m, int64_t k, int64_t n) {
    if (m == 0 || n == 0) return; /* :24 */
    for (int64_t i = 0; i < m; i++) {
        const float *a_row = a + i * k;
        for (int64_t j = 0; j < n; j++) {
            const int8_t *w_row = wq + j * k;
            float acc[VL] = {0};
            int64_t kk = 0;
            for (; kk + VL <= k; kk += VL) /* :42-47 */
                for (int l = 0; l < VL; l++) acc[l] += a_row[kk + l] * (float)w_row[kk + l];
            float sum = lane_sum(acc); /* :49 */
            for (; kk < k; kk++) sum += a_row[kk] * (float)w_row[kk]; /* :50-52 */
            float s = orc_f16_to_f32(scale[j]);                         /* :54 */
            c[i * n + j] = sum * s + (bias ? bias[j] : 0.0f);            /* :55 */
        }
    }
}

/* arctic.zig:609-621: f32 weights, C = A W^T then C += bias */
void orc_linear_f32(const float *a, const float *w, const float *bias, float *c,
                    int64_t m, int64_t k, int64_t n) {
    for (int64_t i = 0; i < m; i++) {
        const float *a_row = a + i * k;
        for (int64_t j = 0; j < n; j++) {
            const float *w_row = w + j * k;
            float acc[VL] = {0};
            int64_t kk = 0;
            for (; kk + VL <= k; kk += VL)
                for (int l = 0; l < VL; l++) acc[l] += a_row[kk + l] * w_row[kk + l];
            float sum = lane_sum(acc);
            for (; kk < k; kk++) sum += a_row[kk] * w_row[kk];
            c[i * n + j] = sum;
        }
    }
    if (bias)
        for (int64_t i = 0; i < m; i++)
            for (int64_t j = 0; j < n; j++) c[i * n + j] += bias[j];
}

/* ------------------------------------------------------------------ */
/* A4 LayerNorm: layernorm.zig:26-117                                  */
/* ------------------------------------------------------------------ */
void orc_layernorm(const float *x_all, const float *gamma, const float *beta, float *y_all,
                   int64_t rows, int64_t n, float eps) {
    float *tmp = (float *)malloc(sizeof(float) * (size_t)n);
    for (int64_t r = 0; r < rows; r++) {
        /* copy first so in-place calls (x == y) read the original row */
        memcpy(tmp, x_all + r * n, sizeof(float) * (size_t)n);
        const float *x = tmp;
        float *y = y_all + r * n;
        float acc[VL] = {0};
        int64_t i = 0;
        for (; i + VL <= n; i += VL)
            for (int l = 0; l < VL; l++) acc[l] += x[i + l];
        float sum = lane_sum(acc);
        for (; i < n; i++) sum += x[i];
        float mean = sum / (float)n; /* :71 */
        float vacc[VL] = {0};
        i = 0;
        for (; i + VL <= n; i += VL)
            for (int l = 0; l < VL; l++) {
                float d = x[i + l] - mean;
                vacc[l] += d * d;
            }
        float var_sum = lane_sum(vacc);
        for (; i < n; i++) {
            float d = x[i] - mean;
            var_sum += d * d;
        }
        float variance = var_sum / (float)n;          /* :92 */
        float inv_std = 1.0f / sqrtf(variance + eps); /* :95 */
        for (i = 0; i < n; i++) {
            float normalized = (x[i] - mean) * inv_std; /* :105, :113 */
            y[i] = normalized * gamma[i] + beta[i];     /* :107, :114 */
        }
    }
    free(tmp);
}

/* ------------------------------------------------------------------ */
/* A8 GELU (tanh form with std.math.tanh): arctic.zig:750-756          */
/* ------------------------------------------------------------------ */
float orc_gelu(float x) {
    const float sqrt_2_over_pi = 0.7978845608f;
    const float coeff = 0.044715f;
    float inner = sqrt_2_over_pi * (x + coeff * x * x * x);
    return 0.5f * x * (1.0f + tanhf(inner));
}

/* ------------------------------------------------------------------ */
/* A10 L2 normalise: arctic.zig:851-863                                */
/* ------------------------------------------------------------------ */
void orc_l2_normalize(float *v, int64_t n) {
    float norm_sq = 0.0f;
    for (int64_t i = 0; i < n; i++) norm_sq += v[i] * v[i];
    float norm = sqrtf(norm_sq);
    if (norm > 1e-12f)
        for (int64_t i = 0; i < n; i++) v[i] /= norm;
}

/* ------------------------------------------------------------------ */
/* A6 attention core for one head: arctic.zig:660-713                  */
/* ------------------------------------------------------------------ */
void orc_attention_head(const float *q, const float *k, const float *v, float *out,
                        int64_t L, int64_t ld, int64_t head_dim, float *scores) {
    const float scale = 1.0f / sqrtf((float)head_dim); /* :649 */
    for (int64_t i = 0; i < L; i++) /* :675 Q_h K_h^T */
        for (int64_t j = 0; j < L; j++) {
            float s = 0.0f;
            for (int64_t d = 0; d < head_dim; d++) s += q[i * ld + d] * k[j * ld + d];
            scores[i * L + j] = s;
        }
    for (int64_t t = 0; t < L * L; t++) scores[t] *= scale; /* :678-680 */
    for (int64_t i = 0; i < L; i++) {                      /* :683-703 */
        float *row = scores + i * L;
        float mx = row[0];
        for (int64_t j = 1; j < L; j++)
            if (row[j] > mx) mx = row[j];
        float sum = 0.0f;
        for (int64_t j = 0; j < L; j++) {
            row[j] = expf(row[j] - mx);
            sum += row[j];
        }
        for (int64_t j = 0; j < L; j++) row[j] /= sum;
    }
    for (int64_t i = 0; i < L; i++) /* :707 P V_h */
        for (int64_t d = 0; d < head_dim; d++) {
            float s = 0.0f;
            for (int64_t j = 0; j < L; j++) s += scores[i * L + j] * v[j * ld + d];
            out[i * ld + d] = s;
        }
}

/* ------------------------------------------------------------------ */
/* A3 embeddings: arctic.zig:484-585                                   */
/* ------------------------------------------------------------------ */
static void write_row(float *dst, const tzh_mat_view *w, int64_t row, int64_t cols) {
    if (w->dtype == TZH_F32) { /* :486-489 */
        memcpy(dst, (const float *)w->data + row * cols, sizeof(float) * (size_t)cols);
    } else { /* :490-508 */
        const int8_t *q = (const int8_t *)w->data + row * cols;
        float s = orc_f16_to_f32(w->scale[row]);
        for (int64_t i = 0; i < cols; i++) dst[i] = (float)q[i] * s;
    }
}

static void add_row(float *dst, const tzh_mat_view *w, int64_t row, int64_t cols) {
    if (w->dtype == TZH_F32) { /* :514-517 */
        const float *d = (const float *)w->data + row * cols;
        for (int64_t i = 0; i < cols; i++) dst[i] += d[i];
    } else { /* :518-537 */
        const int8_t *q = (const int8_t *)w->data + row * cols;
        float s = orc_f16_to_f32(w->scale[row]);
        for (int64_t i = 0; i < cols; i++) dst[i] = dst[i] + (float)q[i] * s;
    }
}

void orc_embeddings(float *out, const uint32_t *ids, int64_t L, const tzh_arctic_weights *w) {
    const int64_t h = w->config.hidden_size;
    for (int64_t p = 0; p < L; p++) { /* :553-558 */
        float *row = out + p * h;
        write_row(row, &w->word_embeddings, ids[p], h);
        add_row(row, &w->position_embeddings, p, h);
        add_row(row, &w->token_type_embeddings, 0, h);
    }
    orc_layernorm(out, w->layer_norm_gamma, w->layer_norm_beta, out, L, h,
                  w->config.layer_norm_eps); /* :561-584 */
}

/* ------------------------------------------------------------------ */
/* A5/A6/A7/A9/A11 forward: arctic.zig:599-898                         */
/* ------------------------------------------------------------------ */
typedef struct {
    float *hidden, *q, *k, *v, *scores, *attn_out, *ffn, *tmp, *enc_in, *enc_out, *layer_in;
} orc_ctx; /* InferenceContext, arctic.zig:408-482 */

static int ctx_init(orc_ctx *c, const tzh_arctic_config *cfg, int64_t L) {
    int64_t h = cfg->hidden_size, inter = cfg->intermediate_size;
    c->hidden = malloc(sizeof(float) * L * h);
    c->q = malloc(sizeof(float) * L * h);
    c->k = malloc(sizeof(float) * L * h);
    c->v = malloc(sizeof(float) * L * h);
    c->scores = malloc(sizeof(float) * L * L);
    c->attn_out = malloc(sizeof(float) * L * h);
    c->ffn = malloc(sizeof(float) * L * inter);
    c->tmp = malloc(sizeof(float) * L * h);
    c->enc_in = malloc(sizeof(float) * L * h);
    c->enc_out = malloc(sizeof(float) * L * h);
    c->layer_in = malloc(sizeof(float) * L * h);
    return (c->hidden && c->q && c->k && c->v && c->scores && c->attn_out && c->ffn && c->tmp &&
            c->enc_in && c->enc_out && c->layer_in) ? 0 : -1;
}

static void ctx_free(orc_ctx *c) {
    free(c->hidden); free(c->q); free(c->k); free(c->v); free(c->scores); free(c->attn_out);
    free(c->ffn); free(c->tmp); free(c->enc_in); free(c->enc_out); free(c->layer_in);
}

/* arctic.zig:599-635 */
static void linear(float *out, const float *in, const tzh_mat_view *w, const float *bias,
                   int64_t L, int64_t in_f, int64_t out_f) {
    if (w->dtype == TZH_F32)
        orc_linear_f32(in, (const float *)w->data, bias, out, L, in_f, out_f);
    else
        orc_matmul_w8a32(in, (const int8_t *)w->data, w->scale, bias, out, L, in_f, out_f);
}

/* arctic.zig:639-747 */
static void self_attention(float *output, const float *input, const tzh_attention_weights *aw,
                           const tzh_arctic_config *cfg, orc_ctx *c, int64_t L) {
    const int64_t h = cfg->hidden_size, heads = cfg->num_attention_heads, hd = h / heads;
    linear(c->q, input, &aw->query_weight, aw->query_bias, L, h, h);
    linear(c->k, input, &aw->key_weight, aw->key_bias, L, h, h);
    linear(c->v, input, &aw->value_weight, aw->value_bias, L, h, h);
    for (int64_t hh = 0; hh < heads; hh++)
        orc_attention_head(c->q + hh * hd, c->k + hh * hd, c->v + hh * hd, c->attn_out + hh * hd,
                           L, h, hd, c->scores);
    linear(c->tmp, c->attn_out, &aw->output_weight, aw->output_bias, L, h, h); /* :716 */
    for (int64_t i = 0; i < L * h; i++) output[i] = input[i] + c->tmp[i];     /* :719-721 */
    orc_layernorm(output, aw->output_ln_gamma, aw->output_ln_beta, output, L, h,
                  cfg->layer_norm_eps);
}

/* arctic.zig:760-810 */
static void feed_forward(float *output, const float *input, const tzh_ffn_weights *fw,
                         const tzh_arctic_config *cfg, orc_ctx *c, int64_t L) {
    const int64_t h = cfg->hidden_size, inter = cfg->intermediate_size;
    linear(c->ffn, input, &fw->intermediate_weight, fw->intermediate_bias, L, h, inter);
    for (int64_t i = 0; i < L * inter; i++) c->ffn[i] = orc_gelu(c->ffn[i]);
    linear(c->tmp, c->ffn, &fw->output_weight, fw->output_bias, L, inter, h);
    for (int64_t i = 0; i < L * h; i++) output[i] = input[i] + c->tmp[i];
    orc_layernorm(output, fw->output_ln_gamma, fw->output_ln_beta, output, L, h,
                  cfg->layer_norm_eps);
}

static int check_cfg(const tzh_arctic_weights *w, int64_t L) {
    const tzh_arctic_config *cfg = &w->config;
    if (L <= 0 || L > cfg->max_position_embeddings) return -1;
    if (cfg->hidden_size <= 0 || cfg->num_attention_heads <= 0 ||
        cfg->hidden_size % cfg->num_attention_heads)
        return -1;
    return 0;
}

static void run_encoder(const tzh_arctic_weights *w, const uint32_t *ids, int64_t L,
                        int32_t n_layers, orc_ctx *c) {
    const tzh_arctic_config *cfg = &w->config;
    const int64_t h = cfg->hidden_size;
    orc_embeddings(c->enc_in, ids, L, w); /* :888 */
    const float *input = c->enc_in;
    for (int32_t l = 0; l < n_layers; l++) { /* :830-848 */
        if (l > 0) {
            memcpy(c->layer_in, c->enc_out, sizeof(float) * L * h);
            input = c->layer_in;
        }
        self_attention(c->hidden, input, &w->layers[l].attention, cfg, c, L); /* :822 */
        feed_forward(c->enc_out, c->hidden, &w->layers[l].ffn, cfg, c, L);    /* :825 */
    }
    if (n_layers == 0) memcpy(c->enc_out, c->enc_in, sizeof(float) * L * h);
}

int orc_arctic_forward(const tzh_arctic_weights *w, const uint32_t *ids, int64_t L, float *out) {
    if (check_cfg(w, L)) return -1;
    orc_ctx c;
    if (ctx_init(&c, &w->config, L)) { ctx_free(&c); return -1; }
    const int64_t h = w->config.hidden_size;
    run_encoder(w, ids, L, w->config.num_hidden_layers, &c);
    memcpy(out, c.enc_out, sizeof(float) * h); /* :894 CLS */
    orc_l2_normalize(out, h);                  /* :897 */
    ctx_free(&c);
    return 0;
}

int orc_arctic_hidden(const tzh_arctic_weights *w, const uint32_t *ids, int64_t L,
                      int32_t n_layers_run, float *hidden_out) {
    if (check_cfg(w, L) || n_layers_run < 0 || n_layers_run > w->config.num_hidden_layers)
        return -1;
    orc_ctx c;
    if (ctx_init(&c, &w->config, L)) { ctx_free(&c); return -1; }
    run_encoder(w, ids, L, n_layers_run, &c);
    memcpy(hidden_out, c.enc_out, sizeof(float) * L * w->config.hidden_size);
    ctx_free(&c);
    return 0;
}

int orc_arctic_forward_batch(const tzh_arctic_weights *w, const uint32_t *ids,
                             const int64_t *offsets, const int32_t *lengths, int32_t batch,
                             float *out, int32_t nthreads) {
    if (batch <= 0) return 0; /* :967 */
    const int64_t h = w->config.hidden_size;
    int32_t threads = nthreads < 1 ? 1 : nthreads;
    if (threads > batch) threads = batch;          /* threading.zig:142 */
    int32_t per = (batch + threads - 1) / threads; /* threading.zig:143 */
    int err = 0;
#pragma omp parallel num_threads(threads) reduction(| : err)
    {
        int t = 0;
#ifdef _OPENMP
        t = omp_get_thread_num();
#endif
        int32_t b0 = t * per, b1 = b0 + per;
        if (b1 > batch) b1 = batch;
        for (int32_t b = b0; b < b1; b++)
            err |= orc_arctic_forward(w, ids + offsets[b], lengths[b], out + (int64_t)b * h) ? 1 : 0;
    }
    return err ? -1 : 0;
}

/* ------------------------------------------------------------------ */
/* Elementwise op semantics: simd.zig:107-315, elementwise.zig:124-207 */
/* ------------------------------------------------------------------ */
static inline float sigmoid_f(float x) { return 1.0f / (1.0f + expf(-x)); }      /* simd.zig:279-281 */
static inline float tanh_f(float x) { return 2.0f * sigmoid_f(2.0f * x) - 1.0f; } /* simd.zig:266-269 */
static inline double sigmoid_d(double x) { return 1.0 / (1.0 + exp(-x)); }
static inline double tanh_d(double x) { return 2.0 * sigmoid_d(2.0 * x) - 1.0; }

static int unary_supported(int32_t op) {
    switch (op) { /* elementwise.zig:148-168 */
    case TZH_OP_NEG: case TZH_OP_ABS: case TZH_OP_EXP: case TZH_OP_LOG: case TZH_OP_SQRT:
    case TZH_OP_RSQRT: case TZH_OP_SIN: case TZH_OP_COS: case TZH_OP_TANH: case TZH_OP_SIGMOID:
    case TZH_OP_RELU: case TZH_OP_GELU: case TZH_OP_SILU: case TZH_OP_SOFTPLUS:
    case TZH_OP_FLOOR: case TZH_OP_CEIL: case TZH_OP_ROUND:
        return 1;
    default:
        return 0;
    }
}

static int binary_supported(int32_t op) {
    switch (op) { /* elementwise.zig:196-207 */
    case TZH_OP_ADD: case TZH_OP_SUB: case TZH_OP_MUL: case TZH_OP_DIV: case TZH_OP_POW:
    case TZH_OP_MAX: case TZH_OP_MIN:
        return 1;
    default:
        return 0;
    }
}

static int reduce_supported(int32_t op) {
    switch (op) { /* reduce.zig:188-196 */
    case TZH_OP_SUM: case TZH_OP_MEAN: case TZH_OP_PROD: case TZH_OP_REDUCE_MAX:
    case TZH_OP_REDUCE_MIN:
        return 1;
    default:
        return 0;
    }
}

float orc_unary_f32(int32_t op, float x) {
    switch (op) {
    case TZH_OP_NEG: return -x;
    case TZH_OP_ABS: return fabsf(x);
    case TZH_OP_EXP: return expf(x);
    case TZH_OP_LOG: return logf(x);
    case TZH_OP_SQRT: return sqrtf(x);
    case TZH_OP_RSQRT: return 1.0f / sqrtf(x);
    case TZH_OP_SIN: return sinf(x);
    case TZH_OP_COS: return cosf(x);
    case TZH_OP_TANH: return tanh_f(x);
    case TZH_OP_SIGMOID: return sigmoid_f(x);
    case TZH_OP_RELU: return fmaxf(x, 0.0f);
    case TZH_OP_GELU: { /* simd.zig:283-290 */
        const float k0 = (float)0.7978845608028654, k1 = 0.044715f;
        float x3 = x * x * x;
        float inner = k0 * (x + k1 * x3);
        return 0.5f * x * (1.0f + tanh_f(inner));
    }
    case TZH_OP_SILU: return x * sigmoid_f(x);
    case TZH_OP_SOFTPLUS: return logf(1.0f + expf(x));
    case TZH_OP_FLOOR: return floorf(x);
    case TZH_OP_CEIL: return ceilf(x);
    case TZH_OP_ROUND: return roundf(x);
    default: return NAN;
    }
}

double orc_unary_f64(int32_t op, double x) {
    switch (op) {
    case TZH_OP_NEG: return -x;
    case TZH_OP_ABS: return fabs(x);
    case TZH_OP_EXP: return exp(x);
    case TZH_OP_LOG: return log(x);
    case TZH_OP_SQRT: return sqrt(x);
    case TZH_OP_RSQRT: return 1.0 / sqrt(x);
    case TZH_OP_SIN: return sin(x);
    case TZH_OP_COS: return cos(x);
    case TZH_OP_TANH: return tanh_d(x);
    case TZH_OP_SIGMOID: return sigmoid_d(x);
    case TZH_OP_RELU: return fmax(x, 0.0);
    case TZH_OP_GELU: {
        const double k0 = 0.7978845608028654, k1 = 0.044715;
        double x3 = x * x * x;
        double inner = k0 * (x + k1 * x3);
        return 0.5 * x * (1.0 + tanh_d(inner));
    }
    case TZH_OP_SILU: return x * sigmoid_d(x);
    case TZH_OP_SOFTPLUS: return log(1.0 + exp(x));
    case TZH_OP_FLOOR: return floor(x);
    case TZH_OP_CEIL: return ceil(x);
    case TZH_OP_ROUND: return round(x);
    default: return NAN;
    }
}

float orc_binary_f32(int32_t op, float a, float b) {
    switch (op) {
    case TZH_OP_ADD: return a + b;
    case TZH_OP_SUB: return a - b;
    case TZH_OP_MUL: return a * b;
    case TZH_OP_DIV: return a / b;
    case TZH_OP_POW: return powf(a, b);
    case TZH_OP_MAX: return fmaxf(a, b);
    case TZH_OP_MIN: return fminf(a, b);
    default: return NAN;
    }
}

double orc_binary_f64(int32_t op, double a, double b) {
    switch (op) {
    case TZH_OP_ADD: return a + b;
    case TZH_OP_SUB: return a - b;
    case TZH_OP_MUL: return a * b;
    case TZH_OP_DIV: return a / b;
    case TZH_OP_POW: return pow(a, b);
    case TZH_OP_MAX: return fmax(a, b);
    case TZH_OP_MIN: return fmin(a, b);
    default: return NAN;
    }
}

/* ------------------------------------------------------------------ */
/* A12-A15 executor: executor.zig:29-196, 327-360; reduce.zig:13-96    */
/* ------------------------------------------------------------------ */
static int64_t numel_of(int32_t ndim, const int64_t *shape) {
    int64_t n = 1;
    for (int32_t i = 0; i < ndim; i++) n *= shape[i];
    return n;
}

static int same_shape(int32_t na, const int64_t *a, int32_t nb, const int64_t *b) {
    if (na != nb) return 0;
    for (int32_t i = 0; i < na; i++)
        if (a[i] != b[i]) return 0;
    return 1;
}

typedef struct {
    const tzh_node *tape;
    int32_t n_nodes;
    const tzh_leaf *leaves;
    int32_t n_leaves;
    int32_t dtype;
    size_t es;
} eval_env;

static int eval_node(const eval_env *env, int32_t idx, void *out);

/* executor.zig:551-578: leaves are used in place, everything else is
 * evaluated into a fresh temporary. */
static int input_data(const eval_env *env, int32_t idx, const void **data, void **owned) {
    const tzh_node *n = &env->tape[idx];
    *owned = NULL;
    if (n->kind == TZH_NODE_TENSOR) {
        *data = env->leaves[n->leaf].data;
        return 0;
    }
    size_t bytes = (size_t)numel_of(n->ndim, n->shape) * env->es;
    void *buf = malloc(bytes ? bytes : env->es);
    if (!buf) return TZH_ERR_OUT_OF_MEMORY;
    int rc = eval_node(env, idx, buf);
    if (rc) { free(buf); return rc; }
    *data = buf;
    *owned = buf;
    return 0;
}

/* strides.zig:92-121 broadcast strides of src into an out of rank `ond` */
static void bcast_strides(int32_t snd, const int64_t *sshape, int32_t ond, int64_t *st) {
    int64_t cs[TZH_MAX_RANK];
    int64_t s = 1;
    for (int32_t i = snd - 1; i >= 0; i--) { cs[i] = s; s *= sshape[i]; }
    for (int32_t i = 0; i < ond; i++) {
        int32_t si = i - (ond - snd);
        st[i] = (si >= 0 && sshape[si] != 1) ? cs[si] : 0;
    }
}

static int check_broadcast(const tzh_node *n, const tzh_node *l, const tzh_node *r) {
    int32_t nd = l->ndim > r->ndim ? l->ndim : r->ndim; /* shape.zig:168-204 */
    if (n->ndim != nd) return TZH_ERR_SHAPE;
    for (int32_t i = 0; i < nd; i++) {
        int64_t a = (i - (nd - l->ndim) >= 0) ? l->shape[i - (nd - l->ndim)] : 1;
        int64_t b = (i - (nd - r->ndim) >= 0) ? r->shape[i - (nd - r->ndim)] : 1;
        if (a != b && a != 1 && b != 1) return TZH_ERR_SHAPE;
        if (n->shape[i] != (a > b ? a : b)) return TZH_ERR_SHAPE;
        /* @max(0, 1) = 1: the result has an element the empty operand
           cannot supply; executor.zig:139-144 would index past its slice
           (a bounds panic in a safe build), so this is an error here */
        if ((a == 0 || b == 0) && n->shape[i] != 0) return TZH_ERR_SHAPE;
    }
    return 0;
}

#define DEF_APPLY(T, SUF)                                                                       \
    static void unary_##SUF(int32_t op, const T *in, T *out, int64_t n) {                        \
        for (int64_t i = 0; i < n; i++) out[i] = orc_unary_##SUF(op, in[i]);                     \
    }                                                                                          \
    static void binary_##SUF(const tzh_node *nd, const tzh_node *ln, const tzh_node *rn,         \
                             const T *l, const T *r, T *out) {                                  \
        int64_t on = numel_of(nd->ndim, nd->shape);                                             \
        int64_t lnum = numel_of(ln->ndim, ln->shape), rnum = numel_of(rn->ndim, rn->shape);      \
        int32_t op = nd->op;                                                                    \
        if (lnum == rnum && lnum == on) { /* executor.zig:136-138 */                             \
            for (int64_t i = 0; i < on; i++) out[i] = orc_binary_##SUF(op, l[i], r[i]);          \
        } else if (lnum == 1) { /* :139-141 */                                                  \
            for (int64_t i = 0; i < on; i++) out[i] = orc_binary_##SUF(op, l[0], r[i]);          \
        } else if (rnum == 1) { /* :142-144 */                                                  \
            for (int64_t i = 0; i < on; i++) out[i] = orc_binary_##SUF(op, l[i], r[0]);          \
        } else { /* :145-196 general broadcast */                                               \
            int64_t ls[TZH_MAX_RANK], rs[TZH_MAX_RANK];                                         \
            bcast_strides(ln->ndim, ln->shape, nd->ndim, ls);                                   \
            bcast_strides(rn->ndim, rn->shape, nd->ndim, rs);                                   \
            for (int64_t f = 0; f < on; f++) {                                                  \
                int64_t rem = f, lo = 0, ro = 0;                                                \
                for (int32_t d = nd->ndim - 1; d >= 0; d--) {                                   \
                    int64_t ix = rem % nd->shape[d];                                            \
                    rem /= nd->shape[d];                                                        \
                    lo += ix * ls[d];                                                           \
                    ro += ix * rs[d];                                                           \
                }                                                                               \
                out[f] = orc_binary_##SUF(op, l[lo], r[ro]);                                    \
            }                                                                                   \
        }                                                                                       \
    }                                                                                          \
    static T red_ident_##SUF(int32_t op) {                                                       \
        switch (op) {                                                                           \
        case TZH_OP_PROD: return (T)1;                                                          \
        case TZH_OP_REDUCE_MAX: return (T)-INFINITY;                                            \
        case TZH_OP_REDUCE_MIN: return (T)INFINITY;                                             \
        default: return (T)0;                                                                   \
        }                                                                                       \
    }                                                                                          \
    static T red_apply_##SUF(int32_t op, T acc, T v) {                                           \
        switch (op) {                                                                           \
        case TZH_OP_PROD: return acc * v;                                                       \
        case TZH_OP_REDUCE_MAX: return orc_binary_##SUF(TZH_OP_MAX, acc, v);                    \
        case TZH_OP_REDUCE_MIN: return orc_binary_##SUF(TZH_OP_MIN, acc, v);                    \
        default: return acc + v;                                                                \
        }                                                                                       \
    }                                                                                          \
    /* reduce.zig:13-48 (vector lanes, ordered lane combine, remainder, mean) */                 \
    static T reduce_all_##SUF(int32_t op, const T *in, int64_t n) {                              \
        if (n == 0) return red_ident_##SUF(op);                                                 \
        enum { L_ = 64 / sizeof(T) };                                                           \
        T acc[L_];                                                                              \
        for (int l = 0; l < L_; l++) acc[l] = red_ident_##SUF(op);                              \
        int64_t i = 0;                                                                          \
        for (; i + L_ <= n; i += L_)                                                            \
            for (int l = 0; l < L_; l++) acc[l] = red_apply_##SUF(op, acc[l], in[i + l]);       \
        T a = acc[0];                                                                           \
        for (int l = 1; l < L_; l++) a = red_apply_##SUF(op, a, acc[l]);                        \
        for (; i < n; i++) a = red_apply_##SUF(op, a, in[i]);                                   \
        if (op == TZH_OP_MEAN) a = a / (T)n;                                                    \
        return a;                                                                               \
    }                                                                                          \
    /* reduce.zig:52-95 */                                                                      \
    static void reduce_axis_##SUF(int32_t op, const T *in, T *out, int32_t ndim,                \
                                  const int64_t *shape, int32_t axis) {                         \
        int64_t outer = 1, inner = 1, rsz = shape[axis];                                        \
        for (int32_t i = 0; i < axis; i++) outer *= shape[i];                                   \
        for (int32_t i = axis + 1; i < ndim; i++) inner *= shape[i];                            \
        for (int64_t o = 0; o < outer; o++)                                                     \
            for (int64_t in_ = 0; in_ < inner; in_++) {                                         \
                T acc = red_ident_##SUF(op);                                                    \
                for (int64_t r = 0; r < rsz; r++)                                               \
                    acc = red_apply_##SUF(op, acc, in[o * rsz * inner + r * inner + in_]);      \
                if (op == TZH_OP_MEAN) acc = acc / (T)rsz;                                      \
                out[o * inner + in_] = acc;                                                     \
            }                                                                                   \
    }

DEF_APPLY(float, f32)
DEF_APPLY(double, f64)

static int eval_node(const eval_env *env, int32_t idx, void *out) {
    const tzh_node *n = &env->tape[idx];
    const int is64 = env->dtype == TZH_F64;
    int64_t on = numel_of(n->ndim, n->shape);
    if (n->ndim < 0 || n->ndim > TZH_MAX_RANK) return TZH_ERR_SHAPE;
    switch (n->kind) {
    case TZH_NODE_TENSOR: { /* executor.zig:57-60 */
        if (n->leaf < 0 || n->leaf >= env->n_leaves) return TZH_ERR_INVALID_ARGS;
        const tzh_leaf *lf = &env->leaves[n->leaf];
        if (!same_shape(lf->ndim, lf->shape, n->ndim, n->shape)) return TZH_ERR_SHAPE;
        memcpy(out, lf->data, (size_t)on * env->es);
        return 0;
    }
    case TZH_NODE_CONSTANT: /* executor.zig:61-64 */
        for (int64_t i = 0; i < on; i++) {
            if (is64) ((double *)out)[i] = n->value;
            else ((float *)out)[i] = (float)n->value;
        }
        return 0;
    case TZH_NODE_UNARY: { /* executor.zig:95-111 */
        if (!unary_supported(n->op)) return TZH_ERR_UNSUPPORTED_OP;
        if (n->lhs < 0 || n->lhs >= idx) return TZH_ERR_INVALID_ARGS;
        const tzh_node *c = &env->tape[n->lhs];
        if (!same_shape(c->ndim, c->shape, n->ndim, n->shape)) return TZH_ERR_SHAPE;
        const void *d; void *own;
        int rc = input_data(env, n->lhs, &d, &own);
        if (rc) return rc;
        if (is64) unary_f64(n->op, (const double *)d, (double *)out, on);
        else unary_f32(n->op, (const float *)d, (float *)out, on);
        free(own);
        return 0;
    }
    case TZH_NODE_BINARY: { /* executor.zig:113-196 */
        if (!binary_supported(n->op)) return TZH_ERR_UNSUPPORTED_OP;
        if (n->lhs < 0 || n->lhs >= idx || n->rhs < 0 || n->rhs >= idx) return TZH_ERR_INVALID_ARGS;
        const tzh_node *l = &env->tape[n->lhs], *r = &env->tape[n->rhs];
        int rc = check_broadcast(n, l, r);
        if (rc) return rc;
        const void *ld, *rd; void *lo, *ro;
        rc = input_data(env, n->lhs, &ld, &lo);
        if (rc) return rc;
        rc = input_data(env, n->rhs, &rd, &ro);
        if (rc) { free(lo); return rc; }
        if (is64) binary_f64(n, l, r, (const double *)ld, (const double *)rd, (double *)out);
        else binary_f32(n, l, r, (const float *)ld, (const float *)rd, (float *)out);
        free(lo);
        free(ro);
        return 0;
    }
    case TZH_NODE_REDUCE: { /* executor.zig:326-360 */
        if (!reduce_supported(n->op)) return TZH_ERR_UNSUPPORTED_OP;
        if (n->lhs < 0 || n->lhs >= idx) return TZH_ERR_INVALID_ARGS;
        const tzh_node *c = &env->tape[n->lhs];
        if (n->axis < -1 || n->axis >= c->ndim) return TZH_ERR_SHAPE;
        const void *d; void *own;
        int rc = input_data(env, n->lhs, &d, &own);
        if (rc) return rc;
        int64_t cn = numel_of(c->ndim, c->shape);
        if (n->axis < 0) {
            if (is64) ((double *)out)[0] = reduce_all_f64(n->op, (const double *)d, cn);
            else ((float *)out)[0] = reduce_all_f32(n->op, (const float *)d, cn);
            for (int64_t i = 1; i < on; i++) { /* keepdims all-ones shape holds one value */
                if (is64) ((double *)out)[i] = ((double *)out)[0];
                else ((float *)out)[i] = ((float *)out)[0];
            }
        } else {
            if (is64) reduce_axis_f64(n->op, (const double *)d, (double *)out, c->ndim, c->shape, n->axis);
            else reduce_axis_f32(n->op, (const float *)d, (float *)out, c->ndim, c->shape, n->axis);
        }
        free(own);
        return 0;
    }
    default:
        return TZH_ERR_UNSUPPORTED_OP;
    }
}

int orc_eval(const tzh_node *tape, int32_t n_nodes, const tzh_leaf *leaves, int32_t n_leaves,
             int32_t dtype, void *out) {
    if (!tape || n_nodes <= 0 || !out) return TZH_ERR_INVALID_ARGS;
    if (dtype != TZH_F32 && dtype != TZH_F64) return TZH_ERR_UNSUPPORTED_DTYPE;
    eval_env env = {tape, n_nodes, leaves, n_leaves, dtype, dtype == TZH_F64 ? 8u : 4u};
    return eval_node(&env, n_nodes - 1, out);
}

void orc_chain_add_mul_exp(const float *a, const float *b_row, const float *c, float *out,
                           int64_t rows, int64_t cols, float *tmp1, float *tmp2) {
    /* pass 1: t2 = a + b (general broadcast path, executor.zig:152-196) */
    for (int64_t i = 0; i < rows; i++)
        for (int64_t j = 0; j < cols; j++) tmp2[i * cols + j] = a[i * cols + j] + b_row[j];
    /* pass 2: t1 = t2 * c (elementwise.zig:39-65) */
    for (int64_t i = 0; i < rows * cols; i++) tmp1[i] = tmp2[i] * c[i];
    /* pass 3: out = exp(t1) (elementwise.zig:13-36) */
    for (int64_t i = 0; i < rows * cols; i++) out[i] = expf(tmp1[i]);
}

void orc_unary_vec_f32(int32_t op, const float *x, float *y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = orc_unary_f32(op, x[i]);
}

void orc_binary_vec_f32(int32_t op, const float *a, const float *b, float *y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = orc_binary_f32(op, a[i], b[i]);
}

void orc_gelu_vec(const float *x, float *y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = orc_gelu(x[i]);
}
