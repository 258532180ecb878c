/*
 * moonlight_oracle.c -- CPU restatement of floyd's quantized Moonlight path.
 * TEST INFRASTRUCTURE ONLY (see moonlight_oracle.h): the product never calls it.
 *
 * Build: oracle/Makefile (gcc -O3 -march=x86-64-v3 -fopenmp -ffp-contract=off).
 */
#include "moonlight_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------ */
/* synthetic inputs                                                          */
/* ------------------------------------------------------------------------ */

uint64_t orc_splitmix64_at(uint64_t seed, uint64_t k) {
    uint64_t z = seed + (k + 1) * 0x9E3779B97F4A7C15ULL;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

float orc_bf16_round(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7F800000u) == 0x7F800000u) return x; /* inf / nan unchanged */
    u += 0x7FFFu + ((u >> 16) & 1u);                 /* round to nearest even */
    u &= 0xFFFF0000u;
    memcpy(&x, &u, 4);
    return x;
}

void orc_fill_normal(float *out, int64_t n, uint64_t seed, double mean,
                     double std, int bf16) {
    const double two_pi = 6.283185307179586476925286766559;
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        uint64_t a = orc_splitmix64_at(seed, 2 * (uint64_t)i);
        uint64_t b = orc_splitmix64_at(seed, 2 * (uint64_t)i + 1);
        double u1 = ((double)(a >> 11) + 1.0) * 0x1.0p-53; /* (0, 1] */
        double u2 = (double)(b >> 11) * 0x1.0p-53;         /* [0, 1) */
        double z = sqrt(-2.0 * log(u1)) * cos(two_pi * u2);
        float v = (float)(mean + std * z);
        out[i] = bf16 ? orc_bf16_round(v) : v;
    }
}

/* ------------------------------------------------------------------------ */
/* packing: tools/convert_moonlight.py:46-66                                */
/* numpy float32 semantics: amax/qmax and w/s are f32 IEEE ops, np.maximum   */
/* against the weak python float 1e-8 (-> 1e-8f), np.rint = round-half-even. */
/* ------------------------------------------------------------------------ */

static float row_scale(const float *w, int cols, float qmax) {
    float amax = 0.0f;
    for (int c = 0; c < cols; ++c) {
        float a = fabsf(w[c]);
        if (a > amax) amax = a;
    }
    float s = amax / qmax;
    return s > 1e-8f ? s : 1e-8f;
}

void orc_quant_int8(const float *w, int rows, int cols, uint8_t *q, float *s) {
    #pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) {
        const float *row = w + (int64_t)r * cols;
        float scale = row_scale(row, cols, 127.0f);
        s[r] = scale;
        for (int c = 0; c < cols; ++c) {
            float v = rintf(row[c] / scale);
            if (v < -128.0f) v = -128.0f;
            if (v > 127.0f) v = 127.0f;
            q[(int64_t)r * cols + c] = (uint8_t)(int8_t)v;
        }
    }
}

void orc_quant_int4(const float *w, int rows, int cols, uint8_t *q, float *s) {
    int row_bytes = (cols + 1) / 2;
    #pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) {
        const float *row = w + (int64_t)r * cols;
        uint8_t *dst = q + (int64_t)r * row_bytes;
        float scale = row_scale(row, cols, 7.0f);
        s[r] = scale;
        memset(dst, 0, (size_t)row_bytes);
        for (int c = 0; c < cols; ++c) {
            float v = rintf(row[c] / scale);
            if (v < -8.0f) v = -8.0f;
            if (v > 7.0f) v = 7.0f;
            uint8_t nib = (uint8_t)((int)v + 8);
            dst[c / 2] |= (c & 1) ? (uint8_t)(nib << 4) : nib;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* matmul: moonlight_kernels.metal:43-130, the tests' serial reference       */
/* (tests/test_moonlight_metal_primitives.c:33-74): f32 serial sum, scale    */
/* applied once after the sum.                                               */
/* ------------------------------------------------------------------------ */

static float dot_row(int fmt, const void *w, int o, const float *x, int in_width) {
    float sum = 0.0f;
    if (fmt == 0) {
        const float *row = (const float *)w + (int64_t)o * in_width;
        for (int i = 0; i < in_width; ++i) sum += x[i] * row[i];
    } else if (fmt == 1) {
        const int8_t *row = (const int8_t *)w + (int64_t)o * in_width;
        for (int i = 0; i < in_width; ++i) sum += x[i] * (float)row[i];
    } else {
        int row_bytes = (in_width + 1) / 2;
        const uint8_t *row = (const uint8_t *)w + (int64_t)o * row_bytes;
        for (int i = 0; i < in_width; ++i) {
            uint8_t packed = row[i / 2];
            int value = (i & 1) ? (packed >> 4) - 8 : (packed & 15) - 8;
            sum += x[i] * (float)value;
        }
    }
    return sum;
}

void orc_matmul(int fmt, const void *w, const float *s, const float *x,
                float *y, int out_width, int in_width, int rows, int threads) {
    int64_t total = (int64_t)rows * out_width;
#ifdef _OPENMP
    if (threads < 1) threads = 1;
    #pragma omp parallel for schedule(static) num_threads(threads)
#else
    (void)threads;
#endif
    for (int64_t idx = 0; idx < total; ++idx) {
        int r = (int)(idx / out_width);
        int o = (int)(idx % out_width);
        float sum = dot_row(fmt, w, o, x + (int64_t)r * in_width, in_width);
        y[idx] = fmt == 0 ? sum : sum * s[o];
    }
}

int orc_detect_format(int64_t byte_count, int out_width, int in_width) {
    if (byte_count == (int64_t)out_width * in_width) return 1;
    if (byte_count == (int64_t)out_width * ((in_width + 1) / 2)) return 2;
    return -1;
}

/* Dequantised element, moonlight_kernels.metal:202-216: q * s[row]. */
static float weight_value(int fmt, const void *w, const float *s, int row,
                          int col, int width) {
    if (fmt == 0) return ((const float *)w)[(int64_t)row * width + col];
    if (fmt == 1)
        return (float)((const int8_t *)w)[(int64_t)row * width + col] * s[row];
    int row_bytes = (width + 1) / 2;
    uint8_t packed = ((const uint8_t *)w)[(int64_t)row * row_bytes + col / 2];
    int value = (col & 1) ? (packed >> 4) - 8 : (packed & 15) - 8;
    return (float)value * s[row];
}

/* ------------------------------------------------------------------------ */
/* elementwise: rmsnorm (moonlight_kernels.metal:23-41, the tests'           */
/* rmsnorm_reference at tests/test_moonlight_metal_mla.c:77-90), RoPE        */
/* (moonlight_kernels.metal:132-200, rope_reference at :92-108), SiLU        */
/* (moonlight_kernels.metal:533-541).                                        */
/* ------------------------------------------------------------------------ */

void orc_rmsnorm(const float *x, const float *w, float *y, int rows, int width,
                 float eps) {
    for (int r = 0; r < rows; ++r) {
        const float *src = x + (int64_t)r * width;
        float sum = 0.0f;
        for (int c = 0; c < width; ++c) sum += src[c] * src[c];
        float scale = 1.0f / sqrtf(sum / (float)width + eps);
        for (int c = 0; c < width; ++c)
            y[(int64_t)r * width + c] = src[c] * scale * w[c];
    }
}

float orc_rope_inv_freq(float theta, int pair, int width) {
    return powf(theta, -2.0f * (float)pair / (float)width);
}

void orc_rope(const float *in, float *out, int width, int position,
              float theta) {
    int half = width / 2;
    for (int p = 0; p < half; ++p) {
        float angle = (float)position * orc_rope_inv_freq(theta, p, width);
        float c = cosf(angle), s = sinf(angle);
        float first = in[2 * p], second = in[2 * p + 1];
        out[p] = first * c - second * s;
        out[half + p] = second * c + first * s;
    }
}

float orc_silu_mul(float gate, float up) {
    return gate / (1.0f + expf(-gate)) * up;
}

/* ------------------------------------------------------------------------ */
/* routing: moonlight_route_sigmoid_topk (moonlight_kernels.metal:469-512)   */
/* = moe_route_select + moe_route_finalize (moe_route.h:47-99) with          */
/* MOE_SCORE_SIGMOID: bias for selection only, strict '>' so the lower      */
/* index wins ties, weights from unbiased scores, /(sum + 1e-20) then        */
/* * routed_scale.                                                           */
/* ------------------------------------------------------------------------ */

/* Router score 1 / (1 + e^-x) with e^-x correctly rounded to f32 (exp in
 * double, rounded once).  moe_route.h:12-14 calls glibc expf, which is not
 * correctly rounded for about 0.06 % of inputs (measured over [-12, 12]):
 * there the two scores differ by one ulp.  Selection ids are unaffected unless
 * two selection scores tie within that ulp; weights may differ by a few ulp. */
static float route_sigmoid(float x) {
    return 1.0f / (1.0f + (float)exp(-(double)x));
}

void orc_route_sigmoid_topk(const float *logits, const float *bias, int rows,
                            int experts, int top_k, int normalize,
                            float routed_scale, int *ids, float *weights) {
    float scores[1024];
    for (int r = 0; r < rows; ++r) {
        const float *lg = logits + (int64_t)r * experts;
        int *id = ids + (int64_t)r * top_k;
        float *wt = weights + (int64_t)r * top_k;
        for (int e = 0; e < experts; ++e) scores[e] = route_sigmoid(lg[e]);
        for (int k = 0; k < top_k; ++k) {
            int best = -1;
            float best_value = -INFINITY;
            for (int e = 0; e < experts; ++e) {
                int taken = 0;
                for (int j = 0; j < k; ++j) taken |= id[j] == e;
                float v = scores[e] + (bias ? bias[e] : 0.0f);
                if (!taken && v > best_value) {
                    best = e;
                    best_value = v;
                }
            }
            id[k] = best;
            wt[k] = best >= 0 ? scores[best] : 0.0f;
        }
        float denom = 1.0f;
        if (normalize) {
            float sum = 0.0f;
            for (int k = 0; k < top_k; ++k) sum += wt[k];
            denom = sum + 1e-20f;
        }
        for (int k = 0; k < top_k; ++k) wt[k] = wt[k] / denom * routed_scale;
    }
}

int orc_route_tables(const int *ids, int rows, int top_k, int experts,
                     int max_batch, int *unique, int *counts, int *expert_rows,
                     int *expert_slots) {
    unsigned char seen[1024] = {0};
    int n_unique = 0;
    memset(counts, 0, (size_t)experts * sizeof(int));
    for (int r = 0; r < rows; ++r) {
        for (int k = 0; k < top_k; ++k) {
            int e = ids[(int64_t)r * top_k + k];
            if (e < 0 || e >= experts) return -1;
            if (!seen[e]) {
                seen[e] = 1;
                unique[n_unique++] = e;
            }
            int j = counts[e]++;
            expert_rows[(int64_t)e * max_batch + j] = r;
            expert_slots[(int64_t)e * max_batch + j] = k;
        }
    }
    return n_unique;
}

/* ------------------------------------------------------------------------ */
/* named-tensor model                                                        */
/* ------------------------------------------------------------------------ */

typedef struct {
    char *name;
    int dtype;
    const void *data;
    int64_t numel, nbytes;
} OrcTensor;

struct OrcModel {
    OrcConfig cfg;
    int context_size;
    OrcTensor *tensors;
    int count, cap;
    int *hash;
    int hash_cap;
    float *latent_kv; /* [layers][ctx][kv_lora_rank] */
    float *rope_kv;   /* [layers][ctx][qk_rope_dim]  */
    int *kv_lengths;
    int position;
};

static uint64_t name_hash(const char *s) {
    uint64_t h = 1469598103934665603ULL;
    while (*s) {
        h ^= (unsigned char)*s++;
        h *= 1099511628211ULL;
    }
    return h;
}

static void rehash(OrcModel *m) {
    free(m->hash);
    m->hash_cap = 64;
    while (m->hash_cap < m->count * 2 + 2) m->hash_cap <<= 1;
    m->hash = malloc((size_t)m->hash_cap * sizeof(int));
    for (int i = 0; i < m->hash_cap; ++i) m->hash[i] = -1;
    for (int i = 0; i < m->count; ++i) {
        uint64_t h = name_hash(m->tensors[i].name) & (uint64_t)(m->hash_cap - 1);
        while (m->hash[h] >= 0) h = (h + 1) & (uint64_t)(m->hash_cap - 1);
        m->hash[h] = i;
    }
}

static const OrcTensor *find(const OrcModel *m, const char *name) {
    if (!m->hash) return NULL;
    uint64_t h = name_hash(name) & (uint64_t)(m->hash_cap - 1);
    while (m->hash[h] >= 0) {
        const OrcTensor *t = &m->tensors[m->hash[h]];
        if (!strcmp(t->name, name)) return t;
        h = (h + 1) & (uint64_t)(m->hash_cap - 1);
    }
    return NULL;
}

OrcModel *orc_model_create(const OrcConfig *config, int context_size) {
    OrcModel *m = calloc(1, sizeof(*m));
    if (!m) return NULL;
    m->cfg = *config;
    m->context_size = context_size;
    size_t lat = (size_t)config->layer_count * context_size * config->kv_lora_rank;
    size_t rope = (size_t)config->layer_count * context_size * config->qk_rope_dim;
    m->latent_kv = calloc(lat, sizeof(float));
    m->rope_kv = calloc(rope, sizeof(float));
    m->kv_lengths = calloc((size_t)config->layer_count, sizeof(int));
    if (!m->latent_kv || !m->rope_kv || !m->kv_lengths) {
        orc_model_destroy(m);
        return NULL;
    }
    return m;
}

void orc_model_destroy(OrcModel *m) {
    if (!m) return;
    for (int i = 0; i < m->count; ++i) free(m->tensors[i].name);
    free(m->tensors);
    free(m->hash);
    free(m->latent_kv);
    free(m->rope_kv);
    free(m->kv_lengths);
    free(m);
}

int orc_model_add_tensor(OrcModel *m, const char *name, int dtype,
                         const void *data, int64_t numel, int64_t nbytes) {
    if (!m || !name || !data) return 0;
    if (m->count == m->cap) {
        int cap = m->cap ? m->cap * 2 : 256;
        OrcTensor *t = realloc(m->tensors, (size_t)cap * sizeof(OrcTensor));
        if (!t) return 0;
        m->tensors = t;
        m->cap = cap;
    }
    OrcTensor *t = &m->tensors[m->count++];
    t->name = strdup(name);
    t->dtype = dtype;
    t->data = data;
    t->numel = numel;
    t->nbytes = nbytes;
    if (m->count * 2 + 2 > m->hash_cap) rehash(m);
    else {
        uint64_t h = name_hash(name) & (uint64_t)(m->hash_cap - 1);
        while (m->hash[h] >= 0) h = (h + 1) & (uint64_t)(m->hash_cap - 1);
        m->hash[h] = m->count - 1;
    }
    return 1;
}

void orc_model_reset(OrcModel *m) {
    memset(m->kv_lengths, 0, (size_t)m->cfg.layer_count * sizeof(int));
    m->position = 0;
}

int orc_model_kv_length(const OrcModel *m, int layer) {
    if (!m || layer < 0 || layer >= m->cfg.layer_count) return 0;
    return m->kv_lengths[layer];
}

int orc_model_set_kv(OrcModel *m, int layer, const float *latent,
                     const float *rope, int length) {
    if (!m || layer < 0 || layer >= m->cfg.layer_count || length < 0 ||
        length > m->context_size) return 0;
    size_t lw = (size_t)m->cfg.kv_lora_rank, rw = (size_t)m->cfg.qk_rope_dim;
    memcpy(m->latent_kv + (size_t)layer * m->context_size * lw, latent,
           (size_t)length * lw * sizeof(float));
    memcpy(m->rope_kv + (size_t)layer * m->context_size * rw, rope,
           (size_t)length * rw * sizeof(float));
    m->kv_lengths[layer] = length;
    if (m->position < length) m->position = length;
    return 1;
}

int orc_model_copy_kv(const OrcModel *m, int layer, float *latent, float *rope,
                      int capacity) {
    if (!m || layer < 0 || layer >= m->cfg.layer_count ||
        capacity < m->kv_lengths[layer]) return 0;
    size_t lw = (size_t)m->cfg.kv_lora_rank, rw = (size_t)m->cfg.qk_rope_dim;
    int n = m->kv_lengths[layer];
    memcpy(latent, m->latent_kv + (size_t)layer * m->context_size * lw,
           (size_t)n * lw * sizeof(float));
    memcpy(rope, m->rope_kv + (size_t)layer * m->context_size * rw,
           (size_t)n * rw * sizeof(float));
    return 1;
}

/* resolve_matrix (moonlight_metal.m:129-162). */
typedef struct {
    int fmt;
    const void *w;
    const float *s;
} OrcMatrix;

static int resolve(const OrcModel *m, const char *name, int in_width,
                   int out_width, OrcMatrix *mat) {
    char scale_name[600];
    const OrcTensor *t = find(m, name);
    if (!t) return 0;
    mat->w = t->data;
    mat->s = NULL;
    if (t->dtype == 2) {
        if (t->numel != (int64_t)in_width * out_width) return 0;
        mat->fmt = 0;
        return 1;
    }
    if (t->dtype != 3) return 0;
    snprintf(scale_name, sizeof(scale_name), "%s.qs", name);
    const OrcTensor *st = find(m, scale_name);
    if (!st || st->dtype != 2 || st->numel != out_width) return 0;
    mat->s = (const float *)st->data;
    mat->fmt = orc_detect_format(t->nbytes, out_width, in_width);
    return mat->fmt > 0;
}

static const float *vector(const OrcModel *m, const char *name, int64_t numel) {
    const OrcTensor *t = find(m, name);
    if (!t || t->dtype != 2 || t->numel != numel) return NULL;
    return (const float *)t->data;
}

static int g_threads = 1;

void orc_set_threads(int threads) { g_threads = threads > 0 ? threads : 1; }

static void mm(const OrcMatrix *mat, const float *x, float *y, int rows,
               int in_width, int out_width) {
    orc_matmul(mat->fmt, mat->w, mat->s, x, y, out_width, in_width, rows, g_threads);
}

int orc_named_matmul(const OrcModel *m, const char *name, const float *x,
                     int rows, int in_width, int out_width, float *y) {
    OrcMatrix mat;
    if (!resolve(m, name, in_width, out_width, &mat)) return 0;
    mm(&mat, x, y, rows, in_width, out_width);
    return 1;
}

/* encode_attention_buffer (moonlight_metal.m:287-440) with the kernels
 * cache_append (moonlight_kernels.metal:132-170), rope_query (:172-200),
 * absorb_query (:218-245), scores (:247-282), latent_context (:284-343),
 * decode_value (:345-375). */
int orc_attention(OrcModel *m, int layer, const float *x, int rows,
                  int position, float *out) {
    const OrcConfig *c = &m->cfg;
    char name[512];
    OrcMatrix qm, kvam, kvbm, om;
    int heads = c->head_count, nope = c->qk_nope_dim, rope = c->qk_rope_dim;
    int vdim = c->value_dim, lw = c->kv_lora_rank;
    int hw = nope + rope, qw = heads * hw, cw = lw + rope, ctxw = heads * vdim;
    if (layer < 0 || layer >= c->layer_count || c->q_lora_rank ||
        position != m->kv_lengths[layer] || position + rows > m->context_size)
        return 0;
    snprintf(name, sizeof(name), "model.layers.%d.self_attn.q_proj.weight", layer);
    if (!resolve(m, name, c->hidden_size, qw, &qm)) return 0;
    snprintf(name, sizeof(name), "model.layers.%d.self_attn.kv_a_proj_with_mqa.weight", layer);
    if (!resolve(m, name, c->hidden_size, cw, &kvam)) return 0;
    snprintf(name, sizeof(name), "model.layers.%d.self_attn.kv_b_proj.weight", layer);
    if (!resolve(m, name, lw, heads * (nope + vdim), &kvbm)) return 0;
    snprintf(name, sizeof(name), "model.layers.%d.self_attn.o_proj.weight", layer);
    if (!resolve(m, name, ctxw, c->hidden_size, &om)) return 0;
    snprintf(name, sizeof(name), "model.layers.%d.self_attn.kv_a_layernorm.weight", layer);
    const float *kv_norm = vector(m, name, lw);
    if (!kv_norm) return 0;

    float *q = malloc((size_t)rows * qw * sizeof(float));
    float *comp = malloc((size_t)rows * cw * sizeof(float));
    float *ctx = malloc((size_t)rows * ctxw * sizeof(float));
    float rope_buf[512];
    mm(&qm, x, q, rows, c->hidden_size, qw);
    mm(&kvam, x, comp, rows, c->hidden_size, cw);

    float *lat_base = m->latent_kv + (size_t)layer * m->context_size * lw;
    float *rope_base = m->rope_kv + (size_t)layer * m->context_size * rope;
    for (int r = 0; r < rows; ++r) {
        const float *src = comp + (int64_t)r * cw;
        orc_rmsnorm(src, kv_norm, lat_base + (size_t)(position + r) * lw, 1, lw,
                    c->rms_norm_epsilon);
        orc_rope(src + lw, rope_base + (size_t)(position + r) * rope, rope,
                 position + r, c->rope_theta);
        for (int h = 0; h < heads; ++h) {
            float *qh = q + ((int64_t)r * heads + h) * hw;
            orc_rope(qh + nope, rope_buf, rope, position + r, c->rope_theta);
            memcpy(qh + nope, rope_buf, (size_t)rope * sizeof(float));
        }
    }

    float attention_scale = 1.0f / sqrtf((float)(nope + rope));
    /* rows are independent once every cache row is written: threads split
     * the rows, each (row, head) computed exactly as in the serial order */
#ifdef _OPENMP
    #pragma omp parallel num_threads(g_threads)
#endif
    {
    float *qa = malloc((size_t)lw * sizeof(float));
    float *lc = malloc((size_t)lw * sizeof(float));
    float *scores = malloc((size_t)(position + rows) * sizeof(float));
#ifdef _OPENMP
    #pragma omp for schedule(dynamic, 1)
#endif
    for (int r = 0; r < rows; ++r) {
        int keys = position + r + 1;
        for (int h = 0; h < heads; ++h) {
            const float *qh = q + ((int64_t)r * heads + h) * hw;
            int wrow = h * (nope + vdim);
            for (int l = 0; l < lw; ++l) {
                float sum = 0.0f;
                for (int cc = 0; cc < nope; ++cc)
                    sum += qh[cc] * weight_value(kvbm.fmt, kvbm.w, kvbm.s,
                                                 wrow + cc, l, lw);
                qa[l] = sum;
            }
            float maximum = -INFINITY;
            for (int k = 0; k < keys; ++k) {
                const float *lat = lat_base + (size_t)k * lw;
                const float *rp = rope_base + (size_t)k * rope;
                float score = 0.0f;
                for (int l = 0; l < lw; ++l) score += qa[l] * lat[l];
                for (int cc = 0; cc < rope; ++cc) score += qh[nope + cc] * rp[cc];
                scores[k] = score * attention_scale;
                if (scores[k] > maximum) maximum = scores[k];
            }
            float denom = 0.0f;
            for (int k = 0; k < keys; ++k) denom += expf(scores[k] - maximum);
            for (int l = 0; l < lw; ++l) lc[l] = 0.0f;
            for (int k = 0; k < keys; ++k) {
                float p = expf(scores[k] - maximum) / denom;
                const float *lat = lat_base + (size_t)k * lw;
                for (int l = 0; l < lw; ++l) lc[l] += p * lat[l];
            }
            float *ch = ctx + ((int64_t)r * heads + h) * vdim;
            for (int v = 0; v < vdim; ++v) {
                float sum = 0.0f;
                for (int l = 0; l < lw; ++l)
                    sum += lc[l] * weight_value(kvbm.fmt, kvbm.w, kvbm.s,
                                                wrow + nope + v, l, lw);
                ch[v] = sum;
            }
        }
    }
    free(qa);
    free(lc);
    free(scores);
    }
    mm(&om, ctx, out, rows, ctxw, c->hidden_size);
    m->kv_lengths[layer] = position + rows;
    if (m->position < position + rows) m->position = position + rows;
    free(q);
    free(comp);
    free(ctx);
    return 1;
}

/* One SwiGLU FFN: down(silu(gate x) * up x), moonlight_metal.m:442-483. */
static int ffn(const OrcModel *m, const char *prefix, const float *x, int rows,
               int width, float *out) {
    const OrcConfig *c = &m->cfg;
    char name[512];
    OrcMatrix g, u, d;
    snprintf(name, sizeof(name), "%s.gate_proj.weight", prefix);
    if (!resolve(m, name, c->hidden_size, width, &g)) return 0;
    snprintf(name, sizeof(name), "%s.up_proj.weight", prefix);
    if (!resolve(m, name, c->hidden_size, width, &u)) return 0;
    snprintf(name, sizeof(name), "%s.down_proj.weight", prefix);
    if (!resolve(m, name, width, c->hidden_size, &d)) return 0;
    float *gate = malloc((size_t)rows * width * sizeof(float));
    float *up = malloc((size_t)rows * width * sizeof(float));
    mm(&g, x, gate, rows, c->hidden_size, width);
    mm(&u, x, up, rows, c->hidden_size, width);
    for (int64_t i = 0; i < (int64_t)rows * width; ++i)
        gate[i] = orc_silu_mul(gate[i], up[i]);
    mm(&d, gate, out, rows, width, c->hidden_size);
    free(gate);
    free(up);
    return 1;
}

int orc_dense_mlp(OrcModel *m, int layer, const float *x, int rows, float *out) {
    char prefix[256];
    snprintf(prefix, sizeof(prefix), "model.layers.%d.mlp", layer);
    return ffn(m, prefix, x, rows, m->cfg.dense_intermediate_size, out);
}

/* moe_route_fixed + moe_route_finalize (moe_route.h:76-99) with sigmoid
 * scores: the weights of the given ids are their unbiased scores, then
 * /(sum + 1e-20) when normalising, then * routed_scale. */
int orc_route_fixed(const float *logits, int rows, int experts, int top_k,
                    int normalize, float routed_scale, const int *ids,
                    float *weights) {
    for (int r = 0; r < rows; ++r) {
        const float *lg = logits + (int64_t)r * experts;
        const int *id = ids + (int64_t)r * top_k;
        float *wt = weights + (int64_t)r * top_k;
        for (int k = 0; k < top_k; ++k) {
            if (id[k] < 0 || id[k] >= experts) return 0;
            wt[k] = route_sigmoid(lg[id[k]]);
        }
        float denom = 1.0f;
        if (normalize) {
            float sum = 0.0f;
            for (int k = 0; k < top_k; ++k) sum += wt[k];
            denom = sum + 1e-20f;
        }
        for (int k = 0; k < top_k; ++k) wt[k] = wt[k] / denom * routed_scale;
    }
    return 1;
}

static int moe_layer(OrcModel *m, int layer, const float *x, int rows,
                     const int *fixed_ids, int *route_ids, float *route_weights,
                     float *router_logits, float *routed, float *shared, float *out);

/* moonlight_test_moe (moonlight_metal.m:1520-1733); routed sum in slot order
 * per row as quantized_moe_reference (tests/test_moonlight_metal_moe.c:83-149),
 * then routed + shared. */
int orc_moe_layer(OrcModel *m, int layer, const float *x, int rows,
                  int *route_ids, float *route_weights, float *router_logits,
                  float *routed, float *shared, float *out) {
    return moe_layer(m, layer, x, rows, NULL, route_ids, route_weights,
                     router_logits, routed, shared, out);
}

/* The same layer with caller-given expert ids (orc_route_fixed). */
int orc_moe_layer_fixed(OrcModel *m, int layer, const float *x, int rows,
                        const int *fixed_ids, float *route_weights, float *out) {
    return moe_layer(m, layer, x, rows, fixed_ids, NULL, route_weights, NULL,
                     NULL, NULL, out);
}

static int moe_layer(OrcModel *m, int layer, const float *x, int rows,
                     const int *fixed_ids, int *route_ids, float *route_weights,
                     float *router_logits, float *routed, float *shared, float *out) {
    const OrcConfig *c = &m->cfg;
    char name[512];
    OrcMatrix router;
    int H = c->hidden_size, E = c->expert_count, K = c->experts_per_token;
    if (layer < c->first_dense_layer_count || layer >= c->layer_count) return 0;
    snprintf(name, sizeof(name), "model.layers.%d.mlp.gate.weight", layer);
    if (!resolve(m, name, H, E, &router)) return 0;
    snprintf(name, sizeof(name), "model.layers.%d.mlp.gate.e_score_correction_bias", layer);
    const float *bias = vector(m, name, E);
    if (!bias) return 0;
    float *logits = router_logits ? router_logits : malloc((size_t)rows * E * sizeof(float));
    int *ids = route_ids ? route_ids : malloc((size_t)rows * K * sizeof(int));
    float *wts = route_weights ? route_weights : malloc((size_t)rows * K * sizeof(float));
    float *rt = routed ? routed : malloc((size_t)rows * H * sizeof(float));
    float *sh = shared ? shared : malloc((size_t)rows * H * sizeof(float));
    float *y = malloc((size_t)H * sizeof(float));
    int ok = 1;
    mm(&router, x, logits, rows, H, E);
    if (fixed_ids) {
        memcpy(ids, fixed_ids, (size_t)rows * K * sizeof(int));
        ok = orc_route_fixed(logits, rows, E, K, c->normalize_topk, c->routed_scale, ids, wts);
    } else {
        orc_route_sigmoid_topk(logits, bias, rows, E, K, c->normalize_topk,
                               c->routed_scale, ids, wts);
    }
    memset(rt, 0, (size_t)rows * H * sizeof(float));
    for (int r = 0; r < rows && ok; ++r) {
        for (int k = 0; k < K && ok; ++k) {
            int e = ids[r * K + k];
            char prefix[256];
            snprintf(prefix, sizeof(prefix), "model.layers.%d.mlp.experts.%d", layer, e);
            ok = ffn(m, prefix, x + (int64_t)r * H, 1, c->moe_intermediate_size, y);
            for (int d = 0; ok && d < H; ++d) rt[(int64_t)r * H + d] += wts[r * K + k] * y[d];
        }
    }
    if (ok) {
        char prefix[256];
        snprintf(prefix, sizeof(prefix), "model.layers.%d.mlp.shared_experts", layer);
        ok = ffn(m, prefix, x, rows, c->moe_intermediate_size * c->shared_expert_count, sh);
    }
    if (ok)
        for (int64_t i = 0; i < (int64_t)rows * H; ++i) out[i] = rt[i] + sh[i];
    if (!router_logits) free(logits);
    if (!route_ids) free(ids);
    if (!route_weights) free(wts);
    if (!routed) free(rt);
    if (!shared) free(sh);
    free(y);
    return ok;
}

/* run_tokens_fast (moonlight_metal.m:1892-1986) with the block order of
 * encode_attention_block (:678-706): h = x + attn(norm(x)); x' = h + mlp(norm(h)). */
static int forward(OrcModel *m, const int *ids, int rows, int start_position,
                   const int *fixed_trace, float *layer_outputs, int *route_trace,
                   float *last_logits);

int orc_forward(OrcModel *m, const int *ids, int rows, int start_position,
                float *layer_outputs, int *route_trace, float *last_logits) {
    return forward(m, ids, rows, start_position, NULL, layer_outputs, route_trace,
                   last_logits);
}

/* The same forward with every MoE layer routed to the given experts
 * (fixed_trace [layers][rows][experts_per_token], orc_moe_layer_fixed). */
int orc_forward_routes(OrcModel *m, const int *ids, int rows, int start_position,
                       const int *fixed_trace, float *layer_outputs, float *last_logits) {
    return forward(m, ids, rows, start_position, fixed_trace, layer_outputs, NULL,
                   last_logits);
}

static int forward(OrcModel *m, const int *ids, int rows, int start_position,
                   const int *fixed_trace, float *layer_outputs, int *route_trace,
                   float *last_logits) {
    const OrcConfig *c = &m->cfg;
    int H = c->hidden_size, K = c->experts_per_token;
    char name[512];
    const float *embed = vector(m, "model.embed_tokens.weight", (int64_t)c->vocab_size * H);
    const float *final_norm = vector(m, "model.norm.weight", H);
    OrcMatrix head;
    if (!embed || !final_norm || !resolve(m, "lm_head.weight", H, c->vocab_size, &head))
        return 0;
    size_t bytes = (size_t)rows * H * sizeof(float);
    float *x = malloc(bytes), *norm = malloc(bytes), *tmp = malloc(bytes);
    int ok = 1;
    for (int r = 0; r < rows; ++r) {
        if (ids[r] < 0 || ids[r] >= c->vocab_size) { ok = 0; break; }
        memcpy(x + (int64_t)r * H, embed + (int64_t)ids[r] * H, (size_t)H * sizeof(float));
    }
    for (int layer = 0; ok && layer < c->layer_count; ++layer) {
        snprintf(name, sizeof(name), "model.layers.%d.input_layernorm.weight", layer);
        const float *w_in = vector(m, name, H);
        snprintf(name, sizeof(name), "model.layers.%d.post_attention_layernorm.weight", layer);
        const float *w_post = vector(m, name, H);
        if (!w_in || !w_post) { ok = 0; break; }
        orc_rmsnorm(x, w_in, norm, rows, H, c->rms_norm_epsilon);
        if (!orc_attention(m, layer, norm, rows, start_position, tmp)) { ok = 0; break; }
        for (int64_t i = 0; i < (int64_t)rows * H; ++i) x[i] += tmp[i];
        orc_rmsnorm(x, w_post, norm, rows, H, c->rms_norm_epsilon);
        if (layer < c->first_dense_layer_count) {
            ok = orc_dense_mlp(m, layer, norm, rows, tmp);
        } else {
            if (fixed_trace) {
                ok = orc_moe_layer_fixed(m, layer, norm, rows,
                                         fixed_trace + (int64_t)layer * rows * K, NULL, tmp);
            } else {
                int *trace = route_trace ? route_trace + (int64_t)layer * rows * K : NULL;
                ok = orc_moe_layer(m, layer, norm, rows, trace, NULL, NULL, NULL, NULL, tmp);
            }
        }
        if (!ok) break;
        for (int64_t i = 0; i < (int64_t)rows * H; ++i) x[i] += tmp[i];
        if (layer_outputs)
            memcpy(layer_outputs + (int64_t)layer * rows * H, x, bytes);
    }
    if (ok) {
        orc_rmsnorm(x + (int64_t)(rows - 1) * H, final_norm, norm, 1, H, c->rms_norm_epsilon);
        mm(&head, norm, last_logits, 1, H, c->vocab_size);
        m->position = start_position + rows;
    }
    free(x);
    free(norm);
    free(tmp);
    return ok;
}

/* ---- next-token choice (moonlight_chat.c:89-131) -------------------------- */

double orc_random_unit(uint64_t *state) {
    uint64_t x = *state;
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    *state = x;
    return (double)(x >> 11) * (1.0 / 9007199254740992.0);
}

typedef struct {
    float p;
    int token;
} OrcCandidate;

/* descending probability; equal probabilities keep token order */
static int orc_candidate_cmp(const void *left, const void *right) {
    const OrcCandidate *a = (const OrcCandidate *)left, *b = (const OrcCandidate *)right;
    if (a->p < b->p) return 1;
    if (a->p > b->p) return -1;
    return (a->token > b->token) - (a->token < b->token);
}

int orc_choose_token(const float *logits, int vocab, float temperature, float top_p,
                     uint64_t *rng) {
    int best = 0;
    for (int t = 1; t < vocab; ++t)
        if (logits[t] > logits[best]) best = t;
    if (temperature <= 0.0f) return best;
    const float maximum = logits[best];
    OrcCandidate *c = (OrcCandidate *)malloc((size_t)vocab * sizeof(OrcCandidate));
    if (!c) return -1;
    double total = 0.0;
    for (int t = 0; t < vocab; ++t) {
        c[t].p = expf((logits[t] - maximum) / temperature);
        c[t].token = t;
        total += c[t].p;
    }
    const float ftotal = (float)total;
    for (int t = 0; t < vocab; ++t) c[t].p /= ftotal;
    qsort(c, (size_t)vocab, sizeof(*c), orc_candidate_cmp);
    double kept = 0.0;
    int count = 0;
    do {
        kept += c[count++].p;
    } while (count < vocab && kept < top_p);
    const double sample = orc_random_unit(rng) * kept;
    double cumulative = 0.0;
    int token = c[count - 1].token;
    for (int i = 0; i < count; ++i) {
        cumulative += c[i].p;
        if (cumulative >= sample) {
            token = c[i].token;
            break;
        }
    }
    free(c);
    return token;
}
