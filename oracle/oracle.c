/*
 * oracle.c -- CPU restatement of the reference's decision-path forward.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h).  Each function names the
 * reference lines it follows.  Built by oracle/Makefile into
 * oracle/_build/liboracle_*.so; the product never links it.
 */
#include "oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ f16 */

/* IEEE binary16 from binary32, round to nearest even (half::f16::from_f32). */
uint16_t orc_f32_to_f16(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    uint32_t sign = (u >> 16) & 0x8000u;
    uint32_t exp = (u >> 23) & 0xffu;
    uint32_t man = u & 0x7fffffu;
    if (exp == 0xffu) return (uint16_t)(sign | 0x7c00u | (man ? (0x200u | (man >> 13)) : 0u));
    int e = (int)exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        uint32_t m = man | 0x800000u;
        int shift = 14 - e;
        uint32_t h = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    uint32_t h = sign | ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)h;
}

float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t exp = ((uint32_t)h >> 10) & 0x1fu;
    uint32_t man = (uint32_t)h & 0x3ffu;
    uint32_t u;
    if (exp == 0) {
        if (man == 0) {
            u = sign;
        } else {
            int e = -1;
            do {
                e++;
                man <<= 1;
            } while (!(man & 0x400u));
            man &= 0x3ffu;
            u = sign | ((uint32_t)(112 - e) << 23) | (man << 13);
        }
    } else if (exp == 31) {
        u = sign | 0x7f800000u | (man << 13);
    } else {
        u = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static inline float r16(float x) { return orc_f16_to_f32(orc_f32_to_f16(x)); }

/* ------------------------------------------------------------------ rng */

/* tests/reference.rs:17-28: xorshift64, uniform in [-1, 1). */
float orc_rng_next(uint64_t *s) {
    uint64_t v = *s;
    v ^= v << 13;
    v ^= v >> 7;
    v ^= v << 17;
    *s = v;
    return ((float)(v >> 40) / (float)(1ull << 24)) * 2.0f - 1.0f;
}

void orc_rng_values(uint64_t *s, float *out, size_t n, float scale) {
    for (size_t i = 0; i < n; i++) out[i] = orc_rng_next(s) * scale;
}

/* --------------------------------------------------------- block formats */

/* model.rs:408-431: scale = max|v| / 127 (stored f16), q = round(v / scale)
 * clamped to +-127, with the reciprocal taken of the f32 scale. */
int orc_quantize_q8(const float *v, size_t n, uint8_t *data, uint8_t *scales) {
    if (n % 32) return -1;
    for (size_t b = 0; b < n / 32; b++) {
        const float *blk = v + 32 * b;
        float amax = 0.0f;
        for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(blk[j]));
        float d = amax / 127.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint16_t h = orc_f32_to_f16(d);
        scales[2 * b] = (uint8_t)(h & 0xff);
        scales[2 * b + 1] = (uint8_t)(h >> 8);
        for (int j = 0; j < 32; j++) {
            float q = roundf(blk[j] * id);
            if (q < -127.0f) q = -127.0f;
            if (q > 127.0f) q = 127.0f;
            data[32 * b + j] = (uint8_t)(int8_t)q;
        }
    }
    return 0;
}

/* model.rs:435-466: scale = (signed value of largest magnitude) / -8,
 * q = clamp(trunc(v / scale + 8.5), 0, 15); byte j holds element j in the
 * low nibble and element j + 16 in the high nibble. */
int orc_quantize_q4(const float *v, size_t n, uint8_t *data, uint8_t *scales) {
    if (n % 32) return -1;
    for (size_t b = 0; b < n / 32; b++) {
        const float *blk = v + 32 * b;
        float mx = 0.0f, amax = 0.0f;
        for (int j = 0; j < 32; j++) {
            if (fabsf(blk[j]) > amax) {
                amax = fabsf(blk[j]);
                mx = blk[j];
            }
        }
        float d = mx / -8.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint16_t h = orc_f32_to_f16(d);
        scales[2 * b] = (uint8_t)(h & 0xff);
        scales[2 * b + 1] = (uint8_t)(h >> 8);
        for (int j = 0; j < 16; j++) {
            int lo = (int)(blk[j] * id + 8.5f);
            int hi = (int)(blk[j + 16] * id + 8.5f);
            lo = lo < 0 ? 0 : (lo > 15 ? 15 : lo);
            hi = hi < 0 ? 0 : (hi > 15 ? 15 : hi);
            data[16 * b + j] = (uint8_t)(lo | (hi << 4));
        }
    }
    return 0;
}

/* model.rs:507-525 */
float orc_get(int dtype, const uint8_t *data, const uint8_t *scales, size_t i) {
    if (dtype == ORC_F16) return orc_f16_to_f32((uint16_t)(data[2 * i] | (data[2 * i + 1] << 8)));
    size_t b = i / 32;
    float d = orc_f16_to_f32((uint16_t)(scales[2 * b] | (scales[2 * b + 1] << 8)));
    if (dtype == ORC_Q8) return (float)(int8_t)data[i] * d;
    size_t j = i % 32;
    uint8_t byte = data[b * 16 + j % 16];
    int q = j < 16 ? (byte & 0xf) : (byte >> 4);
    return ((float)q - 8.0f) * d;
}

/* ---------------------------------------------------------------- model */

typedef struct {
    int present;
    int64_t rows, cols;
    float *w; /* dequantized, row-major */
} orc_tensor;

enum {
    T_ATTN_NORM,
    T_QKV,
    T_Q_NORM,
    T_K_NORM,
    T_O,
    T_POST_ATTN_NORM,
    T_FFN_NORM,
    T_GATE,
    T_UP,
    T_DOWN,
    T_POST_FFN_NORM,
    T_PL_GATE,
    T_PL_PROJ,
    T_PL_NORM,
    T_OUT_SCALE,
    T_COUNT
};
static const char *LAYER_NAMES[T_COUNT] = {"attn_norm", "qkv", "q_norm", "k_norm",
                                           "o", "post_attn_norm", "ffn_norm", "gate",
                                           "up", "down", "post_ffn_norm", "pl_gate",
                                           "pl_proj", "pl_norm", "out_scale"};

struct orc_model {
    orc_config cfg;
    int gpu;
    /* Kernel-faithful attention (orc_model_set_attention_tiles): key tile,
     * chunk lengths in tiles for sliding / global layers, lazy-rescale
     * threshold in log2 units; key_tile = 0 is the plain softmax. */
    int key_tile, chunk_sliding, chunk_global;
    float tau;
    orc_tensor embed, final_norm, pl_model_proj, pl_proj_norm, per_layer_table;
    orc_tensor layer[ORC_MAX_LAYERS][T_COUNT];
};

static int has_kv(const orc_config *c, int l) { return c->kv_source[l] == l; }
static int64_t qkv_width(const orc_config *c, int l) {
    int64_t hd = c->head_dim[l];
    return has_kv(c, l) ? (int64_t)(c->heads + 2 * c->kv_heads) * hd : (int64_t)c->heads * hd;
}

orc_model *orc_model_new(const orc_config *cfg, int gpu_rounding) {
    if (cfg->layers <= 0 || cfg->layers > ORC_MAX_LAYERS) return NULL;
    orc_model *m = (orc_model *)calloc(1, sizeof(orc_model));
    if (!m) return NULL;
    m->cfg = *cfg;
    m->gpu = gpu_rounding;
    return m;
}

int orc_model_set_attention_tiles(orc_model *m, int key_tile, int chunk_sliding, int chunk_global, float tau) {
    if (key_tile < 0 || (key_tile > 0 && (chunk_sliding <= 0 || chunk_global <= 0 || tau < 0.0f))) return -1;
    m->key_tile = key_tile;
    m->chunk_sliding = chunk_sliding;
    m->chunk_global = chunk_global;
    m->tau = tau;
    return 0;
}

static void tensor_free(orc_tensor *t) {
    free(t->w);
    t->w = NULL;
    t->present = 0;
}

void orc_model_free(orc_model *m) {
    if (!m) return;
    tensor_free(&m->embed);
    tensor_free(&m->final_norm);
    tensor_free(&m->pl_model_proj);
    tensor_free(&m->pl_proj_norm);
    tensor_free(&m->per_layer_table);
    for (int l = 0; l < ORC_MAX_LAYERS; l++)
        for (int k = 0; k < T_COUNT; k++) tensor_free(&m->layer[l][k]);
    free(m);
}

static orc_tensor *lookup(orc_model *m, const char *name, int *is_linear) {
    *is_linear = 0;
    if (!strcmp(name, "embed")) return &m->embed;
    if (!strcmp(name, "final_norm")) return &m->final_norm;
    if (!strcmp(name, "pl_model_proj")) {
        *is_linear = 1;
        return &m->pl_model_proj;
    }
    if (!strcmp(name, "pl_proj_norm")) return &m->pl_proj_norm;
    if (!strcmp(name, "per_layer_table")) return &m->per_layer_table;
    int l;
    char rest[64];
    if (sscanf(name, "blk.%d.%63s", &l, rest) != 2) return NULL;
    if (l < 0 || l >= m->cfg.layers) return NULL;
    for (int k = 0; k < T_COUNT; k++) {
        if (!strcmp(rest, LAYER_NAMES[k])) {
            *is_linear = (k == T_QKV || k == T_O || k == T_GATE || k == T_UP || k == T_DOWN || k == T_PL_GATE ||
                          k == T_PL_PROJ);
            return &m->layer[l][k];
        }
    }
    return NULL;
}

int orc_model_set(orc_model *m, const char *name, int dtype, int64_t rows, int64_t cols,
                  const uint8_t *data, const uint8_t *scales) {
    int lin;
    orc_tensor *t = lookup(m, name, &lin);
    if (!t) return -1;
    int64_t n = rows * cols;
    tensor_free(t);
    t->w = (float *)malloc((size_t)n * sizeof(float));
    if (!t->w) return -2;
    const int round16 = m->gpu && lin;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++) {
        float v = orc_get(dtype, data, scales, (size_t)i);
        /* matmul.wgsl decodes linear weights to f16 pairs. */
        t->w[i] = round16 ? r16(v) : v;
    }
    t->rows = rows;
    t->cols = cols;
    t->present = 1;
    return 0;
}

int orc_model_missing(const orc_model *m, char *buf, size_t len) {
    int count = 0;
    size_t at = 0;
    if (buf && len) buf[0] = 0;
#define MISS(s)                                                               \
    do {                                                                      \
        count++;                                                              \
        if (buf && at < len) at += (size_t)snprintf(buf + at, len - at, "%s\n", s); \
    } while (0)
    if (!m->embed.present) MISS("embed");
    if (!m->final_norm.present) MISS("final_norm");
    const int pl = m->cfg.per_layer_dim > 0;
    if (pl && !m->pl_model_proj.present) MISS("pl_model_proj");
    if (pl && !m->pl_proj_norm.present) MISS("pl_proj_norm");
    if (pl && !m->per_layer_table.present) MISS("per_layer_table");
    for (int l = 0; l < m->cfg.layers; l++) {
        for (int k = 0; k < T_COUNT; k++) {
            if (k == T_K_NORM && !has_kv(&m->cfg, l)) continue;
            if (k >= T_PL_GATE && !pl) continue;
            if (!m->layer[l][k].present) {
                char nm[64];
                snprintf(nm, sizeof nm, "blk.%d.%s", l, LAYER_NAMES[k]);
                MISS(nm);
            }
        }
    }
#undef MISS
    return count;
}

/* reference.rs:141-148 */
static void rmsnorm(const float *x, int64_t n, const float *w, float eps, float offset, float *y) {
    float ms = 0.0f;
    for (int64_t i = 0; i < n; i++) ms += x[i] * x[i];
    ms /= (float)n;
    float inv = 1.0f / sqrtf(ms + eps);
    for (int64_t i = 0; i < n; i++) y[i] = x[i] * inv * (w ? offset + w[i] : 1.0f);
}

/* reference.rs:150-157: y[t][n] = sum_k x[t][k] W[n][k].  Four rows share
 * each weight row; the k sum is a vectorised reduction. */
static void linear(const float *x, int64_t t, int64_t k, const float *w, int64_t n, float *y) {
#pragma omp parallel for schedule(static)
    for (int64_t i0 = 0; i0 < t; i0 += 4) {
        int64_t ni = t - i0 < 4 ? t - i0 : 4;
        const float *x0 = x + i0 * k;
        const float *x1 = x0 + (ni > 1 ? k : 0);
        const float *x2 = x0 + (ni > 2 ? 2 * k : 0);
        const float *x3 = x0 + (ni > 3 ? 3 * k : 0);
        for (int64_t c = 0; c < n; c++) {
            const float *wr = w + c * k;
            float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
#pragma omp simd reduction(+ : a0, a1, a2, a3)
            for (int64_t kk = 0; kk < k; kk++) {
                float wv = wr[kk];
                a0 += x0[kk] * wv;
                a1 += x1[kk] * wv;
                a2 += x2[kk] * wv;
                a3 += x3[kk] * wv;
            }
            y[i0 * n + c] = a0;
            if (ni > 1) y[(i0 + 1) * n + c] = a1;
            if (ni > 2) y[(i0 + 2) * n + c] = a2;
            if (ni > 3) y[(i0 + 3) * n + c] = a3;
        }
    }
}

void orc_linear(const float *x, int64_t t, int64_t k, const float *w, int64_t n, float *y) { linear(x, t, k, w, n, y); }

/* reference.rs:159-168: pairs (i, i + hd/2) for i < rope_dims/2. */
static void rope(float *v, int64_t hd, int32_t pos, float theta, int64_t rope_dims) {
    int64_t half = hd / 2;
    for (int64_t i = 0; i < rope_dims / 2; i++) {
        float ang = (float)pos * powf(theta, -(float)i / (float)half);
        float s = sinf(ang), c = cosf(ang);
        float a = v[i], b = v[i + half];
        v[i] = a * c - b * s;
        v[i + half] = b * c + a * s;
    }
}

/* reference.rs:170-172 */
static float gelu(float x) {
    return 0.5f * x * (1.0f + tanhf(0.7978845608f * (x + 0.044715f * x * x * x)));
}

/* attention.wgsl:73-76 (group bits above SEQ_GROUP_SHIFT); for one group it
 * is reference.rs:284-286. */
static int visible(int32_t qp, int32_t qs, int32_t kp, int32_t ks, int sliding, int32_t window) {
    int same_group = ((ks ^ qs) >> ORC_SEQ_GROUP_SHIFT) == 0;
    return same_group && ((ks & 0xfff) == 0 || ks == qs) && kp <= qp &&
           (!sliding || (qp - kp) < window);
}

static void round_rows(float *v, int64_t n) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++) v[i] = r16(v[i]);
}

static void norm_rows(const float *x, int64_t t, int64_t d, const orc_tensor *w, float eps,
                      float offset, float *y) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < t; i++) rmsnorm(x + i * d, d, w->w, eps, offset, y + i * d);
}

/* One query row of one head, with the rounding points of an f16 flash
 * kernel instead of the reference's f32 softmax (reference.rs:284-300,
 * shaders/attention.wgsl:55,240-252 keep P in f32): keys are taken in
 * cache-row order in tiles of `kt`; the running max (log2 units, rounded up
 * to a whole number) moves only when a tile's max exceeds it by more than
 * `tau`; a probability is 2^frac(x) 2^(floor(x) - m) for x = s log2(e); each is
 * rounded to f16 before both the sum and the P.V product, whose f32 sum is
 * taken per tile and then added to O (one MFMA per tile); the key range is
 * cut at absolute multiples of `chunk` tiles, each chunk's O / l is rounded
 * to f16, and chunks are merged with weights l_c 2^(m_c - M) (one chunk:
 * its f16 row unchanged).  `s` holds the visible keys' scores, `idx` their
 * rows (ascending). */
static void attend_tiled(const float *s, const int64_t *idx, int64_t n, const float *V, int64_t vstride,
                         int64_t hd, int kt, int chunk, float tau, float *out, float *acc, float *part) {
    const float LOG2E = 1.4426950408889634f;
    int64_t r = 0;
    int nchunks = 0;
    float cm[64], cl[64];
    while (r < n) {
        const int64_t c = idx[r] / kt / chunk;
        float m = -INFINITY, l = 0.0f;
        for (int64_t e = 0; e < hd; e++) acc[e] = 0.0f;
        while (r < n && idx[r] / kt / chunk == c) {
            const int64_t tile = idx[r] / kt;
            int64_t r1 = r;
            float mt = -INFINITY;
            while (r1 < n && idx[r1] / kt == tile) mt = fmaxf(mt, s[r1++]);
            mt *= LOG2E;
            const int grow = mt > m + tau;
            const float m_new = grow ? ceilf(mt) : m; /* whole powers of two */
            const float m_use = m_new == -INFINITY ? 0.0f : m_new;
            if (grow && m != -INFINITY) {
                const float alpha = exp2f(m - m_use);
                l *= alpha;
                for (int64_t e = 0; e < hd; e++) acc[e] *= alpha;
            }
            /* the tile's P.V in its own f32 sum, then added to O, as one
             * MFMA over the tile's keys adds to the accumulator */
            float psum = 0.0f, *tacc = acc + hd;
            for (int64_t e = 0; e < hd; e++) tacc[e] = 0.0f;
            for (; r < r1; r++) {
                /* 2^frac(x) * 2^(floor(x) - m): exact power-of-two scaling under another max */
                const float x = fmaxf(s[r] * LOG2E, -16384.0f), xi = floorf(x);
                const float p = r16(ldexpf(exp2f(x - xi), (int)(xi - m_use)));
                psum += p;
                const float *vj = V + idx[r] * vstride;
                for (int64_t e = 0; e < hd; e++) tacc[e] += p * vj[e];
            }
            for (int64_t e = 0; e < hd; e++) acc[e] += tacc[e];
            l += psum;
            m = m_new;
        }
        if (nchunks >= 64) break; /* more chunks than the kernel's work lists make */
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
        for (int64_t e = 0; e < hd; e++) part[nchunks * hd + e] = r16(acc[e] * inv);
        cm[nchunks] = m;
        cl[nchunks] = l;
        nchunks++;
    }
    if (nchunks == 0) {
        for (int64_t e = 0; e < hd; e++) out[e] = 0.0f;
        return;
    }
    if (nchunks == 1) {
        for (int64_t e = 0; e < hd; e++) out[e] = part[e];
        return;
    }
    float M = -INFINITY, L = 0.0f;
    for (int k = 0; k < nchunks; k++) M = fmaxf(M, cm[k]);
    for (int64_t e = 0; e < hd; e++) acc[e] = 0.0f;
    for (int k = 0; k < nchunks; k++) {
        const float w = cl[k] * exp2f(cm[k] - M);
        L += w;
        for (int64_t e = 0; e < hd; e++) acc[e] += part[k * hd + e] * w;
    }
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    for (int64_t e = 0; e < hd; e++) out[e] = r16(acc[e] * inv);
}

/* reference.rs:175-349, without Gemma 4's per-layer inputs. */
int orc_forward(const orc_model *m, const uint32_t *ids, const int32_t *pos, const int32_t *seq,
                int64_t t, float *hidden) {
    const orc_config *c = &m->cfg;
    if (orc_model_missing(m, NULL, 0)) return -1;
    int64_t d = c->d, H = c->heads, KV = c->kv_heads;
    for (int64_t i = 0; i < t; i++)
        if ((int64_t)ids[i] >= c->vocab) return -2;
    int64_t max_hd = 0, max_ff = 0, max_qkv = 0;
    for (int l = 0; l < c->layers; l++) {
        if (c->head_dim[l] > max_hd) max_hd = c->head_dim[l];
        if (c->ff[l] > max_ff) max_ff = c->ff[l];
        if (qkv_width(c, l) > max_qkv) max_qkv = qkv_width(c, l);
    }
    float *x = (float *)malloc((size_t)(t * d) * 4);
    float *h = (float *)malloc((size_t)(t * d) * 4);
    float *a = (float *)malloc((size_t)(t * d) * 4);
    float *qkv = (float *)malloc((size_t)(t * max_qkv) * 4);
    float *q = (float *)malloc((size_t)(t * H * max_hd) * 4);
    float *att = (float *)malloc((size_t)(t * H * max_hd) * 4);
    float *g = (float *)malloc((size_t)(t * max_ff) * 4);
    float *u = (float *)malloc((size_t)(t * max_ff) * 4);
    float **kstore = (float **)calloc((size_t)c->layers, sizeof(float *));
    float **vstore = (float **)calloc((size_t)c->layers, sizeof(float *));
    /* Embedding rows, reference.rs:182-189. */
    float sc = sqrtf((float)d);
    for (int64_t i = 0; i < t; i++)
        for (int64_t k = 0; k < d; k++) x[i * d + k] = m->embed.w[(int64_t)ids[i] * d + k] * sc;
    /* Per-layer inputs [t][layers x P], reference.rs:190-215. */
    const int64_t P = c->per_layer_dim, PL = P * c->layers;
    float *pli = NULL;
    if (P > 0) {
        pli = (float *)malloc((size_t)(t * PL) * 4);
        float *xr = (float *)malloc((size_t)(t * d) * 4);
        memcpy(xr, x, (size_t)(t * d) * 4);
        if (m->gpu) round_rows(xr, t * d);
        float *proj = (float *)malloc((size_t)(t * PL) * 4);
        linear(xr, t, d, m->pl_model_proj.w, PL, proj);
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < t; i++) {
            float slice[1024], nv[1024];
            for (int l = 0; l < c->layers; l++) {
                for (int64_t j = 0; j < P; j++) slice[j] = proj[i * PL + l * P + j] / sqrtf((float)d);
                rmsnorm(slice, P, m->pl_proj_norm.w, c->eps, c->norm_offset, nv);
                for (int64_t j = 0; j < P; j++) {
                    /* engine.rs:1370-1381 gathers the table rows as f16 */
                    float tv = m->per_layer_table.w[(int64_t)ids[i] * PL + l * P + j];
                    if (m->gpu) tv = r16(tv);
                    const float e = tv * sqrtf((float)P);
                    pli[i * PL + l * P + j] = (nv[j] + e) / sqrtf(2.0f);
                }
            }
        }
        free(xr);
        free(proj);
    }

    for (int l = 0; l < c->layers; l++) {
        const orc_tensor *L = m->layer[l];
        int64_t hd = c->head_dim[l];
        int sl = c->sliding[l];
        float theta = sl ? c->theta_local : c->theta_global;
        int kvl = has_kv(c, l);
        int64_t hpg = H / KV;
        int64_t qw = qkv_width(c, l);
        int64_t ff = c->ff[l];
        norm_rows(x, t, d, &L[T_ATTN_NORM], c->eps, c->norm_offset, h);
        if (m->gpu) round_rows(h, t * d);
        linear(h, t, d, L[T_QKV].w, qw, qkv);
        if (kvl) {
            kstore[l] = (float *)malloc((size_t)(t * KV * hd) * 4);
            vstore[l] = (float *)malloc((size_t)(t * KV * hd) * 4);
        }
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < t; i++) {
            const float *row = qkv + i * qw;
            for (int64_t hh = 0; hh < H; hh++) {
                float *qh = q + (i * H + hh) * hd;
                rmsnorm(row + hh * hd, hd, L[T_Q_NORM].w, c->eps, c->norm_offset, qh);
                rope(qh, hd, pos[i], theta, c->rope_dims[l]);
                for (int64_t e = 0; e < hd; e++) qh[e] *= c->query_scale;
            }
            if (kvl) {
                for (int64_t gh = 0; gh < KV; gh++) {
                    float *kk = kstore[l] + (i * KV + gh) * hd;
                    rmsnorm(row + (H + gh) * hd, hd, L[T_K_NORM].w, c->eps, c->norm_offset, kk);
                    rope(kk, hd, pos[i], theta, c->rope_dims[l]);
                    float *vv = vstore[l] + (i * KV + gh) * hd;
                    const float *src = row + (H + KV + gh) * hd;
                    if (c->v_norm)
                        rmsnorm(src, hd, NULL, c->eps, 0.0f, vv);
                    else
                        memcpy(vv, src, (size_t)hd * 4);
                }
            }
        }
        if (m->gpu) {
            round_rows(q, t * H * hd);
            if (kvl) {
                round_rows(kstore[l], t * KV * hd);
                round_rows(vstore[l], t * KV * hd);
            }
        }
        const float *K = kstore[c->kv_source[l]];
        const float *V = vstore[c->kv_source[l]];
        if (!K || !V) return -3;
#pragma omp parallel
        {
            float *sc_ = (float *)malloc((size_t)t * 4);
            int64_t *idx = (int64_t *)malloc((size_t)t * 8);
            float *acc_ = (float *)malloc((size_t)(2 * hd) * 4);
            float *part_ = (float *)malloc((size_t)(64 * hd) * 4);
#pragma omp for schedule(dynamic, 8)
            for (int64_t i = 0; i < t; i++) {
                for (int64_t hh = 0; hh < H; hh++) {
                    const float *qh = q + (i * H + hh) * hd;
                    int64_t gh = hh / hpg;
                    int64_t n = 0;
                    for (int64_t j = 0; j < t; j++) {
                        if (!visible(pos[i], seq[i], pos[j], seq[j], sl, c->window)) continue;
                        const float *kj = K + (j * KV + gh) * hd;
                        float s = 0.0f;
                        for (int64_t e = 0; e < hd; e++) s += qh[e] * kj[e];
                        idx[n] = j;
                        sc_[n++] = s;
                    }
                    if (m->key_tile > 0) {
                        attend_tiled(sc_, idx, n, V + gh * hd, KV * hd, hd, m->key_tile,
                                     sl ? m->chunk_sliding : m->chunk_global, m->tau, att + (i * H + hh) * hd,
                                     acc_, part_);
                        continue;
                    }
                    float mx = -3.402823466e38f;
                    for (int64_t r = 0; r < n; r++) mx = fmaxf(mx, sc_[r]);
                    float lsum = 0.0f;
                    for (int64_t r = 0; r < n; r++) lsum += expf(sc_[r] - mx);
                    float *out = att + (i * H + hh) * hd;
                    for (int64_t e = 0; e < hd; e++) out[e] = 0.0f;
                    for (int64_t r = 0; r < n; r++) {
                        float p = expf(sc_[r] - mx) / lsum;
                        const float *vj = V + (idx[r] * KV + gh) * hd;
                        for (int64_t e = 0; e < hd; e++) out[e] += p * vj[e];
                    }
                }
            }
            free(sc_);
            free(idx);
            free(acc_);
            free(part_);
        }
        if (m->gpu) round_rows(att, t * H * hd);
        linear(att, t, H * hd, L[T_O].w, d, a);
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < t; i++) {
            float tmp[8192];
            rmsnorm(a + i * d, d, L[T_POST_ATTN_NORM].w, c->eps, c->norm_offset, tmp);
            for (int64_t k = 0; k < d; k++) x[i * d + k] += tmp[k];
            rmsnorm(x + i * d, d, L[T_FFN_NORM].w, c->eps, c->norm_offset, h + i * d);
        }
        if (m->gpu) round_rows(h, t * d);
        linear(h, t, d, L[T_GATE].w, ff, g);
        linear(h, t, d, L[T_UP].w, ff, u);
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < t * ff; i++) g[i] = gelu(g[i]) * u[i];
        if (m->gpu) round_rows(g, t * ff);
        linear(g, t, ff, L[T_DOWN].w, d, a);
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < t; i++) {
            float tmp[8192];
            rmsnorm(a + i * d, d, L[T_POST_FFN_NORM].w, c->eps, c->norm_offset, tmp);
            for (int64_t k = 0; k < d; k++) x[i * d + k] += tmp[k];
        }
        if (P > 0) {
            /* reference.rs:323-341: x += rmsnorm(pl_proj . (gelu(x . pl_gate) * pli[l])); x *= out_scale. */
            float *xr = (float *)malloc((size_t)(t * d) * 4);
            float *gp = (float *)malloc((size_t)(t * P) * 4);
            memcpy(xr, x, (size_t)(t * d) * 4);
            if (m->gpu) round_rows(xr, t * d);
            linear(xr, t, d, L[T_PL_GATE].w, P, gp);
            for (int64_t i = 0; i < t; i++)
                for (int64_t j = 0; j < P; j++) gp[i * P + j] = gelu(gp[i * P + j]) * pli[i * PL + l * P + j];
            if (m->gpu) round_rows(gp, t * P);
            linear(gp, t, P, L[T_PL_PROJ].w, d, a);
            const float scale = L[T_OUT_SCALE].w[0];
#pragma omp parallel for schedule(static)
            for (int64_t i = 0; i < t; i++) {
                float tmp[8192];
                rmsnorm(a + i * d, d, L[T_PL_NORM].w, c->eps, c->norm_offset, tmp);
                for (int64_t k = 0; k < d; k++) x[i * d + k] = (x[i * d + k] + tmp[k]) * scale;
            }
            free(xr);
            free(gp);
        }
    }
    free(pli);
    norm_rows(x, t, d, &m->final_norm, c->eps, c->norm_offset, hidden);
    for (int l = 0; l < c->layers; l++) {
        free(kstore[l]);
        free(vstore[l]);
    }
    free(kstore);
    free(vstore);
    free(x);
    free(h);
    free(a);
    free(qkv);
    free(q);
    free(att);
    free(g);
    free(u);
    return 0;
}

/* reference.rs:580-590 (and engine.rs:1901-1906 for the softcap). */
int orc_logits(const orc_model *m, const float *rows, int64_t n, float *out) {
    const orc_config *c = &m->cfg;
    int64_t d = c->d, V = c->vocab;
#pragma omp parallel for schedule(static)
    for (int64_t v = 0; v < V; v++) {
        const float *e = m->embed.w + v * d;
        for (int64_t r = 0; r < n; r++) {
            float z = 0.0f;
            for (int64_t i = 0; i < d; i++) z += rows[r * d + i] * e[i];
            if (c->softcap > 0.0f) z = c->softcap * tanhf(z / c->softcap);
            out[r * V + v] = z;
        }
    }
    return 0;
}

/* -------------------------------------------------------------- packing */

/* engine.rs:1479-1482 (layout order) and :1512-1571 (ids, meta, wanted,
 * decoded). */
int orc_pack(const orc_group *groups, int64_t ngroups, int64_t first, int resident,
             uint32_t *ids, int32_t *meta, int64_t *wanted, int64_t *decoded,
             int64_t *n_ids, int64_t *n_wanted, int64_t *n_decoded) {
    int64_t total = 0;
    for (int64_t g = 0; g < ngroups; g++) {
        total += groups[g].prefix_len;
        for (int64_t b = 0; b < groups[g].nbranches; b++) total += groups[g].branches[b].ntokens;
    }
    if (ngroups == 0 || total == 0) return -1;
    int64_t p0 = groups[first].prefix_len;
    int64_t base = resident ? p0 : 0;
    int64_t n = 0, nw = 0, nd = 0;
    for (int64_t k = 0; k < ngroups; k++) {
        int64_t gi = k == 0 ? first : (k <= first ? k - 1 : k);
        const orc_group *g = &groups[gi];
        int64_t p = g->prefix_len;
        if (g->nbranches >= (1 << ORC_SEQ_GROUP_SHIFT)) return -2;
        int32_t seq_hi = (int32_t)(k << ORC_SEQ_GROUP_SHIFT);
        int64_t row_lo = k == 0 ? 0 : base + n;
        if (!(k == 0 && base > 0)) {
            decoded[2 * nd] = gi;
            decoded[2 * nd + 1] = base + n;
            nd++;
            for (int64_t i = 0; i < p; i++) {
                int32_t *mm = meta + 4 * n;
                mm[0] = (int32_t)i;
                mm[1] = seq_hi;
                mm[2] = (int32_t)row_lo;
                mm[3] = (int32_t)(base + n + 1);
                ids[n++] = g->prefix[i];
            }
        }
        for (int64_t bi = 0; bi < g->nbranches; bi++) {
            const orc_branch *br = &g->branches[bi];
            int64_t start = n;
            for (int64_t j = 0; j < br->ntokens; j++) {
                int32_t *mm = meta + 4 * n;
                mm[0] = (int32_t)(p + j);
                mm[1] = seq_hi | (int32_t)(bi + 1);
                mm[2] = (int32_t)row_lo;
                mm[3] = (int32_t)(base + n + 1);
                ids[n++] = br->tokens[j];
            }
            for (int64_t s = 0; s < br->nwant; s++) {
                if (br->want[s] >= br->ntokens) return -3;
                int64_t *w = wanted + 4 * nw++;
                w[0] = gi;
                w[1] = bi;
                w[2] = s;
                w[3] = start + br->want[s];
            }
        }
    }
    *n_ids = n;
    *n_wanted = nw;
    *n_decoded = nd;
    return 0;
}

/* ---------------------------------------------------------------- state */

/* engine.rs:625-641, FNV-1a 64 over model id, a zero byte, then the prefix
 * tokens little-endian. */
uint64_t orc_state_key(const char *model_id, const uint32_t *prefix, int64_t n) {
    uint64_t h = 0xcbf29ce484222325ull;
#define EAT(b)                        \
    do {                              \
        h ^= (uint64_t)(uint8_t)(b);  \
        h *= 0x00000100000001b3ull;   \
    } while (0)
    for (const char *p = model_id; *p; p++) EAT(*p);
    EAT(0);
    for (int64_t i = 0; i < n; i++)
        for (int s = 0; s < 4; s++) EAT(prefix[i] >> (8 * s));
#undef EAT
    return h;
}

/* engine.rs:1967-1974 */
void orc_state_rows(int sliding, int64_t window, int64_t p, int64_t *r0, int64_t *r1) {
    if (sliding && window > 0) {
        *r0 = p > window ? p - window : 0;
        *r1 = p;
    } else {
        *r0 = 0;
        *r1 = p;
    }
}

/* --------------------------------------------------------- readout math */

/* math.rs:5-11 */
void orc_softmax(const float *z, int64_t n, float temperature, double *out) {
    double t = (double)(temperature > 1e-6f ? temperature : 1e-6f);
    float mf = -INFINITY;
    for (int64_t i = 0; i < n; i++) mf = fmaxf(mf, z[i]);
    double m = (double)mf, s = 0.0;
    for (int64_t i = 0; i < n; i++) {
        out[i] = exp(((double)z[i] - m) / t);
        s += out[i];
    }
    for (int64_t i = 0; i < n; i++) out[i] /= s;
}

/* math.rs:14-17 */
double orc_log_sum_exp(const float *z, int64_t n) {
    float mf = -INFINITY;
    for (int64_t i = 0; i < n; i++) mf = fmaxf(mf, z[i]);
    double m = (double)mf, s = 0.0;
    for (int64_t i = 0; i < n; i++) s += exp((double)z[i] - m);
    return m + log(s);
}

/* math.rs:22-29 */
double orc_confidence(const double *p, int64_t n) {
    if (n <= 1) return 1.0;
    double h = 0.0;
    for (int64_t i = 0; i < n; i++)
        if (p[i] > 0.0) h -= p[i] * log(p[i]);
    double c = 1.0 - h / log((double)n);
    return c < 0.0 ? 0.0 : (c > 1.0 ? 1.0 : c);
}

/* math.rs:59-67 */
int64_t orc_argmax(const double *p, int64_t n) {
    int64_t best = 0;
    for (int64_t i = 0; i < n; i++)
        if (p[i] > p[best]) best = i;
    return best;
}

/* math.rs:41-57: identity, rotations, then reversed rotations. */
int64_t orc_option_orders(int64_t k, int64_t n, int64_t *out) {
    int64_t distinct = k <= 1 ? 1 : (k == 2 ? 2 : 2 * k);
    int64_t cnt = n < distinct ? n : distinct;
    for (int64_t r = 0; r < cnt; r++) {
        int64_t base[256];
        for (int64_t i = 0; i < k; i++) base[i] = r >= k ? k - 1 - i : i;
        int64_t sh = k ? r % k : 0;
        for (int64_t i = 0; i < k; i++) out[r * k + i] = base[(i + sh) % k];
    }
    return cnt;
}

/* readout.rs:124-146 */
void orc_label_readout(const float *row, int64_t vocab, const uint32_t *label_ids, int64_t k,
                       float temperature, float *logits, double *probs, double *candidate_mass) {
    for (int64_t i = 0; i < k; i++) logits[i] = row[label_ids[i]];
    double lse_all = orc_log_sum_exp(row, vocab);
    double lse_labels = orc_log_sum_exp(logits, k);
    orc_softmax(logits, k, temperature, probs);
    *candidate_mass = exp(lse_labels - lse_all);
}

static float dotf(const float *a, const float *b, int64_t n) {
    float s = 0.0f;
    for (int64_t i = 0; i < n; i++) s += a[i] * b[i];
    return s;
}

/* readout.rs:30-43 */
void orc_pointer_logits(int64_t d, int64_t dp, const float *w_q, const float *b_q,
                        const float *w_k, const float *b_k, const float *decide,
                        const float *opts, int64_t nopts, float *out) {
    float *q = (float *)malloc((size_t)dp * 4);
    float *kk = (float *)malloc((size_t)dp * 4);
    for (int64_t r = 0; r < dp; r++) q[r] = dotf(w_q + r * d, decide, d) + b_q[r];
    float scale = 1.0f / sqrtf((float)dp);
    for (int64_t o = 0; o < nopts; o++) {
        for (int64_t r = 0; r < dp; r++) kk[r] = dotf(w_k + r * d, opts + o * d, d) + b_k[r];
        out[o] = dotf(kk, q, dp) * scale;
    }
    free(q);
    free(kk);
}

/* plan.rs:244-271: mean logit per original option over the runs that asked
 * it, accumulated in f64. */
void orc_fold_mean(int64_t k, int64_t nruns, const int64_t *orders, const float *logits,
                   float excluded, float *out) {
    double sum[256] = {0};
    int64_t count[256] = {0};
    for (int64_t r = 0; r < nruns; r++)
        for (int64_t slot = 0; slot < k; slot++) {
            int64_t orig = orders[r * k + slot];
            sum[orig] += (double)logits[r * k + slot];
            count[orig]++;
        }
    for (int64_t o = 0; o < k; o++) out[o] = count[o] ? (float)(sum[o] / (double)count[o]) : excluded;
}
