/*
 * laya.c -- CPU restatement of the reference's bidirectional encoder pass
 * (crates/omg-wgpu/src/laya.rs: LayaEngine::hidden and score).
 *
 * TEST INFRASTRUCTURE ONLY, like oracle.c: nothing in the product links,
 * loads or calls it.
 *
 * What it follows (paths relative to the reference checkout):
 *   pass plan       crates/omg-wgpu/src/laya.rs:1261-1392 (embed, embed_norm,
 *                   per encoder layer qkv / rope / attention / o / add_o_norm /
 *                   wi / wo / add_wo_norm, type_emb, per head layer norm1 /
 *                   in_proj + bias / attention / out_proj / add_out_norm2 /
 *                   l1 + ReLU / l2 / add_l2(_norm1)), rows read from x
 *                   (:1393-1403)
 *   packing         laya.rs:1165-1187 (meta = position, sequence, first row,
 *                   last row + 1)
 *   LayerNorm       shaders/layernorm.wgsl:53-95 (mean, variance around the
 *                   mean, residual add x + a then + rb)
 *   linears         shaders/matmul.wgsl (X and the decoded W rounded to f16,
 *                   f32 accumulation)
 *   GeGLU (erf)     shaders/matmul_gated.wgsl:114-129, Abramowitz & Stegun
 *                   7.1.26 for erf
 *   RoPE            shaders/rope_bi.wgsl:30-49 (pairs (d, d + 32),
 *                   theta^(-2d/64), q scaled after the rotation)
 *   attention       shaders/attention_bi.wgsl (Q, K, V rounded to f16;
 *                   visible = same sequence and |row difference| <= window
 *                   on local layers; f32 softmax; the head layers' attention
 *                   has no 1/sqrt(head_dim) factor, as the reference runs it)
 *   bias_act        shaders/bias_act.wgsl (y = a + bias, ReLU; the last head
 *                   layer's residual (a + bias) + x)
 *   scorer          laya.rs:1442-1485, 1496-1547
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

static inline float h16(float x) { return orc_f16_to_f32(orc_f32_to_f16(x)); }

typedef struct {
    int present;
    int64_t rows, cols;
    float *w;
} ltensor;

enum { E_ATTN_NORM, E_QKV, E_O, E_MLP_NORM, E_WI_VAL, E_WI_GATE, E_WO, E_COUNT };
static const char *ENC_NAMES[E_COUNT] = {"attn_norm", "qkv", "o", "mlp_norm", "wi_val", "wi_gate", "wo"};
enum {
    H_NORM1_W, H_NORM1_B, H_IN_PROJ, H_IN_PROJ_B, H_OUT_PROJ, H_OUT_PROJ_B,
    H_NORM2_W, H_NORM2_B, H_L1, H_L1_B, H_L2, H_L2_B, H_COUNT
};
static const char *HEAD_NAMES[H_COUNT] = {"norm1_w", "norm1_b", "in_proj", "in_proj_b", "out_proj", "out_proj_b",
                                          "norm2_w", "norm2_b", "l1", "l1_b", "l2", "l2_b"};
enum { G_EMBED, G_EMBED_NORM, G_FINAL_NORM, G_TYPE_EMB, G_S_NORM_W, G_S_NORM_B, G_S_L1, G_S_L1_B, G_S_L2, G_S_L2_B,
       G_A_L1, G_A_L1_B, G_A_L2, G_A_L2_B, G_COUNT };
static const char *GLOBAL_NAMES[G_COUNT] = {"embed", "embed_norm", "final_norm", "type_emb", "scorer.norm_w",
                                            "scorer.norm_b", "scorer.l1", "scorer.l1_b", "scorer.l2",
                                            "scorer.l2_b", "act.l1", "act.l1_b", "act.l2", "act.l2_b"};
#define ORC_MAX_HEAD_LAYERS 8

struct orc_laya {
    orc_laya_config cfg;
    ltensor g[G_COUNT];
    ltensor enc[ORC_MAX_LAYERS][E_COUNT];
    ltensor head[ORC_MAX_HEAD_LAYERS][H_COUNT];
};

orc_laya *orc_laya_new(const orc_laya_config *cfg) {
    if (cfg->layers <= 0 || cfg->layers > ORC_MAX_LAYERS || cfg->head_layers < 0 ||
        cfg->head_layers > ORC_MAX_HEAD_LAYERS || cfg->heads <= 0 || cfg->d != cfg->heads * 64)
        return NULL;
    orc_laya *m = (orc_laya *)calloc(1, sizeof(orc_laya));
    if (m) m->cfg = *cfg;
    return m;
}

static void lfree(ltensor *t) {
    free(t->w);
    t->w = NULL;
    t->present = 0;
}

void orc_laya_free(orc_laya *m) {
    if (!m) return;
    for (int k = 0; k < G_COUNT; k++) lfree(&m->g[k]);
    for (int l = 0; l < ORC_MAX_LAYERS; l++)
        for (int k = 0; k < E_COUNT; k++) lfree(&m->enc[l][k]);
    for (int l = 0; l < ORC_MAX_HEAD_LAYERS; l++)
        for (int k = 0; k < H_COUNT; k++) lfree(&m->head[l][k]);
    free(m);
}

/* Which tensors are GPU linears (their decoded weights rounded to f16). */
static ltensor *llookup(orc_laya *m, const char *name, int *gpu_linear) {
    *gpu_linear = 0;
    for (int k = 0; k < G_COUNT; k++)
        if (!strcmp(name, GLOBAL_NAMES[k])) return &m->g[k];
    int l;
    char rest[64];
    if (sscanf(name, "enc.%d.%63s", &l, rest) == 2) {
        if (l < 0 || l >= m->cfg.layers) return NULL;
        for (int k = 0; k < E_COUNT; k++)
            if (!strcmp(rest, ENC_NAMES[k])) {
                *gpu_linear = k == E_QKV || k == E_O || k == E_WI_VAL || k == E_WI_GATE || k == E_WO;
                return &m->enc[l][k];
            }
        return NULL;
    }
    if (sscanf(name, "head.%d.%63s", &l, rest) == 2) {
        if (l < 0 || l >= m->cfg.head_layers) return NULL;
        for (int k = 0; k < H_COUNT; k++)
            if (!strcmp(rest, HEAD_NAMES[k])) {
                *gpu_linear = k == H_IN_PROJ || k == H_OUT_PROJ || k == H_L1 || k == H_L2;
                return &m->head[l][k];
            }
    }
    return NULL;
}

int orc_laya_set(orc_laya *m, const char *name, int dtype, int64_t rows, int64_t cols, const uint8_t *data,
                 const uint8_t *scales) {
    int lin;
    ltensor *t = llookup(m, name, &lin);
    if (!t) return -1;
    const int64_t n = rows * cols;
    lfree(t);
    t->w = (float *)malloc((size_t)n * sizeof(float));
    if (!t->w) return -2;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++) {
        const float v = orc_get(dtype, data, scales, (size_t)i);
        t->w[i] = lin ? h16(v) : v;
    }
    t->rows = rows;
    t->cols = cols;
    t->present = 1;
    return 0;
}

int orc_laya_missing(const orc_laya *m, char *buf, size_t len) {
    int count = 0;
    size_t at = 0;
    if (buf && len) buf[0] = 0;
    char nm[80];
#define LMISS(s)                                                                    \
    do {                                                                            \
        count++;                                                                    \
        if (buf && at < len) at += (size_t)snprintf(buf + at, len - at, "%s\n", s); \
    } while (0)
    for (int k = 0; k < G_COUNT; k++) {
        if (k == G_TYPE_EMB && !m->cfg.type_emb) continue;
        if (k >= G_A_L1 && m->cfg.act_out == 0) continue;
        if (!m->g[k].present) LMISS(GLOBAL_NAMES[k]);
    }
    for (int l = 0; l < m->cfg.layers; l++)
        for (int k = 0; k < E_COUNT; k++) {
            if (k == E_ATTN_NORM && l == 0) continue;
            if (!m->enc[l][k].present) {
                snprintf(nm, sizeof nm, "enc.%d.%s", l, ENC_NAMES[k]);
                LMISS(nm);
            }
        }
    for (int l = 0; l < m->cfg.head_layers; l++)
        for (int k = 0; k < H_COUNT; k++)
            if (!m->head[l][k].present) {
                snprintf(nm, sizeof nm, "head.%d.%s", l, HEAD_NAMES[k]);
                LMISS(nm);
            }
#undef LMISS
    return count;
}

/* layernorm.wgsl:53-95 on one row (b may be NULL). */
void orc_layer_norm(const float *x, int64_t n, const float *w, const float *b, float eps, float *y) {
    float s = 0.0f;
    for (int64_t i = 0; i < n; i++) s += x[i];
    const float mean = s / (float)n;
    float q = 0.0f;
    for (int64_t i = 0; i < n; i++) q += (x[i] - mean) * (x[i] - mean);
    const float inv = 1.0f / sqrtf(q / (float)n + eps);
    for (int64_t i = 0; i < n; i++) y[i] = (x[i] - mean) * inv * w[i] + (b ? b[i] : 0.0f);
}

/* Abramowitz & Stegun 7.1.26 (matmul_gated.wgsl:117-124, laya.rs:1529-1546). */
float orc_erf(float x) {
    const float s = x > 0.0f ? 1.0f : (x < 0.0f ? -1.0f : 0.0f);
    const float a = fabsf(x);
    const float t = 1.0f / (1.0f + 0.3275911f * a);
    const float poly = ((((1.061405429f * t - 1.453152027f) * t + 1.421413741f) * t - 0.284496736f) * t +
                        0.254829592f) * t;
    return s * (1.0f - poly * expf(-a * a));
}

float orc_gelu_erf(float x) { return 0.5f * x * (1.0f + orc_erf(x * 0.70710678118654752f)); }

/* rope_bi.wgsl:30-49 on one 64-wide head row at position pos. */
void orc_rope_bi(float *v, int32_t pos, float theta, float scale) {
    for (int d = 0; d < 32; d++) {
        const float ang = (float)pos * powf(theta, -(float)(2 * d) / 64.0f);
        const float c = cosf(ang), s = sinf(ang);
        const float a = v[d], b = v[d + 32];
        v[d] = (a * c - b * s) * scale;
        v[d + 32] = (b * c + a * s) * scale;
    }
}

/* y[t][n] = f16(x)[t][k] . W[n][k] (W already rounded), f32 sums. */
static void lin16(const float *x, int64_t t, int64_t k, const ltensor *w, float *y) {
    float *xr = (float *)malloc((size_t)(t * k) * sizeof(float));
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < t * k; i++) xr[i] = h16(x[i]);
    orc_linear(xr, t, k, w->w, w->rows, y);
    free(xr);
}

/* attention_bi.wgsl over the packed batch: qkv [t][3d] (f32, rotated),
 * out [t][d]. */
static void attention(const orc_laya *m, const float *qkv, const int32_t *meta, int64_t t, int window, float *out) {
    const int64_t d = m->cfg.d, H = m->cfg.heads;
#pragma omp parallel for schedule(dynamic, 4)
    for (int64_t i = 0; i < t; i++) {
        int64_t lo = meta[4 * i + 2], hi = meta[4 * i + 3];
        if (window > 0) {
            if (lo < i - window) lo = i - window;
            if (hi > i + window + 1) hi = i + window + 1;
        }
        float *p = (float *)malloc((size_t)(hi - lo) * sizeof(float));
        for (int64_t g = 0; g < H; g++) {
            const float *q = qkv + i * 3 * d + g * 64;
            float mx = -INFINITY;
            for (int64_t j = lo; j < hi; j++) {
                const float *k = qkv + j * 3 * d + d + g * 64;
                float s = 0.0f;
                for (int c = 0; c < 64; c++) s += h16(q[c]) * h16(k[c]);
                p[j - lo] = s;
                if (s > mx) mx = s;
            }
            float l = 0.0f;
            for (int64_t j = lo; j < hi; j++) {
                p[j - lo] = expf(p[j - lo] - mx);
                l += p[j - lo];
            }
            float acc[64] = {0};
            for (int64_t j = lo; j < hi; j++) {
                const float *v = qkv + j * 3 * d + 2 * d + g * 64;
                for (int c = 0; c < 64; c++) acc[c] += p[j - lo] * h16(v[c]);
            }
            for (int c = 0; c < 64; c++) out[i * d + g * 64 + c] = acc[c] / l;
        }
        free(p);
    }
}

int orc_laya_hidden(const orc_laya *m, const uint32_t *ids, const int32_t *meta, const int32_t *qtypes, int64_t t,
                    const int64_t *rows, int64_t nrows, float *out) {
    const orc_laya_config *c = &m->cfg;
    if (orc_laya_missing(m, NULL, 0)) return -1;
    const int64_t d = c->d, ff = c->ff, f4 = 4 * d;
    const int64_t wide = ff > f4 ? ff : f4;
    float *x = (float *)malloc((size_t)(t * d) * sizeof(float));
    float *h = (float *)malloc((size_t)(t * d) * sizeof(float));
    float *qkv = (float *)malloc((size_t)(t * 3 * d) * sizeof(float));
    float *at = (float *)malloc((size_t)(t * d) * sizeof(float));
    float *a = (float *)malloc((size_t)(t * d) * sizeof(float));
    float *g = (float *)malloc((size_t)(t * wide) * sizeof(float));
    float *u = (float *)malloc((size_t)(t * wide) * sizeof(float));
    if (!x || !h || !qkv || !at || !a || !g || !u) return -2;
    const ltensor *E = &m->g[G_EMBED];
    /* embed (scale 1) then embed_norm into x (laya.rs:1261-1269). */
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < t; i++) {
        for (int64_t k = 0; k < d; k++) h[i * d + k] = E->w[(int64_t)ids[i] * d + k];
        orc_layer_norm(h + i * d, d, m->g[G_EMBED_NORM].w, NULL, c->eps, x + i * d);
    }
    for (int l = 0; l < c->layers; l++) {
        const ltensor *L = m->enc[l];
        const int last = l + 1 == c->layers;
        lin16(l > 0 ? h : x, t, d, &L[E_QKV], qkv);
        const float theta = c->sliding[l] ? c->theta_local : c->theta_global;
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < t; i++)
            for (int64_t hh = 0; hh < c->heads; hh++) {
                orc_rope_bi(qkv + i * 3 * d + hh * 64, meta[4 * i], theta, 0.125f);
                orc_rope_bi(qkv + i * 3 * d + d + hh * 64, meta[4 * i], theta, 1.0f);
            }
        attention(m, qkv, meta, t, c->sliding[l] ? c->window : 0, at);
        lin16(at, t, d, &L[E_O], a);
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < t; i++) {
            for (int64_t k = 0; k < d; k++) x[i * d + k] += a[i * d + k];
            orc_layer_norm(x + i * d, d, L[E_MLP_NORM].w, NULL, c->eps, h + i * d);
        }
        lin16(h, t, d, &L[E_WI_VAL], g);
        lin16(h, t, d, &L[E_WI_GATE], u);
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < t * ff; i++) g[i] = orc_gelu_erf(g[i]) * u[i];
        lin16(g, t, ff, &L[E_WO], a);
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < t; i++) {
            for (int64_t k = 0; k < d; k++) x[i * d + k] += a[i * d + k];
            if (!last) {
                orc_layer_norm(x + i * d, d, m->enc[l + 1][E_ATTN_NORM].w, NULL, c->eps, h + i * d);
            } else {
                float row[2048];
                orc_layer_norm(x + i * d, d, m->g[G_FINAL_NORM].w, NULL, c->eps, row);
                memcpy(x + i * d, row, (size_t)d * sizeof(float));
            }
        }
    }
    if (c->type_emb) {
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < t; i++)
            for (int64_t k = 0; k < d; k++) x[i * d + k] += m->g[G_TYPE_EMB].w[(int64_t)qtypes[i] * d + k];
    }
    for (int hl = 0; hl < c->head_layers; hl++) {
        const ltensor *Hd = m->head[hl];
        const int last = hl + 1 == c->head_layers;
        if (hl == 0) {
#pragma omp parallel for schedule(static)
            for (int64_t i = 0; i < t; i++)
                orc_layer_norm(x + i * d, d, Hd[H_NORM1_W].w, Hd[H_NORM1_B].w, c->eps, h + i * d);
        }
        lin16(h, t, d, &Hd[H_IN_PROJ], qkv);
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < t; i++)
            for (int64_t k = 0; k < 3 * d; k++) qkv[i * 3 * d + k] += Hd[H_IN_PROJ_B].w[k];
        attention(m, qkv, meta, t, 0, at);
        lin16(at, t, d, &Hd[H_OUT_PROJ], a);
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < t; i++) {
            for (int64_t k = 0; k < d; k++) x[i * d + k] = (x[i * d + k] + a[i * d + k]) + Hd[H_OUT_PROJ_B].w[k];
            orc_layer_norm(x + i * d, d, Hd[H_NORM2_W].w, Hd[H_NORM2_B].w, c->eps, h + i * d);
        }
        lin16(h, t, d, &Hd[H_L1], g);
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < t; i++)
            for (int64_t k = 0; k < f4; k++) {
                const float y = g[i * f4 + k] + Hd[H_L1_B].w[k];
                g[i * f4 + k] = y > 0.0f ? y : 0.0f;
            }
        lin16(g, t, f4, &Hd[H_L2], a);
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < t; i++) {
            if (last) {
                for (int64_t k = 0; k < d; k++) x[i * d + k] = (a[i * d + k] + Hd[H_L2_B].w[k]) + x[i * d + k];
            } else {
                for (int64_t k = 0; k < d; k++) x[i * d + k] = (x[i * d + k] + a[i * d + k]) + Hd[H_L2_B].w[k];
                orc_layer_norm(x + i * d, d, m->head[hl + 1][H_NORM1_W].w, m->head[hl + 1][H_NORM1_B].w, c->eps,
                               h + i * d);
            }
        }
    }
    for (int64_t r = 0; r < nrows; r++) memcpy(out + r * d, x + rows[r] * d, (size_t)d * sizeof(float));
    free(x);
    free(h);
    free(qkv);
    free(at);
    free(a);
    free(g);
    free(u);
    return 0;
}

static float ldot(const float *a, const float *b, int64_t n) {
    float s = 0.0f;
    for (int64_t i = 0; i < n; i++) s += a[i] * b[i];
    return s;
}

static void lsoftmax(const float *z, int64_t n, float *p) {
    float m = -INFINITY, s = 0.0f;
    for (int64_t i = 0; i < n; i++) m = z[i] > m ? z[i] : m;
    for (int64_t i = 0; i < n; i++) {
        p[i] = expf(z[i] - m);
        s += p[i];
    }
    for (int64_t i = 0; i < n; i++) p[i] /= s;
}

static int cmpf(const void *a, const void *b) {
    const float x = *(const float *)a, y = *(const float *)b;
    return x < y ? -1 : (x > y ? 1 : 0);
}

/* laya.rs:1442-1485 on one sequence's rows ([CLS], then the markers). */
void orc_laya_score(const orc_laya *m, const float *rows, int64_t nmarkers, float *logits, float *act) {
    const int64_t d = m->cfg.d;
    float *z = (float *)malloc((size_t)d * sizeof(float));
    float *y = (float *)malloc((size_t)d * sizeof(float));
    for (int64_t j = 0; j < nmarkers; j++) {
        orc_layer_norm(rows + (1 + j) * d, d, m->g[G_S_NORM_W].w, m->g[G_S_NORM_B].w, m->cfg.eps, z);
        for (int64_t r = 0; r < d; r++) y[r] = orc_gelu_erf(ldot(m->g[G_S_L1].w + r * d, z, d) + m->g[G_S_L1_B].w[r]);
        logits[j] = ldot(y, m->g[G_S_L2].w, d) + m->g[G_S_L2_B].w[0];
    }
    free(z);
    free(y);
    if (m->cfg.act_out == 0) {
        *act = NAN;
        return;
    }
    const int64_t k = nmarkers > 2 ? nmarkers : 2;
    float *pad = (float *)malloc((size_t)k * sizeof(float));
    float *p = (float *)malloc((size_t)k * sizeof(float));
    for (int64_t j = 0; j < k; j++) pad[j] = j < nmarkers ? logits[j] : -1e4f;
    lsoftmax(pad, k, p);
    float ent = 0.0f;
    for (int64_t j = 0; j < k; j++) ent += p[j] * logf(p[j] > 1e-9f ? p[j] : 1e-9f);
    const float entropy = -ent / logf((float)k);
    qsort(p, (size_t)k, sizeof(float), cmpf);
    const float top1 = p[k - 1], top2 = p[k - 2];
    const int64_t hid = m->cfg.act_hidden, nout = m->cfg.act_out;
    float *pooled = (float *)malloc((size_t)(d + 4) * sizeof(float));
    memcpy(pooled, rows, (size_t)d * sizeof(float));
    pooled[d] = top1;
    pooled[d + 1] = top1 - top2;
    pooled[d + 2] = entropy;
    pooled[d + 3] = (float)k / 255.0f;
    float *hv = (float *)malloc((size_t)hid * sizeof(float));
    for (int64_t r = 0; r < hid; r++)
        hv[r] = orc_gelu_erf(ldot(m->g[G_A_L1].w + r * (d + 4), pooled, d + 4) + m->g[G_A_L1_B].w[r]);
    float *o = (float *)malloc((size_t)nout * sizeof(float));
    float *po = (float *)malloc((size_t)nout * sizeof(float));
    for (int64_t r = 0; r < nout; r++) o[r] = ldot(m->g[G_A_L2].w + r * hid, hv, hid) + m->g[G_A_L2_B].w[r];
    lsoftmax(o, nout, po);
    *act = po[0];
    free(pad);
    free(p);
    free(pooled);
    free(hv);
    free(o);
    free(po);
}
