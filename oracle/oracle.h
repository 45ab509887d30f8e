/*
 * oracle.h -- CPU restatement of the reference's decision-path forward.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (grande_amd/, include/)
 * links, loads or calls this code.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg use it, and only as the checker / the timed CPU
 * baseline.
 *
 * What each part restates (paths relative to the reference checkout):
 *   f16 conversion      IEEE binary16, round-to-nearest-even, as `half::f16`
 *                       (used by crates/omg-wgpu/src/model.rs:403-406,418-419).
 *   xorshift rng        crates/omg-wgpu/tests/reference.rs:17-38
 *   quantize / get      crates/omg-wgpu/src/model.rs:408-466 (Q8_0, Q4_0),
 *                       model.rs:507-525 (element decode)
 *   forward             crates/omg-wgpu/tests/reference.rs:141-349 (rmsnorm,
 *                       linear, rope, gelu, the per-layer loop), with the
 *                       group-aware visibility of shaders/attention.wgsl:70-76
 *   logits              crates/omg-wgpu/tests/reference.rs:564-598
 *   pack                crates/omg-wgpu/src/engine.rs:1479-1581 (order, meta,
 *                       wanted rows, decoded prefixes)
 *   state bytes / key   crates/omg-wgpu/src/engine.rs:510-580 (GRWS1),
 *                       :625-641 (FNV-1a), :1967-1974 (state_rows)
 *   encoder path        laya.c (crates/omg-wgpu/src/laya.rs hidden + score)
 *   readout math        crates/omg-core/src/math.rs:5-67,
 *                       crates/omg-core/src/readout.rs:30-43,124-146,
 *                       crates/omg-core/src/plan.rs:223-303 (fold)
 *
 * Parity pins for each function are listed in tests/test_oracle.py.
 */
#ifndef OMG_ORACLE_H
#define OMG_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_F16 = 0, ORC_Q8 = 1, ORC_Q4 = 2 };
#define ORC_MAX_LAYERS 64
#define ORC_SEQ_GROUP_SHIFT 12

typedef struct {
    int32_t vocab, d, layers, heads, kv_heads;
    int32_t head_dim[ORC_MAX_LAYERS];
    int32_t ff[ORC_MAX_LAYERS];
    int32_t sliding[ORC_MAX_LAYERS];
    int32_t kv_source[ORC_MAX_LAYERS];
    int32_t rope_dims[ORC_MAX_LAYERS];
    float eps;
    int32_t window;
    float theta_global, theta_local, query_scale, norm_offset;
    int32_t v_norm;
    float softcap;
    int32_t bos;
    int32_t per_layer_dim; /* Gemma 4 per-layer inputs (0 = none) */
} orc_config;

/* ---- scalars ---- */
uint16_t orc_f32_to_f16(float x);
float orc_f16_to_f32(uint16_t h);
float orc_rng_next(uint64_t *state);
void orc_rng_values(uint64_t *state, float *out, size_t n, float scale);

/* ---- block formats ---- */
int orc_quantize_q8(const float *v, size_t n, uint8_t *data, uint8_t *scales);
int orc_quantize_q4(const float *v, size_t n, uint8_t *data, uint8_t *scales);
float orc_get(int dtype, const uint8_t *data, const uint8_t *scales, size_t i);

/* ---- model + forward ---- */
typedef struct orc_model orc_model;
/* gpu_rounding = 1 applies the reference GPU path's rounding points
 * (shaders/matmul.wgsl:9 X and W to f16; attention.wgsl:89-90,115-116 Q/K/V
 * to f16); 0 is the plain f32 forward of tests/reference.rs. */
orc_model *orc_model_new(const orc_config *cfg, int gpu_rounding);
void orc_model_free(orc_model *m);
/* Replace the reference's f32 softmax with the rounding points of an f16
 * flash-attention kernel (keys in tiles of key_tile cache rows; running max
 * moved lazily by more than tau log2 units; P rounded to f16; key ranges
 * cut at absolute multiples of chunk_sliding / chunk_global tiles with
 * f16 O / l partials merged by weight).  key_tile = 0 restores the plain
 * softmax.  Models what the HIP attention kernel computes, so tests can
 * bound its difference from the reference with the same rounding. */
int orc_model_set_attention_tiles(orc_model *m, int key_tile, int chunk_sliding, int chunk_global, float tau);
int orc_model_set(orc_model *m, const char *name, int dtype, int64_t rows, int64_t cols,
                  const uint8_t *data, const uint8_t *scales);
/* Missing tensor names, newline separated, into buf; returns their count. */
int orc_model_missing(const orc_model *m, char *buf, size_t len);
/* Final-norm hidden rows for every token of a packed sequence. */
int orc_forward(const orc_model *m, const uint32_t *ids, const int32_t *pos,
                const int32_t *seq, int64_t t, float *hidden);
/* rows . embed^T (+ softcap) for n rows. */
int orc_logits(const orc_model *m, const float *rows, int64_t n, float *out);

/* ---- packing (engine.rs:1479-1581) ---- */
typedef struct {
    const uint32_t *tokens;
    int64_t ntokens;
    const int64_t *want;
    int64_t nwant;
} orc_branch;
typedef struct {
    const uint32_t *prefix;
    int64_t prefix_len;
    const orc_branch *branches;
    int64_t nbranches;
} orc_group;
/* Outputs: ids[total-base], meta[4*(total-base)], wanted[4*rows]
 * (group, branch, slot, workspace row), decoded[2*ngroups] (group, cache
 * row), counts via *n_ids, *n_wanted, *n_decoded.  Returns 0 or a negative
 * error (-1 empty, -2 too many branches, -3 wanted past branch). */
int orc_pack(const orc_group *groups, int64_t ngroups, int64_t first, int resident,
             uint32_t *ids, int32_t *meta, int64_t *wanted, int64_t *decoded,
             int64_t *n_ids, int64_t *n_wanted, int64_t *n_decoded);

/* ---- state (engine.rs:510-641,1967-1974) ---- */
uint64_t orc_state_key(const char *model_id, const uint32_t *prefix, int64_t n);
void orc_state_rows(int sliding, int64_t window, int64_t p, int64_t *r0, int64_t *r1);

/* ---- readout math (omg-core) ---- */
void orc_softmax(const float *z, int64_t n, float temperature, double *out);
double orc_log_sum_exp(const float *z, int64_t n);
double orc_confidence(const double *p, int64_t n);
int64_t orc_argmax(const double *p, int64_t n);
/* Orders r < min(n, distinct) of k options, row-major into out[count*k]. */
int64_t orc_option_orders(int64_t k, int64_t n, int64_t *out);
/* Label readout of one logits row: label logits, probs, candidate mass. */
void orc_label_readout(const float *row, int64_t vocab, const uint32_t *label_ids, int64_t k,
                       float temperature, float *logits, double *probs, double *candidate_mass);
/* PointerHead::logits (readout.rs:30-43): w_q,w_k [dp,d]. */
void orc_pointer_logits(int64_t d, int64_t dp, const float *w_q, const float *b_q,
                        const float *w_k, const float *b_k, const float *decide,
                        const float *opts, int64_t nopts, float *out);
/* Plan::fold core (plan.rs:244-282): runs of (order[k], logits[k]) -> mean
 * logit per original option (EXCLUDED_LOGIT where never asked). */
void orc_fold_mean(int64_t k, int64_t nruns, const int64_t *orders, const float *logits,
                   float excluded, float *out);

/* ---- bidirectional encoder (laya.c: crates/omg-wgpu/src/laya.rs) ---- */
typedef struct {
    int32_t vocab, d, layers, heads, ff, window, head_layers, type_emb, act_hidden, act_out;
    int32_t sliding[ORC_MAX_LAYERS];
    float theta_global, theta_local, eps;
} orc_laya_config;
typedef struct orc_laya orc_laya;
orc_laya *orc_laya_new(const orc_laya_config *cfg);
void orc_laya_free(orc_laya *m);
int orc_laya_set(orc_laya *m, const char *name, int dtype, int64_t rows, int64_t cols, const uint8_t *data,
                 const uint8_t *scales);
int orc_laya_missing(const orc_laya *m, char *buf, size_t len);
/* x after the head layers at rows[0..nrows) of a packed batch; meta = 4
 * int32 per token (position, sequence, first row, last row + 1). */
int orc_laya_hidden(const orc_laya *m, const uint32_t *ids, const int32_t *meta, const int32_t *qtypes, int64_t t,
                    const int64_t *rows, int64_t nrows, float *out);
/* The host scorer on one sequence's rows ([CLS], then each marker). */
void orc_laya_score(const orc_laya *m, const float *rows, int64_t nmarkers, float *logits, float *act);
/* Pieces, exported for their own pins. */
void orc_layer_norm(const float *x, int64_t n, const float *w, const float *b, float eps, float *y);
float orc_erf(float x);
float orc_gelu_erf(float x);
void orc_rope_bi(float *v, int32_t pos, float theta, float scale);
/* y[t][n] = x[t][k] . w[n][k], f32 (reference.rs:150-157). */
void orc_linear(const float *x, int64_t t, int64_t k, const float *w, int64_t n, float *y);

#ifdef __cplusplus
}
#endif
#endif
