/*
 * omg_hip.h -- C ABI of the MI355X decision-path engine.
 *
 * This is the drop-in boundary for the reference's omg-wgpu engine surface
 * (bokuweb/grande, crates/omg-wgpu): load a checkpoint, run
 * forward(state, branches) as one block-causal pass, read out rows at the
 * wanted positions, and keep / serialise / restore the state's f16 K/V.
 * Each entry point names the reference item it replaces (path:line in the
 * reference checkout).
 *
 * Conventions
 *   - Opaque handles; plain pointers and sizes; no exceptions cross.
 *   - Status: 0 = ok, negative = error class (OMG_E_*); omg_last_error()
 *     returns the calling thread's last message (the reference's anyhow
 *     strings, engine.rs:1503-1581).  Functions returning a handle return
 *     NULL on failure.
 *   - One engine is not thread-safe; callers serialise (the reference's
 *     server gives the engine one thread, omg-server/src/lib.rs:57-99).
 *   - Token ids are uint32 in the checkpoint's vocabulary.
 */
#ifndef OMG_HIP_H
#define OMG_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OMG_OK 0
#define OMG_E_INVALID (-1)  /* bad argument or request */
#define OMG_E_CAPACITY (-2) /* capacity / max_rows / 4095-branch limits */
#define OMG_E_DEVICE (-3)   /* HIP runtime failure */
#define OMG_E_STATE (-4)    /* state bytes rejected */
#define OMG_E_IO (-5)       /* file system */
#define OMG_E_MISSING (-6)  /* tensors missing at finish */

/* model.rs:337-371 Dtype (codes = Dtype::code) */
#define OMG_DTYPE_F16 0
#define OMG_DTYPE_Q8 1
#define OMG_DTYPE_Q4 2

/* omg-core backend.rs:14-20 Want.  OMG_WANT_LABELS and OMG_WANT_LABELS_LSE
 * have no counterpart in the reference, whose Readout::distribution
 * (readout.rs:124-146) reads the full logits row on the host to pick the
 * label columns and take log_sum_exp (math.rs:13-17) for candidate_mass:
 *   LABELS      k floats per row: the logits of the given label ids;
 *   LABELS_LSE  k + 1 floats per row: the same k logits, then the
 *               log-sum-exp of the row over the whole vocabulary (f32), so
 *               candidate_mass = exp(lse(labels) - row[k]) needs no
 *               vocabulary-wide readback. */
#define OMG_WANT_LOGITS 0
#define OMG_WANT_HIDDEN 1
#define OMG_WANT_LABELS 2
#define OMG_WANT_LABELS_LSE 3

/* omg-core backend.rs:92-104 PrefixSource (0 = none yet) */
#define OMG_SRC_NONE 0
#define OMG_SRC_RESIDENT 1
#define OMG_SRC_RAM 2
#define OMG_SRC_DISK 3
#define OMG_SRC_DECODED 4

typedef struct omg_engine omg_engine;
typedef struct omg_builder omg_builder;

/* omg-core backend.rs:22-30 BranchTokens: tokens + ascending wanted indices. */
typedef struct {
    const uint32_t *tokens;
    size_t ntokens;
    const uint32_t *want;
    size_t nwant;
} omg_branch;

/* omg-core backend.rs:38-45 / engine.rs:26-38 Group. */
typedef struct {
    const uint32_t *prefix;
    size_t prefix_len;
    const omg_branch *branches;
    size_t nbranches;
} omg_group;

/* The Backend facts callers read: n_embd / n_vocab / bos (backend.rs:124-128)
 * and the shape the engine was built for (model.rs:27-63). */
typedef struct {
    uint32_t vocab, d, layers, heads, kv_heads, head_dim, bos;
    uint64_t capacity, max_rows;
} omg_config_t;

/* Thread-local message of the last failure on this thread. */
const char *omg_last_error(void);

/* ---- loading (engine.rs:763-1335, backend.rs:28-71) ---- */

/* EngineBuilder::new(Config::from_json(config.json)) (engine.rs:845-869). */
omg_builder *omg_builder_new(const char *config_json);
/* EngineBuilder::push (engine.rs:888-933): one catalogued tensor, encoded as
 * model.rs QTensor (payload + f16 block scales for Q8/Q4). */
int omg_builder_push(omg_builder *b, const char *name, int dtype, const int64_t *shape, size_t ndim,
                     const void *data, size_t nbytes, const void *scales, size_t nscale_bytes);
/* A host checkpoint (model.rs:540-546 Weights): the seeded random weights
 * of tests/reference.rs:106-139 for a config (linears in `linear_dtype`,
 * the embedding in `embed_dtype`), or an exported directory
 * (model.rs:742-795).  Tensors are in the reference's QTensor encoding;
 * omg_weights_get hands out borrowed pointers valid until omg_weights_free. */
typedef struct omg_weights omg_weights;
omg_weights *omg_synth(const char *config_json, uint64_t seed, int linear_dtype, int embed_dtype);
omg_weights *omg_load_dir(const char *dir);
size_t omg_weights_count(const omg_weights *w);
int omg_weights_get(const omg_weights *w, size_t i, const char **name, int *dtype, int64_t *shape,
                    size_t *ndim, const uint8_t **data, size_t *nbytes, const uint8_t **scales,
                    size_t *nscale_bytes);
void omg_weights_free(omg_weights *w);
/* A llama.cpp GGUF file (v2/v3, gemma3) read directly: the metadata and
 * tensor mapping of tools/export_wgpu_gguf.py:112-296 (q / k / v fused per
 * layer, Q8_0 / Q4_0 blocks split into codes and scales, f32 / bf16 to
 * f16).  The reference reaches a GGUF through that export step; this reads
 * the file itself. */
omg_weights *omg_load_gguf(const char *path);
/* Engine::new's loop over the catalogue (engine.rs:1341-1351). */
int omg_builder_push_weights(omg_builder *b, const omg_weights *w);
/* EngineBuilder::missing (engine.rs:875-885): newline-separated names into
 * buf; returns how many are missing. */
size_t omg_builder_missing(omg_builder *b, char *buf, size_t len);
/* EngineBuilder::finish (engine.rs:952-1334).  Consumes the builder even on
 * failure. */
omg_engine *omg_builder_finish(omg_builder *b, size_t capacity, size_t max_rows);
void omg_builder_free(omg_builder *b);
/* WgpuBackend::load for an exported directory: config.json + manifest.json
 * + *.bin (backend.rs:28-71, model.rs:742-795). */
omg_engine *omg_open_dir(const char *dir, size_t capacity, size_t max_rows);
/* An engine straight from a GGUF file (omg_load_gguf's tensors). */
omg_engine *omg_open_gguf(const char *path, size_t capacity, size_t max_rows);
void omg_close(omg_engine *e);
int omg_config(const omg_engine *e, omg_config_t *out);
/* Engine::warmup (engine.rs:1356-1366). */
int omg_warmup(omg_engine *e);

/* ---- the pass (engine.rs:1386-1940) ---- */

/* Engine::evaluate_groups / Backend::evaluate_many (engine.rs:1404-1444,
 * backend.rs:142-152).  Rows are written densely into `out` in (group,
 * branch, want) order; width n_embd (HIDDEN), n_vocab (LOGITS), nlabels
 * (LABELS, with label_ids) or nlabels + 1 (LABELS_LSE).  prefix_sources (may be NULL) gets one
 * OMG_SRC_* per group. */
int omg_evaluate_groups(omg_engine *e, const omg_group *groups, size_t ngroups, int want,
                        const uint32_t *label_ids, size_t nlabels, float *out, size_t out_floats,
                        int *prefix_sources);
/* Readout::Pointer's head (omg-core readout.rs:17-29, PointerHead): two
 * affine maps d -> dp, weights row-major [dp][d] and biases [dp], f32; the
 * engine keeps a device copy.  w_q = NULL clears it. */
int omg_set_pointer_head(omg_engine *e, size_t d, size_t dp, const float *w_q, const float *b_q,
                         const float *w_k, const float *b_k);
/* The roles of wanted rows for omg_evaluate_pointer (readout.rs Mark). */
#define OMG_ROLE_NONE 0   /* Mark::Last: not scored */
#define OMG_ROLE_OPT 1    /* Mark::OptEnd: an option's `</opt>` row */
#define OMG_ROLE_DECIDE 2 /* Mark::Decide: the `<decide>` row */
/* Readout::distribution's pointer branch (readout.rs:149-173) on the
 * device: omg_evaluate_groups with Want::Hidden whose rows are scored by the
 * pointer head (readout.rs:37-44) instead of read back.  roles: one per
 * wanted row in (group, branch, want) order, each branch with exactly one
 * OMG_ROLE_DECIDE row ("no decide row" otherwise).  out: each branch's
 * option logits (its OMG_ROLE_OPT rows in want order), branch after branch
 * in (group, branch) order; *written (may be NULL) = their count. */
int omg_evaluate_pointer(omg_engine *e, const omg_group *groups, size_t ngroups, const uint8_t *roles,
                         size_t nroles, float *out, size_t out_floats, size_t *written, int *prefix_sources);
/* Engine::evaluate (engine.rs:1386-1396): one group. */
int omg_evaluate(omg_engine *e, const uint32_t *prefix, size_t prefix_len, const omg_branch *branches,
                 size_t nbranches, int want, const uint32_t *label_ids, size_t nlabels, float *out,
                 size_t out_floats);
/* Engine::prefix_source (engine.rs:2158-2161): OMG_SRC_* of the last pass. */
int omg_prefix_source(const omg_engine *e);
/* Engine::is_resident (engine.rs:2152-2156). */
int omg_is_resident(const omg_engine *e, const uint32_t *prefix, size_t n);
/* Engine::evict_resident (engine.rs:2163-2166). */
void omg_evict_resident(omg_engine *e);

/* ---- state (engine.rs:499-641, 1942-2150) ---- */

/* Engine::set_state_cache (engine.rs:1945-1954): RAM LRU of `bytes`, files
 * in `dir` (NULL or "" = none), states tagged with `model_id`. */
int omg_set_state_cache(omg_engine *e, size_t bytes, const char *dir, const char *model_id);
/* Engine::save_state + SavedState::to_bytes (engine.rs:1977-1979, 517-534):
 * the GRWS1 bytes of the prefix at cache rows 0..n; free with
 * omg_free_bytes. */
int omg_save_state(omg_engine *e, const uint32_t *prefix, size_t n, const char *model_id, uint8_t **bytes,
                   size_t *len);
/* SavedState::from_bytes + Engine::restore_state (engine.rs:536-579,
 * 2051-2092): the prefix is resident afterwards. */
int omg_restore_state(omg_engine *e, const uint8_t *bytes, size_t len, const char *model_id);
void omg_free_bytes(uint8_t *p);

/* ---- host-side pieces (no GPU needed) ---- */

/* QTensor::quantize_q8 / quantize_q4 (model.rs:408-466); dtype Q8 or Q4. */
int omg_quantize(int dtype, const float *values, size_t n, uint8_t *data, uint8_t *scales);
/* The packing of Engine::run (engine.rs:1512-1571) with `first` laid out
 * first and its prefix resident when `resident`: ids, meta (4 int32 per
 * token: position, sequence id, first key row, own row + 1) and wanted
 * (4 int64 per row: group, branch, slot, workspace row).  Sizes in/out.
 * align <= 1 gives the reference's layout; align > 1 the engine's own,
 * where every group after the first starts on a multiple of `align` cache
 * rows (padding rows: token 0, sequence id -1), unless that needs more
 * than `rows` rows. */
int omg_pack(const omg_group *groups, size_t ngroups, size_t first, int resident, size_t align, size_t rows,
             uint32_t *ids, int32_t *meta, int64_t *wanted, size_t *n_ids, size_t *n_wanted);
/* state_key (engine.rs:625-641): FNV-1a 64 of model id, 0, prefix. */
uint64_t omg_state_key(const char *model_id, const uint32_t *prefix, size_t n);
/* SavedState::from_bytes (engine.rs:536-579) without an engine: 0 and the
 * prefix length / layer count, or OMG_E_STATE with the reason. */
int omg_state_check(const uint8_t *bytes, size_t len, const char *model_id, size_t *prefix_len,
                    size_t *nlayers);

/* ---- measurement (no counterpart in the reference; bench.py and the
 * kernel tests use them) ---- */

/* Pack + upload one request whose first group's prefix is resident (or not)
 * and keep it for omg_pass_launch, which replays the pass's device work
 * (forward + readout at the wanted rows) on the engine's stream with no host
 * transfer.  omg_sync waits for it.  Any evaluate (omg_evaluate_groups,
 * omg_evaluate_pointer) or omg_restore_state in between uploads over the
 * prepared pass's inputs and cancels it: omg_pass_launch, omg_pass_graph
 * and omg_pass_read then fail with "no prepared pass" until the next
 * omg_pass_prepare. */
int omg_pass_prepare(omg_engine *e, const omg_group *groups, size_t ngroups, int want,
                     const uint32_t *label_ids, size_t nlabels, int first_resident);
int omg_pass_launch(omg_engine *e);
/* No counterpart in the reference (it records one command buffer per
 * request, engine.rs:1761-1861): capture the prepared pass's kernel
 * launches into a HIP graph (on != 0), which omg_pass_launch then replays
 * as one submission; on = 0, the next omg_pass_prepare or any evaluate
 * drops it. */
int omg_pass_graph(omg_engine *e, int on);
/* The prepared pass's rows after its launches (waits for them), in wanted
 * order (group, branch, slot), width as omg_evaluate_groups gives them. */
int omg_pass_read(omg_engine *e, float *out, size_t out_floats, size_t *written);
int omg_sync(omg_engine *e);
/* HIP-event time per kernel of every launch while on; the report is lines
 * "name launches total_ms". */
int omg_profile(omg_engine *e, int on);
size_t omg_profile_report(omg_engine *e, char *buf, size_t len);
/* No counterpart in the reference, whose pass runs every layer for every
 * row (engine.rs:1674-1751).  By default, from the last layer that writes
 * K/V (the model's last layer, or with Gemma 4's K/V-sharing layers the
 * last layer before them) past its attention, the pass runs for the rows a
 * request reads out only: that layer's attention for the query tiles that
 * hold them, then o, norms, gate/up, down and the per-layer block on the
 * gathered rows, and every later layer on those rows alone (its keys and
 * values are an earlier layer's cache, so no other row reaches them).
 * Every K/V cache is still written for every row.  on != 0 runs every
 * layer for every row as the reference does.  The rows a pass returns are
 * the same bits either way.  From the next pass on. */
int omg_set_full_last_layer(omg_engine *e, int on);

/* Kernel-level entry points on device pointers (the reference's matmul.rs
 * kernel tests): a weight uploaded in the device layout, then
 * Y[m][N] = f16(X)[m][K] . W^T (f32) or act = gelu(X.Wg^T) * (X.Wu^T)
 * (f16).  stream NULL = the null stream. */
typedef struct omg_weight omg_weight;
omg_weight *omg_weight_upload(int dtype, int64_t rows, int64_t cols, const void *data, const void *scales);
void omg_weight_free(omg_weight *w);
int omg_dev_gemm(const omg_weight *w, const void *x_f16, int64_t ldx, int64_t m, float *y, int64_t ldy,
                 void *stream);
int omg_dev_gemm_geglu(const omg_weight *wg, const omg_weight *wu, const void *x_f16, int64_t ldx, int64_t m,
                       void *act_f16, int64_t ldact, void *stream);
/* The label readout on device pointers (logits.wgsl's product, then what
 * readout.rs:124-146 takes from the row): rows f32 [nrows][d] times the
 * embedding `embed` [vocab][d] in f32, softcap applied when > 0, then per
 * row the logits of the device-resident label ids and the log-sum-exp of
 * the full vocabulary row: out f32 [nrows][nlabels + 1].  `rows` must be
 * 16-byte aligned.  Label ids must be below vocab; the device-resident ids
 * are not checked before the launch, and an id past the vocabulary gives
 * NaN in its column.  The full logits and per-workgroup partials live in
 * scratch device memory the call allocates and frees in stream order. */
int omg_dev_label_readout(const omg_weight *embed, const float *rows, int64_t nrows, const uint32_t *labels,
                          int64_t nlabels, float softcap, float *out, void *stream);
/* No counterpart in the reference.  omg_dev_label_readout for callers that
 * cannot allocate (code under HIP graph capture, tight serving loops):
 * same arguments and results, nothing allocated; its scratch is a fixed
 * 16 MiB device array per GPU (4,194,304 floats), which must hold
 * nrows * vocab (rounded up to even) + 2 * nrows * ceil(vocab / 64) floats,
 * else OMG_E_CAPACITY.
 * Calls that overlap on one GPU share that array and race. */
int omg_dev_label_readout_noalloc(const omg_weight *embed, const float *rows, int64_t nrows, const uint32_t *labels,
                                  int64_t nlabels, float softcap, float *out, void *stream);
/* The embedding gather + first norm kernel (embed.wgsl + rmsnorm.wgsl):
 * x[t][d] = deq(E[ids[t]]) * scale (f32), hn[t][d] = f16(rmsnorm(x) * w)
 * with w (f32, d entries) already offset.  Device pointers. */
int omg_dev_embed_norm(const omg_weight *embed, const uint32_t *ids, int64_t t, float scale, const float *w,
                       float eps, float *x, void *hn_f16, void *stream);

/* Kernel-level entry points of the encoder path, on device pointers:
 * the gated GEMM with the exact (erf) GELU (matmul_gated.wgsl GELU_ERF = 1);
 * Y = f16(max(X.W^T + bias, 0)) (matmul.wgsl then bias_act.wgsl mode 1);
 * the fused [q | k | v] projection scattered per 64-wide head as f16 with
 * bias, RoPE from `rope` ([pos][32] (cos, sin) pairs; NULL = none, then
 * `meta` may be NULL) and the q scale (rope_bi.wgsl): q16 / k16
 * [heads][tpad][64], vt [heads][tpad/32][64][32] with key k of a tile at
 * column 8*((k%16)/4) + 4*(k/16) + k%4; and the bidirectional attention
 * over those arrays (attention_bi.wgsl): out [t][heads*64] f16. */
int omg_dev_gemm_geglu_erf(const omg_weight *wg, const omg_weight *wu, const void *x_f16, int64_t ldx, int64_t m,
                           void *act_f16, int64_t ldact, void *stream);
int omg_dev_gemm_bias_relu(const omg_weight *w, const void *x_f16, int64_t ldx, int64_t m, const void *bias_f16,
                           void *y_f16, int64_t ldy, void *stream);
int omg_dev_qkv_heads(const omg_weight *w, const void *x_f16, int64_t ldx, int64_t m, const void *bias_f16,
                      const float *rope, const int32_t *meta, float qscale, int64_t tpad, void *q16, void *k16,
                      void *vt, void *stream);
int omg_dev_attention_bi(const void *q16, const void *k16, const void *vt, const int32_t *meta, int heads, int64_t t,
                         int64_t tpad, int window, void *out_f16, void *stream);

/* ---- the bidirectional encoder path (crates/omg-wgpu/src/laya.rs) ----
 * An mmBERT / ModernBERT encoder with Laya's decision head: every question
 * is one sequence; a request's sequences run as one packed pass isolated by
 * the attention mask; the scorer reads the [CLS] and [MASK] rows on the
 * host. */
typedef struct omg_laya omg_laya;
typedef struct omg_laya_builder omg_laya_builder;

/* laya.rs:468-476 Sequence: token ids, the token index of each option's
 * [MASK] (option order), question type (0 choice, 1 score, 2 noul). */
typedef struct {
    const uint32_t *ids;
    size_t nids;
    const uint32_t *markers;
    size_t nmarkers;
    int qtype;
} omg_laya_seq;

typedef struct {
    uint32_t vocab, d, layers, heads, ff, head_layers, act_out, max_len;
    uint32_t cls, sep, mask, pad;
    uint64_t capacity, max_rows;
} omg_laya_config_t;

/* LayaBuilder::new(config_from_export(config.json)) (laya.rs:312-323,
 * 623-645): the encoder config.json with the agent config under
 * "laya_agent" and the special token ids under "laya_tokens"
 * ({"cls_token": id, ...}; the reference resolves surface forms with its
 * tokenizer, which stays on the caller's side). */
omg_laya_builder *omg_laya_builder_new(const char *config_json);
/* LayaBuilder::push (laya.rs:662-709). */
int omg_laya_builder_push(omg_laya_builder *b, const char *name, int dtype, const int64_t *shape, size_t ndim,
                          const void *data, size_t nbytes, const void *scales, size_t nscale_bytes);
/* LayaEngine::new's loop over the catalogue (laya.rs:1115-1124). */
int omg_laya_builder_push_weights(omg_laya_builder *b, const omg_weights *w);
/* LayaBuilder::missing (laya.rs:651-660). */
size_t omg_laya_builder_missing(omg_laya_builder *b, char *buf, size_t len);
/* LayaBuilder::finish (laya.rs:711-1083); consumes the builder. */
omg_laya *omg_laya_builder_finish(omg_laya_builder *b, size_t capacity, size_t max_rows);
void omg_laya_builder_free(omg_laya_builder *b);
/* Seeded weights for a config (LayaConfig::tensors order, laya.rs:252-305)
 * from the xorshift of tests/reference.rs:17-38: linears U(-1, 1) /
 * sqrt(fan-in), embedding U(-1, 1), type embedding x 0.15, norm weights
 * 1 + U/2, biases U/50; the reference ships no generator for this model. */
omg_weights *omg_laya_synth(const char *config_json, uint64_t seed, int linear_dtype, int embed_dtype);
/* LayaBackend::load for an exported directory (laya/backend.rs:61-91,
 * tools/export_laya.py): config.json (encoder config + laya_agent +
 * laya_tokens), manifest.json, *.bin; the engine is warmed up
 * (laya.rs:1126-1135).  special_ids (cls, sep, mask, pad), when not NULL,
 * replace laya_tokens: the reference resolves their surface forms with
 * the checkpoint's tokenizer, which stays with the caller. */
omg_laya *omg_laya_open_dir(const char *dir, const uint32_t *special_ids, size_t capacity, size_t max_rows);
/* The same directory's tensors as a host checkpoint. */
omg_weights *omg_laya_load_dir(const char *dir, const uint32_t *special_ids);
void omg_laya_close(omg_laya *e);
int omg_laya_config(const omg_laya *e, omg_laya_config_t *out);
/* LayaEngine::warmup (laya.rs:1126-1135). */
int omg_laya_warmup(omg_laya *e);
/* LayaEngine::hidden (laya.rs:1138-1432): per sequence the [CLS] row then
 * each marker's row, d floats each, dense in sequence order. */
int omg_laya_hidden(omg_laya *e, const omg_laya_seq *seqs, size_t n, float *out, size_t out_floats);
/* LayaEngine::evaluate (laya.rs:1435-1485): the scorer's raw logit per
 * marker, dense in sequence order, and the act probability per sequence
 * (NaN without an act head). */
int omg_laya_evaluate(omg_laya *e, const omg_laya_seq *seqs, size_t n, float *logits, size_t nlogits, float *act,
                      size_t nact);
/* LayaConfig::temperature_for (laya.rs:234-248). */
int omg_laya_temperature(const omg_laya *e, int qtype, size_t k, float *out);
/* Measurement, as omg_pass_prepare / omg_pass_launch / omg_sync / omg_profile. */
int omg_laya_prepare(omg_laya *e, const omg_laya_seq *seqs, size_t n);
int omg_laya_launch(omg_laya *e);
int omg_laya_sync(omg_laya *e);
int omg_laya_profile(omg_laya *e, int on);
size_t omg_laya_profile_report(omg_laya *e, char *buf, size_t len);
/* No counterpart in the reference, whose head layers run every row
 * (laya.rs:1346-1392).  By default the last decision-head layer runs past
 * its attention for the read-out rows only (o projection, LayerNorm, l1,
 * l2 on the gathered [CLS] and marker rows); on != 0 runs it for every row.
 * The rows are the same bits either way.  From the next pass on. */
int omg_laya_set_full_last_layer(omg_laya *e, int on);

#ifdef __cplusplus
}
#endif
#endif
