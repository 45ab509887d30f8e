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

/* omg-core backend.rs:14-20 Want; OMG_WANT_LABELS has no counterpart in the
 * reference: logits of the given label ids only (readout.rs:130-133 picks
 * them out of the full row on the host). */
#define OMG_WANT_LOGITS 0
#define OMG_WANT_HIDDEN 1
#define OMG_WANT_LABELS 2

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
void omg_close(omg_engine *e);
int omg_config(const omg_engine *e, omg_config_t *out);
/* Engine::warmup (engine.rs:1356-1366). */
int omg_warmup(omg_engine *e);

/* ---- the pass (engine.rs:1386-1940) ---- */

/* Engine::evaluate_groups / Backend::evaluate_many (engine.rs:1404-1444,
 * backend.rs:142-152).  Rows are written densely into `out` in (group,
 * branch, want) order; width n_embd (HIDDEN), n_vocab (LOGITS) or nlabels
 * (LABELS, with label_ids).  prefix_sources (may be NULL) gets one
 * OMG_SRC_* per group. */
int omg_evaluate_groups(omg_engine *e, const omg_group *groups, size_t ngroups, int want,
                        const uint32_t *label_ids, size_t nlabels, float *out, size_t out_floats,
                        int *prefix_sources);
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
 * (4 int64 per row: group, branch, slot, workspace row).  Sizes in/out. */
int omg_pack(const omg_group *groups, size_t ngroups, size_t first, int resident, uint32_t *ids,
             int32_t *meta, int64_t *wanted, size_t *n_ids, size_t *n_wanted);
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
 * transfer.  omg_sync waits for it. */
int omg_pass_prepare(omg_engine *e, const omg_group *groups, size_t ngroups, int want,
                     const uint32_t *label_ids, size_t nlabels, int first_resident);
int omg_pass_launch(omg_engine *e);
int omg_sync(omg_engine *e);
/* HIP-event time per kernel of every launch while on; the report is lines
 * "name launches total_ms". */
int omg_profile(omg_engine *e, int on);
size_t omg_profile_report(omg_engine *e, char *buf, size_t len);

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
/* The embedding gather + first norm kernel (embed.wgsl + rmsnorm.wgsl):
 * x[t][d] = deq(E[ids[t]]) * scale (f32), hn[t][d] = f16(rmsnorm(x) * w)
 * with w (f32, d entries) already offset.  Device pointers. */
int omg_dev_embed_norm(const omg_weight *embed, const uint32_t *ids, int64_t t, float scale, const float *w,
                       float eps, float *x, void *hn_f16, void *stream);

#ifdef __cplusplus
}
#endif
#endif
