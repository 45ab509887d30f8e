// Launchers for the gfx950 kernels of the decision-path forward.  Every
// launcher checks on the host that the shapes it is given fit what its
// kernel and grid assume, and throws omg::Error otherwise.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <vector>

namespace omg {

typedef _Float16 half_t;

// Storage codes of a device weight (model.rs Dtype::code).
constexpr int F16_DT = 0, Q8_DT = 1, Q4_DT = 2;

// A linear weight on the device, row-major [rows, cols] = [out, in].
//   F16: data = half_t[rows*cols].
//   Q8:  data = int8[rows*cols] (natural order), scales as below.
//   Q4:  data = 16 B per 32-element block, [rows][cols/32][16 B]; inside a
//        block, 32-bit word w holds elements 8w..8w+7 with element 8w+p at
//        bit 4*(p/2) (p even) or 16+4*(p/2) (p odd), so two shifts and a
//        mask yield them as f16 pairs in order.  scales as Q8.
//
// Stage tiles: the same weight again for the decoder GEMMs, cut into
// packets of 32 rows x 64 columns (one K stage of one MFMA row block) so
// that a workgroup's DMA of a stage reads whole contiguous packets instead
// of 32-byte pieces of many rows.  Packet (rb, st) of row block rb and
// stage st sits at (rb * stages + st) * tile_packet_bytes(dtype) in
// `tiles`; inside it, the 8-column group of row r at k-step ks (columns
// 16 ks .. 16 ks + 15 of the stage) and half h (columns 16 ks + 8 h ..
// + 7) sits at (32 h + r) * PK / 64 + ks * PK / 256, so one lane of a
// 32x32x16 MFMA operand (row r, half h) reads all four k-steps of the
// stage as one contiguous 16 / 32 / 64-byte run.  `tscales` holds a
// 128-byte packet per (rb, st): row r's two block scales at 4 r (f16,
// block 2 st in the low half).  Rows past `rows` and columns past `cols`
// are zeros (codes and scales), so they contribute nothing.
struct DevWeight {
    int dtype = 0;
    int64_t rows = 0, cols = 0;
    const void* data = nullptr;
    const uint16_t* scales = nullptr;  // [rows][sld] f16, block b of row r at r * sld + b
    int64_t sld = 0;                   // cols / 32 rounded up to even (the pad holds zeros)
    const uint8_t* tiles = nullptr;    // stage tiles (see above)
    const uint8_t* tscales = nullptr;  // their scale packets (Q8, Q4)
    int64_t stages = 0;                // cols / 64 rounded up
};

// Bytes per stage-tile packet: 32 rows x 64 columns of codes.
constexpr int tile_packet_bytes(int dtype) { return dtype == Q4_DT ? 1024 : (dtype == Q8_DT ? 2048 : 4096); }
constexpr int TILE_SCALE_BYTES = 128;

// Repack one Q4_0 tensor (model.rs layout: byte j = element j | element
// j+16 << 4) into the device layout above.  n = element count.
void repack_q4(const uint8_t* src, uint8_t* dst, int64_t n);

// ---- residual-stream kernels (norm.hip) ----
// x[r] = deq(E[ids[r]]) * sqrt(d) (f32, bit-exact), hn[r] = f16(rmsnorm(x[r]) * w).
void launch_embed_norm(hipStream_t s, const DevWeight& E, const uint32_t* ids, int64_t t,
                       float embed_scale, const float* w, float eps, float* x, half_t* hn);
// y = rmsnorm(a[r]) * w1;  x[r] = (y + x[r]) * scale;  if w2: hn[r] = f16(rmsnorm(x[r]) * w2),
// else if hn: hn[r] = f16(x[r]).  With parts > 1, a[r] is the sum of the
// split-K parts a[z * part_stride + r]: each run of `group` consecutive
// parts added in order (z = 0, 1, ...), then the runs' sums in order
// (parts a multiple of group).
void launch_residual_norm(hipStream_t s, const float* a, const float* w1, float* x, const float* w2,
                          half_t* hn, int64_t t, int64_t d, float eps, float scale, int parts = 1,
                          int64_t part_stride = 0, int group = 1);
// Gemma 4 per-layer inputs (engine.rs:1651-1666, 1728-1750).  pl holds
// f16(x) . pl_model_proj^T as [t][layers x P] and is replaced by
// (rmsnorm(pl * proj_scale) * w + f16(table[ids[t], :]) * emb_scale) * out_scale.
void launch_pl_combine(hipStream_t s, const DevWeight& table, const uint32_t* ids, const float* w, float* pl,
                       int64_t t, int64_t P, int64_t layers, float eps, float proj_scale, float emb_scale,
                       float out_scale);
// out[t][j] = f16(gelu_tanh(g[t][j]) * pl[t][layer * P + j]).
void launch_pl_gate(hipStream_t s, const float* g, const float* pl, half_t* out, int64_t t, int64_t P, int64_t layers,
                    int64_t layer);
// out = f16(x), n % 4 == 0.
void launch_to_f16(hipStream_t s, const float* x, half_t* out, int64_t n);
// Per token: q heads normed + roped + scaled into q16; on K/V layers, k
// heads normed + roped and v heads (optionally normed) into the f16 cache.
struct QkArgs {
    const float* qkv;
    int64_t qkv_stride;
    const int32_t* meta;  // 4 ints per cache row: pos, seq, first key row, own row + 1
    const float* q_norm;
    const float* k_norm;
    const float2* rope;  // [rope_rows][hd/2]: (cos, sin) of pos * inv_freq[i]
    int64_t rope_rows, rope_dims;
    float eps, q_scale;
    int heads, kv_heads, hd;
    bool has_kv, v_norm;
    int64_t t, base, cap_pad;
    half_t* q16;  // [t][heads][hd]
    half_t* kc;   // [kv_heads][cap_pad][hd]
    half_t* vt;   // [kv_heads][cap_pad/64][hd][64], key columns ordered by vt_col
};
void launch_qk_prep(hipStream_t s, const QkArgs& a);
// The q/k/v projection x . W^T with launch_qk_prep's work in its epilogue
// (head_dim 256; a.qkv unused): one launch instead of the f32 product and
// qk_prep, the same rows.
void launch_gemm_qkprep(hipStream_t s, const half_t* x, int64_t ldx, const DevWeight& w, const QkArgs& a, int64_t m);
// out[p][i] = (cos, sin)(float(p) * inv_freq[i]) for p < rows, i < half.
void launch_rope_table(hipStream_t s, const float* inv_freq, int64_t rows, int64_t half, float2* out);
// rows[i] = rmsnorm(x[wanted[i]]) * w, f32.
// rows[i] = final norm of x row wanted[i] (row i without a list).
void launch_final_rows(hipStream_t s, const float* x, const int32_t* wanted, int64_t n, int64_t d,
                       const float* w, float eps, float* rows);
// aw[i] = a[rows[i] - r0] (f16, width wa), xw[i] = x[rows[i] - r0] (f32,
// width wx), i < n; with p, pw[i] = p[rows[i] - r0][po .. po + wp) (row
// stride ps).
void launch_gather_out(hipStream_t s, const half_t* a, int64_t wa, const float* x, int64_t wx, const int32_t* rows,
                       int64_t r0, int64_t n, half_t* aw, float* xw, const float* p = nullptr, int64_t ps = 0,
                       int64_t po = 0, int64_t wp = 0, float* pw = nullptr);
// out[r][j] = rows[r] . deq(E[col(j)]) in f32 (+ softcap), col(j) = cols ? cols[j] : j.
// logits[r][j] = rows[r] . deq(E[cols ? cols[j] : j]) (softcap applied),
// f32 [nrows][ncols]; with `part` (logits_blocks(ncols) x nrows pairs) each
// workgroup's (max, sum of exp) per row for the log-sum-exp.
void launch_logits(hipStream_t s, const DevWeight& E, const float* rows, int64_t nrows, const uint32_t* cols,
                   int64_t ncols, float softcap, float* out, float2* part = nullptr);
int64_t logits_blocks(int64_t ncols);
// The label readout (logits, then launch_label_lse) with its scratch in a
// fixed device array instead of allocated memory: nothing is allocated;
// nrows x vocab + 2 x nrows x logits_blocks(vocab) floats must fit
// label_readout_scratch_floats().
void launch_label_readout_noalloc(hipStream_t s, const DevWeight& E, const float* rows, int64_t nrows,
                                  const uint32_t* labels, int64_t nlabels, float softcap, float* out);
int64_t label_readout_scratch_floats();
// Per row of full-vocabulary logits [nrows][vocab] and the logits kernel's
// partials: the columns `labels`, then log-sum-exp over the whole row, into
// out [nrows][nlabels + 1].
void launch_label_lse(hipStream_t s, const float* logits, int64_t nrows, int64_t vocab, const float2* part,
                      int64_t nblocks, const uint32_t* labels, int64_t nlabels, float* out);
// Readout::Pointer (readout.rs:30-44): proj[r] = W_m h_r + b_m for each row
// r of `rows` with a map m = mat[r] (0: the q map, 1: the k map, -1: none),
// w = [W_q; W_k] row-major [2][dp][d], b = [b_q; b_k]; then for each pair i
// (option row, decide row) out[i] = proj[option] . proj[decide] / sqrt(dp).
void launch_pointer(hipStream_t s, const float* rows, int64_t nrows, int64_t d, const float* w, const float* b,
                    int64_t dp, const int32_t* mat, float* proj, const int2* pairs, int64_t npairs, float* out);
// K/V cache rows <-> the reference's state row format [K heads | V heads] f16.
void launch_kv_gather(hipStream_t s, const half_t* kc, const half_t* vt, int64_t cap_pad, int kv_heads,
                      int hd, int64_t row0, int64_t rows, half_t* out);
void launch_kv_scatter(hipStream_t s, half_t* kc, half_t* vt, int64_t cap_pad, int kv_heads, int hd,
                       int64_t row0, int64_t rows, const half_t* in);

// Column of key k (0..31) inside its 32-key V^T tile of the bidirectional
// encoder's attention: the eight keys one MFMA lane holds probabilities
// for (4g..4g+3 and 16+4g..16+4g+3) are adjacent.
__host__ __device__ inline int vt_col32(int k) { return 8 * ((k % 16) / 4) + 4 * (k / 16) + k % 4; }

// The fused [q | k | v] projection of a bidirectional encoder layer
// (64-wide heads), scattered per head as f16 for the attention kernel:
// bias added, q and k rotated (rope_bi.wgsl) when `rope` is set, q scaled.
struct QkvHeads {
    const float2* rope;   // [max pos + 1][32]: (cos, sin) of pos * inv_freq[i]; null = no rotation
    const int32_t* meta;  // 4 ints per token: pos, seq, first row, last row + 1
    float qscale;
    int64_t dq;           // q width = heads * 64
    int64_t tpad;         // rows of the head arrays (>= t, multiple of 32)
    half_t* q16;          // [heads][tpad][64]
    half_t* k16;          // [heads][tpad][64]
    half_t* vt;           // [heads][tpad / 32][64][32], key columns ordered by vt_col32
};

// ---- MFMA GEMMs (gemm.hip) ----
// y[M][N] (f32) = f16(X)[M][K] . deq(W)[N][K]^T, f32 accumulation.
void launch_gemm(hipStream_t s, const half_t* x, int64_t ldx, const DevWeight& w, float* y, int64_t ldy,
                 int64_t m);
// The same product with K split into `parts` ranges (K % (64 parts) == 0):
// partial p (K range p) goes to y + p * part_stride; the sum is the
// consumer's (launch_residual_norm).  More workgroups for narrow-N, deep-K
// products; each partial's rows are independent of M.
// kfold > 0: inside each range the products of every kfold stages (64 K
// each; the last piece may be shorter) accumulate from zero and these
// piece sums are added in K order — what ranges of one piece each give
// when launch_residual_norm adds them in runs of the pieces per range.
void launch_gemm_splitk(hipStream_t s, const half_t* x, int64_t ldx, const DevWeight& w, float* y, int64_t ldy,
                        int64_t m, int parts, int64_t part_stride, int kfold = 0);
// act[M][F] (f16) = gelu(X . Wg^T) * (X . Wu^T); gelu_tanh, or the exact
// (erf) form when `erf`.
void launch_gemm_geglu(hipStream_t s, const half_t* x, int64_t ldx, const DevWeight& wg,
                       const DevWeight& wu, half_t* act, int64_t ldact, int64_t m, bool erf = false);
// y[M][N] (f16) = max(X . W^T + bias, 0) (bias f16 [N]).
void launch_gemm_bias_relu(hipStream_t s, const half_t* x, int64_t ldx, const DevWeight& w,
                           const uint16_t* bias, half_t* y, int64_t ldy, int64_t m);
// The [q | k | v] projection X . W^T (+ bias) into QkvHeads' arrays.
void launch_gemm_qkv_heads(hipStream_t s, const half_t* x, int64_t ldx, const DevWeight& w,
                           const uint16_t* bias, const QkvHeads& o, int64_t m);

// ---- bidirectional encoder rows and attention (laya.hip) ----
// out[t][h * 64 + c] (f16) = sum over visible keys j of softmax_j(q_t . k_j) v_j[c]:
// visible = same sequence (the span meta[2]..meta[3] of the query row) and,
// when window > 0, |t - j| <= window (attention_bi.wgsl).
void launch_attention_bi(hipStream_t s, const QkvHeads& a, int heads, int64_t t, int window, half_t* out);
// x[r] = LayerNorm(deq(E[ids[r]]); w) (f32), x16[r] = f16(x[r]).
void launch_embed_ln(hipStream_t s, const DevWeight& E, const uint32_t* ids, int64_t t, const float* w,
                     float eps, float* x, half_t* x16);
// x[r] = (x[r] + a[r]) (+ rb);  h16[r] = f16(LayerNorm(x[r]; w, b)).  rb, b may be null.
void launch_add_ln(hipStream_t s, float* x, const float* a, const float* rb, const float* w, const float* b,
                   float eps, int64_t t, int64_t d, half_t* h16);
// x[r] = LayerNorm(x[r] + a[r]; wf);  x[r] += temb[qtypes[r]] (if temb);
// h16[r] = f16(LayerNorm(x[r]; w1, b1)) (if w1).
void launch_add_ln_final(hipStream_t s, float* x, const float* a, const float* wf, const float* temb,
                         const uint32_t* qtypes, const float* w1, const float* b1, float eps, int64_t t,
                         int64_t d, half_t* h16);
// out[i] = (a[rows[i]] + bias) + x[rows[i]] (f32), or x[rows[i]] when a is null.
void launch_gather_rows(hipStream_t s, const float* x, const float* a, const float* bias, const int32_t* rows,
                        int64_t n, int64_t d, float* out);

// Column of cache row `row` inside its 64-row V^T tile.  Within each half
// of 32 keys, key k sits at 8 * ((k % 16) / 4) + 4 * (k / 16) + k % 4: the
// eight keys one MFMA lane holds probabilities for (4g..4g+3 and
// 16+4g..16+4g+3) are then adjacent, so a V^T fragment is one 16-byte read.
__host__ __device__ inline int64_t vt_col(int64_t row) {
    const int64_t k = row % 64, h = k / 32, kk = k % 32;
    return 32 * h + 8 * ((kk % 16) / 4) + 4 * (kk / 16) + kk % 4;
}

// ---- block-causal attention (attention.hip) ----
struct AttnArgs {
    const half_t* q16;   // [t][heads][hd]
    const half_t* kc;    // [kv_heads][cap_pad][hd]
    const half_t* vt;    // [kv_heads][cap_pad/64][hd][64]
    const int32_t* meta; // per cache row
    half_t* out;         // [t][heads][hd]
    half_t* part_o;      // chunk partials: [slot][kv_heads][rows][hd] O / l (f16)
    float* part_ml;      // [slot][kv_heads][rows][2]: running max (log2 units), sum
    int64_t t, base, cap_pad;
    int heads, kv_heads, hd;
    int window;          // 0 = global layer
    // Queries that are not the cache rows [base, base + t) (rows gathered
    // from a pass): their metadata, one int4 per query row, and the end of
    // the cache rows their keys may come from.  Null / 0: meta + base and
    // base + t.
    const int32_t* qmeta;
    int64_t kend;
};
// The pass's attention work: items (query tile, first key tile, end key
// tile, partial slot or -1) and, for split tiles, merges (query tile, first
// slot, slot count, 0).
struct AttnWork {
    std::vector<int4> items, merges;
    int slots = 0;
    int nw = 4;           // waves (16-row query blocks) per work item
    bool aligned = true;  // every query tile's groups start on a key tile
};
// Geometry of the attention work: keys per K/V tile (the unit of chunk and
// of the items' key tile ranges) and query rows per work item (at most:
// 4 waves of 16 rows).
int attention_key_tile();
int attention_rows();
// Build the work of one layer type from the pass's per-token metadata
// (4 ints per token of this pass, in workspace order).  chunk = key tiles
// per split (0 = never split); nw = waves per work item (2 or 4).  A row's
// sums depend on the chunk boundaries alone, which count from its group's
// first key row when its query tile's groups all start on a key tile
// (w.aligned) and from cache row 0 otherwise; with every tile aligned they
// are the same for either nw.
void attention_work(const int32_t* meta, int64_t t, int heads, int kv_heads, int window, int chunk, int nw,
                    AttnWork& w);
void launch_attention(hipStream_t s, const AttnArgs& a, const int4* items, int64_t nitems, int nw);
// The chunk merges of the split query tiles (after launch_attention).
void launch_attention_merge(hipStream_t s, const AttnArgs& a, const int4* merges, int64_t nmerges, int nw);

}  // namespace omg
