// The decision-path engine on one MI355X: the C++ counterpart of
// crates/omg-wgpu/src/engine.rs (EngineBuilder, Engine, SavedState,
// StateCache).  One HIP stream; weights and a capacity-sized workspace live
// in HBM for the life of the engine; a request uploads its token ids and
// per-token metadata, runs the whole network, and reads back only the
// wanted rows.
#pragma once

#include <hip/hip_runtime.h>

#include <array>
#include <map>
#include <memory>
#include <optional>
#include <string>
#include <vector>

#include "common.h"
#include "kernels.h"
#include "model.h"
#include "state.h"

namespace omg {

enum WantKind { WANT_LOGITS = 0, WANT_HIDDEN = 1, WANT_LABELS = 2, WANT_LABELS_LSE = 3 };
enum Source { SRC_NONE = 0, SRC_RESIDENT = 1, SRC_RAM = 2, SRC_DISK = 3, SRC_DECODED = 4 };
// readout.rs Mark: a wanted row that is none of these (Mark::Last), an
// option's `</opt>` (Mark::OptEnd) or the `<decide>` row (Mark::Decide).
enum Role { ROLE_NONE = 0, ROLE_OPT = 1, ROLE_DECIDE = 2 };

// Owned device allocation.
struct DevBuf {
    void* p = nullptr;
    size_t bytes = 0;
    DevBuf() = default;
    explicit DevBuf(size_t n, bool zero = false);
    ~DevBuf();
    DevBuf(const DevBuf&) = delete;
    DevBuf& operator=(const DevBuf&) = delete;
    DevBuf(DevBuf&& o) noexcept : p(o.p), bytes(o.bytes) {
        o.p = nullptr;
        o.bytes = 0;
    }
    DevBuf& operator=(DevBuf&& o) noexcept;
    template <class T>
    T* as() const {
        return static_cast<T*>(p);
    }
};

struct DevTensor {
    DevWeight w;
    DevBuf data, scales, tiles, tscales;
};
// Upload a linear weight in the device layout (Q4 repacked, scale rows
// padded to an even block count) and, when `tiled` (every weight a GEMM
// reads; not the gather-only embedding tables), as stage tiles.
DevTensor upload_weight(const QTensor& t, bool tiled = true);

class Engine;

// engine.rs:763-1335: receives weights one tensor at a time (uploaded as
// they arrive) and allocates the workspace at finish.
class Builder {
   public:
    explicit Builder(Config cfg);
    void push(const std::string& name, const QTensor& t);
    std::vector<std::string> missing() const;
    std::unique_ptr<Engine> finish(int64_t capacity, int64_t max_rows);
    const Config& config() const { return cfg_; }

   private:
    friend class Engine;
    Config cfg_;
    std::map<std::string, std::vector<int64_t>> expected_;
    std::map<std::string, DevTensor> linears_;
    std::map<std::string, DevBuf> norms_;  // f32, norm offset folded in
    std::map<std::string, float> scalars_;  // per-layer output scales (engine.rs:896-901)
};

struct PassPlan {
    int64_t t = 0, base = 0, nrows = 0, nlabels = 0;
    int want = WANT_HIDDEN;
};

class Engine {
   public:
    ~Engine();
    const Config& config() const { return cfg_; }
    int64_t capacity() const { return capacity_; }
    int64_t max_rows() const { return max_rows_; }

    // engine.rs:1404-1444.  Output rows are dense in the caller's (group,
    // branch, want) order; width d (hidden), vocab (logits) or nlabels.
    void evaluate_groups(const GroupIn* groups, int64_t n, int want, const uint32_t* labels, int64_t nlabels,
                         float* out, int64_t out_floats, int* sources);
    void warmup();  // engine.rs:1356-1366

    // Readout::Pointer (omg-core readout.rs:17-44, 149-173) on the device:
    // the head's two affine maps d -> dp (row-major [dp][d] and [dp], f32).
    void set_pointer_head(int64_t d, int64_t dp, const float* w_q, const float* b_q, const float* w_k,
                          const float* b_k);
    // A hidden-state pass whose wanted rows are scored by the head: roles
    // (one per wanted row, (group, branch, want) order) mark each row as an
    // option end (ROLE_OPT), the decide row (ROLE_DECIDE, one per branch) or
    // neither; out gets each branch's option logits in want order, branch
    // after branch.  Returns the logits written.
    int64_t evaluate_pointer(const GroupIn* groups, int64_t n, const uint8_t* roles, int64_t nroles, float* out,
                             int64_t out_floats, int* sources);

    void set_state_cache(size_t bytes, const std::string& dir, const std::string& model_id);
    SavedState save_state(const uint32_t* prefix, int64_t n) { return save_state_at(prefix, n, 0); }
    // The same state serialised straight from the pinned staging buffer as
    // GRWS1 bytes (SavedState::to_bytes's layout) into one malloc'd block
    // the caller frees with std::free.
    std::pair<uint8_t*, size_t> save_state_bytes(const uint32_t* prefix, int64_t n, const std::string& model_id);
    void restore_state(const SavedState& s);
    bool is_resident(const uint32_t* prefix, int64_t n) const;
    int prefix_source() const { return last_source_; }
    void evict_resident() { resident_.reset(); }
    const std::string& model_id() const { return model_id_; }

    // Measurement surface: pack + upload a request once, then replay its
    // device work (forward + readout, no host transfers).
    void prepare(const GroupIn* groups, int64_t n, int want, const uint32_t* labels, int64_t nlabels,
                 bool resident_first);
    void launch_prepared();
    // Capture the prepared pass's launches into a HIP graph (on = true) that
    // launch_prepared then replays as one submission; dropped by the next
    // prepare, by any pass through evaluate, and by on = false.
    void set_graph(bool on);
    // The prepared pass's output rows after its launches (wanted order:
    // group, branch, slot), width as evaluate_groups gives them.
    int64_t read_prepared(float* out, int64_t out_floats);
    void sync();
    void set_profile(bool on);
    std::string profile_report() const;
    // Every layer for every row of the pass (on) or, the default, from the
    // last layer that writes K/V past its attention on, the rows a request
    // reads out only (their tiles' attention, then the rest of that layer
    // and every later layer on the gathered rows): the same rows either
    // way.  Takes effect from the next pass.
    void set_full_last_layer(bool on);
    hipStream_t stream() const { return stream_; }

   private:
    friend class Builder;
    Engine() = default;
    std::pair<int64_t, int> admit(const GroupIn* groups, int64_t n);
    int restore_from_cache(const uint32_t* prefix, int64_t n);
    void remember(const uint32_t* prefix, int64_t n, int64_t row0);
    SavedState save_state_at(const uint32_t* prefix, int64_t n, int64_t row0);
    // Gather the K/V rows of a state of p tokens (cache rows from row0) into
    // h_state_, layer after layer, and synchronise; returns the bytes staged.
    size_t stage_state(int64_t p, int64_t row0);
    std::pair<int64_t, int64_t> state_rows(int64_t layer, int64_t p) const;
    Packed pack_checked(const GroupIn* groups, int64_t n, int64_t first, bool resident) const;
    // A request's pass up to its readout, enqueued (admit, pack, upload,
    // forward, readout of `want`), and the bookkeeping after it ran.
    struct Run {
        Packed pk;
        int64_t first = 0;
        int source = SRC_NONE;
    };
    Run run_pass(const GroupIn* groups, int64_t n, int want, const uint32_t* labels, int64_t nlabels,
                 int64_t out_floats_needed, int64_t out_floats);
    void finish_pass(const GroupIn* groups, int64_t n, const Run& run, int* sources);
    void upload(const Packed& pk, const uint32_t* labels, int64_t nlabels);
    // How an o / down product of K k and width n runs in a pass of t rows:
    // its K splits, each split's K pieces (group, kfold stages each), and
    // whether the pieces run a workgroup each (short passes) or are added
    // in the GEMM's registers.
    struct SplitPlan {
        int splits = 1, group = 1, kfold = 0;
        bool pieces = false;
    };
    SplitPlan split_plan(int64_t k, int64_t n, int64_t t) const;
    void split_product(const char* name, int k, const half_t* x, int64_t kdim, const DevWeight& w, int64_t r0,
                       int64_t t, const SplitPlan& sp);
    struct NormParts {
        float* a;
        int parts;
        int64_t stride;
        int group;
    };
    NormParts norm_parts(const SplitPlan& sp, int64_t r0, int64_t t) const;
    void forward(int64_t base);
    void readout(const PassPlan& plan);
    // One profiled launch (or launcher call) on range k's stream.
    template <class F>
    void step(const char* name, int k, F&& f);

    Config cfg_;
    int64_t capacity_ = 0, max_rows_ = 0, cap_pad_ = 0;
    // Cache rows the workspace holds: the token capacity plus room to start
    // every layout group after the first on a multiple of align_ rows
    // (align_groups), for up to max_rows groups.
    int64_t slots_ = 0, align_ = 1;
    hipStream_t stream_ = nullptr;
    int64_t cus_ = 256;  // compute units of the device
    DevTensor embed_;
    DevBuf final_norm_;
    struct Layer {
        DevTensor qkv, o, gate, up, down;
        DevBuf attn_norm, q_norm, k_norm, post_attn_norm, ffn_norm, post_ffn_norm;
        // per-layer inputs (Gemma 4)
        DevTensor pl_gate, pl_proj;
        DevBuf pl_norm;
        float out_scale = 1.0f;
    };
    std::vector<Layer> layers_;
    // Gemma 4 per-layer inputs: the [vocab, layers x P] token table stays in
    // HBM and is gathered on the device.
    DevTensor pl_model_proj_, pl_table_;
    DevBuf pl_proj_norm_;
    // RoPE (cos, sin) tables, one per (layer type, head_dim); rope_of_[l]
    // indexes the layer's.
    std::vector<DevBuf> rope_tabs_;
    std::vector<int> rope_of_;
    int64_t rope_rows_ = 0;
    // workspace
    DevBuf meta_, x_, hn_, qkv_, q16_, attn_, a_, act_, rows_, logits_, kv_stage_;
    // the pass's inputs in one block (upload): token ids, wanted rows, label ids, work lists
    DevBuf in_;
    size_t in_bytes_ = 0;
    const uint32_t* d_ids_ = nullptr;
    const int32_t* d_wanted_ = nullptr;
    const uint32_t* d_labels_ = nullptr;
    // Label logits + full-row log-sum-exp per wanted row (WANT_LABELS_LSE),
    // and the logits kernel's per-workgroup (max, sum of exp) pairs.
    DevBuf label_lse_, lse_part_;
    DevBuf x16_, pli_, plg_, pl16_;  // per-layer inputs: f16(x), [t][layers x P] f32, gate f32, gated f16
    // attention chunk lengths in key tiles: [0] sliding layers, [1] global
    int attn_chunk_[2] = {0, 0};
    DevBuf part_o_, part_ml_;
    int64_t part_slots_ = 0;  // chunk partial slots part_o_ / part_ml_ hold
    // Sub-passes: a long pass runs as up to MAX_SUB consecutive row ranges,
    // each on a stream of its own, layer by layer; a range's attention at
    // layer l waits for the K/V rows the earlier ranges write at layer l
    // (a row sees only rows before it), so the ranges' kernels overlap and
    // every row's arithmetic is that of the whole pass.
    static constexpr int MAX_SUB = 3;
    struct Sub {
        int64_t r0 = 0, r1 = 0;  // pass-relative rows [r0, r1)
        AttnWork work[2];        // host side of its attention lists per layer type
        const int4* d_items[2] = {nullptr, nullptr};
        const int4* d_merges[2] = {nullptr, nullptr};
        int64_t n_items[2] = {0, 0}, n_merges[2] = {0, 0};
        // The last layer on the answer rows only (out_rows_): the range's
        // share [w0, w1) of the pass's wanted rows and its attention work
        // restricted to the query tiles that hold them.
        int64_t w0 = 0, w1 = 0;
        AttnWork out_work;
        const int4* d_out_items = nullptr;
        const int4* d_out_merges = nullptr;
    };
    Sub sub_[MAX_SUB];
    int nsub_ = 1;
    hipStream_t sub_stream_[MAX_SUB] = {};  // [0] is stream_
    hipEvent_t ev_fork_ = nullptr, ev_join_[MAX_SUB] = {};
    std::vector<hipEvent_t> ev_kv_;  // [range][layer]: the range's K/V rows of the layer are in the cache
    void layer(int64_t l, int k, int64_t base);
    // The answer rows: from layer out_layer_ (the last one that writes K/V)
    // past its attention on, the rest of the pass runs for the rows a
    // request reads out only, gathered into max_rows-row buffers.
    struct RowBufs {
        half_t* aw = nullptr;    // attention output
        float* xw = nullptr;     // stream
        half_t* hw = nullptr;    // normed stream (f16)
        half_t* actw = nullptr;  // gated activations
        float* pw = nullptr;     // product parts
        float* pliw = nullptr;   // per-layer inputs of every layer
        half_t* x16w = nullptr;  // f16(stream)
        float* plgw = nullptr;   // the per-layer gate's product
        half_t* pl16w = nullptr; // gated per-layer inputs
    };
    RowBufs row_bufs(int64_t w0, int64_t W, int64_t ff);
    // Range k's answer rows through layer out_layer_ past its attention.
    void layer_out(int k, const half_t* attn, const float* x, int64_t r0);
    // Layer l past its attention on n gathered rows.
    void rows_post(int64_t l, int k, hipStream_t s, int64_t n, const RowBufs& b);
    // A layer after out_layer_ on the answer rows alone.
    void layer_tail(int64_t l);
    bool full_last_layer_ = false;  // set_full_last_layer
    bool out_rows_ = false;         // this pass runs the answer-row path
    int64_t out_layer_ = 0;         // the last layer with K/V of its own
    int64_t tail_rows_ = 0;         // answer rows of the pass
    int64_t tail_kend_ = 0;         // end of the pass's cache rows
    // the layers after out_layer_: the answer rows' metadata and attention
    // work over them, per layer type
    const int32_t* d_tail_meta_ = nullptr;
    AttnWork tail_work_[2];
    const int4* d_tail_items_[2] = {nullptr, nullptr};
    const int4* d_tail_merges_[2] = {nullptr, nullptr};
    // [max_rows] rows: attention output, stream, normed stream, gated
    // activations, product parts (the most any o / down product makes),
    // queries and (head_dim 512) the f32 q/k/v product
    DevBuf attn_w_, x_w_, hn_w_, act_w_, a_w_, q16_w_, qkv_w_;
    // ... and with per-layer inputs: f16(x), the gate's product, the gated
    // inputs (f16) and the rows' inputs of every layer
    DevBuf x16_w_, plg_w_, pl16_w_, pli_w_;
    std::vector<DevBuf> kc_, vt_;  // per layer that owns K/V
    // pinned host staging
    void* h_in_ = nullptr;
    size_t h_in_bytes_ = 0;
    void* h_out_ = nullptr;
    size_t h_out_bytes_ = 0;
    // pointer head ([q; k] maps) and its per-pass plan / projections
    int64_t ptr_dp_ = 0;
    DevBuf ptr_w_, ptr_b_, ptr_plan_, ptr_proj_, ptr_out_;
    void* h_ptr_ = nullptr;  // pinned plan staging: max_rows row matrices + max_rows row pairs
    // pinned staging of a whole state's K/V rows (save / restore), sized
    // at finish for a state of `capacity` tokens
    void* h_state_ = nullptr;
    size_t h_state_bytes_ = 0;
    // resident prefix / state cache (engine.rs:483-496)
    std::optional<std::vector<uint32_t>> resident_;
    int last_source_ = SRC_NONE;
    StateCache states_;
    std::string state_dir_;
    std::string model_id_ = "hip";
    // measurement
    PassPlan prepared_;
    hipGraphExec_t graph_exec_ = nullptr;
    void drop_graph();
    bool profile_ = false;
    struct Timed {
        const char* name;  // null for the sequence's start event
        hipEvent_t e;
    };
    std::vector<Timed> pending_[MAX_SUB];  // per range's stream
    std::vector<hipEvent_t> event_pool_;
    std::map<std::string, std::pair<int64_t, double>> totals_;
    void collect_profile();
};

}  // namespace omg
