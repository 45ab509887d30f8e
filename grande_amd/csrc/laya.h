// The bidirectional encoder path on one MI355X: the C++ counterpart of
// crates/omg-wgpu/src/laya.rs (LayaConfig, LayaWeights, LayaBuilder,
// LayaEngine).  An mmBERT / ModernBERT encoder plus Laya's decision-head
// layers run on the GPU over one packed batch of sequences (one per
// question); the scorer (LayerNorm -> Linear -> GELU -> Linear(1)) and the
// act head read the [CLS] and [MASK] rows on the host in f32.
#pragma once

#include <hip/hip_runtime.h>

#include <map>
#include <memory>
#include <string>
#include <vector>

#include "common.h"
#include "engine.h"
#include "json.h"
#include "kernels.h"
#include "model.h"

namespace omg {

// laya.rs:47-82.  Token ids of the special tokens are given directly
// (tokenization is the caller's side, as for the decoder path).
struct LayaConfig {
    int64_t vocab = 0, d = 0, layers = 0, heads = 0, ff = 0;
    std::vector<bool> sliding;  // per encoder layer: local attention
    int64_t window = 64;        // inclusive local distance (local_attention / 2)
    float theta_global = 160000.0f, theta_local = 10000.0f, eps = 1e-5f;
    int64_t head_layers = 2;
    bool type_emb = true;
    int64_t act_hidden = 256, act_out = 0;
    int64_t max_len = 512, head_max_len = 192;
    float temperature[3] = {1.0f, 1.0f, 1.0f};
    std::map<std::string, float> temperature_by_options;
    uint32_t cls = 0, sep = 0, mask = 0, pad = 0;

    // laya.rs:88-206 over an encoder config.json carrying the agent config
    // under "laya_agent" and the special token ids under "laya_tokens"
    // (laya.rs:312-323, the exported directory's form).
    static LayaConfig from_json(const Json& v);
    void validate() const;                          // laya.rs:212-231 + this engine's kernels
    int64_t head_dim() const { return heads ? d / heads : 0; }
    std::vector<TensorSpec> tensors() const;        // laya.rs:252-305
    float temperature_for(int qtype, int64_t k) const;  // laya.rs:234-248
};

bool laya_host_tensor(const std::string& name);  // laya.rs:326-328

// A host checkpoint of the encoder path (laya.rs:331-464).
struct LayaWeights {
    LayaConfig config;
    std::map<std::string, QTensor> tensors;
};

// Seeded random weights for a config, in catalogue order, with the
// xorshift generator of tests/reference.rs:17-38: linears uniform in
// [-1, 1) / sqrt(fan-in), the type embedding x 0.15, the embedding x 1.0,
// norm weights 1 + U/2, biases U/50; the GPU linears and the embedding
// quantised to `linear` / `embed`, everything else f16.  (The reference
// has no generator for this model.)
LayaWeights synth_laya(const LayaConfig& cfg, uint64_t seed, Dtype linear, Dtype embed);

// An exported directory (laya.rs:61-91 with tools/export_laya.py's layout:
// config.json with laya_agent, manifest.json, *.bin).  `special` (cls,
// sep, mask, pad), when given, replaces the config's laya_tokens: the
// reference resolves those surface forms with its tokenizer.
LayaWeights load_laya_dir(const std::string& dir, const uint32_t* special);

// One question's sequence (laya.rs:468-476).
struct LayaSeq {
    const uint32_t* ids;
    int64_t n;
    const uint32_t* markers;  // token index of each option's [MASK]
    int64_t nmarkers;
    int qtype;                // 0 choice, 1 score, 2 noul
};

class LayaEngine;

// laya.rs:611-1083: weights arrive one tensor at a time; finish allocates
// the workspace for `capacity` packed tokens and `max_rows` read-back rows.
class LayaBuilder {
   public:
    explicit LayaBuilder(LayaConfig cfg);
    void push(const std::string& name, const QTensor& t);
    std::vector<std::string> missing() const;
    std::unique_ptr<LayaEngine> finish(int64_t capacity, int64_t max_rows);
    const LayaConfig& config() const { return cfg_; }

   private:
    LayaConfig cfg_;
    std::map<std::string, std::vector<int64_t>> expected_;
    std::map<std::string, DevTensor> linears_;
    std::map<std::string, DevBuf> vecs_;                 // f32 on the device
    std::map<std::string, std::vector<float>> host_;     // scorer / act head
};

class LayaEngine {
   public:
    ~LayaEngine();
    const LayaConfig& config() const { return cfg_; }
    int64_t capacity() const { return capacity_; }
    int64_t max_rows() const { return max_rows_; }

    // laya.rs:1138-1432: per sequence the [CLS] row then each marker's row,
    // d wide, dense in sequence order into `out`.
    void hidden(const LayaSeq* seqs, int64_t n, float* out, int64_t out_floats);
    // laya.rs:1435-1485: the scorer's raw logit per marker (dense in
    // sequence order) and the act probability per sequence (NaN without an
    // act head).
    void evaluate(const LayaSeq* seqs, int64_t n, float* logits, int64_t nlogits, float* act, int64_t nact);
    void warmup();  // laya.rs:1126-1135

    // Measurement surface: pack + upload once, then replay the device work.
    void prepare(const LayaSeq* seqs, int64_t n);
    void launch_prepared();
    void sync();
    void set_profile(bool on);
    std::string profile_report() const;
    int64_t prepared_rows() const { return nrows_; }
    // The last decision-head layer past its attention for every row (on)
    // or, the default, for the read-out rows only; the same rows either way.
    void set_full_last_layer(bool on);

   private:
    friend class LayaBuilder;
    LayaEngine() = default;
    int64_t pack(const LayaSeq* seqs, int64_t n);  // returns the token count; fills wanted
    void forward();
    void score(const float* rows, int64_t nmarkers, float* logits, float* act) const;
    template <class F>
    void step(const char* name, F&& f);

    LayaConfig cfg_;
    int64_t capacity_ = 0, max_rows_ = 0, rows_cap_ = 0, tpad_ = 0;
    int64_t t_ = 0, nrows_ = 0;
    hipStream_t stream_ = nullptr;
    DevTensor embed_;
    DevBuf embed_norm_, final_norm_, type_emb_;
    struct Enc {
        DevTensor qkv, o, wi_val, wi_gate, wo;
        DevBuf attn_norm, mlp_norm;
        bool sliding = false;
    };
    struct Head {
        DevTensor in_proj, out_proj, l1, l2;
        DevBuf norm1_w, norm1_b, in_proj_b16, out_proj_b, norm2_w, norm2_b, l1_b16, l2_b;
    };
    std::vector<Enc> enc_;
    std::vector<Head> head_;
    std::map<std::string, std::vector<float>> host_;
    DevBuf rope_local_, rope_global_;
    // workspace
    DevBuf ids_, qtypes_, meta_, x_, a_, h16_, q16_, k16_, vt_, attn16_, act16_, rows_, wanted_;
    // The last head layer on the read-out rows: [max_rows] rows of the
    // attention output, stream, product, normed stream and activations.
    bool full_last_layer_ = false;
    DevBuf attn_w_, x_w_, a_w_, h16_w_, act_w_;
    void* h_in_ = nullptr;
    size_t h_in_bytes_ = 0;
    void* h_out_ = nullptr;
    size_t h_out_bytes_ = 0;
    // measurement
    bool profile_ = false;
    struct Timed {
        const char* name;
        hipEvent_t e;
    };
    std::vector<Timed> pending_;
    std::vector<hipEvent_t> event_pool_;
    std::map<std::string, std::pair<int64_t, double>> totals_;
    void collect_profile();
};

}  // namespace omg
