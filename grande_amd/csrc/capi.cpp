// extern "C" surface of include/omg_hip.h: converts between the C structs
// and the engine's types and turns every omg::Error into a status code plus
// a thread-local message.
#include "../../include/omg_hip.h"

#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "engine.h"
#include "laya.h"

struct omg_builder {
    std::unique_ptr<omg::Builder> b;
};
struct omg_engine {
    std::unique_ptr<omg::Engine> e;
};
struct omg_weight {
    omg::DevTensor t;
};
struct omg_weights {
    std::map<std::string, omg::QTensor> tensors;
    std::vector<const std::pair<const std::string, omg::QTensor>*> order;  // catalogue order
    void index(const std::vector<omg::TensorSpec>& specs) {
        order.clear();
        for (const auto& spec : specs) {
            auto it = tensors.find(spec.name);
            if (it != tensors.end()) order.push_back(&*it);
        }
        auto table = tensors.find("per_layer_table");  // after the catalogue, as set_per_layer_table
        if (table != tensors.end()) order.push_back(&*table);
    }
};
struct omg_laya_builder {
    std::unique_ptr<omg::LayaBuilder> b;
};
struct omg_laya {
    std::unique_ptr<omg::LayaEngine> e;
};

namespace {

thread_local std::string g_err;

template <class F>
int guard(F&& f) {
    try {
        f();
        return OMG_OK;
    } catch (const omg::Error& e) {
        g_err = e.what();
        return e.code;
    } catch (const std::bad_alloc&) {
        g_err = "out of host memory";
        return OMG_E_INVALID;
    } catch (const std::exception& e) {
        g_err = e.what();
        return OMG_E_INVALID;
    }
}

static_assert(OMG_ROLE_NONE == omg::ROLE_NONE && OMG_ROLE_OPT == omg::ROLE_OPT && OMG_ROLE_DECIDE == omg::ROLE_DECIDE,
              "pointer roles");

struct Groups {
    std::vector<std::vector<omg::BranchIn>> branches;
    std::vector<omg::GroupIn> groups;
};

Groups convert(const omg_group* g, size_t n) {
    if (n && !g) omg::fail(omg::E_INVALID, "null groups");
    Groups out;
    out.branches.resize(n);
    for (size_t i = 0; i < n; ++i) {
        if (g[i].prefix_len && !g[i].prefix) omg::fail(omg::E_INVALID, "null prefix");
        if (g[i].nbranches && !g[i].branches) omg::fail(omg::E_INVALID, "null branches");
        for (size_t b = 0; b < g[i].nbranches; ++b) {
            const omg_branch& br = g[i].branches[b];
            if ((br.ntokens && !br.tokens) || (br.nwant && !br.want)) omg::fail(omg::E_INVALID, "null branch data");
            out.branches[i].push_back({br.tokens, int64_t(br.ntokens), br.want, int64_t(br.nwant)});
        }
    }
    for (size_t i = 0; i < n; ++i)
        out.groups.push_back({g[i].prefix, int64_t(g[i].prefix_len), out.branches[i].data(), int64_t(g[i].nbranches)});
    return out;
}

omg::Engine& eng(omg_engine* e) {
    if (!e || !e->e) omg::fail(omg::E_INVALID, "null engine");
    return *e->e;
}

omg::QTensor make_tensor(int dtype, const int64_t* shape, size_t ndim, const void* data, size_t nbytes,
                         const void* scales, size_t nscale) {
    if (dtype < 0 || dtype > 2) omg::fail(omg::E_INVALID, "unknown dtype");
    omg::QTensor t;
    t.dtype = omg::Dtype(dtype);
    t.shape.assign(shape, shape + ndim);
    const uint8_t* d = static_cast<const uint8_t*>(data);
    const uint8_t* s = static_cast<const uint8_t*>(scales);
    if (nbytes && !d) omg::fail(omg::E_INVALID, "null tensor data");
    if (nscale && !s) omg::fail(omg::E_INVALID, "null tensor scales");
    t.data.assign(d, d + nbytes);
    t.scales.assign(s, s + nscale);
    return t;
}

}  // namespace

extern "C" {

const char* omg_last_error(void) { return g_err.c_str(); }

omg_builder* omg_builder_new(const char* config_json) {
    omg_builder* out = nullptr;
    guard([&] {
        if (!config_json) omg::fail(omg::E_INVALID, "null config");
        auto cfg = omg::Config::from_json(omg::Json::parse(config_json));
        out = new omg_builder{std::make_unique<omg::Builder>(std::move(cfg))};
    });
    return out;
}

int omg_builder_push(omg_builder* b, const char* name, int dtype, const int64_t* shape, size_t ndim,
                     const void* data, size_t nbytes, const void* scales, size_t nscale_bytes) {
    return guard([&] {
        if (!b || !b->b || !name || (ndim && !shape)) omg::fail(omg::E_INVALID, "null argument");
        b->b->push(name, make_tensor(dtype, shape, ndim, data, nbytes, scales, nscale_bytes));
    });
}

omg_weights* omg_synth(const char* config_json, uint64_t seed, int linear_dtype, int embed_dtype) {
    omg_weights* out = nullptr;
    guard([&] {
        if (!config_json) omg::fail(omg::E_INVALID, "null config");
        if (linear_dtype < 0 || linear_dtype > 2 || embed_dtype < 0 || embed_dtype > 2)
            omg::fail(omg::E_INVALID, "unknown dtype");
        auto cfg = omg::Config::from_json(omg::Json::parse(config_json));
        auto w = std::make_unique<omg_weights>();
        w->tensors = omg::synth_weights(cfg, seed, omg::Dtype(linear_dtype), omg::Dtype(embed_dtype)).tensors;
        w->index(cfg.tensors());
        out = w.release();
    });
    return out;
}

omg_weights* omg_load_dir(const char* dir) {
    omg_weights* out = nullptr;
    guard([&] {
        if (!dir) omg::fail(omg::E_INVALID, "null dir");
        auto w = std::make_unique<omg_weights>();
        omg::Weights loaded = omg::load_dir(dir);
        w->tensors = std::move(loaded.tensors);
        w->index(loaded.config.tensors());
        out = w.release();
    });
    return out;
}

omg_weights* omg_load_gguf(const char* path) {
    omg_weights* out = nullptr;
    guard([&] {
        if (!path) omg::fail(omg::E_INVALID, "null path");
        auto w = std::make_unique<omg_weights>();
        omg::Weights loaded = omg::load_gguf(path);
        w->tensors = std::move(loaded.tensors);
        w->index(loaded.config.tensors());
        out = w.release();
    });
    return out;
}

omg_engine* omg_open_gguf(const char* path, size_t capacity, size_t max_rows) {
    omg_engine* out = nullptr;
    guard([&] {
        if (!path) omg::fail(omg::E_INVALID, "null path");
        omg::Weights w = omg::load_gguf(path);
        omg::Builder b(w.config);
        for (const auto& kv : w.tensors) b.push(kv.first, kv.second);
        out = new omg_engine{b.finish(int64_t(capacity), int64_t(max_rows))};
    });
    return out;
}

size_t omg_weights_count(const omg_weights* w) { return w ? w->order.size() : 0; }

int omg_weights_get(const omg_weights* w, size_t i, const char** name, int* dtype, int64_t* shape, size_t* ndim,
                    const uint8_t** data, size_t* nbytes, const uint8_t** scales, size_t* nscale_bytes) {
    return guard([&] {
        if (!w || i >= w->order.size()) omg::fail(omg::E_INVALID, "weights index out of range");
        const auto& kv = *w->order[i];
        if (name) *name = kv.first.c_str();
        if (dtype) *dtype = int(kv.second.dtype);
        if (ndim) *ndim = kv.second.shape.size();
        if (shape)
            for (size_t k = 0; k < kv.second.shape.size() && k < 4; ++k) shape[k] = kv.second.shape[k];
        if (data) *data = kv.second.data.data();
        if (nbytes) *nbytes = kv.second.data.size();
        if (scales) *scales = kv.second.scales.data();
        if (nscale_bytes) *nscale_bytes = kv.second.scales.size();
    });
}

void omg_weights_free(omg_weights* w) { delete w; }

int omg_builder_push_weights(omg_builder* b, const omg_weights* w) {
    return guard([&] {
        if (!b || !b->b || !w) omg::fail(omg::E_INVALID, "null argument");
        for (const auto& kv : w->tensors) b->b->push(kv.first, kv.second);
    });
}

size_t omg_builder_missing(omg_builder* b, char* buf, size_t len) {
    if (!b || !b->b) return 0;
    const auto m = b->b->missing();
    std::string s;
    for (const auto& n : m) s += n + "\n";
    if (buf && len) {
        const size_t k = std::min(len - 1, s.size());
        std::memcpy(buf, s.data(), k);
        buf[k] = 0;
    }
    return m.size();
}

omg_engine* omg_builder_finish(omg_builder* b, size_t capacity, size_t max_rows) {
    omg_engine* out = nullptr;
    guard([&] {
        if (!b || !b->b) omg::fail(omg::E_INVALID, "null builder");
        std::unique_ptr<omg::Builder> keep = std::move(b->b);
        delete b;
        out = new omg_engine{keep->finish(int64_t(capacity), int64_t(max_rows))};
    });
    return out;
}

void omg_builder_free(omg_builder* b) { delete b; }

omg_engine* omg_open_dir(const char* dir, size_t capacity, size_t max_rows) {
    omg_engine* out = nullptr;
    guard([&] {
        if (!dir) omg::fail(omg::E_INVALID, "null dir");
        omg::Weights w = omg::load_dir(dir);
        omg::Builder b(w.config);
        for (auto& kv : w.tensors) b.push(kv.first, kv.second);
        out = new omg_engine{b.finish(int64_t(capacity), int64_t(max_rows))};
    });
    return out;
}

void omg_close(omg_engine* e) { delete e; }

int omg_config(const omg_engine* e, omg_config_t* out) {
    return guard([&] {
        if (!e || !e->e || !out) omg::fail(omg::E_INVALID, "null argument");
        const omg::Config& c = e->e->config();
        out->vocab = uint32_t(c.vocab);
        out->d = uint32_t(c.d);
        out->layers = uint32_t(c.layers);
        out->heads = uint32_t(c.heads);
        out->kv_heads = uint32_t(c.kv_heads);
        out->head_dim = uint32_t(c.max_head_dim());
        out->bos = c.bos;
        out->capacity = uint64_t(e->e->capacity());
        out->max_rows = uint64_t(e->e->max_rows());
    });
}

int omg_warmup(omg_engine* e) {
    return guard([&] { eng(e).warmup(); });
}

int omg_evaluate_groups(omg_engine* e, const omg_group* groups, size_t ngroups, int want,
                        const uint32_t* label_ids, size_t nlabels, float* out, size_t out_floats,
                        int* prefix_sources) {
    return guard([&] {
        Groups g = convert(groups, ngroups);
        if (!out && out_floats) omg::fail(omg::E_INVALID, "null output");
        eng(e).evaluate_groups(g.groups.data(), int64_t(ngroups), want, label_ids, int64_t(nlabels), out,
                               int64_t(out_floats), prefix_sources);
    });
}

int omg_set_pointer_head(omg_engine* e, size_t d, size_t dp, const float* w_q, const float* b_q, const float* w_k,
                         const float* b_k) {
    return guard([&] { eng(e).set_pointer_head(int64_t(d), int64_t(dp), w_q, b_q, w_k, b_k); });
}

int omg_evaluate_pointer(omg_engine* e, const omg_group* groups, size_t ngroups, const uint8_t* roles,
                         size_t nroles, float* out, size_t out_floats, size_t* written, int* prefix_sources) {
    return guard([&] {
        Groups g = convert(groups, ngroups);
        if (!out && out_floats) omg::fail(omg::E_INVALID, "null output");
        const int64_t k = eng(e).evaluate_pointer(g.groups.data(), int64_t(ngroups), roles, int64_t(nroles), out,
                                                  int64_t(out_floats), prefix_sources);
        if (written) *written = size_t(k);
    });
}

int omg_evaluate(omg_engine* e, const uint32_t* prefix, size_t prefix_len, const omg_branch* branches,
                 size_t nbranches, int want, const uint32_t* label_ids, size_t nlabels, float* out,
                 size_t out_floats) {
    const omg_group g{prefix, prefix_len, branches, nbranches};
    return omg_evaluate_groups(e, &g, 1, want, label_ids, nlabels, out, out_floats, nullptr);
}

int omg_prefix_source(const omg_engine* e) { return (e && e->e) ? e->e->prefix_source() : OMG_SRC_NONE; }

int omg_is_resident(const omg_engine* e, const uint32_t* prefix, size_t n) {
    return (e && e->e && (prefix || !n)) ? int(e->e->is_resident(prefix, int64_t(n))) : 0;
}

void omg_evict_resident(omg_engine* e) {
    if (e && e->e) e->e->evict_resident();
}

int omg_set_state_cache(omg_engine* e, size_t bytes, const char* dir, const char* model_id) {
    return guard([&] { eng(e).set_state_cache(bytes, dir ? dir : "", model_id ? model_id : ""); });
}

int omg_save_state(omg_engine* e, const uint32_t* prefix, size_t n, const char* model_id, uint8_t** bytes,
                   size_t* len) {
    return guard([&] {
        if (!bytes || !len || (n && !prefix)) omg::fail(omg::E_INVALID, "null argument");
        const auto [p, size] = eng(e).save_state_bytes(prefix, int64_t(n), model_id ? model_id : eng(e).model_id());
        *bytes = p;
        *len = size;
    });
}

int omg_restore_state(omg_engine* e, const uint8_t* bytes, size_t len, const char* model_id) {
    return guard([&] {
        if (!bytes && len) omg::fail(omg::E_INVALID, "null bytes");
        const omg::SavedState s =
            omg::SavedState::from_bytes(bytes, len, model_id ? model_id : eng(e).model_id());
        eng(e).restore_state(s);
    });
}

void omg_free_bytes(uint8_t* p) { std::free(p); }

int omg_quantize(int dtype, const float* values, size_t n, uint8_t* data, uint8_t* scales) {
    return guard([&] {
        if (!values || !data || !scales) omg::fail(omg::E_INVALID, "null argument");
        const std::vector<int64_t> shape{int64_t(n)};
        omg::QTensor t;
        if (dtype == OMG_DTYPE_Q8)
            t = omg::quantize_q8(shape, values);
        else if (dtype == OMG_DTYPE_Q4)
            t = omg::quantize_q4(shape, values);
        else
            omg::fail(omg::E_INVALID, "omg_quantize: dtype must be Q8 or Q4");
        std::memcpy(data, t.data.data(), t.data.size());
        std::memcpy(scales, t.scales.data(), t.scales.size());
    });
}

int omg_pack(const omg_group* groups, size_t ngroups, size_t first, int resident, size_t align, size_t rows,
             uint32_t* ids, int32_t* meta, int64_t* wanted, size_t* n_ids, size_t* n_wanted) {
    return guard([&] {
        if (!n_ids || !n_wanted) omg::fail(omg::E_INVALID, "null sizes");
        if (first >= ngroups) omg::fail(omg::E_INVALID, "first group out of range");
        Groups g = convert(groups, ngroups);
        omg::Packed pk = omg::pack_groups(g.groups.data(), int64_t(ngroups), int64_t(first), resident != 0);
        if (align > 1) pk = omg::align_groups(pk, int64_t(align), int64_t(rows));
        if (pk.ids.size() > *n_ids || pk.wanted.size() > *n_wanted)
            omg::fail(omg::E_CAPACITY, "omg_pack: output arrays too small");
        std::memcpy(ids, pk.ids.data(), pk.ids.size() * 4);
        std::memcpy(meta, pk.meta.data(), pk.meta.size() * 4);
        for (size_t r = 0; r < pk.wanted.size(); ++r)
            for (int k = 0; k < 4; ++k) wanted[4 * r + size_t(k)] = pk.wanted[r][size_t(k)];
        *n_ids = pk.ids.size();
        *n_wanted = pk.wanted.size();
    });
}

uint64_t omg_state_key(const char* model_id, const uint32_t* prefix, size_t n) {
    return omg::state_key(model_id ? model_id : "", prefix, int64_t(n));
}

int omg_state_check(const uint8_t* bytes, size_t len, const char* model_id, size_t* prefix_len, size_t* nlayers) {
    return guard([&] {
        if (!bytes && len) omg::fail(omg::E_INVALID, "null bytes");
        const omg::SavedState s = omg::SavedState::from_bytes(bytes, len, model_id ? model_id : "");
        if (prefix_len) *prefix_len = s.prefix.size();
        if (nlayers) *nlayers = s.layers.size();
    });
}

int omg_pass_prepare(omg_engine* e, const omg_group* groups, size_t ngroups, int want, const uint32_t* label_ids,
                     size_t nlabels, int first_resident) {
    return guard([&] {
        Groups g = convert(groups, ngroups);
        eng(e).prepare(g.groups.data(), int64_t(ngroups), want, label_ids, int64_t(nlabels), first_resident != 0);
    });
}

int omg_pass_launch(omg_engine* e) {
    return guard([&] { eng(e).launch_prepared(); });
}

int omg_pass_read(omg_engine* e, float* out, size_t out_floats, size_t* written) {
    return guard([&] {
        if (!out) omg::fail(omg::E_INVALID, "null output");
        const int64_t n = eng(e).read_prepared(out, int64_t(out_floats));
        if (written) *written = size_t(n);
    });
}

int omg_pass_graph(omg_engine* e, int on) {
    return guard([&] { eng(e).set_graph(on != 0); });
}

int omg_sync(omg_engine* e) {
    return guard([&] { eng(e).sync(); });
}

int omg_profile(omg_engine* e, int on) {
    return guard([&] { eng(e).set_profile(on != 0); });
}

int omg_set_full_last_layer(omg_engine* e, int on) {
    return guard([&] { eng(e).set_full_last_layer(on != 0); });
}

size_t omg_profile_report(omg_engine* e, char* buf, size_t len) {
    if (!e || !e->e) return 0;
    const std::string s = e->e->profile_report();
    if (buf && len) {
        const size_t k = std::min(len - 1, s.size());
        std::memcpy(buf, s.data(), k);
        buf[k] = 0;
    }
    return s.size();
}

omg_weight* omg_weight_upload(int dtype, int64_t rows, int64_t cols, const void* data, const void* scales) {
    omg_weight* out = nullptr;
    guard([&] {
        if (rows <= 0 || cols <= 0 || cols % 32) omg::fail(omg::E_INVALID, "weight: bad shape");
        const int64_t n = rows * cols;
        const int64_t shape[2] = {rows, cols};
        const size_t nbytes = size_t(omg::payload_bytes(omg::Dtype(dtype), n));
        omg::QTensor t = make_tensor(dtype, shape, 2, data, nbytes, scales, dtype == OMG_DTYPE_F16 ? 0 : size_t(n / 32 * 2));
        auto w = std::make_unique<omg_weight>();
        w->t = omg::upload_weight(t);
        out = w.release();
    });
    return out;
}

void omg_weight_free(omg_weight* w) { delete w; }

int omg_dev_gemm(const omg_weight* w, const void* x_f16, int64_t ldx, int64_t m, float* y, int64_t ldy,
                 void* stream) {
    return guard([&] {
        if (!w || !x_f16 || !y) omg::fail(omg::E_INVALID, "null argument");
        omg::launch_gemm(static_cast<hipStream_t>(stream), static_cast<const omg::half_t*>(x_f16), ldx, w->t.w, y, ldy,
                         m);
    });
}

int omg_dev_gemm_geglu(const omg_weight* wg, const omg_weight* wu, const void* x_f16, int64_t ldx, int64_t m,
                       void* act_f16, int64_t ldact, void* stream) {
    return guard([&] {
        if (!wg || !wu || !x_f16 || !act_f16) omg::fail(omg::E_INVALID, "null argument");
        omg::launch_gemm_geglu(static_cast<hipStream_t>(stream), static_cast<const omg::half_t*>(x_f16), ldx, wg->t.w,
                               wu->t.w, static_cast<omg::half_t*>(act_f16), ldact, m);
    });
}

int omg_dev_label_readout(const omg_weight* embed, const float* rows, int64_t nrows, const uint32_t* labels,
                          int64_t nlabels, float softcap, float* out, void* stream) {
    return guard([&] {
        if (!embed || !rows || !labels || !out) omg::fail(omg::E_INVALID, "null argument");
        if (nrows <= 0 || nlabels <= 0) omg::fail(omg::E_INVALID, "label readout: no rows or no labels");
        const hipStream_t s = static_cast<hipStream_t>(stream);
        const int64_t vocab = embed->t.w.rows, nb = omg::logits_blocks(vocab);
        // scratch: the full logits rows, then the per-workgroup partials
        // (float2, on an 8-byte boundary)
        const int64_t nlog = (nrows * vocab + 1) / 2 * 2;
        const size_t bytes = size_t(nlog) * 4 + size_t(nb * nrows) * 8;
        void* scratch = nullptr;
        OMG_HIP(hipMallocAsync(&scratch, bytes, s));
        float* logits = static_cast<float*>(scratch);
        float2* part = reinterpret_cast<float2*>(logits + nlog);
        try {
            omg::launch_logits(s, embed->t.w, rows, nrows, nullptr, vocab, softcap, logits, part);
            omg::launch_label_lse(s, logits, nrows, vocab, part, nb, labels, nlabels, out);
        } catch (...) {
            (void)hipFreeAsync(scratch, s);
            throw;
        }
        OMG_HIP(hipFreeAsync(scratch, s));
    });
}

int omg_dev_label_readout_noalloc(const omg_weight* embed, const float* rows, int64_t nrows, const uint32_t* labels,
                                  int64_t nlabels, float softcap, float* out, void* stream) {
    return guard([&] {
        if (!embed || !rows || !labels || !out) omg::fail(omg::E_INVALID, "null argument");
        omg::launch_label_readout_noalloc(static_cast<hipStream_t>(stream), embed->t.w, rows, nrows, labels, nlabels,
                                          softcap, out);
    });
}

int omg_dev_embed_norm(const omg_weight* embed, const uint32_t* ids, int64_t t, float scale, const float* w,
                       float eps, float* x, void* hn_f16, void* stream) {
    return guard([&] {
        if (!embed || !ids || !w || !x || !hn_f16) omg::fail(omg::E_INVALID, "null argument");
        omg::launch_embed_norm(static_cast<hipStream_t>(stream), embed->t.w, ids, t, scale, w, eps, x,
                               static_cast<omg::half_t*>(hn_f16));
    });
}

int omg_dev_gemm_geglu_erf(const omg_weight* wg, const omg_weight* wu, const void* x_f16, int64_t ldx, int64_t m,
                           void* act_f16, int64_t ldact, void* stream) {
    return guard([&] {
        if (!wg || !wu || !x_f16 || !act_f16) omg::fail(omg::E_INVALID, "null argument");
        omg::launch_gemm_geglu(static_cast<hipStream_t>(stream), static_cast<const omg::half_t*>(x_f16), ldx, wg->t.w,
                               wu->t.w, static_cast<omg::half_t*>(act_f16), ldact, m, true);
    });
}

int omg_dev_gemm_bias_relu(const omg_weight* w, const void* x_f16, int64_t ldx, int64_t m, const void* bias_f16,
                           void* y_f16, int64_t ldy, void* stream) {
    return guard([&] {
        if (!w || !x_f16 || !bias_f16 || !y_f16) omg::fail(omg::E_INVALID, "null argument");
        omg::launch_gemm_bias_relu(static_cast<hipStream_t>(stream), static_cast<const omg::half_t*>(x_f16), ldx, w->t.w,
                                   static_cast<const uint16_t*>(bias_f16), static_cast<omg::half_t*>(y_f16), ldy, m);
    });
}

int omg_dev_qkv_heads(const omg_weight* w, const void* x_f16, int64_t ldx, int64_t m, const void* bias_f16,
                      const float* rope, const int32_t* meta, float qscale, int64_t tpad, void* q16, void* k16,
                      void* vt, void* stream) {
    return guard([&] {
        if (!w || !x_f16) omg::fail(omg::E_INVALID, "null argument");
        omg::QkvHeads o{};
        o.rope = reinterpret_cast<const float2*>(rope);
        o.meta = meta;
        o.qscale = qscale;
        o.dq = w->t.w.rows / 3;
        o.tpad = tpad;
        o.q16 = static_cast<omg::half_t*>(q16);
        o.k16 = static_cast<omg::half_t*>(k16);
        o.vt = static_cast<omg::half_t*>(vt);
        omg::launch_gemm_qkv_heads(static_cast<hipStream_t>(stream), static_cast<const omg::half_t*>(x_f16), ldx,
                                   w->t.w, static_cast<const uint16_t*>(bias_f16), o, m);
    });
}

int omg_dev_attention_bi(const void* q16, const void* k16, const void* vt, const int32_t* meta, int heads, int64_t t,
                         int64_t tpad, int window, void* out_f16, void* stream) {
    return guard([&] {
        omg::QkvHeads o{};
        o.meta = meta;
        o.dq = int64_t(heads) * 64;
        o.tpad = tpad;
        o.q16 = static_cast<omg::half_t*>(const_cast<void*>(q16));
        o.k16 = static_cast<omg::half_t*>(const_cast<void*>(k16));
        o.vt = static_cast<omg::half_t*>(const_cast<void*>(vt));
        omg::launch_attention_bi(static_cast<hipStream_t>(stream), o, heads, t, window,
                                 static_cast<omg::half_t*>(out_f16));
    });
}

/* ---- the bidirectional encoder path ---- */

omg_laya_builder* omg_laya_builder_new(const char* config_json) {
    omg_laya_builder* out = nullptr;
    guard([&] {
        if (!config_json) omg::fail(omg::E_INVALID, "null config");
        auto cfg = omg::LayaConfig::from_json(omg::Json::parse(config_json));
        out = new omg_laya_builder{std::make_unique<omg::LayaBuilder>(std::move(cfg))};
    });
    return out;
}

int omg_laya_builder_push(omg_laya_builder* b, const char* name, int dtype, const int64_t* shape, size_t ndim,
                          const void* data, size_t nbytes, const void* scales, size_t nscale_bytes) {
    return guard([&] {
        if (!b || !b->b || !name || (ndim && !shape)) omg::fail(omg::E_INVALID, "null argument");
        b->b->push(name, make_tensor(dtype, shape, ndim, data, nbytes, scales, nscale_bytes));
    });
}

int omg_laya_builder_push_weights(omg_laya_builder* b, const omg_weights* w) {
    return guard([&] {
        if (!b || !b->b || !w) omg::fail(omg::E_INVALID, "null argument");
        for (const auto& kv : w->tensors) b->b->push(kv.first, kv.second);
    });
}

size_t omg_laya_builder_missing(omg_laya_builder* b, char* buf, size_t len) {
    if (!b || !b->b) return 0;
    const auto m = b->b->missing();
    std::string s;
    for (const auto& n : m) s += n + "\n";
    if (buf && len) {
        const size_t k = s.size() < len - 1 ? s.size() : len - 1;
        std::memcpy(buf, s.data(), k);
        buf[k] = 0;
    }
    return m.size();
}

omg_laya* omg_laya_builder_finish(omg_laya_builder* b, size_t capacity, size_t max_rows) {
    omg_laya* out = nullptr;
    guard([&] {
        if (!b || !b->b) omg::fail(omg::E_INVALID, "null builder");
        std::unique_ptr<omg::LayaBuilder> own = std::move(b->b);
        out = new omg_laya{own->finish(int64_t(capacity), int64_t(max_rows))};
    });
    delete b;
    return out;
}

void omg_laya_builder_free(omg_laya_builder* b) { delete b; }

omg_weights* omg_laya_synth(const char* config_json, uint64_t seed, int linear_dtype, int embed_dtype) {
    omg_weights* out = nullptr;
    guard([&] {
        if (!config_json) omg::fail(omg::E_INVALID, "null config");
        if (linear_dtype < 0 || linear_dtype > 2 || embed_dtype < 0 || embed_dtype > 2)
            omg::fail(omg::E_INVALID, "unknown dtype");
        auto cfg = omg::LayaConfig::from_json(omg::Json::parse(config_json));
        auto w = std::make_unique<omg_weights>();
        w->tensors = omg::synth_laya(cfg, seed, omg::Dtype(linear_dtype), omg::Dtype(embed_dtype)).tensors;
        w->index(cfg.tensors());
        out = w.release();
    });
    return out;
}

omg_weights* omg_laya_load_dir(const char* dir, const uint32_t* special_ids) {
    omg_weights* out = nullptr;
    guard([&] {
        if (!dir) omg::fail(omg::E_INVALID, "null dir");
        omg::LayaWeights lw = omg::load_laya_dir(dir, special_ids);
        auto w = std::make_unique<omg_weights>();
        w->tensors = std::move(lw.tensors);
        w->index(lw.config.tensors());
        out = w.release();
    });
    return out;
}

omg_laya* omg_laya_open_dir(const char* dir, const uint32_t* special_ids, size_t capacity, size_t max_rows) {
    omg_laya* out = nullptr;
    guard([&] {
        if (!dir) omg::fail(omg::E_INVALID, "null dir");
        omg::LayaWeights lw = omg::load_laya_dir(dir, special_ids);
        omg::LayaBuilder b(lw.config);
        for (const auto& kv : lw.tensors) b.push(kv.first, kv.second);
        auto e = b.finish(int64_t(capacity), int64_t(max_rows));
        e->warmup();
        out = new omg_laya{std::move(e)};
    });
    return out;
}

void omg_laya_close(omg_laya* e) { delete e; }

}  // extern "C"

namespace {

omg::LayaEngine& laya(omg_laya* e) {
    if (!e || !e->e) omg::fail(omg::E_INVALID, "null engine");
    return *e->e;
}

std::vector<omg::LayaSeq> laya_seqs(const omg_laya_seq* s, size_t n) {
    if (n && !s) omg::fail(omg::E_INVALID, "null sequences");
    std::vector<omg::LayaSeq> v;
    for (size_t i = 0; i < n; ++i) {
        if ((s[i].nids && !s[i].ids) || (s[i].nmarkers && !s[i].markers)) omg::fail(omg::E_INVALID, "null sequence data");
        v.push_back({s[i].ids, int64_t(s[i].nids), s[i].markers, int64_t(s[i].nmarkers), s[i].qtype});
    }
    return v;
}

}  // namespace

extern "C" {

int omg_laya_hidden(omg_laya* e, const omg_laya_seq* seqs, size_t n, float* out, size_t out_floats) {
    return guard([&] {
        auto v = laya_seqs(seqs, n);
        if (!out) omg::fail(omg::E_INVALID, "null output");
        laya(e).hidden(v.data(), int64_t(n), out, int64_t(out_floats));
    });
}

int omg_laya_evaluate(omg_laya* e, const omg_laya_seq* seqs, size_t n, float* logits, size_t nlogits, float* act,
                      size_t nact) {
    return guard([&] {
        auto v = laya_seqs(seqs, n);
        if ((nlogits && !logits) || (nact && !act)) omg::fail(omg::E_INVALID, "null output");
        laya(e).evaluate(v.data(), int64_t(n), logits, int64_t(nlogits), act, int64_t(nact));
    });
}

int omg_laya_warmup(omg_laya* e) {
    return guard([&] { laya(e).warmup(); });
}

int omg_laya_config(const omg_laya* e, omg_laya_config_t* out) {
    return guard([&] {
        if (!e || !e->e || !out) omg::fail(omg::E_INVALID, "null argument");
        const omg::LayaConfig& c = e->e->config();
        out->vocab = uint32_t(c.vocab);
        out->d = uint32_t(c.d);
        out->layers = uint32_t(c.layers);
        out->heads = uint32_t(c.heads);
        out->ff = uint32_t(c.ff);
        out->head_layers = uint32_t(c.head_layers);
        out->act_out = uint32_t(c.act_out);
        out->max_len = uint32_t(c.max_len);
        out->cls = c.cls;
        out->sep = c.sep;
        out->mask = c.mask;
        out->pad = c.pad;
        out->capacity = uint64_t(e->e->capacity());
        out->max_rows = uint64_t(e->e->max_rows());
    });
}

int omg_laya_temperature(const omg_laya* e, int qtype, size_t k, float* out) {
    return guard([&] {
        if (!e || !e->e || !out) omg::fail(omg::E_INVALID, "null argument");
        if (qtype < 0 || qtype >= 3) omg::fail(omg::E_INVALID, "question type " + std::to_string(qtype));
        *out = e->e->config().temperature_for(qtype, int64_t(k));
    });
}

int omg_laya_prepare(omg_laya* e, const omg_laya_seq* seqs, size_t n) {
    return guard([&] {
        auto v = laya_seqs(seqs, n);
        laya(e).prepare(v.data(), int64_t(n));
    });
}

int omg_laya_launch(omg_laya* e) {
    return guard([&] { laya(e).launch_prepared(); });
}

int omg_laya_sync(omg_laya* e) {
    return guard([&] { laya(e).sync(); });
}

int omg_laya_profile(omg_laya* e, int on) {
    return guard([&] { laya(e).set_profile(on != 0); });
}

int omg_laya_set_full_last_layer(omg_laya* e, int on) {
    return guard([&] { laya(e).set_full_last_layer(on != 0); });
}

size_t omg_laya_profile_report(omg_laya* e, char* buf, size_t len) {
    std::string s;
    guard([&] { s = laya(e).profile_report(); });
    if (buf && len) {
        const size_t k = s.size() < len - 1 ? s.size() : len - 1;
        std::memcpy(buf, s.data(), k);
        buf[k] = 0;
    }
    return s.size();
}

}  // extern "C"
