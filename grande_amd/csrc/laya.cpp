// The encoder path's host side: config, seeded weights, builder, the pass
// plan (laya.rs:1138-1432) and the host scorer (laya.rs:1442-1547).
#include "laya.h"

#include <algorithm>
#include <cmath>
#include <cstring>

namespace omg {

namespace {

int64_t need(const Json& v, const char* k) {
    if (!v.has(k) || !v[k].is_uint()) fail(E_INVALID, std::string("encoder/config.json: missing ") + k);
    return int64_t(v[k].u64(0));
}

int64_t count(const std::vector<int64_t>& s) {
    int64_t n = 1;
    for (int64_t x : s) n *= x;
    return n;
}

bool ends_with(const std::string& s, const char* suf) {
    const size_t n = std::strlen(suf);
    return s.size() >= n && s.compare(s.size() - n, n, suf) == 0;
}

// laya.rs:1496-1547: the host half in f32, sums in order.
std::vector<float> layer_norm(const float* x, int64_t n, const float* w, const float* b, float eps) {
    float mean = 0.0f;
    for (int64_t i = 0; i < n; ++i) mean += x[i];
    mean /= float(n);
    float var = 0.0f;
    for (int64_t i = 0; i < n; ++i) var += (x[i] - mean) * (x[i] - mean);
    var /= float(n);
    const float inv = 1.0f / std::sqrt(var + eps);
    std::vector<float> y(static_cast<size_t>(n));
    for (int64_t i = 0; i < n; ++i) y[size_t(i)] = (x[i] - mean) * inv * w[i] + b[i];
    return y;
}

float dot(const float* a, const float* b, int64_t n) {
    float s = 0.0f;
    for (int64_t i = 0; i < n; ++i) s += a[i] * b[i];
    return s;
}

std::vector<float> linear(const std::vector<float>& x, const std::vector<float>& w, const std::vector<float>& b) {
    const int64_t k = int64_t(x.size()), out = int64_t(b.size());
    std::vector<float> y(static_cast<size_t>(out));
    for (int64_t r = 0; r < out; ++r) y[size_t(r)] = dot(w.data() + r * k, x.data(), k) + b[size_t(r)];
    return y;
}

// Abramowitz & Stegun 7.1.26 (|error| < 1.5e-7), the reference's erf.
float erf_as(float x) {
    const float s = x > 0.0f ? 1.0f : (x < 0.0f ? -1.0f : 0.0f);
    const float a = std::fabs(x);
    const float t = 1.0f / (1.0f + 0.3275911f * a);
    const float poly = ((((1.061405429f * t - 1.453152027f) * t + 1.421413741f) * t - 0.284496736f) * t +
                        0.254829592f) * t;
    return s * (1.0f - poly * std::exp(-a * a));
}

float gelu_erf_host(float x) { return 0.5f * x * (1.0f + erf_as(x * 0.70710678118654752f)); }

std::vector<float> softmax(const std::vector<float>& z) {
    float m = -INFINITY;
    for (float v : z) m = std::max(m, v);
    std::vector<float> e(z.size());
    float s = 0.0f;
    for (size_t i = 0; i < z.size(); ++i) {
        e[i] = std::exp(z[i] - m);
        s += e[i];
    }
    for (float& v : e) v /= s;
    return e;
}

DevBuf upload(const void* src, size_t n) {
    DevBuf b(n);
    OMG_HIP(hipMemcpy(b.p, src, n, hipMemcpyHostToDevice));
    return b;
}

std::vector<float> to_f32(const QTensor& t) {
    std::vector<float> v(size_t(t.numel()));
    for (int64_t i = 0; i < t.numel(); ++i) v[size_t(i)] = t.get(i);
    return v;
}

}  // namespace

// ------------------------------------------------------------------ config

LayaConfig LayaConfig::from_json(const Json& v) {
    if (v["model_type"].s("") != "modernbert")
        fail(E_INVALID, "encoder model_type " + v["model_type"].s("?") + " is not modernbert");
    if (v.has("hidden_activation") && v["hidden_activation"].s("gelu") != "gelu")
        fail(E_INVALID, "encoder hidden_activation " + v["hidden_activation"].s("?") + " is not gelu");
    LayaConfig c;
    c.layers = need(v, "num_hidden_layers");
    const int64_t every = int64_t(v["global_attn_every_n_layers"].u64(3));
    if (v["layer_types"].kind == Json::Array) {
        for (const Json& t : v["layer_types"].arr) c.sliding.push_back(t.s("") == "sliding_attention");
    } else {
        for (int64_t i = 0; i < c.layers; ++i) c.sliding.push_back(every == 0 ? false : i % every != 0);
    }
    if (int64_t(c.sliding.size()) != c.layers)
        fail(E_INVALID, "layer_types has " + std::to_string(c.sliding.size()) + " entries for " +
                            std::to_string(c.layers) + " layers");
    const Json& rope = v["rope_parameters"];
    c.theta_global = float(rope["full_attention"]["rope_theta"].f64(v["global_rope_theta"].f64(160000.0)));
    c.theta_local = float(rope["sliding_attention"]["rope_theta"].f64(v["local_rope_theta"].f64(10000.0)));
    c.eps = float(v["norm_eps"].f64(v["layer_norm_eps"].f64(1e-5)));
    c.vocab = need(v, "vocab_size");
    c.d = need(v, "hidden_size");
    c.heads = need(v, "num_attention_heads");
    c.ff = need(v, "intermediate_size");
    c.window = int64_t(v["local_attention"].u64(128)) / 2;

    const Json& agent = v["laya_agent"];
    if (agent.has("temperature")) {
        const Json& t = agent["temperature"];
        if (t.kind != Json::Array || t.arr.size() != 3)
            fail(E_INVALID, "rl_agent_config.json: temperature must have 3 entries");
        for (int i = 0; i < 3; ++i) c.temperature[i] = float(t.arr[size_t(i)].f64(1.0));
    }
    if (agent["temperature_by_options"].kind == Json::Object)
        for (const auto& kv : agent["temperature_by_options"].obj) c.temperature_by_options[kv.first] = float(kv.second.f64(1.0));
    for (float t : c.temperature)
        if (!std::isfinite(t) || t <= 0.0f) fail(E_INVALID, "calibration temperatures must be finite and positive");
    for (const auto& kv : c.temperature_by_options)
        if (!std::isfinite(kv.second) || kv.second <= 0.0f)
            fail(E_INVALID, "calibration temperatures must be finite and positive");
    c.max_len = int64_t(agent["max_len"].u64(512));
    c.head_max_len = int64_t(agent["head_max_len"].u64(192));
    if (!(4 < c.head_max_len && c.head_max_len < c.max_len))
        fail(E_INVALID, "expected 4 < head_max_len " + std::to_string(c.head_max_len) + " < max_len " +
                            std::to_string(c.max_len));
    c.head_layers = int64_t(agent["head_layers"].u64(2));
    c.type_emb = agent["type_emb"].boolean(true);
    c.act_hidden = 256;
    c.act_out = 0;
    if (!(agent.has("act_head") && agent["act_head"].kind == Json::Bool && !agent["act_head"].b))
        c.act_out = agent["act_costs"].kind == Json::Object ? int64_t(agent["act_costs"].obj.size()) + 1 : 0;
    const Json& tok = v["laya_tokens"];
    auto id = [&](const char* name) -> uint32_t {
        const Json& t = tok[name];
        if (t.is_uint()) return uint32_t(t.u64(0));
        if (t.kind == Json::Object && t["id"].is_uint()) return uint32_t(t["id"].u64(0));
        fail(E_INVALID, std::string("laya_tokens: missing the id of ") + name);
    };
    c.cls = id("cls_token");
    c.sep = id("sep_token");
    c.mask = id("mask_token");
    c.pad = id("pad_token");
    c.validate();
    return c;
}

void LayaConfig::validate() const {
    if (heads <= 0 || d % heads != 0)
        fail(E_INVALID, "hidden_size " + std::to_string(d) + " / heads " + std::to_string(heads));
    if (head_dim() != 64) fail(E_INVALID, "head_dim " + std::to_string(head_dim()) + ": this engine's encoder kernels take 64");
    if (d % 32 != 0 || ff % 32 != 0) fail(E_INVALID, "hidden_size and intermediate_size must be multiples of 32");
    if (d > 2048) fail(E_INVALID, "hidden_size " + std::to_string(d) + " > 2048");
    if (layers <= 0 || vocab <= 0) fail(E_INVALID, "empty encoder");
    if (int64_t(sliding.size()) != layers) fail(E_INVALID, "layer_types length mismatch");
    if (window < 0 || max_len <= 0) fail(E_INVALID, "bad window or max_len");
    if (cls >= vocab || sep >= vocab || mask >= vocab || pad >= vocab) fail(E_INVALID, "special token outside the vocabulary");
}

float LayaConfig::temperature_for(int qtype, int64_t k) const {
    static const char* names[3] = {"choice", "score", "noul"};
    const char* size = k <= 2 ? "2" : (k <= 5 ? "3-5" : (k <= 10 ? "6-10" : "11+"));
    auto it = temperature_by_options.find(std::string(names[qtype]) + ":" + size);
    return it != temperature_by_options.end() ? it->second : temperature[qtype];
}

std::vector<TensorSpec> LayaConfig::tensors() const {
    std::vector<TensorSpec> v{{"embed", {vocab, d}}, {"embed_norm", {d}}, {"final_norm", {d}}};
    if (type_emb) v.push_back({"type_emb", {3, d}});
    for (int64_t l = 0; l < layers; ++l) {
        auto n = [&](const char* s) { return "enc." + std::to_string(l) + "." + s; };
        if (l > 0) v.push_back({n("attn_norm"), {d}});
        v.push_back({n("qkv"), {3 * d, d}});
        v.push_back({n("o"), {d, d}});
        v.push_back({n("mlp_norm"), {d}});
        v.push_back({n("wi_val"), {ff, d}});
        v.push_back({n("wi_gate"), {ff, d}});
        v.push_back({n("wo"), {d, ff}});
    }
    for (int64_t h = 0; h < head_layers; ++h) {
        auto n = [&](const char* s) { return "head." + std::to_string(h) + "." + s; };
        v.push_back({n("norm1_w"), {d}});
        v.push_back({n("norm1_b"), {d}});
        v.push_back({n("in_proj"), {3 * d, d}});
        v.push_back({n("in_proj_b"), {3 * d}});
        v.push_back({n("out_proj"), {d, d}});
        v.push_back({n("out_proj_b"), {d}});
        v.push_back({n("norm2_w"), {d}});
        v.push_back({n("norm2_b"), {d}});
        v.push_back({n("l1"), {4 * d, d}});
        v.push_back({n("l1_b"), {4 * d}});
        v.push_back({n("l2"), {d, 4 * d}});
        v.push_back({n("l2_b"), {d}});
    }
    v.push_back({"scorer.norm_w", {d}});
    v.push_back({"scorer.norm_b", {d}});
    v.push_back({"scorer.l1", {d, d}});
    v.push_back({"scorer.l1_b", {d}});
    v.push_back({"scorer.l2", {1, d}});
    v.push_back({"scorer.l2_b", {1}});
    if (act_out > 0) {
        v.push_back({"act.l1", {act_hidden, d + 4}});
        v.push_back({"act.l1_b", {act_hidden}});
        v.push_back({"act.l2", {act_out, act_hidden}});
        v.push_back({"act.l2_b", {act_out}});
    }
    return v;
}

bool laya_host_tensor(const std::string& name) { return name.rfind("scorer.", 0) == 0 || name.rfind("act.", 0) == 0; }

LayaWeights synth_laya(const LayaConfig& cfg, uint64_t seed, Dtype linear, Dtype embed) {
    cfg.validate();
    Rng r(seed | 1);
    LayaWeights w;
    w.config = cfg;
    std::vector<float> buf;
    for (const TensorSpec& spec : cfg.tensors()) {
        const std::string& nm = spec.name;
        const int64_t n = count(spec.shape);
        buf.resize(size_t(n));
        const bool norm = ends_with(nm, "norm") || ends_with(nm, "norm_w") || ends_with(nm, "norm1_w") ||
                          ends_with(nm, "norm2_w");
        if (spec.shape.size() == 1) {
            for (int64_t i = 0; i < n; ++i) buf[size_t(i)] = norm ? 1.0f + 0.5f * r.next() : 0.02f * r.next();
            w.tensors[nm] = from_f32(spec.shape, buf.data());
            continue;
        }
        // Linears at 1/sqrt(fan-in): the decision-head attention has no
        // 1/sqrt(head_dim) factor (laya.rs:1346-1350), and wider weights
        // saturate its softmax.
        const float scale = nm == "embed" ? 1.0f : (nm == "type_emb" ? 0.15f : 1.0f / std::sqrt(float(spec.shape[1])));
        for (int64_t i = 0; i < n; ++i) buf[size_t(i)] = r.next() * scale;
        const Dtype dt = nm == "embed" ? embed : ((laya_host_tensor(nm) || nm == "type_emb") ? F16 : linear);
        switch (dt) {
            case F16: w.tensors[nm] = from_f32(spec.shape, buf.data()); break;
            case Q8: w.tensors[nm] = quantize_q8(spec.shape, buf.data()); break;
            default: w.tensors[nm] = quantize_q4(spec.shape, buf.data()); break;
        }
    }
    return w;
}

LayaWeights load_laya_dir(const std::string& dir, const uint32_t* special) {
    Json v = Json::parse(read_file(dir + "/config.json"));
    if (special) {
        static const char* names[4] = {"cls_token", "sep_token", "mask_token", "pad_token"};
        Json tok;
        tok.kind = Json::Object;
        for (int i = 0; i < 4; ++i) {
            Json id;
            id.kind = Json::Number;
            id.num = double(special[i]);
            tok.obj[names[i]] = id;
        }
        v.obj["laya_tokens"] = tok;
    }
    LayaWeights w;
    w.config = LayaConfig::from_json(v);
    w.tensors = read_manifest(dir);
    return w;
}

// ----------------------------------------------------------------- builder

LayaBuilder::LayaBuilder(LayaConfig cfg) : cfg_(std::move(cfg)) {
    cfg_.validate();
    for (const TensorSpec& s : cfg_.tensors()) expected_[s.name] = s.shape;
}

void LayaBuilder::push(const std::string& name, const QTensor& t) {
    auto it = expected_.find(name);
    if (it == expected_.end()) fail(E_INVALID, "unexpected tensor " + name);
    if (t.shape != it->second) fail(E_INVALID, name + ": shape mismatch");
    const int64_t n = t.numel();
    if (int64_t(t.data.size()) != payload_bytes(t.dtype, n)) fail(E_INVALID, name + ": payload size mismatch");
    if (t.dtype != F16 && int64_t(t.scales.size()) != n / BLOCK * 2) fail(E_INVALID, name + ": scale size mismatch");
    linears_.erase(name);
    vecs_.erase(name);
    host_.erase(name);
    if (laya_host_tensor(name)) {
        host_[name] = to_f32(t);
        return;
    }
    if (t.shape.size() == 1 && t.dtype != F16) fail(E_INVALID, name + ": 1-D tensors must be f16");
    if (t.shape.size() == 1 || name == "type_emb") {
        // Norm weights, biases and the type embedding are read as f32 (the
        // reference unpacks its f16 pairs to f32, laya.rs:1231-1232).
        const std::vector<float> v = to_f32(t);
        vecs_[name] = upload(v.data(), v.size() * 4);
        if (ends_with(name, "in_proj_b") || ends_with(name, "l1_b"))  // GEMM epilogue biases stay f16
            vecs_[name + ".f16"] = upload(t.data.data(), t.data.size());
        return;
    }
    if (t.shape[1] % 32 != 0) fail(E_INVALID, name + ": inner dimension " + std::to_string(t.shape[1]) + " is not a multiple of 32");
    linears_[name] = upload_weight(t, name != "embed");
}

std::vector<std::string> LayaBuilder::missing() const {
    std::vector<std::string> v;
    for (const auto& kv : expected_)
        if (!linears_.count(kv.first) && !vecs_.count(kv.first) && !host_.count(kv.first)) v.push_back(kv.first);
    return v;
}

std::unique_ptr<LayaEngine> LayaBuilder::finish(int64_t capacity, int64_t max_rows) {
    const auto miss = missing();
    if (!miss.empty()) {
        std::string m = std::to_string(miss.size()) + " tensors missing, e.g.";
        for (size_t i = 0; i < miss.size() && i < 4; ++i) m += " " + miss[i];
        fail(E_MISSING, m);
    }
    if (capacity <= 0 || max_rows <= 0) fail(E_INVALID, "capacity and max_rows must be positive");
    const LayaConfig& c = cfg_;
    std::unique_ptr<LayaEngine> e(new LayaEngine());
    LayaEngine& E = *e;
    E.cfg_ = c;
    E.capacity_ = capacity;
    E.max_rows_ = max_rows;
    // Workspace rows: the tokens plus up to 31 alignment rows before each
    // sequence (every sequence reads back at least its [CLS] row, so there
    // are at most max_rows of them).
    E.rows_cap_ = capacity + 31 * max_rows;
    E.tpad_ = (E.rows_cap_ + 63) / 64 * 64;
    OMG_HIP(hipStreamCreateWithFlags(&E.stream_, hipStreamNonBlocking));
    auto lin = [&](const std::string& n) { return std::move(linears_.at(n)); };
    auto vec = [&](const std::string& n) { return std::move(vecs_.at(n)); };
    E.embed_ = lin("embed");
    E.embed_norm_ = vec("embed_norm");
    E.final_norm_ = vec("final_norm");
    if (c.type_emb) E.type_emb_ = vec("type_emb");
    for (int64_t l = 0; l < c.layers; ++l) {
        auto n = [&](const char* s) { return "enc." + std::to_string(l) + "." + s; };
        LayaEngine::Enc L;
        L.qkv = lin(n("qkv"));
        L.o = lin(n("o"));
        L.wi_val = lin(n("wi_val"));
        L.wi_gate = lin(n("wi_gate"));
        L.wo = lin(n("wo"));
        if (L.wi_val.w.dtype != L.wi_gate.w.dtype)
            fail(E_INVALID, "layer " + std::to_string(l) + ": Wi halves must share a storage type");
        if (l > 0) L.attn_norm = vec(n("attn_norm"));
        L.mlp_norm = vec(n("mlp_norm"));
        L.sliding = c.sliding[size_t(l)];
        E.enc_.push_back(std::move(L));
    }
    for (int64_t h = 0; h < c.head_layers; ++h) {
        auto n = [&](const char* s) { return "head." + std::to_string(h) + "." + s; };
        LayaEngine::Head H;
        H.in_proj = lin(n("in_proj"));
        H.out_proj = lin(n("out_proj"));
        H.l1 = lin(n("l1"));
        H.l2 = lin(n("l2"));
        H.norm1_w = vec(n("norm1_w"));
        H.norm1_b = vec(n("norm1_b"));
        H.in_proj_b16 = vec(n("in_proj_b") + std::string(".f16"));
        H.out_proj_b = vec(n("out_proj_b"));
        H.norm2_w = vec(n("norm2_w"));
        H.norm2_b = vec(n("norm2_b"));
        H.l1_b16 = vec(n("l1_b") + std::string(".f16"));
        H.l2_b = vec(n("l2_b"));
        E.head_.push_back(std::move(H));
    }
    E.host_ = std::move(host_);

    // RoPE (cos, sin) per position below max_len: inv_freq[i] =
    // theta^(-2i / 64) (rope_bi.wgsl:34).
    const int64_t rows = c.max_len;
    auto table = [&](float theta) {
        std::vector<float> f(32);
        for (int i = 0; i < 32; ++i) f[size_t(i)] = std::pow(theta, -float(2 * i) / 64.0f);
        DevBuf inv = upload(f.data(), f.size() * 4);
        DevBuf out(size_t(rows * 32) * 8);
        launch_rope_table(E.stream_, inv.as<float>(), rows, 32, out.as<float2>());
        OMG_HIP(hipStreamSynchronize(E.stream_));
        return out;
    };
    E.rope_local_ = table(c.theta_local);
    E.rope_global_ = table(c.theta_global);

    const int64_t cap = E.rows_cap_, d = c.d, tp = E.tpad_;
    E.ids_ = DevBuf(size_t(cap) * 4);
    E.qtypes_ = DevBuf(size_t(cap) * 4);
    E.meta_ = DevBuf(size_t(cap) * 16, true);
    E.x_ = DevBuf(size_t(cap * d) * 4);
    E.a_ = DevBuf(size_t(cap * d) * 4);
    E.h16_ = DevBuf(size_t(cap * d) * 2);
    // Head arrays are read in whole 32-key tiles: zeroed once so rows past
    // a pass's tokens always hold finite values.
    E.q16_ = DevBuf(size_t(c.heads * tp * 64) * 2, true);
    E.k16_ = DevBuf(size_t(c.heads * tp * 64) * 2, true);
    E.vt_ = DevBuf(size_t(c.heads * tp * 64) * 2, true);
    E.attn16_ = DevBuf(size_t(cap * d) * 2);
    E.act16_ = DevBuf(size_t(cap * std::max(c.ff, 4 * d)) * 2);
    E.rows_ = DevBuf(size_t(max_rows * d) * 4);
    E.wanted_ = DevBuf(size_t(max_rows) * 4);
    E.attn_w_ = DevBuf(size_t(max_rows * d) * 2);
    E.x_w_ = DevBuf(size_t(max_rows * d) * 4);
    E.a_w_ = DevBuf(size_t(max_rows * d) * 4);
    E.h16_w_ = DevBuf(size_t(max_rows * d) * 2);
    E.act_w_ = DevBuf(size_t(max_rows * 4 * d) * 2);
    E.h_in_bytes_ = size_t(cap) * (4 + 4 + 16) + size_t(max_rows) * 4;
    OMG_HIP(hipHostMalloc(&E.h_in_, E.h_in_bytes_, hipHostMallocDefault));
    E.h_out_bytes_ = size_t(max_rows * d) * 4;
    OMG_HIP(hipHostMalloc(&E.h_out_, E.h_out_bytes_, hipHostMallocDefault));
    return e;
}

// ------------------------------------------------------------------ engine

LayaEngine::~LayaEngine() {
    if (stream_) (void)hipStreamSynchronize(stream_);
    for (Timed& t : pending_) (void)hipEventDestroy(t.e);
    for (hipEvent_t ev : event_pool_) (void)hipEventDestroy(ev);
    if (h_in_) (void)hipHostFree(h_in_);
    if (h_out_) (void)hipHostFree(h_out_);
    if (stream_) (void)hipStreamDestroy(stream_);
}

template <class F>
void LayaEngine::step(const char* name, F&& f) {
    if (!profile_) return f();
    auto ev = [&] {
        if (event_pool_.empty()) {
            hipEvent_t e;
            OMG_HIP(hipEventCreateWithFlags(&e, hipEventDisableSystemFence));
            return e;
        }
        hipEvent_t e = event_pool_.back();
        event_pool_.pop_back();
        return e;
    };
    if (pending_.empty()) {
        const hipEvent_t start = ev();
        OMG_HIP(hipEventRecord(start, stream_));
        pending_.push_back(Timed{nullptr, start});
    }
    f();
    const hipEvent_t end = ev();
    OMG_HIP(hipEventRecord(end, stream_));
    pending_.push_back(Timed{name, end});
}

void LayaEngine::collect_profile() {
    for (size_t i = 1; i < pending_.size(); ++i) {
        float ms = 0.0f;
        OMG_HIP(hipEventElapsedTime(&ms, pending_[i - 1].e, pending_[i].e));
        auto& tot = totals_[pending_[i].name];
        tot.first += 1;
        tot.second += double(ms);
    }
    for (Timed& t : pending_) event_pool_.push_back(t.e);
    pending_.clear();
}

void LayaEngine::set_profile(bool on) {
    sync();
    profile_ = on;
    totals_.clear();
}

std::string LayaEngine::profile_report() const {
    std::string s;
    char line[256];
    for (const auto& kv : totals_) {
        std::snprintf(line, sizeof line, "%s %lld %.6f\n", kv.first.c_str(), (long long)kv.second.first,
                      kv.second.second);
        s += line;
    }
    return s;
}

void LayaEngine::sync() {
    OMG_HIP(hipStreamSynchronize(stream_));
    if (!pending_.empty()) collect_profile();
}

// laya.rs:1138-1209: validate, pack the sequences back to back (meta =
// position, sequence, first row, last row + 1), list the rows to read
// back ([CLS] = each sequence's first token, then its markers) and upload.
int64_t LayaEngine::pack(const LayaSeq* seqs, int64_t n) {
    const LayaConfig& c = cfg_;
    int64_t total = 0;
    for (int64_t i = 0; i < n; ++i) total += seqs[i].n;
    if (total == 0) fail(E_INVALID, "empty request");
    if (total > capacity_)
        fail(E_CAPACITY, std::to_string(total) + " tokens exceed the engine capacity " + std::to_string(capacity_));
    sync();
    uint8_t* h = static_cast<uint8_t*>(h_in_);
    uint32_t* ids = reinterpret_cast<uint32_t*>(h);
    uint32_t* qt = ids + rows_cap_;
    int32_t* meta = reinterpret_cast<int32_t*>(qt + rows_cap_);
    int32_t* wanted = meta + 4 * rows_cap_;
    int64_t at = 0, nw = 0;
    for (int64_t si = 0; si < n; ++si) {
        const LayaSeq& s = seqs[si];
        // Each sequence starts on a 32-row boundary, so its rows meet the
        // attention kernel's 32-key tiles the same way in every batch and a
        // sequence's results do not depend on its neighbours.  Rows between
        // sequences are padding: a sequence of their own, seen by nothing.
        for (; at % 32 != 0; ++at) {
            ids[at] = c.pad;
            qt[at] = 0;
            meta[4 * at] = 0;
            meta[4 * at + 1] = -1;
            meta[4 * at + 2] = int32_t(at);
            meta[4 * at + 3] = int32_t(at + 1);
        }
        if (s.n <= 0) fail(E_INVALID, "sequence " + std::to_string(si) + " is empty");
        if (s.n > c.max_len)
            fail(E_INVALID, "sequence " + std::to_string(si) + ": " + std::to_string(s.n) + " tokens > max_len " +
                                std::to_string(c.max_len));
        if (s.qtype < 0 || s.qtype >= 3) fail(E_INVALID, "sequence " + std::to_string(si) + ": question type " + std::to_string(s.qtype));
        const int64_t start = at;
        for (int64_t i = 0; i < s.n; ++i) {
            if (int64_t(s.ids[i]) >= c.vocab)
                fail(E_INVALID, "token id " + std::to_string(s.ids[i]) + " outside the vocabulary of " + std::to_string(c.vocab));
            ids[at] = s.ids[i];
            qt[at] = uint32_t(s.qtype);
            meta[4 * at] = int32_t(i);
            meta[4 * at + 1] = int32_t(si);
            meta[4 * at + 2] = int32_t(start);
            meta[4 * at + 3] = int32_t(start + s.n);
            ++at;
        }
        if (nw + 1 + s.nmarkers > max_rows_)
            fail(E_CAPACITY, "more rows requested than the engine reads back (" + std::to_string(max_rows_) + ")");
        wanted[nw++] = int32_t(start);
        for (int64_t j = 0; j < s.nmarkers; ++j) {
            if (int64_t(s.markers[j]) >= s.n)
                fail(E_INVALID, "sequence " + std::to_string(si) + ": marker " + std::to_string(s.markers[j]) +
                                    " past its " + std::to_string(s.n) + " tokens");
            wanted[nw++] = int32_t(start + s.markers[j]);
        }
    }
    OMG_HIP(hipMemcpyAsync(ids_.p, ids, size_t(at) * 4, hipMemcpyHostToDevice, stream_));
    OMG_HIP(hipMemcpyAsync(qtypes_.p, qt, size_t(at) * 4, hipMemcpyHostToDevice, stream_));
    OMG_HIP(hipMemcpyAsync(meta_.p, meta, size_t(at) * 16, hipMemcpyHostToDevice, stream_));
    OMG_HIP(hipMemcpyAsync(wanted_.p, wanted, size_t(nw) * 4, hipMemcpyHostToDevice, stream_));
    t_ = at;
    nrows_ = nw;
    return total;
}

// laya.rs:1261-1392, one dispatch per step except where a reference step's
// neighbours fold in: the residual adds ride in the following LayerNorm,
// RoPE and the q scale in the q/k/v projection's epilogue, the in_proj and
// l1 biases (and l1's ReLU) in their GEMMs' epilogues, and the last encoder
// layer's final norm + type embedding + the first head norm in one pass.
void LayaEngine::forward() {
    const LayaConfig& c = cfg_;
    const int64_t t = t_, d = c.d;
    const int heads = int(c.heads);
    float* x = x_.as<float>();
    float* a = a_.as<float>();
    half_t* h16 = h16_.as<half_t>();
    half_t* attn = attn16_.as<half_t>();
    half_t* act = act16_.as<half_t>();
    const int32_t* meta = meta_.as<int32_t>();
    QkvHeads qh{};
    qh.meta = meta;
    qh.dq = d;
    qh.tpad = tpad_;
    qh.q16 = q16_.as<half_t>();
    qh.k16 = k16_.as<half_t>();
    qh.vt = vt_.as<half_t>();
    step("embed_ln", [&] { launch_embed_ln(stream_, embed_.w, ids_.as<uint32_t>(), t, embed_norm_.as<float>(), c.eps, x, h16); });
    const Head* h0 = head_.empty() ? nullptr : &head_[0];
    for (size_t l = 0; l < enc_.size(); ++l) {
        const Enc& L = enc_[l];
        const bool last = l + 1 == enc_.size();
        qh.rope = (L.sliding ? rope_local_ : rope_global_).as<float2>();
        qh.qscale = 0.125f;  // 64^-0.5 (laya.rs:1285)
        step("mm_qkv", [&] { launch_gemm_qkv_heads(stream_, h16, d, L.qkv.w, nullptr, qh, t); });
        step("attention", [&] { launch_attention_bi(stream_, qh, heads, t, L.sliding ? int(c.window) : 0, attn); });
        step("mm_o", [&] { launch_gemm(stream_, attn, d, L.o.w, a, d, t); });
        step("add_o_norm", [&] { launch_add_ln(stream_, x, a, nullptr, L.mlp_norm.as<float>(), nullptr, c.eps, t, d, h16); });
        step("mm_wi", [&] {
            launch_gemm_geglu(stream_, h16, d, L.wi_val.w, L.wi_gate.w, act, c.ff, t, true);
        });
        step("mm_wo", [&] { launch_gemm(stream_, act, c.ff, L.wo.w, a, d, t); });
        if (!last) {
            step("add_wo_norm", [&] {
                launch_add_ln(stream_, x, a, nullptr, enc_[l + 1].attn_norm.as<float>(), nullptr, c.eps, t, d, h16);
            });
        } else {
            step("final_norm", [&] {
                launch_add_ln_final(stream_, x, a, final_norm_.as<float>(), c.type_emb ? type_emb_.as<float>() : nullptr,
                                    qtypes_.as<uint32_t>(), h0 ? h0->norm1_w.as<float>() : nullptr,
                                    h0 ? h0->norm1_b.as<float>() : nullptr, c.eps, t, d, h16);
            });
        }
    }
    // Decision-head layers: no rotation, no q scale (laya.rs:1346-1350 runs
    // attention_bi straight on the biased projection).
    qh.rope = nullptr;
    qh.qscale = 1.0f;
    for (size_t hl = 0; hl < head_.size(); ++hl) {
        const Head& H = head_[hl];
        const bool last = hl + 1 == head_.size();
        step("mm_in", [&] { launch_gemm_qkv_heads(stream_, h16, d, H.in_proj.w, H.in_proj_b16.as<uint16_t>(), qh, t); });
        step("head_attention", [&] { launch_attention_bi(stream_, qh, heads, t, 0, attn); });
        if (last && !full_last_layer_ && nrows_ > 0) {
            // Past its attention the last layer feeds only the read-out
            // rows: they are gathered (attention output, stream) and the
            // rest of the layer runs on them; every step is per row, so
            // they come out as the full layer leaves them.
            const int64_t n = nrows_;
            half_t* aw = attn_w_.as<half_t>();
            float* xw = x_w_.as<float>();
            float* pw = a_w_.as<float>();
            half_t* hw = h16_w_.as<half_t>();
            half_t* actw = act_w_.as<half_t>();
            step("gather_out", [&] { launch_gather_out(stream_, attn, d, x, d, wanted_.as<int32_t>(), 0, n, aw, xw); });
            step("mm_out_out", [&] { launch_gemm(stream_, aw, d, H.out_proj.w, pw, d, n); });
            step("add_out_norm2_out", [&] {
                launch_add_ln(stream_, xw, pw, H.out_proj_b.as<float>(), H.norm2_w.as<float>(), H.norm2_b.as<float>(),
                              c.eps, n, d, hw);
            });
            step("mm_l1_out", [&] { launch_gemm_bias_relu(stream_, hw, d, H.l1.w, H.l1_b16.as<uint16_t>(), actw, 4 * d, n); });
            step("mm_l2_out", [&] { launch_gemm(stream_, actw, 4 * d, H.l2.w, pw, d, n); });
            step("rows", [&] { launch_gather_rows(stream_, xw, pw, H.l2_b.as<float>(), nullptr, n, d, rows_.as<float>()); });
            break;
        }
        step("mm_out", [&] { launch_gemm(stream_, attn, d, H.out_proj.w, a, d, t); });
        step("add_out_norm2", [&] {
            launch_add_ln(stream_, x, a, H.out_proj_b.as<float>(), H.norm2_w.as<float>(), H.norm2_b.as<float>(), c.eps,
                          t, d, h16);
        });
        step("mm_l1", [&] { launch_gemm_bias_relu(stream_, h16, d, H.l1.w, H.l1_b16.as<uint16_t>(), act, 4 * d, t); });
        step("mm_l2", [&] { launch_gemm(stream_, act, 4 * d, H.l2.w, a, d, t); });
        if (!last) {
            const Head& N = head_[hl + 1];
            step("add_l2_norm1", [&] {
                launch_add_ln(stream_, x, a, H.l2_b.as<float>(), N.norm1_w.as<float>(), N.norm1_b.as<float>(), c.eps, t,
                              d, h16);
            });
        } else {
            step("rows", [&] {
                launch_gather_rows(stream_, x, a, H.l2_b.as<float>(), wanted_.as<int32_t>(), nrows_, d,
                                   rows_.as<float>());
            });
        }
    }
    if (head_.empty())
        step("rows", [&] { launch_gather_rows(stream_, x, nullptr, nullptr, wanted_.as<int32_t>(), nrows_, d, rows_.as<float>()); });
}

void LayaEngine::prepare(const LayaSeq* seqs, int64_t n) { pack(seqs, n); }

void LayaEngine::set_full_last_layer(bool on) {
    sync();
    full_last_layer_ = on;
}

void LayaEngine::launch_prepared() {
    if (t_ == 0) fail(E_INVALID, "nothing prepared");
    forward();
}

void LayaEngine::hidden(const LayaSeq* seqs, int64_t n, float* out, int64_t out_floats) {
    int64_t want = 0;
    for (int64_t i = 0; i < n; ++i) want += 1 + seqs[i].nmarkers;
    if (out_floats < want * cfg_.d) fail(E_INVALID, "output buffer too small");
    pack(seqs, n);
    forward();
    OMG_HIP(hipMemcpyAsync(h_out_, rows_.p, size_t(nrows_ * cfg_.d) * 4, hipMemcpyDeviceToHost, stream_));
    sync();
    std::memcpy(out, h_out_, size_t(nrows_ * cfg_.d) * 4);
}

void LayaEngine::score(const float* rows, int64_t nmarkers, float* logits, float* act) const {
    const LayaConfig& c = cfg_;
    const int64_t d = c.d;
    const auto& nw = host_.at("scorer.norm_w");
    const auto& nb = host_.at("scorer.norm_b");
    const auto& l1 = host_.at("scorer.l1");
    const auto& l1b = host_.at("scorer.l1_b");
    const auto& l2 = host_.at("scorer.l2");
    const float l2b = host_.at("scorer.l2_b")[0];
    std::vector<float> lg(static_cast<size_t>(nmarkers));
    for (int64_t j = 0; j < nmarkers; ++j) {
        std::vector<float> z = layer_norm(rows + (1 + j) * d, d, nw.data(), nb.data(), c.eps);
        z = linear(z, l1, l1b);
        for (float& v : z) v = gelu_erf_host(v);
        lg[size_t(j)] = dot(z.data(), l2.data(), d) + l2b;
        logits[j] = lg[size_t(j)];
    }
    if (c.act_out == 0) {
        *act = NAN;
        return;
    }
    // Confidence features of the untempered softmax, one-option questions
    // padded to two slots (laya.rs:1464-1480).
    const int64_t k = std::max<int64_t>(nmarkers, 2);
    std::vector<float> padded = lg;
    padded.resize(size_t(k), -1e4f);
    const std::vector<float> p = softmax(padded);
    float ent = 0.0f;
    for (float v : p) ent += v * std::log(std::max(v, 1e-9f));
    const float entropy = -ent / std::log(float(k));
    std::vector<float> sorted = p;
    std::sort(sorted.begin(), sorted.end());
    const float top1 = sorted[size_t(k - 1)], top2 = sorted[size_t(k - 2)];
    std::vector<float> pooled(rows, rows + d);
    pooled.push_back(top1);
    pooled.push_back(top1 - top2);
    pooled.push_back(entropy);
    pooled.push_back(float(k) / 255.0f);
    std::vector<float> h = linear(pooled, host_.at("act.l1"), host_.at("act.l1_b"));
    for (float& v : h) v = gelu_erf_host(v);
    *act = softmax(linear(h, host_.at("act.l2"), host_.at("act.l2_b")))[0];
}

void LayaEngine::evaluate(const LayaSeq* seqs, int64_t n, float* logits, int64_t nlogits, float* act, int64_t nact) {
    int64_t want = 0, rows = 0;
    for (int64_t i = 0; i < n; ++i) {
        want += seqs[i].nmarkers;
        rows += 1 + seqs[i].nmarkers;
    }
    if (nlogits < want || nact < n) fail(E_INVALID, "output buffer too small");
    std::vector<float> h(size_t(rows * cfg_.d));
    hidden(seqs, n, h.data(), int64_t(h.size()));
    int64_t r = 0, j = 0;
    for (int64_t i = 0; i < n; ++i) {
        score(h.data() + r * cfg_.d, seqs[i].nmarkers, logits + j, act + i);
        r += 1 + seqs[i].nmarkers;
        j += seqs[i].nmarkers;
    }
}

void LayaEngine::warmup() {
    const uint32_t ids[3] = {cfg_.cls, cfg_.mask, cfg_.sep};
    const uint32_t marker = 1;
    const LayaSeq s{ids, 3, &marker, 1, 2};
    std::vector<float> out(size_t(2 * cfg_.d));
    hidden(&s, 1, out.data(), int64_t(out.size()));
}

}  // namespace omg
