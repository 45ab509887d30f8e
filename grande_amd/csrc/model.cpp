// Checkpoint description, block formats and the seeded generator
// (crates/omg-wgpu/src/model.rs, crates/omg-wgpu/tests/reference.rs:17-139).
#include "model.h"

#include <cmath>
#include <fstream>
#include <sstream>

namespace omg {

Dtype parse_dtype(const std::string& s) {
    if (s == "f16" || s == "F16") return F16;
    if (s == "q8" || s == "q8_0" || s == "Q8_0") return Q8;
    if (s == "q4" || s == "q4_0" || s == "Q4_0") return Q4;
    fail(E_INVALID, "unsupported dtype " + s);
}

int64_t payload_bytes(Dtype t, int64_t n) { return t == F16 ? n * 2 : (t == Q8 ? n : n / 2); }

// Structural sizes are bounded before anything is sized by them, so a
// hostile config.json is refused instead of exhausting memory.
constexpr int64_t MAX_COUNT = int64_t(1) << 31;

static int64_t need_u64(const Json& v, const char* k, int64_t max = MAX_COUNT) {
    if (!v[k].is_uint()) fail(E_INVALID, std::string("config.json: missing ") + k);
    if (v[k].num > double(max)) fail(E_INVALID, std::string("config.json: ") + k + " too large");
    return int64_t(v[k].num);
}

// An optional unsigned size: absent or not an unsigned integer gives the
// fallback (serde_json's as_u64().unwrap_or, model.rs:66-210); one above
// `max` is refused.
static int64_t opt_u64(const Json& x, int64_t fallback, const char* k, int64_t max = MAX_COUNT) {
    if (!x.is_uint()) return fallback;
    if (x.num > double(max)) fail(E_INVALID, std::string("config.json: ") + k + " too large");
    return int64_t(x.num);
}

// An optional float parameter: finite and within float range.
static double opt_f64(const Json& x, double fallback, const char* k) {
    if (x.kind != Json::Number) return fallback;
    if (!std::isfinite(x.num) || std::fabs(x.num) > 3.0e38) fail(E_INVALID, std::string("config.json: bad ") + k);
    return x.num;
}

Config Config::from_json(const Json& root) {
    const Json& v = root.has("text_config") ? root["text_config"] : root;
    Config c;
    const std::string mt = v["model_type"].s("gemma3_text");
    c.arch = (mt == "gemma4_text" || mt == "gemma4") ? GEMMA4 : GEMMA3;
    c.layers = need_u64(v, "num_hidden_layers", 4096);
    const int64_t L = c.layers;
    if (v["layer_types"].kind == Json::Array) {
        for (const Json& t : v["layer_types"].arr) c.sliding.push_back(t.s("") == "sliding_attention");
    } else {
        const int64_t k = opt_u64(v["_sliding_window_pattern"], 6, "_sliding_window_pattern");
        for (int64_t i = 0; i < L; ++i) c.sliding.push_back(k == 0 ? true : (i + 1) % k != 0);
    }
    if (int64_t(c.sliding.size()) != L)
        fail(E_INVALID, "config.json: layer_types has " + std::to_string(c.sliding.size()) +
                            " entries for " + std::to_string(L) + " layers");
    const Json& rope = v["rope_parameters"];
    c.theta_global = float(opt_f64(rope["full_attention"]["rope_theta"],
                                   opt_f64(v["rope_theta"], 1e6, "rope_theta"), "rope_theta"));
    c.theta_local = float(opt_f64(rope["sliding_attention"]["rope_theta"],
                                  opt_f64(v["rope_local_base_freq"], 1e4, "rope_local_base_freq"), "rope_theta"));
    const int64_t hd_local = need_u64(v, "head_dim", 65536);
    const int64_t hd_global = opt_u64(v["global_head_dim"], hd_local, "global_head_dim", 65536);
    const double rot_local = opt_f64(rope["sliding_attention"]["partial_rotary_factor"], 1.0, "partial_rotary_factor");
    const double rot_global = opt_f64(rope["full_attention"]["partial_rotary_factor"], 1.0, "partial_rotary_factor");
    if (rot_local < 0.0 || rot_local > 1.0 || rot_global < 0.0 || rot_global > 1.0)
        fail(E_INVALID, "config.json: partial_rotary_factor outside [0, 1]");
    for (int64_t i = 0; i < L; ++i) {
        const bool s = c.sliding[size_t(i)];
        const int64_t hd = s ? hd_local : hd_global;
        c.head_dim.push_back(hd);
        c.rope_dims.push_back(int64_t(double(hd) * (s ? rot_local : rot_global)));
    }
    const int64_t shared = opt_u64(v["num_kv_shared_layers"], 0, "num_kv_shared_layers");
    if (shared >= L)
        fail(E_INVALID, "num_kv_shared_layers " + std::to_string(shared) + " >= " +
                            std::to_string(L) + " layers");
    const int64_t first_shared = L - shared;
    for (int64_t i = 0; i < L; ++i) {
        int64_t src = i;
        if (i >= first_shared) {
            for (int64_t j = first_shared - 1; j >= 0; --j)
                if (c.sliding[size_t(j)] == c.sliding[size_t(i)]) {
                    src = j;
                    break;
                }
        }
        if (src >= first_shared && src != i)
            fail(E_INVALID, "layer " + std::to_string(i) + " has no earlier K/V layer of its type to share");
        c.kv_source.push_back(src);
    }
    const Json& ffj = v["intermediate_size"];
    if (ffj.kind == Json::Array) {
        if (int64_t(ffj.arr.size()) != L) fail(E_INVALID, "config.json: intermediate_size length mismatch");
        for (const Json& x : ffj.arr) c.ff.push_back(opt_u64(x, 0, "intermediate_size", int64_t(1) << 24));
    } else if (ffj.kind == Json::Number) {
        const int64_t base = opt_u64(ffj, 0, "intermediate_size", int64_t(1) << 24);
        const bool dbl = v["use_double_wide_mlp"].boolean(false);
        for (int64_t i = 0; i < L; ++i) c.ff.push_back(dbl && i >= first_shared ? 2 * base : base);
    } else {
        fail(E_INVALID, "config.json: missing intermediate_size");
    }
    if (int64_t(c.ff.size()) != L) fail(E_INVALID, "config.json: intermediate_size length mismatch");
    if (c.arch == GEMMA3) {
        const double qps = opt_f64(v["query_pre_attn_scalar"], double(hd_local), "query_pre_attn_scalar");
        if (!(qps > 0.0)) fail(E_INVALID, "config.json: query_pre_attn_scalar must be positive");
        c.query_scale = std::pow(float(qps), -0.5f);
        c.norm_offset = 1.0f;
        c.v_norm = false;
    } else {
        c.query_scale = 1.0f;
        c.norm_offset = 0.0f;
        c.v_norm = true;
    }
    c.norm_offset = float(opt_f64(v["omg_norm_offset"], double(c.norm_offset), "omg_norm_offset"));
    c.vocab = need_u64(v, "vocab_size");
    c.d = need_u64(v, "hidden_size", 65536);
    c.heads = need_u64(v, "num_attention_heads", 1024);
    c.kv_heads = need_u64(v, "num_key_value_heads", 1024);
    c.eps = float(opt_f64(v["rms_norm_eps"], 1e-6, "rms_norm_eps"));
    c.window = opt_u64(v["sliding_window"], 512, "sliding_window");
    c.per_layer_dim = opt_u64(v["hidden_size_per_layer_input"], 0, "hidden_size_per_layer_input", 65536);
    c.softcap = float(opt_f64(v["final_logit_softcapping"], 0.0, "final_logit_softcapping"));
    c.bos = uint32_t(opt_u64(v["bos_token_id"], 2, "bos_token_id", int64_t(0xffffffff)));
    return c;
}

void Config::validate() const {
    if (layers <= 0) fail(E_INVALID, "num_hidden_layers must be positive");
    if (kv_heads == 0 || heads % kv_heads != 0)
        fail(E_INVALID, "num_key_value_heads " + std::to_string(kv_heads) +
                            " must divide num_attention_heads " + std::to_string(heads));
    const int64_t hpg = heads / kv_heads;
    // The attention kernel packs 16 query rows per wavefront as
    // (16 / hpg) tokens x hpg heads of one KV head.
    if (!(hpg == 1 || hpg == 2 || hpg == 4 || hpg == 8 || hpg == 16))
        fail(E_INVALID, "query heads per KV head must divide 16");
    for (int64_t i = 0; i < layers; ++i) {
        const int64_t hd = head_dim[size_t(i)];
        if (hd != 256 && hd != 512)
            fail(E_INVALID, "layer " + std::to_string(i) + ": head_dim " + std::to_string(hd) +
                                " (this engine's attention kernels are built for 256 and 512)");
        if (rope_dims[size_t(i)] > hd || rope_dims[size_t(i)] % 2)
            fail(E_INVALID, "layer " + std::to_string(i) + ": rope_dims " +
                                std::to_string(rope_dims[size_t(i)]));
        if (kv_source[size_t(i)] != i && head_dim[size_t(kv_source[size_t(i)])] != hd)
            fail(E_INVALID, "layer " + std::to_string(i) + ": shares K/V across head_dims");
    }
    if (d % 32 != 0) fail(E_INVALID, "hidden_size must be a multiple of 32");
    // The residual / final norms hold one row per wavefront in registers.
    if (d > 4096) fail(E_INVALID, "hidden_size " + std::to_string(d) + " above 4096 (the row norms' register rows)");
    if (vocab <= 0) fail(E_INVALID, "vocab_size must be positive");
    for (int64_t f : ff)
        if (f % 32 != 0 || f <= 0) fail(E_INVALID, "intermediate_size must be a positive multiple of 32");
    if (per_layer_dim < 0 || per_layer_dim % 32 != 0 || per_layer_dim > 1024)
        fail(E_INVALID, "hidden_size_per_layer_input must be a multiple of 32, at most 1024");
    if (window < 0) fail(E_INVALID, "sliding_window must be >= 0");
}

int64_t Config::qkv_width(int64_t l) const {
    const int64_t hd = head_dim[size_t(l)];
    return has_kv(l) ? (heads + 2 * kv_heads) * hd : heads * hd;
}

int64_t Config::max_head_dim() const {
    int64_t m = 0;
    for (int64_t h : head_dim) m = std::max(m, h);
    return m;
}
int64_t Config::max_ff() const {
    int64_t m = 0;
    for (int64_t f : ff) m = std::max(m, f);
    return m;
}
int64_t Config::max_qkv() const {
    int64_t m = 0;
    for (int64_t l = 0; l < layers; ++l) m = std::max(m, qkv_width(l));
    return m;
}

std::vector<TensorSpec> Config::tensors() const {
    std::vector<TensorSpec> v;
    v.push_back({"embed", {vocab, d}});
    v.push_back({"final_norm", {d}});
    if (per_layer_dim > 0) {
        v.push_back({"pl_model_proj", {per_layer_dim * layers, d}});
        v.push_back({"pl_proj_norm", {per_layer_dim}});
    }
    for (int64_t l = 0; l < layers; ++l) {
        const int64_t hd = head_dim[size_t(l)], f = ff[size_t(l)];
        auto n = [&](const char* s) { return "blk." + std::to_string(l) + "." + s; };
        v.push_back({n("attn_norm"), {d}});
        v.push_back({n("qkv"), {qkv_width(l), d}});
        v.push_back({n("q_norm"), {hd}});
        if (has_kv(l)) v.push_back({n("k_norm"), {hd}});
        v.push_back({n("o"), {d, heads * hd}});
        v.push_back({n("post_attn_norm"), {d}});
        v.push_back({n("ffn_norm"), {d}});
        v.push_back({n("gate"), {f, d}});
        v.push_back({n("up"), {f, d}});
        v.push_back({n("down"), {d, f}});
        v.push_back({n("post_ffn_norm"), {d}});
        if (per_layer_dim > 0) {
            v.push_back({n("pl_gate"), {per_layer_dim, d}});
            v.push_back({n("pl_proj"), {d, per_layer_dim}});
            v.push_back({n("pl_norm"), {d}});
            v.push_back({n("out_scale"), {1}});
        }
    }
    return v;
}

int64_t QTensor::numel() const {
    int64_t n = 1;
    for (int64_t s : shape) n *= s;
    return n;
}

float QTensor::get(int64_t i) const {
    if (dtype == F16) return f16_to_f32(uint16_t(data[size_t(2 * i)] | (data[size_t(2 * i + 1)] << 8)));
    const int64_t b = i / BLOCK;
    const float d = f16_to_f32(uint16_t(scales[size_t(2 * b)] | (scales[size_t(2 * b + 1)] << 8)));
    if (dtype == Q8) return float(int8_t(data[size_t(i)])) * d;
    const int64_t j = i % BLOCK;
    const uint8_t byte = data[size_t(b * 16 + j % 16)];
    const int q = j < 16 ? (byte & 0xf) : (byte >> 4);
    return (float(q) - 8.0f) * d;
}

static int64_t count(const std::vector<int64_t>& shape) {
    int64_t n = 1;
    for (int64_t s : shape) n *= s;
    return n;
}

static void put_scale(std::vector<uint8_t>& s, float d) {
    const uint16_t h = f32_to_f16(d);
    s.push_back(uint8_t(h & 0xff));
    s.push_back(uint8_t(h >> 8));
}

QTensor quantize_q8(const std::vector<int64_t>& shape, const float* v) {
    const int64_t n = count(shape);
    if (n % BLOCK) fail(E_INVALID, "q8: " + std::to_string(n) + " values is not a multiple of 32");
    QTensor t;
    t.dtype = Q8;
    t.shape = shape;
    t.data.reserve(size_t(n));
    t.scales.reserve(size_t(n / BLOCK * 2));
    for (int64_t b = 0; b < n / BLOCK; ++b) {
        const float* blk = v + b * BLOCK;
        float amax = 0.0f;
        for (int j = 0; j < BLOCK; ++j) amax = std::max(amax, std::fabs(blk[j]));
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        put_scale(t.scales, d);
        for (int j = 0; j < BLOCK; ++j) {
            // Rust's f32::round rounds half away from zero, as std::round.
            float q = std::round(blk[j] * id);
            q = std::min(127.0f, std::max(-127.0f, q));
            t.data.push_back(uint8_t(int8_t(q)));
        }
    }
    return t;
}

QTensor quantize_q4(const std::vector<int64_t>& shape, const float* v) {
    const int64_t n = count(shape);
    if (n % BLOCK) fail(E_INVALID, "q4: " + std::to_string(n) + " values is not a multiple of 32");
    QTensor t;
    t.dtype = Q4;
    t.shape = shape;
    t.data.reserve(size_t(n / 2));
    t.scales.reserve(size_t(n / BLOCK * 2));
    for (int64_t b = 0; b < n / BLOCK; ++b) {
        const float* blk = v + b * BLOCK;
        float mx = 0.0f, amax = 0.0f;
        for (int j = 0; j < BLOCK; ++j)
            if (std::fabs(blk[j]) > amax) {
                amax = std::fabs(blk[j]);
                mx = blk[j];
            }
        const float d = mx / -8.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        put_scale(t.scales, d);
        for (int j = 0; j < BLOCK / 2; ++j) {
            // `as i32` truncates toward zero; then clamp to a nibble.
            const int lo = std::min(15, std::max(0, int(blk[j] * id + 8.5f)));
            const int hi = std::min(15, std::max(0, int(blk[j + BLOCK / 2] * id + 8.5f)));
            t.data.push_back(uint8_t(lo | (hi << 4)));
        }
    }
    return t;
}

QTensor from_f32(const std::vector<int64_t>& shape, const float* v) {
    const int64_t n = count(shape);
    QTensor t;
    t.dtype = F16;
    t.shape = shape;
    t.data.resize(size_t(2 * n));
    for (int64_t i = 0; i < n; ++i) {
        const uint16_t h = f32_to_f16(v[i]);
        t.data[size_t(2 * i)] = uint8_t(h & 0xff);
        t.data[size_t(2 * i + 1)] = uint8_t(h >> 8);
    }
    return t;
}

Weights synth_weights(const Config& cfg, uint64_t seed, Dtype linear, Dtype embed) {
    Rng r(seed | 1);
    Weights w;
    w.config = cfg;
    std::vector<float> buf;
    auto tensor = [&](const std::vector<int64_t>& shape, float scale, Dtype dt) {
        const int64_t n = count(shape);
        buf.resize(size_t(n));
        for (int64_t i = 0; i < n; ++i) buf[size_t(i)] = r.next() * scale;
        switch (dt) {
            case F16: return from_f32(shape, buf.data());
            case Q8: return quantize_q8(shape, buf.data());
            default: return quantize_q4(shape, buf.data());
        }
    };
    const float base = cfg.norm_offset == 0.0f ? 1.0f : 0.0f;
    for (const TensorSpec& spec : cfg.tensors()) {
        const std::string& nm = spec.name;
        if (nm == "embed") {
            w.tensors[nm] = tensor(spec.shape, 1.0f, embed);
        } else if (nm.size() >= 9 && nm.compare(nm.size() - 9, 9, "out_scale") == 0) {
            const float v = 0.6f + 0.2f * r.next();
            w.tensors[nm] = from_f32({1}, &v);
        } else if (spec.shape.size() == 1) {
            const int64_t n = spec.shape[0];
            buf.resize(size_t(n));
            for (int64_t i = 0; i < n; ++i) buf[size_t(i)] = r.next() * 0.5f + base;
            w.tensors[nm] = from_f32(spec.shape, buf.data());
        } else {
            const float scale = spec.shape[1] == cfg.d ? 0.15f : 0.08f;
            w.tensors[nm] = tensor(spec.shape, scale, linear);
        }
    }
    // reference.rs:132-133: the per-layer token table comes after the catalogue.
    if (cfg.per_layer_dim > 0) w.tensors["per_layer_table"] = tensor({cfg.vocab, cfg.per_layer_dim * cfg.layers}, 1.0f, linear);
    return w;
}

std::string read_file(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) fail(E_IO, "cannot read " + path);
    std::ostringstream ss;
    ss << f.rdbuf();
    return ss.str();
}

Weights load_dir(const std::string& dir) {
    Weights w;
    w.config = Config::from_json(Json::parse(read_file(dir + "/config.json")));
    w.config.validate();
    w.tensors = read_manifest(dir);
    return w;
}

std::map<std::string, QTensor> read_manifest(const std::string& dir) {
    std::map<std::string, QTensor> out;
    const Json man = Json::parse(read_file(dir + "/manifest.json"));
    if (man["files"].kind != Json::Array) fail(E_INVALID, "manifest.json: missing files");
    // One manifest entry (model.rs:758-794) out of its file's bytes.
    auto entry = [&](const Json& e, const std::string& bytes) {
        QTensor t;
        const std::string name = e["name"].s("");
        t.dtype = parse_dtype(e["dtype"].s(""));
        for (const Json& s : e["shape"].arr) t.shape.push_back(int64_t(s.u64(0)));
        auto slice = [&](uint64_t off, uint64_t n) {
            if (off + n > bytes.size())
                fail(E_INVALID, name + ": byte range " + std::to_string(off) + ".." +
                                    std::to_string(off + n) + " outside the file");
            return std::vector<uint8_t>(bytes.begin() + long(off), bytes.begin() + long(off + n));
        };
        t.data = slice(e["offset"].u64(0), e["nbytes"].u64(0));
        t.scales = slice(e["scales_offset"].u64(0), e["scales_nbytes"].u64(0));
        const int64_t n = t.numel();
        if (int64_t(t.data.size()) != payload_bytes(t.dtype, n))
            fail(E_INVALID, name + ": " + std::to_string(t.data.size()) + " payload bytes, expected " +
                                std::to_string(payload_bytes(t.dtype, n)));
        const int64_t want_scales = t.dtype == F16 ? 0 : n / BLOCK * 2;
        if (int64_t(t.scales.size()) != want_scales)
            fail(E_INVALID, name + ": " + std::to_string(t.scales.size()) + " scale bytes, expected " +
                                std::to_string(want_scales));
        return t;
    };
    for (const Json& file : man["files"].arr) {
        const std::string bytes = read_file(dir + "/" + file["path"].s(""));
        for (const Json& e : file["tensors"].arr) out[e["name"].s("")] = entry(e, bytes);
    }
    // The per-layer token table, in a file of its own (backend.rs:50-57).
    const Json& plt = man["per_layer_table"];
    if (plt.kind == Json::Object) {
        const std::string path = plt["path"].s("");
        if (path.empty()) fail(E_INVALID, "manifest: per_layer_table has no path");
        out["per_layer_table"] = entry(plt, read_file(dir + "/" + path));
    }
    return out;
}

}  // namespace omg
