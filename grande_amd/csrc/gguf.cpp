// A llama.cpp GGUF file read straight into a host checkpoint: the mapping
// tools/export_wgpu_gguf.py:112-296 performs on the way to an exported
// directory (metadata -> the HF-style text config Config::from_json reads;
// q / k / v fused into one qkv tensor per layer; Q8_0 / Q4_0 blocks split
// into codes and f16 scales; f32 / bf16 tensors to f16), done in C++ so a
// GGUF loads without the export step.  Gemma 3 and Gemma 4 text models.
#include <cmath>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "model.h"

namespace omg {

namespace {

// GGUF value types (gguf.constants.GGUFValueType).
enum { V_U8, V_I8, V_U16, V_I16, V_U32, V_I32, V_F32, V_BOOL, V_STR, V_ARR, V_U64, V_I64, V_F64 };
// ggml tensor types used by these checkpoints.
enum { G_F32 = 0, G_F16 = 1, G_Q4_0 = 2, G_Q8_0 = 8, G_BF16 = 30 };

struct Reader {
    const uint8_t* p;
    size_t n, at = 0;
    const uint8_t* take(size_t k) {
        if (k > n - at) fail(E_INVALID, "gguf: truncated file");
        const uint8_t* r = p + at;
        at += k;
        return r;
    }
    template <class T>
    T get() {
        T v;
        std::memcpy(&v, take(sizeof(T)), sizeof(T));
        return v;
    }
    std::string str() {
        const uint64_t k = get<uint64_t>();
        if (k > (1u << 30)) fail(E_INVALID, "gguf: string too long");
        const uint8_t* s = take(size_t(k));
        return std::string(reinterpret_cast<const char*>(s), size_t(k));
    }
};

// A metadata value as JSON (numbers, strings, bools and arrays of them).
Json value(Reader& r, uint32_t type, int depth = 0) {
    Json v;
    auto num = [&](double x) {
        v.kind = Json::Number;
        v.num = x;
    };
    switch (type) {
        case V_U8: num(r.get<uint8_t>()); break;
        case V_I8: num(r.get<int8_t>()); break;
        case V_U16: num(r.get<uint16_t>()); break;
        case V_I16: num(r.get<int16_t>()); break;
        case V_U32: num(r.get<uint32_t>()); break;
        case V_I32: num(r.get<int32_t>()); break;
        case V_F32: num(r.get<float>()); break;
        case V_U64: num(double(r.get<uint64_t>())); break;
        case V_I64: num(double(r.get<int64_t>())); break;
        case V_F64: num(r.get<double>()); break;
        case V_BOOL:
            v.kind = Json::Bool;
            v.b = r.get<uint8_t>() != 0;
            break;
        case V_STR:
            v.kind = Json::String;
            v.str = r.str();
            break;
        case V_ARR: {
            if (depth > 2) fail(E_INVALID, "gguf: nested arrays too deep");
            const uint32_t et = r.get<uint32_t>();
            const uint64_t k = r.get<uint64_t>();
            if (k > (1u << 28)) fail(E_INVALID, "gguf: array too long");
            v.kind = Json::Array;
            // Token tables are large and not needed here: skip string arrays.
            if (et == V_STR) {
                for (uint64_t i = 0; i < k; ++i) r.str();
                break;
            }
            v.arr.reserve(size_t(k));
            for (uint64_t i = 0; i < k; ++i) v.arr.push_back(value(r, et, depth + 1));
            break;
        }
        default: fail(E_INVALID, "gguf: unknown value type " + std::to_string(type));
    }
    return v;
}

struct TensorInfo {
    std::vector<int64_t> shape;  // [rows, cols] order (GGUF lists ne[0] = cols first)
    uint32_t type = 0;
    uint64_t offset = 0;
    int64_t numel() const {
        int64_t k = 1;
        for (int64_t x : shape) k *= x;
        return k;
    }
};

uint16_t f32_to_f16_bits(float x) { return f32_to_f16(x); }  // round to nearest even

}  // namespace

Weights load_gguf(const std::string& path) {
    const std::string file = read_file(path);
    Reader r{reinterpret_cast<const uint8_t*>(file.data()), file.size()};
    if (std::memcmp(r.take(4), "GGUF", 4) != 0) fail(E_INVALID, path + ": not a GGUF file");
    const uint32_t version = r.get<uint32_t>();
    if (version < 2 || version > 3) fail(E_INVALID, "gguf: version " + std::to_string(version) + " (2 or 3 supported)");
    const uint64_t ntensors = r.get<uint64_t>(), nkv = r.get<uint64_t>();
    std::map<std::string, Json> kv;
    for (uint64_t i = 0; i < nkv; ++i) {
        const std::string key = r.str();
        kv[key] = value(r, r.get<uint32_t>());
    }
    std::map<std::string, TensorInfo> infos;
    for (uint64_t i = 0; i < ntensors; ++i) {
        const std::string name = r.str();
        TensorInfo t;
        const uint32_t nd = r.get<uint32_t>();
        if (nd == 0 || nd > 4) fail(E_INVALID, "gguf: " + name + " has " + std::to_string(nd) + " dims");
        std::vector<int64_t> ne(nd);
        // Every dimension positive and the element count below 2^40 (the
        // byte counts below then cannot overflow); the file size bounds it
        // further once the tensor's bytes are located.
        uint64_t count = 1;
        for (uint32_t k = 0; k < nd; ++k) {
            const uint64_t x = r.get<uint64_t>();
            if (x == 0 || x > (uint64_t(1) << 40) || count > (uint64_t(1) << 40) / x)
                fail(E_INVALID, "gguf: " + name + " has an invalid shape");
            count *= x;
            ne[k] = int64_t(x);
        }
        t.shape.assign(ne.rbegin(), ne.rend());
        t.type = r.get<uint32_t>();
        t.offset = r.get<uint64_t>();
        infos[name] = t;
    }
    const uint64_t align = kv.count("general.alignment") ? kv["general.alignment"].u64(32) : 32;
    if (align == 0 || align > (1u << 20) || (align & (align - 1)) != 0)
        fail(E_INVALID, "gguf: general.alignment must be a power of two up to 2^20");
    const size_t data0 = (r.at + align - 1) / align * align;

    const std::string arch = kv["general.architecture"].s("");
    if (arch != "gemma3" && arch != "gemma4")
        fail(E_INVALID, "gguf: architecture " + arch + " (gemma3 and gemma4 supported)");
    const bool g4 = arch == "gemma4";
    auto g = [&](const std::string& k) -> const Json& {
        static const Json none;
        auto it = kv.find(arch + "." + k);
        return it == kv.end() ? none : it->second;
    };
    auto need = [&](const std::string& k) {
        const Json& v = g(k);
        if (v.kind != Json::Number || !std::isfinite(v.num)) fail(E_INVALID, "gguf: missing " + arch + "." + k);
        return v.num;
    };
    // A count from the metadata: a whole number in [0, 2^31).
    auto count = [&](double x, const std::string& k) {
        if (!(x >= 0.0 && x < 2147483648.0) || x != std::floor(x)) fail(E_INVALID, "gguf: bad " + arch + "." + k);
        return int64_t(x);
    };
    if (!infos.count("token_embd.weight")) fail(E_INVALID, "gguf: missing token_embd.weight");
    const int64_t layers = count(need("block_count"), "block_count");
    const int64_t d = count(need("embedding_length"), "embedding_length");
    const int64_t heads = count(need("attention.head_count"), "attention.head_count");
    const Json& kvh = g("attention.head_count_kv");
    const Json& kvh0 = kvh.kind == Json::Array ? kvh[size_t(0)] : kvh;
    if (kvh0.kind != Json::Number) fail(E_INVALID, "gguf: missing " + arch + ".attention.head_count_kv");
    const int64_t kv_heads = count(kvh0.num, "attention.head_count_kv");
    const int64_t vocab = infos["token_embd.weight"].shape[0];

    // export_wgpu_gguf.py:130-171: the text config the exported directory
    // carries (GGUF norm weights already include Gemma 3's +1).
    Json cfg;
    cfg.kind = Json::Object;
    auto setn = [&](const char* k, double x) {
        Json v;
        v.kind = Json::Number;
        v.num = x;
        cfg.obj[k] = v;
    };
    {
        Json mt;
        mt.kind = Json::String;
        mt.str = g4 ? "gemma4_text" : "gemma3_text";
        cfg.obj["model_type"] = mt;
    }
    setn("vocab_size", double(vocab));
    setn("hidden_size", double(d));
    setn("num_hidden_layers", double(layers));
    setn("num_attention_heads", double(heads));
    setn("num_key_value_heads", double(kv_heads));
    const double hd_full = need("attention.key_length");
    const double hd_swa = g("attention.key_length_swa").f64(hd_full);
    setn("head_dim", hd_swa);
    setn("global_head_dim", hd_full);
    const Json& ff = g("feed_forward_length");
    if (ff.kind == Json::Array) {
        cfg.obj["intermediate_size"] = ff;
    } else {
        setn("intermediate_size", need("feed_forward_length"));
    }
    Json types;
    types.kind = Json::Array;
    const Json& pat = g("attention.sliding_window_pattern");
    for (int64_t i = 0; i < layers; ++i) {
        bool swa;
        if (pat.kind == Json::Array) {
            if (int64_t(pat.arr.size()) != layers)
                fail(E_INVALID, "gguf: attention.sliding_window_pattern has the wrong length");
            const Json& e = pat.arr[size_t(i)];
            swa = e.kind == Json::Bool ? e.b : e.num != 0.0;
        } else {
            const int64_t k = count(pat.f64(6.0), "attention.sliding_window_pattern");
            swa = k == 0 ? true : (i + 1) % k != 0;
        }
        Json t;
        t.kind = Json::String;
        t.str = swa ? "sliding_attention" : "full_attention";
        types.arr.push_back(t);
    }
    cfg.obj["layer_types"] = types;
    setn("sliding_window", need("attention.sliding_window"));
    setn("rms_norm_eps", need("attention.layer_norm_rms_epsilon"));
    setn("rope_theta", need("rope.freq_base"));
    setn("rope_local_base_freq", g("rope.freq_base_swa").f64(10000.0));
    setn("final_logit_softcapping", g("final_logit_softcapping").f64(0.0));
    if (g4) {
        // export_wgpu_gguf.py:140-171: partial RoPE on the global layers is
        // carried by rope_freqs (1.0 for rotated pairs, 1e30 for the rest);
        // K/V sharing and the per-layer inputs by their own keys.
        double rot_full = 1.0;
        auto rf = infos.find("rope_freqs.weight");
        if (rf != infos.end()) {
            if (rf->second.type != G_F32) fail(E_INVALID, "gguf: rope_freqs.weight must be f32");
            const int64_t n = rf->second.numel();
            if (data0 > file.size() || rf->second.offset > file.size() - data0 ||
                uint64_t(n) * 4 > file.size() - data0 - rf->second.offset)
                fail(E_INVALID, "gguf: rope_freqs.weight past the end of the file");
            int64_t rotated = 0;
            for (int64_t i = 0; i < n; ++i) {
                float f;
                std::memcpy(&f, file.data() + data0 + rf->second.offset + 4 * i, 4);
                rotated += f < 1e10f;
            }
            rot_full = double(rotated) * 2.0 / hd_full;
        }
        Json rope;
        rope.kind = Json::Object;
        Json full, slide, x;
        full.kind = slide.kind = Json::Object;
        x.kind = Json::Number;
        x.num = need("rope.freq_base");
        full.obj["rope_theta"] = x;
        x.num = rot_full;
        full.obj["partial_rotary_factor"] = x;
        x.num = g("rope.freq_base_swa").f64(10000.0);
        slide.obj["rope_theta"] = x;
        rope.obj["full_attention"] = full;
        rope.obj["sliding_attention"] = slide;
        cfg.obj["rope_parameters"] = rope;
        setn("num_kv_shared_layers", g("attention.shared_kv_layers").f64(0.0));
        setn("hidden_size_per_layer_input", g("embedding_length_per_layer_input").f64(0.0));
    } else {
        setn("query_pre_attn_scalar", g("attention.query_pre_attn_scalar").f64(hd_swa));
    }
    setn("bos_token_id", kv.count("tokenizer.ggml.bos_token_id") ? kv["tokenizer.ggml.bos_token_id"].num : 2.0);
    setn("omg_norm_offset", 0.0);

    Weights w;
    w.config = Config::from_json(cfg);
    w.config.validate();

    auto bytes_of = [&](const std::string& name) -> std::pair<const uint8_t*, TensorInfo> {
        auto it = infos.find(name);
        if (it == infos.end()) fail(E_MISSING, "gguf: missing tensor " + name);
        const TensorInfo& t = it->second;
        const int64_t n = t.numel();
        int64_t nb;
        switch (t.type) {
            case G_F32: nb = n * 4; break;
            case G_F16:
            case G_BF16: nb = n * 2; break;
            case G_Q8_0: nb = n / 32 * 34; break;
            case G_Q4_0: nb = n / 32 * 18; break;
            default: fail(E_INVALID, "gguf: " + name + " has unsupported type " + std::to_string(t.type));
        }
        if ((t.type == G_Q8_0 || t.type == G_Q4_0) && n % 32 != 0) fail(E_INVALID, "gguf: " + name + " not in whole blocks");
        if (data0 > file.size() || t.offset > file.size() - data0 || uint64_t(nb) > file.size() - data0 - t.offset)
            fail(E_INVALID, "gguf: " + name + " past the end of the file");
        return {reinterpret_cast<const uint8_t*>(file.data()) + data0 + t.offset, t};
    };
    // One or more GGUF tensors (rows concatenated) as one QTensor of `shape`.
    auto convert = [&](const std::vector<std::string>& names, const std::vector<int64_t>& shape) {
        QTensor q;
        q.shape = shape;
        uint32_t type = 0;
        for (size_t i = 0; i < names.size(); ++i) {
            auto [p, t] = bytes_of(names[i]);
            if (i == 0) type = t.type;
            if (t.type != type) fail(E_INVALID, "gguf: cannot fuse tensors of mixed types (" + names[0] + ")");
            const int64_t n = t.numel();
            if (type == G_Q8_0 || type == G_Q4_0) {
                q.dtype = type == G_Q8_0 ? Q8 : Q4;
                const int64_t bb = type == G_Q8_0 ? 34 : 18;
                for (int64_t b = 0; b < n / 32; ++b) {
                    q.scales.insert(q.scales.end(), p + b * bb, p + b * bb + 2);
                    q.data.insert(q.data.end(), p + b * bb + 2, p + (b + 1) * bb);
                }
            } else {
                q.dtype = F16;
                for (int64_t e = 0; e < n; ++e) {
                    uint16_t h;
                    if (type == G_F16) {
                        std::memcpy(&h, p + 2 * e, 2);
                    } else {
                        float f;
                        if (type == G_F32) {
                            std::memcpy(&f, p + 4 * e, 4);
                        } else {  // bf16: the upper half of an f32
                            const uint32_t u = uint32_t(p[2 * e]) << 16 | uint32_t(p[2 * e + 1]) << 24;
                            std::memcpy(&f, &u, 4);
                        }
                        h = f32_to_f16_bits(f);
                    }
                    q.data.push_back(uint8_t(h & 0xff));
                    q.data.push_back(uint8_t(h >> 8));
                }
            }
        }
        if (q.numel() * (q.dtype == F16 ? 2 : 1) != int64_t(q.data.size()) * (q.dtype == Q4 ? 2 : 1))
            fail(E_INVALID, "gguf: " + names[0] + " size does not match its shape");
        return q;
    };
    const Config& c = w.config;
    w.tensors["embed"] = convert({"token_embd.weight"}, {vocab, d});
    w.tensors["final_norm"] = convert({"output_norm.weight"}, {d});
    const int64_t pl = c.per_layer_dim;
    if (pl > 0) {
        w.tensors["pl_model_proj"] = convert({"per_layer_model_proj.weight"}, {pl * layers, d});
        w.tensors["pl_proj_norm"] = convert({"per_layer_proj_norm.weight"}, {pl});
        const int64_t rows = infos.count("per_layer_token_embd.weight") ? infos["per_layer_token_embd.weight"].shape[0] : 0;
        if (rows != vocab) fail(E_INVALID, "gguf: per_layer_token_embd.weight rows must match the vocabulary");
        w.tensors["per_layer_table"] = convert({"per_layer_token_embd.weight"}, {vocab, pl * layers});
    }
    for (int64_t l = 0; l < layers; ++l) {
        const std::string b = "blk." + std::to_string(l) + ".";
        const int64_t hd = c.head_dim[size_t(l)], ffl = c.ff[size_t(l)];
        const bool own = c.has_kv(l);
        std::vector<std::string> qkv{b + "attn_q.weight"};
        if (own) {
            qkv.push_back(b + "attn_k.weight");
            qkv.push_back(b + "attn_v.weight");
        }
        w.tensors[b + "attn_norm"] = convert({b + "attn_norm.weight"}, {d});
        w.tensors[b + "qkv"] = convert(qkv, {c.qkv_width(l), d});
        w.tensors[b + "q_norm"] = convert({b + "attn_q_norm.weight"}, {hd});
        if (own) w.tensors[b + "k_norm"] = convert({b + "attn_k_norm.weight"}, {hd});
        w.tensors[b + "o"] = convert({b + "attn_output.weight"}, {d, heads * hd});
        w.tensors[b + "post_attn_norm"] = convert({b + "post_attention_norm.weight"}, {d});
        w.tensors[b + "ffn_norm"] = convert({b + "ffn_norm.weight"}, {d});
        w.tensors[b + "gate"] = convert({b + "ffn_gate.weight"}, {ffl, d});
        w.tensors[b + "up"] = convert({b + "ffn_up.weight"}, {ffl, d});
        w.tensors[b + "down"] = convert({b + "ffn_down.weight"}, {d, ffl});
        w.tensors[b + "post_ffn_norm"] = convert({b + "post_ffw_norm.weight"}, {d});
        if (pl > 0) {
            w.tensors[b + "pl_gate"] = convert({b + "inp_gate.weight"}, {pl, d});
            w.tensors[b + "pl_proj"] = convert({b + "proj.weight"}, {d, pl});
            w.tensors[b + "pl_norm"] = convert({b + "post_norm.weight"}, {d});
            w.tensors[b + "out_scale"] = convert({b + "layer_output_scale.weight"}, {1});
        }
    }
    (void)version;
    return w;
}

}  // namespace omg
