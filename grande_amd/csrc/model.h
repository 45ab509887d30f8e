// Checkpoint description and host-side tensors: the C++ counterpart of
// crates/omg-wgpu/src/model.rs (Config, Dtype, QTensor, Weights, Manifest).
#pragma once

#include <cstdint>
#include <map>
#include <string>
#include <vector>

#include "json.h"

namespace omg {

enum Arch { GEMMA3 = 0, GEMMA4 = 1 };

// model.rs:337-371. Codes match the reference's shader QUANT constant.
enum Dtype { F16 = 0, Q8 = 1, Q4 = 2 };
constexpr int64_t BLOCK = 32;
Dtype parse_dtype(const std::string& s);
int64_t payload_bytes(Dtype t, int64_t n);

struct TensorSpec {
    std::string name;
    std::vector<int64_t> shape;
};

// model.rs:27-63: every per-layer property as a vector so one code path
// covers sliding/global layers, shared K/V and partial RoPE.
struct Config {
    Arch arch = GEMMA3;
    int64_t vocab = 0, d = 0, layers = 0, heads = 0, kv_heads = 0;
    std::vector<int64_t> head_dim, ff;
    std::vector<bool> sliding;
    std::vector<int64_t> kv_source, rope_dims;
    float eps = 1e-6f;
    int64_t window = 512;
    float theta_global = 1e6f, theta_local = 1e4f, query_scale = 1.0f, norm_offset = 0.0f;
    bool v_norm = false;
    int64_t per_layer_dim = 0;
    float softcap = 0.0f;
    uint32_t bos = 2;

    static Config from_json(const Json& v);      // model.rs:66-210
    void validate() const;                        // model.rs:213-254 + this engine's kernels
    bool has_kv(int64_t l) const { return kv_source[size_t(l)] == l; }
    int64_t qkv_width(int64_t l) const;           // model.rs:262-269
    int64_t max_head_dim() const;
    int64_t max_ff() const;
    int64_t max_qkv() const;
    std::vector<TensorSpec> tensors() const;      // model.rs:277-314
};

// model.rs:375-538: raw little-endian payload plus f16 block scales.
struct QTensor {
    Dtype dtype = F16;
    std::vector<int64_t> shape;
    std::vector<uint8_t> data, scales;
    int64_t numel() const;
    float get(int64_t i) const;  // model.rs:507-525
};

QTensor quantize_q8(const std::vector<int64_t>& shape, const float* v);  // model.rs:408-431
QTensor quantize_q4(const std::vector<int64_t>& shape, const float* v);  // model.rs:435-466
QTensor from_f32(const std::vector<int64_t>& shape, const float* v);     // model.rs:403-406

// tests/reference.rs:17-38: the seeded xorshift generator.
struct Rng {
    uint64_t s;
    explicit Rng(uint64_t seed) : s(seed) {}
    float next() {
        s ^= s << 13;
        s ^= s >> 7;
        s ^= s << 17;
        return (float(s >> 40) / float(uint64_t(1) << 24)) * 2.0f - 1.0f;
    }
};

// A whole host checkpoint (model.rs:540-646).
struct Weights {
    Config config;
    std::map<std::string, QTensor> tensors;
};

// tests/reference.rs:106-139: random weights of a config in catalogue order,
// norms 1-D f16 around (norm_offset == 0 ? 1 : 0), linears at 0.15 (input
// width d) or 0.08, the embedding at 1.0.
Weights synth_weights(const Config& cfg, uint64_t seed, Dtype linear, Dtype embed);

// model.rs:742-795 + tools/export_wgpu_gguf.py: config.json + manifest.json
// + *.bin.  Reads every catalogued tensor of an exported directory.
Weights load_dir(const std::string& dir);
// A llama.cpp GGUF file (v2/v3, gemma3): its metadata as the text config
// and its tensors in the catalogue's names, as
// tools/export_wgpu_gguf.py:112-296 maps them (q / k / v fused).
Weights load_gguf(const std::string& path);

// The tensors of an exported directory's manifest.json + *.bin files.
std::map<std::string, QTensor> read_manifest(const std::string& dir);

std::string read_file(const std::string& path);

}  // namespace omg
