// The decision-path engine: request packing, the per-layer launch plan,
// readout, resident prefix and the f16 K/V state machinery
// (crates/omg-wgpu/src/engine.rs).
#include "engine.h"

#include <cstring>

#include <sys/stat.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <fstream>

// Most split-K partials of one product (a_ holds this many).
#ifndef OMG_KSPLIT
#define OMG_KSPLIT 4
#endif

namespace omg {

// ---------------------------------------------------------------- device

DevBuf::DevBuf(size_t n, bool zero) : bytes(n) {
    OMG_HIP(hipMalloc(&p, std::max<size_t>(n, 16)));
    if (zero) OMG_HIP(hipMemset(p, 0, std::max<size_t>(n, 16)));
}
DevBuf::~DevBuf() {
    if (p) (void)hipFree(p);
}
DevBuf& DevBuf::operator=(DevBuf&& o) noexcept {
    if (this != &o) {
        if (p) (void)hipFree(p);
        p = o.p;
        bytes = o.bytes;
        o.p = nullptr;
        o.bytes = 0;
    }
    return *this;
}

static DevBuf upload_bytes(const void* src, size_t n) {
    DevBuf b(n);
    if (n) OMG_HIP(hipMemcpy(b.p, src, n, hipMemcpyHostToDevice));
    return b;
}

DevTensor upload_weight(const QTensor& t, bool tiled) {
    if (t.shape.size() != 2 || t.shape[1] % 32 != 0) fail(E_INVALID, "weight: expected [rows, cols % 32 == 0]");
    DevTensor d;
    d.w.dtype = int(t.dtype);
    d.w.rows = t.shape[0];
    d.w.cols = t.shape[1];
    const int64_t n = d.w.rows * d.w.cols, kb = d.w.cols / BLOCK;
    std::vector<uint8_t> rep;
    if (t.dtype == Q4) {
        rep.resize(t.data.size());
        repack_q4(t.data.data(), rep.data(), n);
    }
    const uint8_t* src = t.dtype == Q4 ? rep.data() : t.data.data();  // row-major device bytes
    d.data = upload_bytes(src, t.data.size());
    if (t.dtype != F16) {
        // Scale rows padded to an even count of blocks (zeros in the pad).
        d.w.sld = (kb + 1) / 2 * 2;
        std::vector<uint8_t> sc(size_t(d.w.rows * d.w.sld) * 2, 0);
        for (int64_t r = 0; r < d.w.rows; ++r)
            std::memcpy(sc.data() + r * d.w.sld * 2, t.scales.data() + r * kb * 2, size_t(kb) * 2);
        d.scales = upload_bytes(sc.data(), sc.size());
    }
    d.w.data = d.data.p;
    d.w.scales = d.scales.as<uint16_t>();
    if (!tiled) return d;

    // Stage tiles (kernels.h): from the row-major device bytes above.
    const int64_t rb = (d.w.rows + 31) / 32, st = (d.w.cols + 63) / 64;
    const int PK = tile_packet_bytes(d.w.dtype);
    const int64_t row_bytes = t.dtype == Q4 ? d.w.cols / 2 : (t.dtype == Q8 ? d.w.cols : 2 * d.w.cols);
    const int CB = PK / 32, piece = CB / 8;  // bytes of one row per stage, per (k-step, half)
    std::vector<uint8_t> tiles(size_t(rb * st * PK), 0);
    std::vector<uint8_t> tsc(t.dtype == F16 ? 0 : size_t(rb * st * TILE_SCALE_BYTES), 0);
    for (int64_t r = 0; r < d.w.rows; ++r) {
        const int64_t b = r / 32, rr = r % 32;
        for (int64_t s = 0; s < st; ++s) {
            uint8_t* pk = tiles.data() + (b * st + s) * PK;
            for (int ks = 0; ks < 4; ++ks)
                for (int h = 0; h < 2; ++h) {
                    const int64_t at = s * CB + ks * (CB / 4) + h * piece;
                    if (at + piece <= row_bytes)
                        std::memcpy(pk + (32 * h + rr) * (PK / 64) + ks * (PK / 256), src + r * row_bytes + at,
                                    size_t(piece));
                }
            if (t.dtype != F16)
                for (int64_t blk = 2 * s; blk < 2 * s + 2 && blk < kb; ++blk)
                    std::memcpy(tsc.data() + (b * st + s) * TILE_SCALE_BYTES + rr * 4 + (blk - 2 * s) * 2,
                                t.scales.data() + (r * kb + blk) * 2, 2);
        }
    }
    d.tiles = upload_bytes(tiles.data(), tiles.size());
    if (!tsc.empty()) d.tscales = upload_bytes(tsc.data(), tsc.size());
    d.w.tiles = d.tiles.as<uint8_t>();
    d.w.tscales = d.tscales.as<uint8_t>();
    d.w.stages = st;
    return d;
}

// --------------------------------------------------------------- builder

Builder::Builder(Config cfg) : cfg_(std::move(cfg)) {
    cfg_.validate();
    for (const TensorSpec& s : cfg_.tensors()) expected_[s.name] = s.shape;
    // engine.rs:938-947 (set_per_layer_table): [vocab, layers x P].
    if (cfg_.per_layer_dim > 0) expected_["per_layer_table"] = {cfg_.vocab, cfg_.per_layer_dim * cfg_.layers};
}

void Builder::push(const std::string& name, const QTensor& t) {
    auto it = expected_.find(name);
    if (it == expected_.end()) fail(E_INVALID, "unexpected tensor " + name);
    if (t.shape != it->second) fail(E_INVALID, name + ": shape mismatch");
    const int64_t n = t.numel();
    if (int64_t(t.data.size()) != payload_bytes(t.dtype, n)) fail(E_INVALID, name + ": payload size mismatch");
    if (t.dtype != F16 && int64_t(t.scales.size()) != n / BLOCK * 2) fail(E_INVALID, name + ": scale size mismatch");
    if (name.size() >= 9 && name.compare(name.size() - 9, 9, "out_scale") == 0) {
        // A per-layer scalar (engine.rs:896-901), applied as is.
        if (t.dtype != F16 || n != 1) fail(E_INVALID, name + ": expected one f16 value");
        scalars_[name] = t.get(0);
        return;
    }
    if (t.shape.size() == 1) {
        // Norm weights are applied as (offset + w) in f32 (rmsnorm.wgsl:34-39).
        if (t.dtype != F16) fail(E_INVALID, name + ": 1-D tensors must be f16");
        std::vector<float> v(static_cast<size_t>(n));
        for (int64_t i = 0; i < n; ++i) v[size_t(i)] = cfg_.norm_offset + t.get(i);
        norms_[name] = upload_bytes(v.data(), v.size() * 4);
        linears_.erase(name);
        return;
    }
    if (t.shape[1] % 32 != 0) fail(E_INVALID, name + ": inner dimension is not a multiple of 32");
    // The embedding tables are only gathered by rows (and the token table
    // read by the readout's own kernel), never fed to a GEMM.
    linears_[name] = upload_weight(t, name != "embed" && name != "per_layer_table");
    norms_.erase(name);
}

std::vector<std::string> Builder::missing() const {
    std::vector<std::string> v;
    for (const auto& kv : expected_)
        if (!linears_.count(kv.first) && !norms_.count(kv.first) && !scalars_.count(kv.first)) v.push_back(kv.first);
    return v;
}

std::unique_ptr<Engine> Builder::finish(int64_t capacity, int64_t max_rows) {
    const auto miss = missing();
    if (!miss.empty()) {
        std::string m = std::to_string(miss.size()) + " tensors missing, e.g.";
        for (size_t i = 0; i < miss.size() && i < 4; ++i) m += " " + miss[i];
        fail(E_MISSING, m);
    }
    if (capacity <= 0 || max_rows <= 0) fail(E_INVALID, "capacity and max_rows must be positive");
    std::unique_ptr<Engine> e(new Engine());
    Engine& E = *e;
    const Config& c = cfg_;
    E.cfg_ = c;
    E.capacity_ = capacity;
    E.max_rows_ = max_rows;
    // Groups start on a key tile and a query tile of the attention kernel.
    E.align_ = std::max<int64_t>(attention_key_tile(), attention_rows() / (c.heads / c.kv_heads));
    E.slots_ = capacity + (E.align_ - 1) * max_rows;
    E.cap_pad_ = (E.slots_ + 63) / 64 * 64;
    OMG_HIP(hipStreamCreateWithFlags(&E.stream_, hipStreamNonBlocking));
    // The sub-pass streams (default priority, like stream_) and their
    // fork / join / K/V-ready events (no timing).
    E.sub_stream_[0] = E.stream_;
    for (int k = 1; k < Engine::MAX_SUB; ++k)
        OMG_HIP(hipStreamCreateWithFlags(&E.sub_stream_[k], hipStreamNonBlocking));
    OMG_HIP(hipEventCreateWithFlags(&E.ev_fork_, hipEventDisableTiming));
    for (int k = 0; k < Engine::MAX_SUB; ++k) OMG_HIP(hipEventCreateWithFlags(&E.ev_join_[k], hipEventDisableTiming));
    E.ev_kv_.assign(size_t(Engine::MAX_SUB * cfg_.layers), nullptr);
    for (hipEvent_t& ev : E.ev_kv_) OMG_HIP(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
    {
        int dev = 0, cus = 0;
        OMG_HIP(hipGetDevice(&dev));
        OMG_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
        E.cus_ = cus > 0 ? cus : 256;
    }
    auto take_lin = [&](const std::string& n) { return std::move(linears_.at(n)); };
    auto take_norm = [&](const std::string& n) { return std::move(norms_.at(n)); };
    if (linears_.count("embed") == 0) fail(E_INVALID, "embed must be a 2-D tensor");
    E.embed_ = take_lin("embed");
    E.final_norm_ = take_norm("final_norm");
    for (int64_t l = 0; l < c.layers; ++l) {
        auto n = [&](const char* s) { return "blk." + std::to_string(l) + "." + s; };
        Engine::Layer L;
        L.qkv = take_lin(n("qkv"));
        L.o = take_lin(n("o"));
        L.gate = take_lin(n("gate"));
        L.up = take_lin(n("up"));
        L.down = take_lin(n("down"));
        if (L.gate.w.dtype != L.up.w.dtype)
            fail(E_INVALID, "layer " + std::to_string(l) + ": gate and up projections must share a storage type");
        L.attn_norm = take_norm(n("attn_norm"));
        L.q_norm = take_norm(n("q_norm"));
        if (c.has_kv(l)) L.k_norm = take_norm(n("k_norm"));
        L.post_attn_norm = take_norm(n("post_attn_norm"));
        L.ffn_norm = take_norm(n("ffn_norm"));
        L.post_ffn_norm = take_norm(n("post_ffn_norm"));
        if (c.per_layer_dim > 0) {
            L.pl_gate = take_lin(n("pl_gate"));
            L.pl_proj = take_lin(n("pl_proj"));
            L.pl_norm = take_norm(n("pl_norm"));
            L.out_scale = scalars_.at(n("out_scale"));
        }
        E.layers_.push_back(std::move(L));
    }
    if (c.per_layer_dim > 0) {
        E.pl_model_proj_ = take_lin("pl_model_proj");
        E.pl_proj_norm_ = take_norm("pl_proj_norm");
        E.pl_table_ = take_lin("per_layer_table");
    }
    // RoPE inverse frequencies theta^(-i / (hd/2)) (reference.rs:159-168)
    // and the rotation (cos, sin) per position, one table per (layer type,
    // head_dim): positions stay below the capacity (every token of a pass
    // has its own cache row).
    const int64_t hd = c.max_head_dim();
    const int64_t cap = E.slots_, d = c.d;
    // positions count within a group, so they stay below the token capacity
    E.rope_rows_ = capacity;
    {
        std::vector<std::pair<bool, int64_t>> keys;
        std::vector<DevBuf> freqs;
        for (int64_t l = 0; l < c.layers; ++l) {
            const std::pair<bool, int64_t> key{c.sliding[size_t(l)], c.head_dim[size_t(l)]};
            auto it = std::find(keys.begin(), keys.end(), key);
            if (it == keys.end()) {
                const int64_t half = key.second / 2;
                const float theta = key.first ? c.theta_local : c.theta_global;
                std::vector<float> f(static_cast<size_t>(half));
                for (int64_t i = 0; i < half; ++i) f[size_t(i)] = std::pow(theta, -float(i) / float(half));
                freqs.push_back(upload_bytes(f.data(), f.size() * 4));
                E.rope_tabs_.emplace_back(size_t(capacity * half) * 8);
                launch_rope_table(E.stream_, freqs.back().as<float>(), capacity, half,
                                  E.rope_tabs_.back().as<float2>());
                keys.push_back(key);
                it = keys.end() - 1;
            }
            E.rope_of_.push_back(int(it - keys.begin()));
        }
        OMG_HIP(hipStreamSynchronize(E.stream_));
    }
    E.meta_ = DevBuf(size_t(E.cap_pad_) * 16, true);
    E.x_ = DevBuf(size_t(cap * d) * 4);
    E.hn_ = DevBuf(size_t(cap * d) * 2);
    E.qkv_ = DevBuf(size_t(cap * c.max_qkv()) * 4);
    E.q16_ = DevBuf(size_t(cap * c.heads * hd) * 2);
    E.attn_ = DevBuf(size_t(cap * c.heads * hd) * 2);
    // a_ holds up to OMG_KSPLIT split-K partials of the o / down products.
    E.a_ = DevBuf(size_t(cap * d) * 4 * OMG_KSPLIT);
    E.act_ = DevBuf(size_t(cap * c.max_ff()) * 2);
    E.rows_ = DevBuf(size_t(max_rows * d) * 4);
    // the last layer on the answer rows (layer_out)
    E.attn_w_ = DevBuf(size_t(max_rows * c.heads * hd) * 2);
    E.x_w_ = DevBuf(size_t(max_rows * d) * 4);
    E.hn_w_ = DevBuf(size_t(max_rows * d) * 2);
    E.act_w_ = DevBuf(size_t(max_rows * c.max_ff()) * 2);
    E.q16_w_ = DevBuf(size_t(max_rows * c.heads * hd) * 2);
    E.qkv_w_ = DevBuf(size_t(max_rows * c.max_qkv()) * 4);
    if (c.per_layer_dim > 0) {
        E.x16_w_ = DevBuf(size_t(max_rows * d) * 2);
        E.plg_w_ = DevBuf(size_t(max_rows * c.per_layer_dim) * 4);
        E.pl16_w_ = DevBuf(size_t(max_rows * c.per_layer_dim) * 2);
        E.pli_w_ = DevBuf(size_t(max_rows * c.per_layer_dim * c.layers) * 4);
    }
    // The answer-row path starts at the last layer that writes K/V (Gemma
    // 4's K/V-sharing layers read an earlier layer's cache).
    for (int64_t l = 0; l < c.layers; ++l)
        if (c.has_kv(l)) E.out_layer_ = l;
    {
        int most = OMG_KSPLIT;  // the most parts of an o / down product (K splits x pieces)
        for (int64_t l = 0; l < c.layers; ++l)
            for (const int64_t kd : {c.heads * c.head_dim[size_t(l)], c.ff[size_t(l)]}) {
                const Engine::SplitPlan p = E.split_plan(kd, d, 1);
                most = std::max(most, p.splits * p.group);
            }
        E.a_w_ = DevBuf(size_t(max_rows * d) * 4 * size_t(most));
    }
    const int64_t width = std::max(c.vocab, d);
    E.logits_ = DevBuf(size_t(max_rows * width) * 4);
    E.label_lse_ = DevBuf(size_t(max_rows * (c.vocab + 1)) * 4);
    E.lse_part_ = DevBuf(size_t(logits_blocks(c.vocab) * max_rows) * 8);
    E.kv_stage_ = DevBuf(size_t(E.cap_pad_ * 2 * c.kv_heads * hd) * 2);
    if (c.per_layer_dim > 0) {
        const int64_t P = c.per_layer_dim;
        E.x16_ = DevBuf(size_t(cap * d) * 2);
        E.pli_ = DevBuf(size_t(cap * P * c.layers) * 4);
        E.plg_ = DevBuf(size_t(cap * P) * 4);
        E.pl16_ = DevBuf(size_t(cap * P) * 2);
    }
    // Attention work: query tiles' key ranges are split at fixed multiples
    // of `chunk` key tiles: 256 keys on sliding layers (a range is at most
    // window + branch long), at least 384 keys and at most ~8 chunks over
    // the cache on global layers.  Measured at C2 (same box): global chunks
    // of 384 keys against 512: cold pass -0.4%, warm -0.4%, one-branch -1%;
    // 256 keys: short passes -1.3 / -1.9% but the cold pass +0.5%; 448 and
    // 320 keys (after the GEMM changes): cold +0.3% and +1.6%; sliding
    // chunks of 384 or 512 keys: every pass 2.5-6% slower.
    {
        const int64_t kt = attention_key_tile();
        // (the global chunk follows the token capacity, not the padded rows)
        const int64_t key_tiles = (capacity + 63) / 64 * 64 / kt;
        const int64_t tpb = attention_rows() / (c.heads / c.kv_heads);
        const int64_t qtiles = (cap + tpb - 1) / tpb;
        E.attn_chunk_[0] = int(256 / kt);
        E.attn_chunk_[1] = int(std::max<int64_t>(384 / kt, (key_tiles + 7) / 8));
        // The pass inputs (ids, wanted rows, labels, both layer types'
        // work lists) and the chunk partials start sized for a few chunks
        // per query tile and grow with the passes that need more (upload).
        E.in_bytes_ = size_t(cap) * 4 + size_t(max_rows) * 4 + size_t(c.vocab) * 4 + size_t(qtiles * 5) * 16 * 2 + 64;
        E.in_ = DevBuf(E.in_bytes_);
        E.part_slots_ = qtiles * 4;
        E.part_o_ = DevBuf(size_t(E.part_slots_ * c.kv_heads * attention_rows()) * size_t(hd) * 2);
        E.part_ml_ = DevBuf(size_t(E.part_slots_ * c.kv_heads * attention_rows()) * 2 * 4);
        (void)key_tiles;
    }
    // The K/V cache starts zeroed: a masked key's probability is exactly 0
    // and its V row must be finite for the 0 * V product to vanish.
    for (int64_t l = 0; l < c.layers; ++l) {
        if (c.has_kv(l)) {
            const size_t bytes = size_t(c.kv_heads * E.cap_pad_ * c.head_dim[size_t(l)]) * 2;
            E.kc_.emplace_back(bytes, true);
            E.vt_.emplace_back(bytes, true);
        } else {
            E.kc_.emplace_back();
            E.vt_.emplace_back();
        }
    }
    E.h_in_bytes_ = size_t(cap) * 16 + E.in_bytes_;
    OMG_HIP(hipHostMalloc(&E.h_in_, E.h_in_bytes_, hipHostMallocDefault));
    E.h_out_bytes_ = size_t(max_rows * (width + 1)) * 4;  // + 1: the log-sum-exp after vocab labels
    OMG_HIP(hipHostMalloc(&E.h_out_, E.h_out_bytes_, hipHostMallocDefault));
    for (int64_t l = 0; l < c.layers; ++l) {
        if (!c.has_kv(l)) continue;
        const auto [r0, r1] = E.state_rows(l, capacity);
        E.h_state_bytes_ += size_t((r1 - r0) * 2 * c.kv_heads * c.head_dim[size_t(l)] * 2);
    }
    if (E.h_state_bytes_) OMG_HIP(hipHostMalloc(&E.h_state_, E.h_state_bytes_, hipHostMallocDefault));
    OMG_HIP(hipDeviceSynchronize());
    return e;
}

// ---------------------------------------------------------------- engine

Engine::~Engine() {
    for (hipStream_t s : sub_stream_)
        if (s) (void)hipStreamSynchronize(s);
    if (graph_exec_) (void)hipGraphExecDestroy(graph_exec_);
    for (auto& list : pending_)
        for (Timed& t : list) (void)hipEventDestroy(t.e);
    for (hipEvent_t ev : event_pool_) (void)hipEventDestroy(ev);
    for (hipEvent_t ev : ev_kv_)
        if (ev) (void)hipEventDestroy(ev);
    for (hipEvent_t ev : ev_join_)
        if (ev) (void)hipEventDestroy(ev);
    if (ev_fork_) (void)hipEventDestroy(ev_fork_);
    for (int k = 1; k < MAX_SUB; ++k)
        if (sub_stream_[k]) (void)hipStreamDestroy(sub_stream_[k]);
    if (h_in_) (void)hipHostFree(h_in_);
    if (h_out_) (void)hipHostFree(h_out_);
    if (h_ptr_) (void)hipHostFree(h_ptr_);
    if (h_state_) (void)hipHostFree(h_state_);
    if (stream_) (void)hipStreamDestroy(stream_);
}

// Measurement mode: one event after each launch on its range's stream; a
// launch's time is the interval since the previous event of the same
// stream, so back-to-back launches pay for one event each rather than two.
template <class F>
void Engine::step(const char* name, int k, F&& f) {
    if (!profile_) {
        f();
        return;
    }
    auto ev = [&]() {
        if (event_pool_.empty()) {
            hipEvent_t e;
            // No system-scope release at the timestamp: it would write back L2
            // between the launches being timed.
            OMG_HIP(hipEventCreateWithFlags(&e, hipEventDisableSystemFence));
            return e;
        }
        hipEvent_t e = event_pool_.back();
        event_pool_.pop_back();
        return e;
    };
    const hipStream_t s = sub_stream_[k];
    std::vector<Timed>& pend = pending_[k];
    if (pend.empty()) {
        const hipEvent_t start = ev();
        OMG_HIP(hipEventRecord(start, s));
        pend.push_back(Timed{nullptr, start});
    }
    f();
    const hipEvent_t end = ev();
    OMG_HIP(hipEventRecord(end, s));
    pend.push_back(Timed{name, end});
}

void Engine::collect_profile() {
    for (auto& pend : pending_) {
        for (size_t i = 1; i < pend.size(); ++i) {
            float ms = 0.0f;
            OMG_HIP(hipEventElapsedTime(&ms, pend[i - 1].e, pend[i].e));
            auto& tot = totals_[pend[i].name];
            tot.first += 1;
            tot.second += double(ms);
        }
        for (Timed& t : pend) event_pool_.push_back(t.e);
        pend.clear();
    }
}

void Engine::set_profile(bool on) {
    sync();
    profile_ = on;
    totals_.clear();
}

void Engine::set_full_last_layer(bool on) {
    sync();
    full_last_layer_ = on;
}

std::string Engine::profile_report() const {
    std::string s;
    char line[256];
    for (const auto& kv : totals_) {
        std::snprintf(line, sizeof line, "%s %lld %.6f\n", kv.first.c_str(), (long long)kv.second.first,
                      kv.second.second);
        s += line;
    }
    return s;
}

void Engine::sync() {
    // (every pass joins its ranges' streams into stream_)
    OMG_HIP(hipStreamSynchronize(stream_));
    collect_profile();
}

std::pair<int64_t, int64_t> Engine::state_rows(int64_t layer, int64_t p) const {
    if (cfg_.sliding[size_t(layer)] && cfg_.window > 0) return {std::max<int64_t>(0, p - cfg_.window), p};
    return {0, p};
}

bool Engine::is_resident(const uint32_t* prefix, int64_t n) const {
    if (n == 0 || !resident_) return false;
    return int64_t(resident_->size()) == n && std::equal(prefix, prefix + n, resident_->begin());
}

std::pair<int64_t, int> Engine::admit(const GroupIn* groups, int64_t n) {
    for (int64_t i = 0; i < n; ++i)
        if (is_resident(groups[i].prefix, groups[i].prefix_len)) return {i, SRC_RESIDENT};
    for (int64_t i = 0; i < n; ++i) {
        const int src = restore_from_cache(groups[i].prefix, groups[i].prefix_len);
        if (src != SRC_NONE) return {i, src};
    }
    return {0, SRC_NONE};
}

Packed Engine::pack_checked(const GroupIn* groups, int64_t n, int64_t first, bool resident) const {
    int64_t total = 0;
    for (int64_t g = 0; g < n; ++g) {
        total += groups[g].prefix_len;
        for (int64_t b = 0; b < groups[g].nbranches; ++b) total += groups[g].branches[b].ntokens;
    }
    if (total > capacity_)
        fail(E_CAPACITY, std::to_string(total) + " tokens exceed the engine capacity " + std::to_string(capacity_));
    // the reference's layout, then groups moved onto aligned rows
    Packed pk = align_groups(pack_groups(groups, n, first, resident), align_, slots_);
    if (int64_t(pk.wanted.size()) > max_rows_)
        fail(E_CAPACITY, std::to_string(pk.wanted.size()) + " rows requested, engine reads back at most " +
                             std::to_string(max_rows_));
    for (uint32_t id : pk.ids)
        if (int64_t(id) >= cfg_.vocab)
            fail(E_INVALID, "token id " + std::to_string(id) + " outside the vocabulary of " + std::to_string(cfg_.vocab));
    return pk;
}

// Passes of at most this many tokens run 2-wave attention items.
constexpr int64_t SHORT_ATTN_ROWS = 1024;
// Row ranges (Engine::Sub): passes of more than MID_ROWS rows run as two
// ranges, the first 55% of the rows (each cut rounded up to a 64-row cache
// tile), or as three cut at 40% and 72% when the model is at least WIDE_D
// wide or the pass at least 3 * SUB_ROWS rows.  Measured (same box): the
// 4B model's 16,320-token pass in three even ranges 169.9 -> 159.0 ms (an
// earlier build), its 8,320-row warm pass in two even ones 96.3 -> 91.9
// ms, in three at 40 / 72% another 87.1 -> 85.3 ms; the 270M model's 2,384-token cold
// pass with two ranges cut at 40 / 45 / 50 / 55 / 60 / 75 / 86% gave
// +1.3 / +2.3 / +2.7 / +3.5 / +2.4 / -2.4 / -4.4% questions/s against one
// range (an even split measured 0.5% slower before this build's kernel
// changes), three at 40 / 72% 6.6% below two; two at 55% took the 1B
// model's 2,384-token pass 5.78 -> 5.45 ms and E2B's 2,663-token pass
// 17.17 -> 15.96 ms, three at 40 / 72% another -1.2% and -3.7%.  Three
// ranges of the 4B model's 16,320-token pass cut at 40 / 72% rather than
// evenly: 150.1 -> 149.4 ms.
constexpr int64_t MID_ROWS = 1024;
constexpr int64_t WIDE_D = 1024;
constexpr int64_t SUB_ROWS = 4096;
// Passes of at most this many rows run deep-K products a piece per
// workgroup (split_plan).
constexpr int64_t CHUNKED_ROWS = 512;

void Engine::upload(const Packed& pk, const uint32_t* labels, int64_t nlabels) {
    const int64_t t = pk.total - pk.base, nr = int64_t(pk.wanted.size());
    // Everything that can reject the request is checked before the first
    // write to the device: a refused request leaves the cache and its
    // metadata as they were.
    if (nlabels > 0) {
        if (!labels) fail(E_INVALID, "label readout without label ids");
        if (nlabels > cfg_.vocab) fail(E_INVALID, "more labels than vocabulary rows");
        for (int64_t i = 0; i < nlabels; ++i)
            if (int64_t(labels[i]) >= cfg_.vocab) fail(E_INVALID, "label id outside the vocabulary");
    }
    // The pass writes cache rows and their metadata from pk.base on: a
    // resident prefix reaching past that is gone from here on, whatever
    // happens to the rest of the pass.
    if (resident_ && int64_t(resident_->size()) > pk.base) resident_.reset();
    // A captured pass reads the work lists and buffers this upload may move.
    drop_graph();
    // Row ranges (Engine::Sub): from MID_ROWS rows two or three (see
    // there), cut where a
    // cache row is a multiple of 64 (no V^T tile of the
    // cache holds rows of two ranges), each longer than CHUNKED_ROWS (no
    // range takes the short passes' one-chunk-per-workgroup products, whose
    // partials share one area).  One range while profiling: the kernels'
    // times are then those of the pass's launches alone.
    static_assert(MAX_SUB == 3, "three ranges at most");
    int ns = 1;
    if (!profile_ && t > MID_ROWS) ns = cfg_.d >= WIDE_D || t >= 3 * SUB_ROWS ? 3 : 2;
    // First row of range k of n (pass-relative), k = 1 .. n - 1.
    auto cut = [&](int k, int n) -> int64_t {
        const int64_t pct = n == 3 ? (k == 1 ? 40 : 72) : 55;
        return (pk.base + t * pct / 100 + 63) / 64 * 64 - pk.base;
    };
    for (; ns > 1; --ns) {
        bool ok = true;
        int64_t prev = 0;
        for (int k = 1; k <= ns; ++k) {
            const int64_t r = k == ns ? t : cut(k, ns);
            ok = ok && r - prev > CHUNKED_ROWS;
            sub_[k - 1].r0 = prev;
            sub_[k - 1].r1 = r;
            prev = r;
        }
        if (ok) break;
    }
    if (ns == 1) {
        sub_[0].r0 = 0;
        sub_[0].r1 = t;
    }
    nsub_ = ns;
    // Attention work lists per range and layer type.  Short ranges run
    // 2-wave items (twice the items: more of the chip busy) when every
    // query tile is aligned, which keeps each row's chunk boundaries, and
    // so its sums, those of 4-wave items, and when the 2-wave workgroups
    // number no more than the CUs: an item's K / V buffers take the same
    // LDS at either width (a CU holds two at head_dim 256, one at 512), so
    // 2-wave workgroups that have to share CUs run half the waves per CU.
    // The ranges' chunk partials take disjoint slots (they run at once).
    int64_t slots = 0;
    for (int k = 0; k < ns; ++k) {
        Sub& sb = sub_[k];
        const int64_t rt = sb.r1 - sb.r0;
        int64_t most = 0;
        for (int kind = 0; kind < 2; ++kind) {
            const int window = kind == 0 ? int(cfg_.window) : 0;
            AttnWork& w = sb.work[kind];
            const int32_t* meta = pk.meta.data() + 4 * sb.r0;
            attention_work(meta, rt, int(cfg_.heads), int(cfg_.kv_heads), window, attn_chunk_[kind],
                           rt <= SHORT_ATTN_ROWS ? 2 : 4, w);
            if (w.nw == 2 && (!w.aligned || int64_t(w.items.size()) * cfg_.kv_heads > cus_))
                attention_work(meta, rt, int(cfg_.heads), int(cfg_.kv_heads), window, attn_chunk_[kind], 4, w);
            for (int4& it : w.items)
                if (it.w >= 0) it.w += int(slots);
            for (int4& m : w.merges) m.y += int(slots);
            most = std::max<int64_t>(most, w.slots);
        }
        slots += most;
    }
    // The last layer on the answer rows only (layer_out): wanted rows in
    // ascending order (each range's share is one run of the list).  Its attention runs the items
    // of the query tiles that hold those rows, the same items a full pass
    // runs for them.
    bool asc = true;
    for (int64_t r = 1; r < nr; ++r) asc = asc && pk.wanted[size_t(r)][3] >= pk.wanted[size_t(r - 1)][3];
    out_rows_ = !full_last_layer_ && nr > 0 && asc;
    if (out_rows_) {
        const int64_t ol = out_layer_;
        const int kind = (cfg_.sliding[size_t(ol)] && cfg_.window > 0) ? 0 : 1;
        int64_t i = 0;
        for (int k = 0; k < ns; ++k) {
            Sub& sb = sub_[k];
            sb.w0 = i;
            while (i < nr && pk.wanted[size_t(i)][3] < sb.r1) ++i;
            sb.w1 = i;
            const AttnWork& w = sb.work[kind];
            const int64_t tpb = int64_t(w.nw) * 16 / (cfg_.heads / cfg_.kv_heads);
            std::vector<char> tile(size_t((sb.r1 - sb.r0 + tpb - 1) / tpb), 0);
            for (int64_t j = sb.w0; j < sb.w1; ++j) tile[size_t((pk.wanted[size_t(j)][3] - sb.r0) / tpb)] = 1;
            sb.out_work.items.clear();
            sb.out_work.merges.clear();
            sb.out_work.nw = w.nw;
            for (const int4& it : w.items)
                if (it.x >= 0 && tile[size_t(it.x)]) sb.out_work.items.push_back(it);
            for (const int4& m : w.merges)
                if (tile[size_t(m.x)]) sb.out_work.merges.push_back(m);
        }
    }
    // The layers after out_layer_ on the answer rows alone: their metadata
    // rows, and per layer type attention items over them (partial slots
    // after the ranges').
    std::vector<int32_t> tail_meta;
    tail_rows_ = 0;
    if (out_rows_ && out_layer_ + 1 < cfg_.layers) {
        tail_rows_ = nr;
        tail_meta.resize(size_t(nr) * 4);
        for (int64_t i = 0; i < nr; ++i)
            std::memcpy(&tail_meta[size_t(i) * 4], pk.meta.data() + 4 * pk.wanted[size_t(i)][3], 16);
        int64_t most = 0;
        for (int kind = 0; kind < 2; ++kind) {
            AttnWork& w = tail_work_[kind];
            const int window = kind == 0 ? int(cfg_.window) : 0;
            attention_work(tail_meta.data(), nr, int(cfg_.heads), int(cfg_.kv_heads), window, attn_chunk_[kind], 2, w);
            if (!w.aligned || int64_t(w.items.size()) * cfg_.kv_heads > cus_)
                attention_work(tail_meta.data(), nr, int(cfg_.heads), int(cfg_.kv_heads), window, attn_chunk_[kind],
                               4, w);
            for (int4& it : w.items)
                if (it.w >= 0) it.w += int(slots);
            for (int4& m : w.merges) m.y += int(slots);
            most = std::max<int64_t>(most, w.slots);
        }
        slots += most;
    }
    tail_kend_ = pk.base + t;
    // The pass's inputs go to the device in two copies: the cache metadata
    // of its rows, and one block [ids | wanted rows | labels | per range and
    // layer type: work items, merges] (16-byte aligned parts).
    auto a16 = [](size_t n) { return (n + 15) / 16 * 16; };
    size_t in_bytes = 0;
    auto part = [&](size_t n) {
        const size_t o = in_bytes;
        in_bytes += a16(n);
        return o;
    };
    const size_t o_ids = part(size_t(t) * 4), o_wanted = part(size_t(nr) * 4), o_labels = part(size_t(nlabels) * 4);
    size_t o_items[MAX_SUB][2], o_merges[MAX_SUB][2], o_out_items[MAX_SUB], o_out_merges[MAX_SUB];
    for (int k = 0; k < ns; ++k) {
        for (int kind = 0; kind < 2; ++kind) {
            o_items[k][kind] = part(sub_[k].work[kind].items.size() * 16);
            o_merges[k][kind] = part(sub_[k].work[kind].merges.size() * 16);
        }
        o_out_items[k] = part(out_rows_ ? sub_[k].out_work.items.size() * 16 : 0);
        o_out_merges[k] = part(out_rows_ ? sub_[k].out_work.merges.size() * 16 : 0);
    }
    const size_t o_tail_meta = part(tail_meta.size() * 4);
    size_t o_tail_items[2], o_tail_merges[2];
    for (int kind = 0; kind < 2; ++kind) {
        o_tail_items[kind] = part(tail_rows_ ? tail_work_[kind].items.size() * 16 : 0);
        o_tail_merges[kind] = part(tail_rows_ ? tail_work_[kind].merges.size() * 16 : 0);
    }
    const size_t meta_bytes = a16(size_t(t) * 16);
    // The previous pass may still read the staging buffer; from here the
    // stream is idle (its ranges' streams joined it), so buffers can grow.
    OMG_HIP(hipStreamSynchronize(stream_));
    if (meta_bytes + in_bytes > h_in_bytes_) {
        OMG_HIP(hipHostFree(h_in_));
        h_in_ = nullptr;
        h_in_bytes_ = 0;
        OMG_HIP(hipHostMalloc(&h_in_, (meta_bytes + in_bytes) * 2, hipHostMallocDefault));
        h_in_bytes_ = (meta_bytes + in_bytes) * 2;
    }
    if (in_bytes > in_bytes_) {
        in_ = DevBuf(in_bytes * 2);
        in_bytes_ = in_bytes * 2;
    }
    if (slots > part_slots_) {
        part_slots_ = slots;
        const size_t rows = size_t(part_slots_ * cfg_.kv_heads * attention_rows());
        part_o_ = DevBuf(rows * size_t(cfg_.max_head_dim()) * 2);
        part_ml_ = DevBuf(rows * 2 * 4);
    }
    uint8_t* h = static_cast<uint8_t*>(h_in_);
    std::memcpy(h, pk.meta.data(), size_t(t) * 16);
    uint8_t* hb = h + meta_bytes;
    std::memcpy(hb + o_ids, pk.ids.data(), size_t(t) * 4);
    int32_t* w = reinterpret_cast<int32_t*>(hb + o_wanted);
    for (int64_t r = 0; r < nr; ++r) w[r] = int32_t(pk.wanted[size_t(r)][3]);
    if (nlabels > 0) std::memcpy(hb + o_labels, labels, size_t(nlabels) * 4);
    for (int k = 0; k < ns; ++k)
        for (int kind = 0; kind < 2; ++kind) {
            const AttnWork& wk = sub_[k].work[kind];
            if (!wk.items.empty()) std::memcpy(hb + o_items[k][kind], wk.items.data(), wk.items.size() * 16);
            if (!wk.merges.empty()) std::memcpy(hb + o_merges[k][kind], wk.merges.data(), wk.merges.size() * 16);
        }
    if (out_rows_)
        for (int k = 0; k < ns; ++k) {
            const AttnWork& wk = sub_[k].out_work;
            if (!wk.items.empty()) std::memcpy(hb + o_out_items[k], wk.items.data(), wk.items.size() * 16);
            if (!wk.merges.empty()) std::memcpy(hb + o_out_merges[k], wk.merges.data(), wk.merges.size() * 16);
        }
    if (tail_rows_) {
        std::memcpy(hb + o_tail_meta, tail_meta.data(), tail_meta.size() * 4);
        for (int kind = 0; kind < 2; ++kind) {
            const AttnWork& wk = tail_work_[kind];
            if (!wk.items.empty()) std::memcpy(hb + o_tail_items[kind], wk.items.data(), wk.items.size() * 16);
            if (!wk.merges.empty()) std::memcpy(hb + o_tail_merges[kind], wk.merges.data(), wk.merges.size() * 16);
        }
    }
    OMG_HIP(hipMemcpyAsync(meta_.as<uint8_t>() + pk.base * 16, h, size_t(t) * 16, hipMemcpyHostToDevice, stream_));
    OMG_HIP(hipMemcpyAsync(in_.p, hb, in_bytes, hipMemcpyHostToDevice, stream_));
    uint8_t* d = in_.as<uint8_t>();
    d_ids_ = reinterpret_cast<const uint32_t*>(d + o_ids);
    d_wanted_ = reinterpret_cast<const int32_t*>(d + o_wanted);
    d_labels_ = reinterpret_cast<const uint32_t*>(d + o_labels);
    for (int k = 0; k < ns; ++k)
        for (int kind = 0; kind < 2; ++kind) {
            Sub& sb = sub_[k];
            sb.d_items[kind] = reinterpret_cast<const int4*>(d + o_items[k][kind]);
            sb.d_merges[kind] = reinterpret_cast<const int4*>(d + o_merges[k][kind]);
            sb.n_items[kind] = int64_t(sb.work[kind].items.size());
            sb.n_merges[kind] = int64_t(sb.work[kind].merges.size());
        }
    for (int k = 0; k < ns; ++k) {
        sub_[k].d_out_items = reinterpret_cast<const int4*>(d + o_out_items[k]);
        sub_[k].d_out_merges = reinterpret_cast<const int4*>(d + o_out_merges[k]);
    }
    d_tail_meta_ = reinterpret_cast<const int32_t*>(d + o_tail_meta);
    for (int kind = 0; kind < 2; ++kind) {
        d_tail_items_[kind] = reinterpret_cast<const int4*>(d + o_tail_items[kind]);
        d_tail_merges_[kind] = reinterpret_cast<const int4*>(d + o_tail_merges[kind]);
    }
}

// K splits of the o / down products (output width n <= 2048): their tiles
// are few (128 output columns each) and each runs K / 64 stages in series;
// the splits run side by side and the residual norm adds them.  Widths up
// to 1280 split in two from K 1024 (measured on the 270M model's o and
// down, K 1024 / 2048 at n 640: both the 2,384-token cold pass and the
// 384-token warm pass gain, the warm one most), and every width splits
// one per 2048 of K from K 8192 (4096 above n 1280), at most OMG_KSPLIT
// (Gemma 4 E2B's K 4096 / 6144 / 12288 at n 1536).  Whole 64-wide stages
// per split.  A function of the shape only, so a row's sums do not depend
// on the pass (rows over a resident prefix stay bit-equal to a full pass).
static int ksplit(int64_t k, int64_t n) {
    if (n > 2048 || k < 1024) return 1;
    int s = 1;
    if (k >= (n > 1280 ? 4096 : 8192))
        s = int(std::min<int64_t>(OMG_KSPLIT, k / 2048));
    else if (n <= 1280)
        s = 2;
    while (s > 1 && k % (64 * s) != 0) --s;
    return s;
}

// K pieces of the o / down products, a function of the shape only: a
// split of deep K (at least 3,072, in whole 1,024-wide pieces: the 4B
// model's down projection, the E2B double-wide down in its 4 splits) is
// cut into `group` pieces whose products accumulate from zero; the pieces'
// sums are added in K order, then the splits' sums in order.  Long passes add a split's pieces in the GEMM's
// registers (kfold, one partial per split); short ones run a piece per
// workgroup, which fills the chip (10 x 20 x 2 = 400 workgroups at the 4B
// one-branch pass instead of 40), and the residual norm adds the pieces in
// the same runs — bit-equal rows either way.
// Measured and not kept (same box): pieces of 8 stages for every split of
// at least 32 (the 4B and E2B o, the E2B down): the 4B one-branch pass
// 4.08 -> 3.79 ms (o 13.8 -> 7.3 us), but adding pieces in registers
// drains the MFMA pipeline at every piece boundary: the 4B cold pass
// 155.9 -> 160.8 ms, E2B cold 16.55 -> 16.71 ms, warm 7.58 -> 7.67 ms;
// pieces of 4 stages on the 270M model's o and down: its cold pass 1.0 and
// 1.3 us slower per product, its warm pass 0.5 and 1.1 us faster.
// 3,072 rather than 4,096 (same box): the E2B double-wide down on its
// answer rows 19.4 -> 10.3 us, cold pass 8.05 -> 7.98 ms, warm 4.92 -> 4.83 ms.
constexpr int64_t DEEP_PIECE_K = 1024, DEEP_MIN_K = 3072;

Engine::SplitPlan Engine::split_plan(int64_t k, int64_t n, int64_t t) const {
    SplitPlan p;
    p.splits = ksplit(k, n);
    const int64_t kr = k / p.splits;
    if (kr < DEEP_MIN_K || kr % DEEP_PIECE_K != 0) return p;
    p.group = int(kr / DEEP_PIECE_K);
    p.kfold = int(DEEP_PIECE_K / 64);
    // a piece per workgroup: the parts (t x n floats each) fit in a_
    // (OMG_KSPLIT x slots x n floats); one range (ranges are longer)
    p.pieces = t <= CHUNKED_ROWS && nsub_ == 1 && int64_t(p.splits) * p.group * t <= int64_t(OMG_KSPLIT) * slots_;
    return p;
}

// Range k's rows [r0, r0 + t) of y = x . W^T (x already offset to the
// range) into the parts of a_ that norm_parts describes.
void Engine::split_product(const char* name, int k, const half_t* x, int64_t kdim, const DevWeight& w, int64_t r0,
                           int64_t t, const SplitPlan& sp) {
    const int64_t d = cfg_.d;
    const hipStream_t s = sub_stream_[k];
    if (sp.pieces) {
        float* a = a_.as<float>();  // one range: r0 = 0
        step(name, k, [&] { launch_gemm_splitk(s, x, kdim, w, a, d, t, sp.splits * sp.group, t * d); });
        return;
    }
    float* a = a_.as<float>() + r0 * d;
    step(name, k, [&] { launch_gemm_splitk(s, x, kdim, w, a, d, t, sp.splits, slots_ * d, sp.kfold); });
}

// Where split_product left a product's parts for the residual norm: a_
// offset to the range's rows, the part count and stride, and the run
// length the norm adds first.
Engine::NormParts Engine::norm_parts(const SplitPlan& sp, int64_t r0, int64_t t) const {
    const int64_t d = cfg_.d;
    if (sp.pieces) return NormParts{a_.as<float>(), sp.splits * sp.group, t * d, sp.group};
    return NormParts{a_.as<float>() + r0 * d, sp.splits, slots_ * d, 1};
}

// The pass's ranges on their streams: the ranges fork from stream_ (whose
// queue holds the pass's input copies), run layer by layer (host order:
// layer-major, so every stream has work queued), and join stream_ before
// the readout.
void Engine::forward(int64_t base) {
    const Config& c = cfg_;
    const int64_t d = c.d, P = c.per_layer_dim;
    const int ns = nsub_;
    if (ns > 1) {
        OMG_HIP(hipEventRecord(ev_fork_, stream_));
        for (int k = 1; k < ns; ++k) OMG_HIP(hipStreamWaitEvent(sub_stream_[k], ev_fork_, 0));
    }
    for (int k = 0; k < ns; ++k) {
        const Sub& sb = sub_[k];
        const int64_t r0 = sb.r0, t = sb.r1 - sb.r0;
        const hipStream_t s = sub_stream_[k];
        step("embed_norm", k, [&] {
            launch_embed_norm(s, embed_.w, d_ids_ + r0, t, std::sqrt(float(d)), layers_[0].attn_norm.as<float>(),
                              c.eps, x_.as<float>() + r0 * d, hn_.as<half_t>() + r0 * d);
        });
        if (P > 0) {
            // Per-layer inputs of every layer at once (engine.rs:1651-1666).
            const int64_t pw = P * c.layers;
            step("pl_in", k, [&] { launch_to_f16(s, x_.as<float>() + r0 * d, x16_.as<half_t>() + r0 * d, t * d); });
            step("mm_pl_model_proj", k, [&] {
                launch_gemm(s, x16_.as<half_t>() + r0 * d, d, pl_model_proj_.w, pli_.as<float>() + r0 * pw, pw, t);
            });
            step("pl_combine", k, [&] {
                launch_pl_combine(s, pl_table_.w, d_ids_ + r0, pl_proj_norm_.as<float>(), pli_.as<float>() + r0 * pw,
                                  t, P, c.layers, c.eps, 1.0f / std::sqrt(float(d)), std::sqrt(float(P)),
                                  1.0f / std::sqrt(2.0f));
            });
        }
    }
    const int64_t full_layers = out_rows_ ? out_layer_ + 1 : c.layers;
    for (int64_t l = 0; l < full_layers; ++l)
        for (int k = 0; k < ns; ++k) layer(l, k, base);
    if (ns > 1) {
        for (int k = 1; k < ns; ++k) {
            OMG_HIP(hipEventRecord(ev_join_[k], sub_stream_[k]));
            OMG_HIP(hipStreamWaitEvent(stream_, ev_join_[k], 0));
        }
    }
    // Past the last layer that writes K/V, the answer rows alone.
    if (tail_rows_ > 0)
        for (int64_t l = full_layers; l < c.layers; ++l) layer_tail(l);
}

// Layer l of range k (rows [r0, r1) of the pass, cache rows from base + r0).
void Engine::layer(int64_t l, int k, int64_t pass_base) {
    const Config& c = cfg_;
    const int64_t d = c.d, P = c.per_layer_dim;
    const Sub& sb = sub_[k];
    const int64_t r0 = sb.r0, t = sb.r1 - sb.r0, base = pass_base + r0;
    const hipStream_t s = sub_stream_[k];
    Layer& L = layers_[size_t(l)];
    const int64_t hd = c.head_dim[size_t(l)], qw = c.qkv_width(l), ff = c.ff[size_t(l)];
    // Range k's part of a per-row buffer starts at r0 rows of the buffer's
    // widest layer: widths vary by layer (Gemma 4: head_dim 256 / 512, the
    // double-wide MLP), and ranges run different layers at once, so
    // offsets of r0 rows of this layer's width would overlap a range still
    // on a narrower or wider layer.  Within the range rows are contiguous
    // at this layer's width.
    const int64_t qw_row = c.max_qkv(), hd_row = c.max_head_dim(), ff_row = c.max_ff();
    const int64_t src = c.kv_source[size_t(l)];
    half_t* hn = hn_.as<half_t>() + r0 * d;
    float* x = x_.as<float>() + r0 * d;
    QkArgs q{};
    q.qkv = qkv_.as<float>() + r0 * qw_row;
    q.qkv_stride = qw;
    q.meta = meta_.as<int32_t>();
    q.q_norm = L.q_norm.as<float>();
    q.k_norm = c.has_kv(l) ? L.k_norm.as<float>() : nullptr;
    q.rope = rope_tabs_[size_t(rope_of_[size_t(l)])].as<float2>();
    q.rope_rows = rope_rows_;
    q.rope_dims = c.rope_dims[size_t(l)];
    q.eps = c.eps;
    q.q_scale = c.query_scale;
    q.heads = int(c.heads);
    q.kv_heads = int(c.kv_heads);
    q.hd = int(hd);
    q.has_kv = c.has_kv(l);
    q.v_norm = c.v_norm;
    q.t = t;
    q.base = base;
    q.cap_pad = cap_pad_;
    q.q16 = q16_.as<half_t>() + r0 * c.heads * hd_row;
    q.kc = kc_[size_t(src)].as<half_t>();
    q.vt = vt_[size_t(src)].as<half_t>();
    if (hd == 256) {
        // qk_prep's norms, RoPE and cache writes in the product's epilogue
        step("mm_qkv", k, [&] { launch_gemm_qkprep(s, hn, d, L.qkv.w, q, t); });
    } else {
        step("mm_qkv", k, [&] { launch_gemm(s, hn, d, L.qkv.w, qkv_.as<float>() + r0 * qw_row, qw, t); });
        step("qk_prep", k, [&] { launch_qk_prep(s, q); });
    }
    if (nsub_ > 1) {
        // This range's K/V rows of layer l are in the cache; the later
        // ranges' attention reads them.
        if (k + 1 < nsub_) OMG_HIP(hipEventRecord(ev_kv_[size_t(k * c.layers + l)], s));
        for (int j = 0; j < k; ++j) OMG_HIP(hipStreamWaitEvent(s, ev_kv_[size_t(j * c.layers + l)], 0));
    }
    AttnArgs att{};
    att.q16 = q.q16;
    att.kc = q.kc;
    att.vt = q.vt;
    att.meta = meta_.as<int32_t>();
    att.out = attn_.as<half_t>() + r0 * c.heads * hd_row;
    att.t = t;
    att.base = base;
    att.cap_pad = cap_pad_;
    att.heads = int(c.heads);
    att.kv_heads = int(c.kv_heads);
    att.hd = int(hd);
    att.window = c.sliding[size_t(l)] ? int(c.window) : 0;
    att.part_o = part_o_.as<half_t>();
    att.part_ml = part_ml_.as<float>();
    const int kind = (c.sliding[size_t(l)] && c.window > 0) ? 0 : 1;
    const int nw = sb.work[kind].nw;
    if (out_rows_ && l == out_layer_) {
        // The last layer that writes K/V: attention for the query tiles of
        // the answer rows, then the rest on those rows alone.
        const int64_t ni = int64_t(sb.out_work.items.size()), nm = int64_t(sb.out_work.merges.size());
        if (ni > 0) step("attention_out", k, [&] { launch_attention(s, att, sb.d_out_items, ni, nw); });
        if (nm > 0) step("attention_merge_out", k, [&] { launch_attention_merge(s, att, sb.d_out_merges, nm, nw); });
        layer_out(k, att.out, x, r0);
        return;
    }
    step("attention", k, [&] { launch_attention(s, att, sb.d_items[kind], sb.n_items[kind], nw); });
    if (sb.n_merges[kind] > 0)
        step("attention_merge", k, [&] { launch_attention_merge(s, att, sb.d_merges[kind], sb.n_merges[kind], nw); });
    const SplitPlan po = split_plan(c.heads * hd, d, t), pd = split_plan(ff, d, t);
    const NormParts no = norm_parts(po, r0, t), nd = norm_parts(pd, r0, t);
    split_product("mm_o", k, att.out, c.heads * hd, L.o.w, r0, t, po);
    step("norm", k, [&] {
        launch_residual_norm(s, no.a, L.post_attn_norm.as<float>(), x, L.ffn_norm.as<float>(), hn, t, d, c.eps, 1.0f,
                             no.parts, no.stride, no.group);
    });
    half_t* act = act_.as<half_t>() + r0 * ff_row;
    step("mm_gate_up", k, [&] { launch_gemm_geglu(s, hn, d, L.gate.w, L.up.w, act, ff, t); });
    split_product("mm_down", k, act, ff, L.down.w, r0, t, pd);
    // The last layer's stream is normed at the wanted rows only (readout).
    const float* next = l + 1 < c.layers ? layers_[size_t(l + 1)].attn_norm.as<float>() : nullptr;
    half_t* next_hn = next ? hn : nullptr;
    if (P == 0) {
        step("norm", k, [&] {
            launch_residual_norm(s, nd.a, L.post_ffn_norm.as<float>(), x, next, next_hn, t, d, c.eps, 1.0f, nd.parts,
                                 nd.stride, nd.group);
        });
        return;
    }
    // Per-layer input block (engine.rs:1733-1750): the stream after the
    // feed-forward, as f16, gates the layer's slice of the inputs.
    half_t* x16 = x16_.as<half_t>() + r0 * d;
    step("norm", k, [&] {
        launch_residual_norm(s, nd.a, L.post_ffn_norm.as<float>(), x, nullptr, x16, t, d, c.eps, 1.0f, nd.parts,
                             nd.stride, nd.group);
    });
    float* plg = plg_.as<float>() + r0 * P;
    half_t* pl16 = pl16_.as<half_t>() + r0 * P;
    float* pli = pli_.as<float>() + r0 * P * c.layers;
    step("mm_pl_gate", k, [&] { launch_gemm(s, x16, d, L.pl_gate.w, plg, P, t); });
    step("pl_gate", k, [&] { launch_pl_gate(s, plg, pli, pl16, t, P, c.layers, l); });
    float* a = a_.as<float>() + r0 * d;
    step("mm_pl_proj", k, [&] { launch_gemm(s, pl16, P, L.pl_proj.w, a, d, t); });
    step("norm", k, [&] {
        launch_residual_norm(s, a, L.pl_norm.as<float>(), x, next, next_hn, t, d, c.eps, L.out_scale);
    });
}

// Range k's answer rows [w0, w1) through layer out_layer_ (the last that
// writes K/V) past its attention: gathered (attention output f16, stream
// f32, with per-layer inputs the rows' inputs of every layer) into rows
// w0.. of the answer-row buffers, then the rest of the layer on them.
void Engine::layer_out(int k, const half_t* attn, const float* x, int64_t r0) {
    const Config& c = cfg_;
    const Sub& sb = sub_[k];
    const int64_t n = sb.w1 - sb.w0;
    if (n == 0) return;
    const int64_t l = out_layer_, d = c.d, P = c.per_layer_dim;
    const int64_t W = c.heads * c.head_dim[size_t(l)];
    const hipStream_t s = sub_stream_[k];
    RowBufs b = row_bufs(sb.w0, W, c.ff[size_t(l)]);
    step("gather_out", k, [&] {
        launch_gather_out(s, attn, W, x, d, d_wanted_ + sb.w0, r0, n, b.aw, b.xw,
                          P > 0 ? pli_.as<float>() + r0 * P * c.layers : nullptr, P * c.layers, 0, P * c.layers,
                          b.pliw);
    });
    rows_post(l, k, s, n, b);
}

// The answer-row buffers from row w0 on, for a layer of attention width W
// and feed-forward width ff.
Engine::RowBufs Engine::row_bufs(int64_t w0, int64_t W, int64_t ff) {
    const Config& c = cfg_;
    const int64_t d = c.d, P = c.per_layer_dim;
    RowBufs b;
    b.aw = attn_w_.as<half_t>() + w0 * W;
    b.xw = x_w_.as<float>() + w0 * d;
    b.hw = hn_w_.as<half_t>() + w0 * d;
    b.actw = act_w_.as<half_t>() + w0 * ff;
    b.pw = a_w_.as<float>() + w0 * d;
    if (P > 0) {
        b.pliw = pli_w_.as<float>() + w0 * P * c.layers;
        b.x16w = x16_w_.as<half_t>() + w0 * d;
        b.plgw = plg_w_.as<float>() + w0 * P;
        b.pl16w = pl16_w_.as<half_t>() + w0 * P;
    }
    return b;
}

// Layer l past its attention on n gathered rows (attention output b.aw),
// on stream s: o, the residual norms, gate/up, down and the per-layer-input
// block, the last norm writing the next layer's normed rows to b.hw (after
// the model's last layer only the stream).  The products' K splits are the
// full pass's (a function of the shape); a deep product's K pieces run a
// workgroup each, their parts [splits x group][max_rows][d] in a_w_, and
// the norm adds them in the long pass's order.  Every step is per row and
// does not depend on the other rows of its launch, so the rows are those of
// the full layer.
void Engine::rows_post(int64_t l, int k, hipStream_t s, int64_t n, const RowBufs& b) {
    const Config& c = cfg_;
    const int64_t d = c.d, P = c.per_layer_dim;
    const Layer& L = layers_[size_t(l)];
    const int64_t W = c.heads * c.head_dim[size_t(l)], ff = c.ff[size_t(l)];
    const int64_t stride = max_rows_ * d;
    auto product = [&](const char* name, const half_t* in, int64_t kd, const DevWeight& w) {
        const SplitPlan p = split_plan(kd, d, n);
        const int parts = p.splits * p.group;
        step(name, k, [&] { launch_gemm_splitk(s, in, kd, w, b.pw, d, n, parts, stride); });
        return NormParts{b.pw, parts, stride, p.group};
    };
    const NormParts no = product("mm_o_out", b.aw, W, L.o.w);
    step("norm_out", k, [&] {
        launch_residual_norm(s, no.a, L.post_attn_norm.as<float>(), b.xw, L.ffn_norm.as<float>(), b.hw, n, d, c.eps,
                             1.0f, no.parts, no.stride, no.group);
    });
    step("mm_gate_up_out", k, [&] { launch_gemm_geglu(s, b.hw, d, L.gate.w, L.up.w, b.actw, ff, n); });
    const NormParts nd = product("mm_down_out", b.actw, ff, L.down.w);
    const float* next = l + 1 < c.layers ? layers_[size_t(l + 1)].attn_norm.as<float>() : nullptr;
    half_t* next_hn = next ? b.hw : nullptr;
    if (P == 0) {
        step("norm_out", k, [&] {
            launch_residual_norm(s, nd.a, L.post_ffn_norm.as<float>(), b.xw, next, next_hn, n, d, c.eps, 1.0f,
                                 nd.parts, nd.stride, nd.group);
        });
        return;
    }
    // The per-layer input block on the rows (as in layer()).
    step("norm_out", k, [&] {
        launch_residual_norm(s, nd.a, L.post_ffn_norm.as<float>(), b.xw, nullptr, b.x16w, n, d, c.eps, 1.0f,
                             nd.parts, nd.stride, nd.group);
    });
    step("mm_pl_gate_out", k, [&] { launch_gemm(s, b.x16w, d, L.pl_gate.w, b.plgw, P, n); });
    step("pl_gate_out", k, [&] { launch_pl_gate(s, b.plgw, b.pliw, b.pl16w, n, P, c.layers, l); });
    step("mm_pl_proj_out", k, [&] { launch_gemm(s, b.pl16w, P, L.pl_proj.w, b.pw, d, n); });
    step("norm_out", k, [&] {
        launch_residual_norm(s, b.pw, L.pl_norm.as<float>(), b.xw, next, next_hn, n, d, c.eps, L.out_scale);
    });
}

// Layer l after the last layer that writes K/V, on the answer rows alone
// (every range's, gathered by layer_out; their normed rows in hn_w_): no
// other row's output reaches them any more, since the layer's keys and
// values are an earlier layer's cache.  Its queries are those rows', with
// their own metadata (d_tail_meta_); the attention items are built over
// them alone.
void Engine::layer_tail(int64_t l) {
    const Config& c = cfg_;
    const int64_t n = tail_rows_, d = c.d;
    const hipStream_t s = stream_;
    Layer& L = layers_[size_t(l)];
    const int64_t hd = c.head_dim[size_t(l)], qw = c.qkv_width(l);
    const int64_t src = c.kv_source[size_t(l)];
    RowBufs b = row_bufs(0, c.heads * hd, c.ff[size_t(l)]);
    QkArgs q{};
    q.qkv = qkv_w_.as<float>();
    q.qkv_stride = qw;
    q.meta = d_tail_meta_;
    q.q_norm = L.q_norm.as<float>();
    q.k_norm = nullptr;
    q.rope = rope_tabs_[size_t(rope_of_[size_t(l)])].as<float2>();
    q.rope_rows = rope_rows_;
    q.rope_dims = c.rope_dims[size_t(l)];
    q.eps = c.eps;
    q.q_scale = c.query_scale;
    q.heads = int(c.heads);
    q.kv_heads = int(c.kv_heads);
    q.hd = int(hd);
    q.has_kv = false;
    q.v_norm = c.v_norm;
    q.t = n;
    q.base = 0;
    q.cap_pad = cap_pad_;
    q.q16 = q16_w_.as<half_t>();
    q.kc = kc_[size_t(src)].as<half_t>();
    q.vt = vt_[size_t(src)].as<half_t>();
    if (hd == 256) {
        step("mm_qkv_out", 0, [&] { launch_gemm_qkprep(s, b.hw, d, L.qkv.w, q, n); });
    } else {
        step("mm_qkv_out", 0, [&] { launch_gemm(s, b.hw, d, L.qkv.w, qkv_w_.as<float>(), qw, n); });
        step("qk_prep_out", 0, [&] { launch_qk_prep(s, q); });
    }
    AttnArgs att{};
    att.q16 = q.q16;
    att.kc = q.kc;
    att.vt = q.vt;
    att.meta = meta_.as<int32_t>();
    att.qmeta = d_tail_meta_;
    att.kend = tail_kend_;
    att.out = b.aw;
    att.t = n;
    att.base = 0;
    att.cap_pad = cap_pad_;
    att.heads = int(c.heads);
    att.kv_heads = int(c.kv_heads);
    att.hd = int(hd);
    att.window = c.sliding[size_t(l)] ? int(c.window) : 0;
    att.part_o = part_o_.as<half_t>();
    att.part_ml = part_ml_.as<float>();
    const int kind = (c.sliding[size_t(l)] && c.window > 0) ? 0 : 1;
    const AttnWork& w = tail_work_[kind];
    const int64_t ni = int64_t(w.items.size()), nm = int64_t(w.merges.size());
    if (ni > 0) step("attention_out", 0, [&] { launch_attention(s, att, d_tail_items_[kind], ni, w.nw); });
    if (nm > 0) step("attention_merge_out", 0, [&] { launch_attention_merge(s, att, d_tail_merges_[kind], nm, w.nw); });
    rows_post(l, 0, s, n, b);
}

void Engine::readout(const PassPlan& p) {
    if (p.nrows == 0) return;
    const Config& c = cfg_;
    // (after layer_out the answer rows' stream is x_w_, in wanted order)
    step("final_rows", 0, [&] {
        launch_final_rows(stream_, out_rows_ ? x_w_.as<float>() : x_.as<float>(), out_rows_ ? nullptr : d_wanted_,
                          p.nrows, c.d, final_norm_.as<float>(), c.eps, rows_.as<float>());
    });
    if (p.want == WANT_LOGITS) {
        step("logits", 0, [&] {
            launch_logits(stream_, embed_.w, rows_.as<float>(), p.nrows, nullptr, c.vocab, c.softcap,
                          logits_.as<float>());
        });
    } else if (p.want == WANT_LABELS) {
        step("logits", 0, [&] {
            launch_logits(stream_, embed_.w, rows_.as<float>(), p.nrows, d_labels_, p.nlabels,
                          c.softcap, logits_.as<float>());
        });
    } else if (p.want == WANT_LABELS_LSE) {
        // Readout::distribution (readout.rs:124-146) needs the label logits
        // and the log-sum-exp of the whole row: every logit is computed,
        // only k + 1 floats per row leave the device.
        step("logits", 0, [&] {
            launch_logits(stream_, embed_.w, rows_.as<float>(), p.nrows, nullptr, c.vocab, c.softcap,
                          logits_.as<float>(), lse_part_.as<float2>());
        });
        step("label_lse", 0, [&] {
            launch_label_lse(stream_, logits_.as<float>(), p.nrows, c.vocab, lse_part_.as<float2>(),
                             logits_blocks(c.vocab), d_labels_, p.nlabels, label_lse_.as<float>());
        });
    }
}

Engine::Run Engine::run_pass(const GroupIn* groups, int64_t n, int want, const uint32_t* labels, int64_t nlabels,
                             int64_t out_floats_needed, int64_t out_floats) {
    Run run;
    // This pass's upload moves the inputs a prepared pass reads (ids, meta,
    // work lists, labels): that pass is gone, and launching or reading it
    // fails until the next prepare.
    prepared_ = PassPlan{};
    auto [first, source] = admit(groups, n);
    run.first = first;
    run.source = source;
    run.pk = pack_checked(groups, n, first, source != SRC_NONE);
    if (out_floats_needed > out_floats)
        fail(E_INVALID, "output buffer holds " + std::to_string(out_floats) + " floats, " +
                            std::to_string(out_floats_needed) + " needed");
    const bool by_label = want == WANT_LABELS || want == WANT_LABELS_LSE;
    upload(run.pk, labels, by_label ? nlabels : 0);
    const int64_t t = run.pk.total - run.pk.base;
    forward(run.pk.base);
    readout(PassPlan{t, run.pk.base, int64_t(run.pk.wanted.size()), nlabels, want});
    return run;
}

void Engine::finish_pass(const GroupIn* groups, int64_t n, const Run& run, int* sources) {
    // engine.rs:1928-1939: cache rows 0..p0 now hold the first group's
    // prefix; every prefix decoded here goes to the state cache.
    const GroupIn& g0 = groups[run.first];
    resident_ = std::vector<uint32_t>(g0.prefix, g0.prefix + g0.prefix_len);
    for (const auto& dgrp : run.pk.decoded)
        remember(groups[dgrp.first].prefix, groups[dgrp.first].prefix_len, dgrp.second);
    const int source = run.source == SRC_NONE ? SRC_DECODED : run.source;
    if (sources)
        for (int64_t g = 0; g < n; ++g) sources[g] = g == run.first ? source : SRC_DECODED;
    last_source_ = source;
}

// Offsets of each group's and branch's first wanted row in the caller's
// (group, branch, want) order.
static void want_offsets(const GroupIn* groups, int64_t n, std::vector<int64_t>& goff,
                         std::vector<std::vector<int64_t>>& boff) {
    goff.assign(static_cast<size_t>(n) + 1, 0);
    boff.assign(static_cast<size_t>(n), {});
    for (int64_t g = 0; g < n; ++g) {
        int64_t acc = 0;
        for (int64_t b = 0; b < groups[g].nbranches; ++b) {
            boff[size_t(g)].push_back(acc);
            acc += groups[g].branches[b].nwant;
        }
        goff[size_t(g) + 1] = goff[size_t(g)] + acc;
    }
}

void Engine::evaluate_groups(const GroupIn* groups, int64_t n, int want, const uint32_t* labels,
                             int64_t nlabels, float* out, int64_t out_floats, int* sources) {
    if (n <= 0) fail(E_INVALID, "empty request");
    if (want != WANT_LOGITS && want != WANT_HIDDEN && want != WANT_LABELS && want != WANT_LABELS_LSE)
        fail(E_INVALID, "unknown want");
    const bool by_label = want == WANT_LABELS || want == WANT_LABELS_LSE;
    if (by_label && (nlabels <= 0 || !labels)) fail(E_INVALID, "label readout without label ids");
    const int64_t width = want == WANT_HIDDEN   ? cfg_.d
                          : want == WANT_LOGITS ? cfg_.vocab
                          : want == WANT_LABELS ? nlabels
                                                : nlabels + 1;
    int64_t nwant = 0;
    for (int64_t g = 0; g < n; ++g)
        for (int64_t b = 0; b < groups[g].nbranches; ++b) nwant += groups[g].branches[b].nwant;
    const Run run = run_pass(groups, n, want, labels, nlabels, nwant * width, out_floats);
    const Packed& pk = run.pk;
    const int64_t nrows = int64_t(pk.wanted.size());
    if (nrows) {
        const DevBuf& src = want == WANT_HIDDEN ? rows_ : want == WANT_LABELS_LSE ? label_lse_ : logits_;
        OMG_HIP(hipMemcpyAsync(h_out_, src.p, size_t(nrows * width) * 4, hipMemcpyDeviceToHost, stream_));
    }
    sync();
    // Dense output in the caller's (group, branch, want) order.
    std::vector<int64_t> goff;
    std::vector<std::vector<int64_t>> boff;
    want_offsets(groups, n, goff, boff);
    const float* h = static_cast<const float*>(h_out_);
    for (int64_t r = 0; r < nrows; ++r) {
        const auto& w = pk.wanted[size_t(r)];
        const int64_t dst = goff[size_t(w[0])] + boff[size_t(w[0])][size_t(w[1])] + w[2];
        std::memcpy(out + dst * width, h + r * width, size_t(width) * 4);
    }
    finish_pass(groups, n, run, sources);
}

void Engine::set_pointer_head(int64_t d, int64_t dp, const float* w_q, const float* b_q, const float* w_k,
                              const float* b_k) {
    if (!w_q) {  // no head
        ptr_dp_ = 0;
        return;
    }
    if (!b_q || !w_k || !b_k) fail(E_INVALID, "pointer head: null weight");
    if (d != cfg_.d) fail(E_INVALID, "pointer head: input width " + std::to_string(d) + ", model width " +
                                         std::to_string(cfg_.d));
    if (dp <= 0 || dp > 65536) fail(E_INVALID, "pointer head: projection width out of range");
    OMG_HIP(hipStreamSynchronize(stream_));  // a pass may still read the old head
    const size_t wb = size_t(dp * d) * 4, bb = size_t(dp) * 4;
    ptr_w_ = DevBuf(2 * wb);
    ptr_b_ = DevBuf(2 * bb);
    ptr_proj_ = DevBuf(size_t(max_rows_ * dp) * 4);
    if (!ptr_plan_.p) {
        const size_t plan = size_t((max_rows_ + 1) / 2 * 2) * 4 + size_t(max_rows_) * 8;
        ptr_plan_ = DevBuf(plan);
        ptr_out_ = DevBuf(size_t(max_rows_) * 4);
        OMG_HIP(hipHostMalloc(&h_ptr_, plan, hipHostMallocDefault));
    }
    OMG_HIP(hipMemcpy(ptr_w_.p, w_q, wb, hipMemcpyHostToDevice));
    OMG_HIP(hipMemcpy(ptr_w_.as<uint8_t>() + wb, w_k, wb, hipMemcpyHostToDevice));
    OMG_HIP(hipMemcpy(ptr_b_.p, b_q, bb, hipMemcpyHostToDevice));
    OMG_HIP(hipMemcpy(ptr_b_.as<uint8_t>() + bb, b_k, bb, hipMemcpyHostToDevice));
    ptr_dp_ = dp;
}

int64_t Engine::evaluate_pointer(const GroupIn* groups, int64_t n, const uint8_t* roles, int64_t nroles,
                                 float* out, int64_t out_floats, int* sources) {
    if (ptr_dp_ <= 0) fail(E_INVALID, "pointer readout without a pointer head");
    if (n <= 0) fail(E_INVALID, "empty request");
    std::vector<int64_t> goff;
    std::vector<std::vector<int64_t>> boff;
    want_offsets(groups, n, goff, boff);
    const int64_t nwant = goff[size_t(n)];
    if (nroles != nwant || (nwant && !roles))
        fail(E_INVALID, "pointer readout: " + std::to_string(nroles) + " roles for " + std::to_string(nwant) +
                            " wanted rows");
    // readout.rs:149-173 per branch: the `</opt>` rows in order and exactly
    // one `<decide>` row.
    int64_t nlogits = 0;
    for (int64_t g = 0; g < n; ++g)
        for (int64_t b = 0; b < groups[g].nbranches; ++b) {
            const uint8_t* r = roles + goff[size_t(g)] + boff[size_t(g)][size_t(b)];
            int decide = 0;
            for (int64_t s = 0; s < groups[g].branches[b].nwant; ++s) {
                if (r[s] > ROLE_DECIDE) fail(E_INVALID, "pointer readout: unknown role");
                decide += r[s] == ROLE_DECIDE;
                nlogits += r[s] == ROLE_OPT;
            }
            if (decide != 1) fail(E_INVALID, decide ? "pointer readout: more than one decide row" : "no decide row");
        }
    const Run run = run_pass(groups, n, WANT_HIDDEN, nullptr, 0, nlogits, out_floats);
    const Packed& pk = run.pk;
    const int64_t nrows = int64_t(pk.wanted.size());
    // The plan: per wanted row (workspace order) its map (0 = q for the
    // decide row, 1 = k for an option, -1 = none); per logit (caller order)
    // the option row and its branch's decide row.
    int32_t* mat = static_cast<int32_t*>(h_ptr_);
    const int64_t mat_slots = (max_rows_ + 1) / 2 * 2;  // the pairs start 8-byte aligned
    int2* pairs = reinterpret_cast<int2*>(mat + mat_slots);
    std::vector<int32_t> ws_row(size_t(nwant), -1);  // caller index -> workspace row
    for (int64_t r = 0; r < nrows; ++r) {
        const auto& w = pk.wanted[size_t(r)];
        const int64_t c = goff[size_t(w[0])] + boff[size_t(w[0])][size_t(w[1])] + w[2];
        ws_row[size_t(c)] = int32_t(r);
        mat[r] = roles[c] == ROLE_DECIDE ? 0 : roles[c] == ROLE_OPT ? 1 : -1;
    }
    int64_t k = 0;
    for (int64_t g = 0; g < n; ++g)
        for (int64_t b = 0; b < groups[g].nbranches; ++b) {
            const int64_t c0 = goff[size_t(g)] + boff[size_t(g)][size_t(b)], nw = groups[g].branches[b].nwant;
            int32_t decide = -1;
            for (int64_t s = 0; s < nw; ++s)
                if (roles[c0 + s] == ROLE_DECIDE) decide = ws_row[size_t(c0 + s)];
            for (int64_t s = 0; s < nw; ++s)
                if (roles[c0 + s] == ROLE_OPT) pairs[k++] = int2{ws_row[size_t(c0 + s)], decide};
        }
    int32_t* d_mat = ptr_plan_.as<int32_t>();
    int2* d_pairs = reinterpret_cast<int2*>(d_mat + mat_slots);
    OMG_HIP(hipMemcpyAsync(d_mat, mat, size_t(nrows) * 4, hipMemcpyHostToDevice, stream_));
    if (nlogits) OMG_HIP(hipMemcpyAsync(d_pairs, pairs, size_t(nlogits) * 8, hipMemcpyHostToDevice, stream_));
    step("pointer", 0, [&] {
        launch_pointer(stream_, rows_.as<float>(), nrows, cfg_.d, ptr_w_.as<float>(), ptr_b_.as<float>(), ptr_dp_,
                       d_mat, ptr_proj_.as<float>(), d_pairs, nlogits, ptr_out_.as<float>());
    });
    if (nlogits) OMG_HIP(hipMemcpyAsync(h_out_, ptr_out_.p, size_t(nlogits) * 4, hipMemcpyDeviceToHost, stream_));
    sync();
    if (nlogits) std::memcpy(out, h_out_, size_t(nlogits) * 4);
    finish_pass(groups, n, run, sources);
    return nlogits;
}

void Engine::warmup() {
    const uint32_t bos = cfg_.bos < uint32_t(cfg_.vocab) ? cfg_.bos : 0;
    const uint32_t tok = 0, want = 0;
    BranchIn b{&tok, 1, &want, 1};
    GroupIn g{&bos, 1, &b, 1};
    std::vector<float> out(size_t(cfg_.vocab));
    evaluate_groups(&g, 1, WANT_LOGITS, nullptr, 0, out.data(), int64_t(out.size()), nullptr);
}

void Engine::prepare(const GroupIn* groups, int64_t n, int want, const uint32_t* labels, int64_t nlabels,
                     bool resident_first) {
    if (n <= 0) fail(E_INVALID, "empty request");
    if (want != WANT_LOGITS && want != WANT_HIDDEN && want != WANT_LABELS && want != WANT_LABELS_LSE)
        fail(E_INVALID, "unknown want");
    const bool by_label = want == WANT_LABELS || want == WANT_LABELS_LSE;
    if (by_label && (nlabels <= 0 || !labels)) fail(E_INVALID, "label readout without label ids");
    if (resident_first && !is_resident(groups[0].prefix, groups[0].prefix_len))
        fail(E_INVALID, "prepare: group 0's prefix is not resident");
    Packed pk = pack_checked(groups, n, 0, resident_first);
    upload(pk, labels, by_label ? nlabels : 0);
    prepared_ = PassPlan{pk.total - pk.base, pk.base, int64_t(pk.wanted.size()), nlabels, want};
    sync();
}

void Engine::launch_prepared() {
    if (prepared_.t <= 0) fail(E_INVALID, "no prepared pass");
    if (graph_exec_ && !profile_) {
        OMG_HIP(hipGraphLaunch(graph_exec_, stream_));
        return;
    }
    forward(prepared_.base);
    readout(prepared_);
}

// The pass is kernels only (no copies or memsets between prepare and the
// readout), so its captured graph replays exactly the launches above; the
// work lists and buffers it reads stay where prepare put them until the
// next prepare or evaluate, which drops the graph.
void Engine::set_graph(bool on) {
    drop_graph();
    if (!on) return;
    if (prepared_.t <= 0) fail(E_INVALID, "no prepared pass");
    if (profile_) fail(E_INVALID, "graph capture while profiling");
    sync();
    hipGraph_t g = nullptr;
    OMG_HIP(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal));
    try {
        forward(prepared_.base);
        readout(prepared_);
    } catch (...) {
        (void)hipStreamEndCapture(stream_, &g);
        if (g) (void)hipGraphDestroy(g);
        throw;
    }
    OMG_HIP(hipStreamEndCapture(stream_, &g));
    const hipError_t err = hipGraphInstantiate(&graph_exec_, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (err != hipSuccess) {
        graph_exec_ = nullptr;
        fail(E_DEVICE, std::string("hipGraphInstantiate: ") + hipGetErrorString(err));
    }
}

int64_t Engine::read_prepared(float* out, int64_t out_floats) {
    const PassPlan& p = prepared_;
    if (p.t <= 0) fail(E_INVALID, "no prepared pass");
    const int64_t width = p.want == WANT_HIDDEN   ? cfg_.d
                          : p.want == WANT_LOGITS ? cfg_.vocab
                          : p.want == WANT_LABELS ? p.nlabels
                                                  : p.nlabels + 1;
    if (p.nrows * width > out_floats) fail(E_INVALID, "output buffer too small for the prepared pass's rows");
    const DevBuf& src = p.want == WANT_HIDDEN ? rows_ : p.want == WANT_LABELS_LSE ? label_lse_ : logits_;
    sync();
    if (p.nrows) OMG_HIP(hipMemcpy(out, src.p, size_t(p.nrows * width) * 4, hipMemcpyDeviceToHost));
    return p.nrows * width;
}

void Engine::drop_graph() {
    if (graph_exec_) {
        (void)hipStreamSynchronize(stream_);
        (void)hipGraphExecDestroy(graph_exec_);
        graph_exec_ = nullptr;
    }
}

// ----------------------------------------------------------- state cache

void Engine::set_state_cache(size_t bytes, const std::string& dir, const std::string& model_id) {
    states_ = StateCache{};
    states_.budget = bytes;
    state_dir_ = dir;
    model_id_ = model_id;
}

SavedState Engine::save_state_at(const uint32_t* prefix, int64_t p, int64_t row0) {
    const Config& c = cfg_;
    if (row0 + p > slots_) fail(E_INVALID, "state rows outside the cache");
    SavedState s;
    s.prefix.assign(prefix, prefix + p);
    stage_state(p, row0);
    size_t off = 0;
    for (int64_t l = 0; l < c.layers; ++l) {
        if (!c.has_kv(l)) continue;
        const auto [r0, r1] = state_rows(l, p);
        const size_t n = size_t((r1 - r0) * 2 * c.kv_heads * c.head_dim[size_t(l)] * 2);
        const uint8_t* src = static_cast<const uint8_t*>(h_state_) + off;
        s.layers.push_back(SavedState::Layer{uint32_t(l), uint32_t(r0), std::vector<uint8_t>(src, src + n)});
        off += n;
    }
    return s;
}

std::pair<uint8_t*, size_t> Engine::save_state_bytes(const uint32_t* prefix, int64_t p, const std::string& model_id) {
    const Config& c = cfg_;
    if (p > capacity_) fail(E_INVALID, "state rows outside the cache");
    const size_t staged = stage_state(p, 0);
    int64_t nl = 0;
    for (int64_t l = 0; l < c.layers; ++l) nl += c.has_kv(l);
    const size_t len = 6 + 4 + model_id.size() + 4 + 4 * size_t(p) + 4 + 12 * size_t(nl) + staged;
    uint8_t* out = static_cast<uint8_t*>(std::malloc(len));
    if (!out) fail(E_INVALID, "out of host memory");
    uint8_t* w = out;
    auto u32 = [&](uint32_t v) {
        for (int i = 0; i < 4; ++i) *w++ = uint8_t(v >> (8 * i));
    };
    const char magic[6] = {'G', 'R', 'W', 'S', '1', '\0'};
    std::memcpy(w, magic, 6);
    w += 6;
    u32(uint32_t(model_id.size()));
    std::memcpy(w, model_id.data(), model_id.size());
    w += model_id.size();
    u32(uint32_t(p));
    for (int64_t i = 0; i < p; ++i) u32(prefix[i]);
    u32(uint32_t(nl));
    size_t off = 0;
    for (int64_t l = 0; l < c.layers; ++l) {
        if (!c.has_kv(l)) continue;
        const auto [r0, r1] = state_rows(l, p);
        const size_t n = size_t((r1 - r0) * 2 * c.kv_heads * c.head_dim[size_t(l)] * 2);
        u32(uint32_t(l));
        u32(uint32_t(r0));
        u32(uint32_t(n));
        std::memcpy(w, static_cast<const uint8_t*>(h_state_) + off, n);
        w += n;
        off += n;
    }
    return {out, len};
}

size_t Engine::stage_state(int64_t p, int64_t row0) {
    const Config& c = cfg_;
    sync();
    // Every layer's rows are gathered into the device stage and copied to
    // the pinned staging buffer in stream order (a layer's gather waits for
    // the previous copy), then synchronised once.
    size_t off = 0;
    for (int64_t l = 0; l < c.layers; ++l) {
        if (!c.has_kv(l)) continue;
        const auto [r0, r1] = state_rows(l, p);
        const int64_t hd = c.head_dim[size_t(l)];
        const size_t n = size_t((r1 - r0) * 2 * c.kv_heads * hd * 2);
        if (off + n > h_state_bytes_) fail(E_STATE, "state larger than the staging buffer");
        if (n) {
            launch_kv_gather(stream_, kc_[size_t(l)].as<half_t>(), vt_[size_t(l)].as<half_t>(), cap_pad_,
                             int(c.kv_heads), int(hd), row0 + r0, r1 - r0, kv_stage_.as<half_t>());
            OMG_HIP(hipMemcpyAsync(static_cast<uint8_t*>(h_state_) + off, kv_stage_.p, n, hipMemcpyDeviceToHost,
                                   stream_));
        }
        off += n;
    }
    OMG_HIP(hipStreamSynchronize(stream_));
    return off;
}

void Engine::restore_state(const SavedState& s) {
    const Config& c = cfg_;
    const int64_t p = int64_t(s.prefix.size());
    if (p > capacity_)
        fail(E_STATE, "state of " + std::to_string(p) + " tokens exceeds the engine capacity " + std::to_string(capacity_));
    for (const SavedState::Layer& L : s.layers) {
        const int64_t l = L.layer;
        if (l >= c.layers || !c.has_kv(l))
            fail(E_STATE, "state has K/V for layer " + std::to_string(l) + ", which owns none");
    }
    sync();
    for (const SavedState::Layer& L : s.layers) {
        const int64_t l = L.layer, hd = c.head_dim[size_t(l)];
        const int64_t row_bytes = 2 * c.kv_heads * hd * 2;
        const auto [r0, r1] = state_rows(l, p);
        if (int64_t(L.row0) != r0 || int64_t(L.bytes.size()) != (r1 - r0) * row_bytes)
            fail(E_STATE, "state layer " + std::to_string(l) + ": " + std::to_string(L.bytes.size()) + " bytes at row " +
                              std::to_string(L.row0) + ", expected " + std::to_string((r1 - r0) * row_bytes) +
                              " at " + std::to_string(r0));
    }
    // All layers' rows into the pinned staging buffer, then per layer a
    // copy to the device stage and the scatter into the cache, in stream
    // order (a layer's copy waits for the previous scatter); one sync.
    size_t total = 0;
    for (const SavedState::Layer& L : s.layers) total += L.bytes.size();
    if (total > h_state_bytes_) fail(E_STATE, "state larger than the staging buffer");
    // The cache rows and their metadata change from here on: no prefix is
    // resident until the restore completes, and a prepared pass (which may
    // read those rows) is gone.
    resident_.reset();
    prepared_ = PassPlan{};
    drop_graph();
    size_t off = 0;
    for (const SavedState::Layer& L : s.layers) {
        std::memcpy(static_cast<uint8_t*>(h_state_) + off, L.bytes.data(), L.bytes.size());
        off += L.bytes.size();
    }
    off = 0;
    for (const SavedState::Layer& L : s.layers) {
        const int64_t l = L.layer, hd = c.head_dim[size_t(l)];
        const auto [r0, r1] = state_rows(l, p);
        if (r1 > r0) {
            OMG_HIP(hipMemcpyAsync(kv_stage_.p, static_cast<const uint8_t*>(h_state_) + off, L.bytes.size(),
                                   hipMemcpyHostToDevice, stream_));
            launch_kv_scatter(stream_, kc_[size_t(l)].as<half_t>(), vt_[size_t(l)].as<half_t>(), cap_pad_,
                              int(c.kv_heads), int(hd), r0, r1 - r0, kv_stage_.as<half_t>());
        }
        off += L.bytes.size();
    }
    OMG_HIP(hipStreamSynchronize(stream_));
    std::vector<int32_t> meta(size_t(4 * p));
    for (int64_t i = 0; i < p; ++i) {
        meta[size_t(4 * i)] = int32_t(i);
        meta[size_t(4 * i + 1)] = 0;
        meta[size_t(4 * i + 2)] = 0;
        meta[size_t(4 * i + 3)] = int32_t(i + 1);
    }
    if (p) OMG_HIP(hipMemcpy(meta_.p, meta.data(), meta.size() * 4, hipMemcpyHostToDevice));
    resident_ = s.prefix;
}

int Engine::restore_from_cache(const uint32_t* prefix, int64_t n) {
    if (n == 0 || !(states_.budget > 0 || !state_dir_.empty())) return SRC_NONE;
    const std::vector<uint32_t> key(prefix, prefix + n);
    if (auto s = states_.get(key)) {
        try {
            restore_state(*s);
            return SRC_RAM;
        } catch (const Error&) {
            return SRC_NONE;
        }
    }
    if (state_dir_.empty()) return SRC_NONE;
    char name[64];
    std::snprintf(name, sizeof name, "/%016llx.state", (unsigned long long)state_key(model_id_, prefix, n));
    std::ifstream f(state_dir_ + name, std::ios::binary);
    if (!f) return SRC_NONE;
    std::vector<uint8_t> bytes((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
    try {
        SavedState s = SavedState::from_bytes(bytes.data(), bytes.size(), model_id_);
        if (s.prefix != key) return SRC_NONE;
        restore_state(s);
        states_.put(std::move(s));
        return SRC_DISK;
    } catch (const Error&) {
        return SRC_NONE;
    }
}

void Engine::remember(const uint32_t* prefix, int64_t n, int64_t row0) {
    if (n == 0 || !(states_.budget > 0 || !state_dir_.empty())) return;
    SavedState s = save_state_at(prefix, n, row0);
    if (!state_dir_.empty()) {
        ::mkdir(state_dir_.c_str(), 0755);
        char name[64];
        std::snprintf(name, sizeof name, "/%016llx.state", (unsigned long long)state_key(model_id_, prefix, n));
        const std::vector<uint8_t> bytes = s.to_bytes(model_id_);
        std::ofstream f(state_dir_ + name, std::ios::binary);
        if (!f) fail(E_IO, "writing " + state_dir_ + name);
        f.write(reinterpret_cast<const char*>(bytes.data()), std::streamsize(bytes.size()));
    }
    states_.put(std::move(s));
}

}  // namespace omg
