// Request packing (engine.rs:1512-1571) and the GRWS1 state bytes, state
// LRU and state key (engine.rs:503-641): host code only.
#include "state.h"

#include <cstring>

namespace omg {

// ------------------------------------------------------------------ pack

Packed pack_groups(const GroupIn* groups, int64_t n, int64_t first, bool resident) {
    Packed pk;
    for (int64_t g = 0; g < n; ++g) {
        pk.total += groups[g].prefix_len;
        for (int64_t b = 0; b < groups[g].nbranches; ++b) pk.total += groups[g].branches[b].ntokens;
    }
    if (n == 0 || pk.total == 0) fail(E_INVALID, "empty request");
    const int64_t p0 = groups[first].prefix_len;
    pk.base = resident ? p0 : 0;
    pk.ids.reserve(size_t(pk.total - pk.base));
    pk.meta.reserve(size_t(4 * (pk.total - pk.base)));
    auto push = [&](int64_t pos, int32_t seq, int64_t row_lo, uint32_t tok) {
        const int64_t row = pk.base + int64_t(pk.ids.size());
        pk.meta.push_back(int32_t(pos));
        pk.meta.push_back(seq);
        pk.meta.push_back(int32_t(row_lo));
        pk.meta.push_back(int32_t(row + 1));
        pk.ids.push_back(tok);
    };
    for (int64_t k = 0; k < n; ++k) {
        const int64_t gi = k == 0 ? first : (k <= first ? k - 1 : k);
        const GroupIn& g = groups[gi];
        if (g.nbranches >= (int64_t(1) << SEQ_GROUP_SHIFT))
            fail(E_CAPACITY, std::to_string(g.nbranches) + " branches in one group; the engine addresses at most " +
                                 std::to_string((1 << SEQ_GROUP_SHIFT) - 1));
        const int32_t seq_hi = int32_t(k << SEQ_GROUP_SHIFT);
        const int64_t row_lo = k == 0 ? 0 : pk.base + int64_t(pk.ids.size());
        if (!(k == 0 && pk.base > 0)) {
            pk.decoded.push_back({gi, pk.base + int64_t(pk.ids.size())});
            for (int64_t i = 0; i < g.prefix_len; ++i) push(i, seq_hi, row_lo, g.prefix[i]);
        }
        for (int64_t bi = 0; bi < g.nbranches; ++bi) {
            const BranchIn& b = g.branches[bi];
            const int64_t start = int64_t(pk.ids.size());
            for (int64_t j = 0; j < b.ntokens; ++j)
                push(g.prefix_len + j, seq_hi | int32_t(bi + 1), row_lo, b.tokens[j]);
            for (int64_t s = 0; s < b.nwant; ++s) {
                if (int64_t(b.want[s]) >= b.ntokens)
                    fail(E_INVALID, "branch " + std::to_string(bi) + ": wanted position " + std::to_string(b.want[s]) +
                                        " past its " + std::to_string(b.ntokens) + " tokens");
                pk.wanted.push_back({gi, bi, s, start + int64_t(b.want[s])});
            }
        }
    }
    return pk;
}

// ----------------------------------------------------------------- state

size_t SavedState::byte_len() const {
    size_t n = prefix.size() * 4;
    for (const Layer& l : layers) n += l.bytes.size();
    return n;
}

static void put_u32(std::vector<uint8_t>& o, uint32_t v) {
    for (int i = 0; i < 4; ++i) o.push_back(uint8_t(v >> (8 * i)));
}

std::vector<uint8_t> SavedState::to_bytes(const std::string& model_id) const {
    std::vector<uint8_t> out;
    out.reserve(byte_len() + 64 + model_id.size());
    const char magic[6] = {'G', 'R', 'W', 'S', '1', '\0'};
    out.insert(out.end(), magic, magic + 6);
    put_u32(out, uint32_t(model_id.size()));
    out.insert(out.end(), model_id.begin(), model_id.end());
    put_u32(out, uint32_t(prefix.size()));
    for (uint32_t t : prefix) put_u32(out, t);
    put_u32(out, uint32_t(layers.size()));
    for (const Layer& l : layers) {
        put_u32(out, l.layer);
        put_u32(out, l.row0);
        put_u32(out, uint32_t(l.bytes.size()));
        out.insert(out.end(), l.bytes.begin(), l.bytes.end());
    }
    return out;
}

SavedState SavedState::from_bytes(const uint8_t* b, size_t n, const std::string& model_id) {
    size_t at = 0;
    auto take = [&](size_t k) {
        if (at + k > n) fail(E_STATE, "state file truncated");
        const uint8_t* p = b + at;
        at += k;
        return p;
    };
    auto u32 = [&]() {
        const uint8_t* p = take(4);
        return uint32_t(p[0]) | uint32_t(p[1]) << 8 | uint32_t(p[2]) << 16 | uint32_t(p[3]) << 24;
    };
    if (std::memcmp(take(6), "GRWS1\0", 6) != 0) fail(E_STATE, "not a omg state file");
    const uint32_t idn = u32();
    const uint8_t* id = take(idn);
    if (std::string(reinterpret_cast<const char*>(id), idn) != model_id)
        fail(E_STATE, "state file is for a different model");
    SavedState s;
    const uint32_t np = u32();
    const uint8_t* pp = take(size_t(np) * 4);
    for (uint32_t i = 0; i < np; ++i)
        s.prefix.push_back(uint32_t(pp[4 * i]) | uint32_t(pp[4 * i + 1]) << 8 | uint32_t(pp[4 * i + 2]) << 16 |
                           uint32_t(pp[4 * i + 3]) << 24);
    const uint32_t nl = u32();
    for (uint32_t i = 0; i < nl; ++i) {
        Layer l;
        l.layer = u32();
        l.row0 = u32();
        const uint32_t len = u32();
        const uint8_t* d = take(len);
        l.bytes.assign(d, d + len);
        s.layers.push_back(std::move(l));
    }
    return s;
}

std::optional<SavedState> StateCache::get(const std::vector<uint32_t>& prefix) {
    for (size_t i = 0; i < entries.size(); ++i) {
        if (entries[i].prefix == prefix) {
            SavedState s = std::move(entries[i]);
            entries.erase(entries.begin() + long(i));
            entries.push_back(s);
            return s;
        }
    }
    return std::nullopt;
}

void StateCache::put(SavedState s) {
    const size_t len = s.byte_len();
    if (len > budget) return;
    for (size_t i = 0; i < entries.size(); ++i)
        if (entries[i].prefix == s.prefix) {
            used -= entries[i].byte_len();
            entries.erase(entries.begin() + long(i));
            break;
        }
    while (used + len > budget && !entries.empty()) {
        used -= entries.front().byte_len();
        entries.erase(entries.begin());
    }
    used += len;
    entries.push_back(std::move(s));
}

uint64_t state_key(const std::string& model_id, const uint32_t* prefix, int64_t n) {
    uint64_t h = 0xcbf29ce484222325ull;
    auto eat = [&](uint8_t b) {
        h ^= b;
        h *= 0x00000100000001b3ull;
    };
    for (char c : model_id) eat(uint8_t(c));
    eat(0);
    for (int64_t i = 0; i < n; ++i)
        for (int s = 0; s < 4; ++s) eat(uint8_t(prefix[i] >> (8 * s)));
    return h;
}

// ----------------------------------------------------------- alignment

Packed align_groups(const Packed& pk, int64_t align, int64_t rows) {
    const int64_t n = int64_t(pk.ids.size());
    if (align <= 1 || n == 0) return pk;
    // New pass index of every token: groups after the first move up to the
    // next multiple of `align` (absolute cache row, the base included).
    std::vector<int64_t> at(static_cast<size_t>(n));
    int64_t used = 0, group = pk.meta[1] >> SEQ_GROUP_SHIFT;
    for (int64_t i = 0; i < n; ++i) {
        const int64_t k = pk.meta[size_t(4 * i + 1)] >> SEQ_GROUP_SHIFT;
        if (k != group) {
            group = k;
            const int64_t row = pk.base + used;
            used += (align - row % align) % align;
        }
        at[size_t(i)] = used++;
    }
    if (pk.base + used > rows || used == n) return pk;
    Packed out;
    out.base = pk.base;
    out.total = pk.base + used;
    out.ids.assign(size_t(used), 0u);
    out.meta.resize(size_t(4 * used));
    for (int64_t j = 0; j < used; ++j) {
        // padding: position 0, no group, its own first key row
        const int64_t row = pk.base + j;
        out.meta[size_t(4 * j)] = 0;
        out.meta[size_t(4 * j + 1)] = -1;
        out.meta[size_t(4 * j + 2)] = int32_t(row);
        out.meta[size_t(4 * j + 3)] = int32_t(row + 1);
    }
    // a group's first key row moves with its first token
    int64_t lo_old = -1, lo_new = -1;
    for (int64_t i = 0; i < n; ++i) {
        const int64_t j = at[size_t(i)], row = pk.base + j;
        const int32_t* m = &pk.meta[size_t(4 * i)];
        if (m[2] != lo_old) {
            lo_old = m[2];
            // the first group's key rows start at 0 (its resident prefix)
            lo_new = lo_old < pk.base ? lo_old : pk.base + at[size_t(lo_old - pk.base)];
        }
        out.ids[size_t(j)] = pk.ids[size_t(i)];
        out.meta[size_t(4 * j)] = m[0];
        out.meta[size_t(4 * j + 1)] = m[1];
        out.meta[size_t(4 * j + 2)] = int32_t(lo_new);
        out.meta[size_t(4 * j + 3)] = int32_t(row + 1);
    }
    for (const auto& w : pk.wanted) out.wanted.push_back({w[0], w[1], w[2], at[size_t(w[3])]});
    // A group with no tokens at the end of the pass records the row past
    // the last token: it maps to the row past the new layout.
    for (const auto& d : pk.decoded) {
        const int64_t i = d.second - pk.base;
        out.decoded.push_back({d.first, pk.base + (i < n ? at[size_t(i)] : used)});
    }
    return out;
}

}  // namespace omg
