// Request packing and the state format: host-only parts of
// crates/omg-wgpu/src/engine.rs (no device code), shared by the engine and
// the CPU sanitizer harness of the parsers.
#pragma once

#include <array>
#include <cstdint>
#include <optional>
#include <string>
#include <utility>
#include <vector>

#include "host_common.h"

namespace omg {

// engine.rs:21-24: bits of a sequence id that number the branch; the bits
// above number the group within the pass.
constexpr int SEQ_GROUP_SHIFT = 12;

struct BranchIn {
    const uint32_t* tokens;
    int64_t ntokens;
    const uint32_t* want;
    int64_t nwant;
};
struct GroupIn {
    const uint32_t* prefix;
    int64_t prefix_len;
    const BranchIn* branches;
    int64_t nbranches;
};

// One pass's packed layout (engine.rs:1512-1571).
struct Packed {
    int64_t base = 0, total = 0;
    std::vector<uint32_t> ids;
    std::vector<int32_t> meta;                        // 4 per token: pos, seq, first key row, row + 1
    std::vector<std::array<int64_t, 4>> wanted;       // group, branch, slot, workspace row
    std::vector<std::pair<int64_t, int64_t>> decoded; // group, cache row of its prefix
};
// Order: `first`, then the other groups in order (engine.rs:1479-1482).
Packed pack_groups(const GroupIn* groups, int64_t n, int64_t first, bool resident);

// The engine's own layout on top of the reference's: every layout group
// after the first starts at a cache row that is a multiple of `align` (the
// attention kernel's key tile and query tile, so a group meets its keys in
// the same tiles as when it runs alone and no query tile holds two
// groups), with padding rows between (token 0, sequence id -1: a group no
// query belongs to, so nothing sees them).  Wanted and decoded rows move
// with their groups.  Returns the packing unchanged when the padded pass
// would need more than `rows` cache rows.
Packed align_groups(const Packed& pk, int64_t align, int64_t rows);

// engine.rs:503-580: a prefix's K/V rows as f16 per layer that owns K/V.
struct SavedState {
    std::vector<uint32_t> prefix;
    struct Layer {
        uint32_t layer, row0;
        std::vector<uint8_t> bytes;
    };
    std::vector<Layer> layers;
    size_t byte_len() const;
    std::vector<uint8_t> to_bytes(const std::string& model_id) const;
    static SavedState from_bytes(const uint8_t* b, size_t n, const std::string& model_id);
};

// engine.rs:582-620: LRU keyed by the exact prefix, most recent last.
struct StateCache {
    size_t budget = 0, used = 0;
    std::vector<SavedState> entries;
    std::optional<SavedState> get(const std::vector<uint32_t>& prefix);
    void put(SavedState s);
};

uint64_t state_key(const std::string& model_id, const uint32_t* prefix, int64_t n);  // engine.rs:625-641

}  // namespace omg
