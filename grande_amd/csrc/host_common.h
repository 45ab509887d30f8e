// Host-side helpers with no HIP dependency: error reporting across the C
// ABI and IEEE half conversion on the host.  The parsers and the state
// format build from this alone (also into the CPU sanitizer harness).
#pragma once

#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>

namespace omg {

// Every failure inside the library is an omg::Error; the C ABI catches it,
// stores the message in a thread-local slot and returns the status code.
struct Error : std::runtime_error {
    int code;
    Error(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

enum Status {
    OK = 0,
    E_INVALID = -1,   // bad argument / request (engine.rs:1503-1581 bail!s)
    E_CAPACITY = -2,  // capacity / max_rows / branch-count limits
    E_DEVICE = -3,    // HIP runtime failure
    E_STATE = -4,     // state bytes rejected (engine.rs:536-579)
    E_IO = -5,        // file system
    E_MISSING = -6,   // tensors missing at finish
};

[[noreturn]] inline void fail(int code, const std::string& msg) { throw Error(code, msg); }


// IEEE binary16 <-> binary32 on the host, round to nearest even; the scale
// rounding of model.rs:418-419,452.
inline uint16_t f32_to_f16(float x) {
    uint32_t u;
    std::memcpy(&u, &x, 4);
    const uint32_t sign = (u >> 16) & 0x8000u;
    const int32_t exp = int32_t((u >> 23) & 0xffu);
    uint32_t man = u & 0x7fffffu;
    if (exp == 0xff) return uint16_t(sign | 0x7c00u | (man ? 0x200u | (man >> 13) : 0u));
    const int32_t e = exp - 112;  // rebias 127 -> 15
    if (e >= 31) return uint16_t(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return uint16_t(sign);
        const uint32_t full = man | 0x800000u;
        const int sh = 14 - e;
        uint32_t h = full >> sh;
        const uint32_t rest = full & ((1u << sh) - 1u), mid = 1u << (sh - 1);
        if (rest > mid || (rest == mid && (h & 1u))) ++h;
        return uint16_t(sign | h);
    }
    uint32_t h = sign | (uint32_t(e) << 10) | (man >> 13);
    const uint32_t rest = man & 0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) ++h;
    return uint16_t(h);
}

inline float f16_to_f32(uint16_t h) {
    const uint32_t sign = uint32_t(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu, man = h & 0x3ffu, u;
    if (exp == 0) {
        if (man == 0) {
            u = sign;
        } else {
            int sh = 0;
            while (!(man & 0x400u)) {
                man <<= 1;
                ++sh;
            }
            u = sign | (uint32_t(113 - sh) << 23) | ((man & 0x3ffu) << 13);
        }
    } else if (exp == 31) {
        u = sign | 0x7f800000u | (man << 13);
    } else {
        u = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

}  // namespace omg
