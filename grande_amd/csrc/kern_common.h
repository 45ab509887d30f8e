// Device-side helpers shared by the gfx950 kernels: vector types for the
// MFMA builtins, wave64 reductions and the weight decoders.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "kernels.h"

namespace omg {

typedef half_t half8 __attribute__((ext_vector_type(8)));
typedef half_t half4 __attribute__((ext_vector_type(4)));
typedef half_t half2v __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int WAVE = 64;


__device__ inline float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, WAVE));
    return v;
}

// Max over the four lanes l, l ^ 16, l ^ 32, l ^ 48 (one row of an MFMA
// 16x16 result) without LDS: v_permlane16_swap / v_permlane32_swap with both
// operands the same value return the pair {x[l], x[l ^ 16]} (resp. ^ 32).
__device__ inline float max_lanes_16_32(float v) {
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    const auto p = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    const float m = fmaxf(__builtin_bit_cast(float, uint32_t(p[0])), __builtin_bit_cast(float, uint32_t(p[1])));
    const uint32_t w = __builtin_bit_cast(uint32_t, m);
    const auto q = __builtin_amdgcn_permlane32_swap(w, w, false, false);
    return fmaxf(__builtin_bit_cast(float, uint32_t(q[0])), __builtin_bit_cast(float, uint32_t(q[1])));
}

// Sum over the same four lanes.
__device__ inline float sum_lanes_16_32(float v) {
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    const auto p = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    const float m = __builtin_bit_cast(float, uint32_t(p[0])) + __builtin_bit_cast(float, uint32_t(p[1]));
    const uint32_t w = __builtin_bit_cast(uint32_t, m);
    const auto q = __builtin_amdgcn_permlane32_swap(w, w, false, false);
    return __builtin_bit_cast(float, uint32_t(q[0])) + __builtin_bit_cast(float, uint32_t(q[1]));
}

// Sum over the wave, the same bits in every lane: within each row of 16
// lanes by DPP (quad swaps, then half-row and row mirrors: each step adds
// two equal-shaped partial sums, so lanes that pair up get the same result),
// then across rows with the permlane swaps above.  No LDS round trips.
template <int CTRL>
__device__ inline float dpp_f32(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
__device__ inline float wave_sum(float v) {
    v += dpp_f32<0xb1>(v);   // quad_perm [1, 0, 3, 2]
    v += dpp_f32<0x4e>(v);   // quad_perm [2, 3, 0, 1]
    v += dpp_f32<0x141>(v);  // row_half_mirror
    v += dpp_f32<0x140>(v);  // row_mirror
    return sum_lanes_16_32(v);
}

// f16 of an f32 value that is first rounded to f32: the empty asm hides
// the producing multiply from the conversion, which the compiler may
// otherwise fuse into one mixed-precision FMA (a single rounding to f16)
// in some template instances and not in others.
__device__ inline half_t f16_rounded(float v) {
    asm("" : "+v"(v));
    return half_t(v);
}

__device__ inline float half_bits_to_f32(uint16_t h) {
    return float(__builtin_bit_cast(half_t, h));
}

__device__ inline half2v as_half2(uint32_t u) { return __builtin_bit_cast(half2v, u); }

// (a & mask) | bits in one instruction (gfx9 VOP3 encodings take no
// literal and one scalar operand: the mask sits in a VGPR, the bits in an
// SGPR).
__device__ inline uint32_t and_or(uint32_t a, uint32_t mask, uint32_t bits) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(mask), "s"(bits));
    return r;
}

// One Q4 device word (elements 8w..8w+7, see kernels.h) as eight f16 values
// (q - 8) * d.  Each nibble pair is or-ed into the mantissa of an f16 whose
// mantissa step at the nibble's position is 1: nibbles at bits 0-3 under
// 1024.0 (0x6400), nibbles at bits 4-7 under 64.0 (0x5400); the upper two
// pairs take one shift by 8 first.  base + q is exact and subtracting
// base + 8 leaves q - 8 exactly; the only rounding is the product with d,
// as in the reference's f16 decode (shaders/weight.wgsl:50-54).
__device__ inline half8 dq4_word(uint32_t w, half2v dd) {
    const half2v o0 = {half_t(1032.0f), half_t(1032.0f)}, o1 = {half_t(72.0f), half_t(72.0f)};
    const uint32_t u = w >> 8;
    const half2v h0 = (as_half2(and_or(w, 0x000F000Fu, 0x64006400u)) - o0) * dd;
    const half2v h1 = (as_half2(and_or(w, 0x00F000F0u, 0x54005400u)) - o1) * dd;
    const half2v h2 = (as_half2(and_or(u, 0x000F000Fu, 0x64006400u)) - o0) * dd;
    const half2v h3 = (as_half2(and_or(u, 0x00F000F0u, 0x54005400u)) - o1) * dd;
    return half8{h0.x, h0.y, h1.x, h1.y, h2.x, h2.y, h3.x, h3.y};
}

// The same four elements as f32: element 8w+p of a Q4 device word.
__device__ inline float q4_elem_f32(uint32_t w, int p, float d) {
    const int sh = (p & 1) ? 16 + 4 * (p >> 1) : 4 * (p >> 1);
    return (float((w >> sh) & 0xfu) - 8.0f) * d;
}

// Eight Q8 codes (two little-endian words) times the block scale, f16.
// Each signed byte b is flipped to b + 128, placed under the exponent byte
// of 1024.0 (0x64) with a byte permute, and 1152 is subtracted: b exactly,
// so the only rounding is the product with d, as in shaders/weight.wgsl.
__device__ inline half2v q8_pair(uint32_t flipped, uint32_t sel) {
    return as_half2(__builtin_amdgcn_perm(0x64646464u, flipped, sel));
}
__device__ inline half8 dq8_words(uint32_t w0, uint32_t w1, half2v dd) {
    const half2v off = {half_t(1152.0f), half_t(1152.0f)};
    const uint32_t a = w0 ^ 0x80808080u, b = w1 ^ 0x80808080u;
    const half2v h0 = (q8_pair(a, 0x04010400u) - off) * dd;
    const half2v h1 = (q8_pair(a, 0x04030402u) - off) * dd;
    const half2v h2 = (q8_pair(b, 0x04010400u) - off) * dd;
    const half2v h3 = (q8_pair(b, 0x04030402u) - off) * dd;
    return half8{h0.x, h0.y, h1.x, h1.y, h2.x, h2.y, h3.x, h3.y};
}

// Elements (row, c..c+3) (c % 4 == 0) of a device weight, f32.
template <int DT>
__device__ inline void load4_f32(const DevWeight& w, int64_t row, int64_t c, float v[4]) {
    const int64_t e = row * w.cols + c;
    if constexpr (DT == F16_DT) {
        const uint2 u = *reinterpret_cast<const uint2*>(static_cast<const half_t*>(w.data) + e);
        const half2v a = as_half2(u.x), b = as_half2(u.y);
        v[0] = float(a.x);
        v[1] = float(a.y);
        v[2] = float(b.x);
        v[3] = float(b.y);
    } else if constexpr (DT == Q8_DT) {
        const float d = half_bits_to_f32(w.scales[row * w.sld + c / 32]);
        const uint32_t u = *reinterpret_cast<const uint32_t*>(static_cast<const uint8_t*>(w.data) + e);
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = float(int8_t(u >> (8 * i))) * d;
    } else {
        const int j = int(c % 32);
        const float d = half_bits_to_f32(w.scales[row * w.sld + c / 32]);
        const uint32_t word = static_cast<const uint32_t*>(w.data)[(e / 32) * 4 + j / 8];
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = q4_elem_f32(word, (j % 8) + i, d);
    }
}

}  // namespace omg
