// Kernels of the bidirectional encoder path (crates/omg-wgpu/src/laya.rs,
// the mmBERT / ModernBERT encoder with Laya's decision head): attention
// within each packed sequence (attention_bi.wgsl), the LayerNorm row
// kernels with their fused residual adds (layernorm.wgsl, bias_act.wgsl,
// embed.wgsl) and the gather of the rows the host scorer reads.
//
// Attention layout.  The [q | k | v] GEMM epilogue writes, per head, q and
// k as [tpad][64] f16 rows and v as 32-key tiles of V^T ([64 dims][32
// keys], keys ordered by vt_col32).  A workgroup of four waves owns 64
// query rows of one head; each wave owns 16 of them and keeps their q
// fragments in registers.  Key tiles of 32 rows stream through a two-slot
// LDS ring by DMA (buffer_load ... lds): K tile 4 KB (128 B rows, 16 B
// chunk c of row r at c ^ ((r >> 1) & 7)) and V^T tile 4 KB (64 B rows,
// chunk c at c ^ ((r >> 1) & 3)), so the rows one fragment read serves at
// once hit distinct banks (the decoder attention's V^T tiles measured 33.5%
// of their LDS cycles in bank conflicts with c ^ ((r >> 2) & 3), 7.3% with
// this swizzle).  Per tile and wave: S^T = K Q^T (4 MFMA 16x16x32),
// online softmax down the key axis (each lane owns one query column and
// eight keys; the other keys of the column sit in lanes l ^ 16, l ^ 32),
// O^T += V^T P^T (4 MFMA), with P^T taken straight from the score
// registers thanks to the V^T key order.
//
// Visibility needs no key metadata: sequences are contiguous row spans
// (laya.rs:1165-1187 packs them so), so a key is visible to query t iff it
// lies in t's span [meta[2], meta[3]) and, on local layers, within
// |t - j| <= window.
#include <cmath>
#include <string>

#include "common.h"
#include "kern_common.h"

namespace omg {

namespace {

constexpr int B_KT = 32;     // keys per tile
constexpr int B_HD = 64;     // head dim
constexpr int B_ROWS = 64;   // query rows per workgroup
constexpr int B_T = 256;     // threads per workgroup
constexpr int B_TILE = B_KT * B_HD * 2;  // bytes of one K or V^T tile
constexpr float LOG2E = 1.4426950408889634f;

typedef __attribute__((address_space(3))) void* lds_ptr_t;

__device__ inline __amdgpu_buffer_rsrc_t bi_rsrc(const void* base, int64_t bytes) {
    const int64_t n = bytes < 0 ? 0 : (bytes > 0x7fffffff ? 0x7fffffff : bytes);
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, int(n), 0x00020000);
}

__device__ inline void bi_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

struct BiArgs {
    QkvHeads h;
    int heads;
    int64_t t, nqb;
    int window;
    half_t* out;  // [t][heads * 64]
};

__global__ __launch_bounds__(B_T) void attention_bi_kernel(BiArgs a) {
    __shared__ __attribute__((aligned(16))) uint8_t smem[2 * 2 * B_TILE];
    const int tid = int(threadIdx.x), lane = tid % WAVE;
    const int wave = __builtin_amdgcn_readfirstlane(tid / WAVE);
    // Workgroups go round-robin over the 8 XCDs; give each XCD a run of
    // neighbouring query blocks of one head so they share K/V tiles in L2.
    const int64_t nitems = int64_t(a.heads) * a.nqb;
    const int64_t per_xcd = int64_t(gridDim.x) / 8;
    const int64_t item = int64_t(blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
    if (item >= nitems) return;
    const int64_t head = item / a.nqb, r0 = (item % a.nqb) * B_ROWS;
    const int64_t t = a.t, tpad = a.h.tpad;
    const int64_t W = a.window;

    // The workgroup's key range: the union of its rows' visible spans.
    int64_t lo = 0x7fffffffffffLL, hi = 0;
    {
        const int64_t q = r0 + lane;
        if (q < t) {
            lo = a.h.meta[4 * q + 2];
            hi = a.h.meta[4 * q + 3];
            if (W > 0) {
                lo = lo > q - W ? lo : q - W;
                hi = hi < q + W + 1 ? hi : q + W + 1;
            }
        }
    }
    const int lr = lane % 16, lg = lane / 16;
    // This lane's query (column) and its own span.
    const int64_t q = r0 + 16 * wave + lr;
    int qlo = 0, qhi = 0;
    if (q < t) {
        int64_t l0 = a.h.meta[4 * q + 2], h0 = a.h.meta[4 * q + 3];
        if (W > 0) {
            l0 = l0 > q - W ? l0 : q - W;
            h0 = h0 < q + W + 1 ? h0 : q + W + 1;
        }
        qlo = int(l0);
        qhi = int(h0);
    }
    int klo = int(lo < 0x7fffffff ? lo : 0x7fffffff), khi = int(hi);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        klo = min(klo, __shfl_xor(klo, o, WAVE));
        khi = max(khi, __shfl_xor(khi, o, WAVE));
    }
    klo = __builtin_amdgcn_readfirstlane(klo);
    khi = __builtin_amdgcn_readfirstlane(khi);
    if (khi <= klo) return;
    const int kt0 = klo / B_KT, kt1 = (khi + B_KT - 1) / B_KT;

    // q fragments (B operand): q[lr][32 ks + 8 lg .. + 8].
    half8 qf[2];
    {
        const half_t* qrow = a.h.q16 + (head * tpad + (q < tpad ? q : tpad - 1)) * B_HD;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) qf[ks] = *reinterpret_cast<const half8*>(qrow + 32 * ks + 8 * lg);
    }

    // Per-lane DMA offsets inside one tile: 256 lanes x 16 B each.
    const int slot = wave * WAVE + lane;
    uint32_t koff, voff;
    {
        const int r = slot / 8, c = (slot % 8) ^ ((r >> 1) & 7);
        koff = uint32_t((r * B_HD + c * 8) * 2);
    }
    {
        const int r = slot / 4, c = (slot % 4) ^ ((r >> 1) & 3);
        voff = uint32_t((r * B_KT + c * 8) * 2);
    }
    const half_t* kbase = a.h.k16 + head * tpad * B_HD;
    const half_t* vbase = a.h.vt + head * tpad * B_HD;
    const int64_t hbytes = tpad * B_HD * 2;
    auto issue = [&](int kt) {
        uint8_t* base = smem + (kt & 1) * 2 * B_TILE;
        const __amdgpu_buffer_rsrc_t rk = bi_rsrc(kbase, hbytes);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lds_ptr_t)(base + wave * WAVE * 16), 16, koff, kt * B_TILE, 0,
                                                 0);
        const __amdgpu_buffer_rsrc_t rv = bi_rsrc(vbase, hbytes);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (lds_ptr_t)(base + B_TILE + wave * WAVE * 16), 16, voff,
                                                 kt * B_TILE, 0, 0);
    };

    // Fragment read offsets (bytes inside a tile).
    int kfo[2][2], vfo[4];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const int r = 16 * kb + lr, c = 4 * ks + lg;
            kfo[kb][ks] = r * 128 + ((c ^ ((r >> 1) & 7)) * 16);
        }
#pragma unroll
    for (int db = 0; db < 4; ++db) {
        const int r = 16 * db + lr;
        vfo[db] = r * 64 + ((lg ^ ((r >> 1) & 3)) * 16);
    }

    floatx4 o[4];
#pragma unroll
    for (int db = 0; db < 4; ++db) o[db] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    float m_run = -INFINITY, l_run = 0.0f;

    issue(kt0);
    for (int kt = kt0; kt < kt1; ++kt) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        bi_barrier();
        if (kt + 1 < kt1) issue(kt + 1);
        const uint8_t* K = smem + (kt & 1) * 2 * B_TILE;
        const uint8_t* V = K + B_TILE;
        half8 kf[2][2], vf[4];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) kf[kb][ks] = *reinterpret_cast<const half8*>(K + kfo[kb][ks]);
#pragma unroll
        for (int db = 0; db < 4; ++db) vf[db] = *reinterpret_cast<const half8*>(V + vfo[db]);

        floatx4 s[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            s[kb] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) s[kb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[kb][ks], qf[ks], s[kb], 0, 0, 0);
        }
        // s[kb][r] = score of key kt*32 + 16 kb + 4 lg + r for query q.
        float mt = -INFINITY;
        float sv[2][4];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int j = kt * B_KT + 16 * kb + 4 * lg + r;
                const bool vis = j >= qlo && j < qhi;
                sv[kb][r] = vis ? s[kb][r] * LOG2E : -INFINITY;
                mt = fmaxf(mt, sv[kb][r]);
            }
        mt = max_lanes_16_32(mt);
        const float m_new = fmaxf(m_run, mt);
        const float m_use = m_new == -INFINITY ? 0.0f : m_new;
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
        m_run = m_new;
        float p[2][4], psum = 0.0f;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                p[kb][r] = __builtin_amdgcn_exp2f(sv[kb][r] - m_use);
                psum += p[kb][r];
            }
        l_run = l_run * alpha + psum;
#pragma unroll
        for (int db = 0; db < 4; ++db) o[db] *= alpha;
        const half8 pf = {half_t(p[0][0]), half_t(p[0][1]), half_t(p[0][2]), half_t(p[0][3]),
                          half_t(p[1][0]), half_t(p[1][1]), half_t(p[1][2]), half_t(p[1][3])};
#pragma unroll
        for (int db = 0; db < 4; ++db) o[db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf[db], pf, o[db], 0, 0, 0);
    }

    // o[db][r] = O[q][16 db + 4 lg + r] (unnormalised); l over the column's lanes.
    const float l = sum_lanes_16_32(l_run);
    if (q >= t) return;
    const float inv = 1.0f / l;
    half_t* dst = a.out + q * (int64_t(a.heads) * B_HD) + head * B_HD;
#pragma unroll
    for (int db = 0; db < 4; ++db)
        *reinterpret_cast<half4*>(dst + 16 * db + 4 * lg) =
            half4{half_t(o[db][0] * inv), half_t(o[db][1] * inv), half_t(o[db][2] * inv), half_t(o[db][3] * inv)};
}

// ------------------------------------------------------------ row kernels
//
// One wave64 per row, four rows per workgroup; a row of d <= 2048 f32
// lives in registers as NV float4 per lane (element 4 (k * 64 + lane) + i).

template <int NV>
__device__ inline void ln_stats(const float4 (&v)[NV], int64_t d, int lane, float eps, float& mean, float& inv) {
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k)
        if ((k * WAVE + lane) * 4 < d) s += (v[k].x + v[k].y) + (v[k].z + v[k].w);
    mean = wave_sum(s) / float(d);
    float q = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k)
        if ((k * WAVE + lane) * 4 < d) {
            const float a = v[k].x - mean, b = v[k].y - mean, c = v[k].z - mean, e = v[k].w - mean;
            q += (a * a + b * b) + (c * c + e * e);
        }
    // layernorm.wgsl:74-82: variance around the mean, inverseSqrt(var + eps).
    inv = 1.0f / sqrtf(wave_sum(q) / float(d) + eps);
}

__device__ inline float4 ln_apply(float4 v, float mean, float inv, const float* w, const float* b, int64_t c) {
    const float4 g = *reinterpret_cast<const float4*>(w + c);
    float4 y = make_float4((v.x - mean) * inv * g.x, (v.y - mean) * inv * g.y, (v.z - mean) * inv * g.z,
                           (v.w - mean) * inv * g.w);
    if (b) {
        const float4 bb = *reinterpret_cast<const float4*>(b + c);
        y = make_float4(y.x + bb.x, y.y + bb.y, y.z + bb.z, y.w + bb.w);
    }
    return y;
}

__device__ inline void store_h16(half_t* p, float4 y) {
    *reinterpret_cast<half4*>(p) = half4{half_t(y.x), half_t(y.y), half_t(y.z), half_t(y.w)};
}

// embed.wgsl (scale 1) then layernorm.wgsl without bias (laya.rs:1261-1269).
template <int DT, int NV>
__global__ __launch_bounds__(256) void embed_ln_kernel(DevWeight E, const uint32_t* __restrict__ ids, int64_t t,
                                                       const float* __restrict__ w, float eps, float* __restrict__ x,
                                                       half_t* __restrict__ x16) {
    const int wave = int(threadIdx.x) / WAVE, lane = int(threadIdx.x) % WAVE;
    const int64_t row = int64_t(blockIdx.x) * 4 + wave;
    if (row >= t) return;
    const int64_t d = E.cols, id = ids[row];
    float4 v[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int64_t c = (k * WAVE + lane) * 4;
        float e[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (c < d) load4_f32<DT>(E, id, c, e);
        v[k] = make_float4(e[0], e[1], e[2], e[3]);
    }
    float mean, inv;
    ln_stats<NV>(v, d, lane, eps, mean, inv);
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int64_t c = (k * WAVE + lane) * 4;
        if (c >= d) continue;
        const float4 y = ln_apply(v[k], mean, inv, w, nullptr, c);
        *reinterpret_cast<float4*>(x + row * d + c) = y;
        store_h16(x16 + row * d + c, y);
    }
}

// layernorm.wgsl with `residual`: x += a (+ rb) written back, then the
// norm of the sum into h16 (laya.rs:1334-1335,1359-1360,1380-1381,1390-1391).
template <int NV>
__global__ __launch_bounds__(256) void add_ln_kernel(float* __restrict__ x, const float* __restrict__ a,
                                                     const float* __restrict__ rb, const float* __restrict__ w,
                                                     const float* __restrict__ b, float eps, int64_t t, int64_t d,
                                                     half_t* __restrict__ h16) {
    const int wave = int(threadIdx.x) / WAVE, lane = int(threadIdx.x) % WAVE;
    const int64_t row = int64_t(blockIdx.x) * 4 + wave;
    if (row >= t) return;
    float4 v[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int64_t c = (k * WAVE + lane) * 4;
        v[k] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (c >= d) continue;
        float4 e = *reinterpret_cast<const float4*>(x + row * d + c);
        const float4 f = *reinterpret_cast<const float4*>(a + row * d + c);
        e = make_float4(e.x + f.x, e.y + f.y, e.z + f.z, e.w + f.w);
        if (rb) {
            const float4 g = *reinterpret_cast<const float4*>(rb + c);
            e = make_float4(e.x + g.x, e.y + g.y, e.z + g.z, e.w + g.w);
        }
        *reinterpret_cast<float4*>(x + row * d + c) = e;
        v[k] = e;
    }
    float mean, inv;
    ln_stats<NV>(v, d, lane, eps, mean, inv);
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int64_t c = (k * WAVE + lane) * 4;
        if (c < d) store_h16(h16 + row * d + c, ln_apply(v[k], mean, inv, w, b, c));
    }
}

// The last encoder layer's add_wo_norm (final norm in place), the type
// embedding added to the encoder output and the first head layer's norm1
// (laya.rs:1308-1323,1340-1343), one pass over the row.
template <int NV>
__global__ __launch_bounds__(256) void add_ln_final_kernel(float* __restrict__ x, const float* __restrict__ a,
                                                           const float* __restrict__ wf, const float* __restrict__ temb,
                                                           const uint32_t* __restrict__ qtypes,
                                                           const float* __restrict__ w1, const float* __restrict__ b1,
                                                           float eps, int64_t t, int64_t d, half_t* __restrict__ h16) {
    const int wave = int(threadIdx.x) / WAVE, lane = int(threadIdx.x) % WAVE;
    const int64_t row = int64_t(blockIdx.x) * 4 + wave;
    if (row >= t) return;
    float4 v[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int64_t c = (k * WAVE + lane) * 4;
        v[k] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (c >= d) continue;
        const float4 e = *reinterpret_cast<const float4*>(x + row * d + c);
        const float4 f = *reinterpret_cast<const float4*>(a + row * d + c);
        v[k] = make_float4(e.x + f.x, e.y + f.y, e.z + f.z, e.w + f.w);
    }
    float mean, inv;
    ln_stats<NV>(v, d, lane, eps, mean, inv);
    const float* te = temb ? temb + int64_t(qtypes[row]) * d : nullptr;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int64_t c = (k * WAVE + lane) * 4;
        if (c >= d) continue;
        float4 y = ln_apply(v[k], mean, inv, wf, nullptr, c);
        if (te) {
            const float4 g = *reinterpret_cast<const float4*>(te + c);
            y = make_float4(y.x + g.x, y.y + g.y, y.z + g.z, y.w + g.w);
        }
        *reinterpret_cast<float4*>(x + row * d + c) = y;
        v[k] = y;
    }
    if (!w1) return;
    ln_stats<NV>(v, d, lane, eps, mean, inv);
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int64_t c = (k * WAVE + lane) * 4;
        if (c < d) store_h16(h16 + row * d + c, ln_apply(v[k], mean, inv, w1, b1, c));
    }
}

// out[i] = (a[r] + bias) + x[r] (bias_act.wgsl mode 0 with `residual`,
// laya.rs:1385-1387), or x[r]; r = rows[i] (i without a list).
__global__ __launch_bounds__(256) void gather_rows_kernel(const float* __restrict__ x, const float* __restrict__ a,
                                                          const float* __restrict__ bias,
                                                          const int32_t* __restrict__ rows, int64_t n, int64_t d,
                                                          float* __restrict__ out) {
    const int64_t i = int64_t(blockIdx.x) * 4 + threadIdx.x / WAVE;
    if (i >= n) return;
    const int64_t r = rows ? rows[i] : i;
    for (int64_t c = int64_t(threadIdx.x % WAVE) * 4; c < d; c += WAVE * 4) {
        float4 v = *reinterpret_cast<const float4*>(x + r * d + c);
        if (a) {
            const float4 f = *reinterpret_cast<const float4*>(a + r * d + c);
            const float4 g = *reinterpret_cast<const float4*>(bias + c);
            v = make_float4((f.x + g.x) + v.x, (f.y + g.y) + v.y, (f.z + g.z) + v.z, (f.w + g.w) + v.w);
        }
        *reinterpret_cast<float4*>(out + i * d + c) = v;
    }
}

int row_nv(int64_t d, const char* what) {
    if (d <= 0 || d % 4 != 0 || d > 2048) fail(E_INVALID, std::string(what) + ": row width must be 4..2048, a multiple of 4");
    return int((d / 4 + WAVE - 1) / WAVE);
}

}  // namespace

void launch_attention_bi(hipStream_t s, const QkvHeads& h, int heads, int64_t t, int window, half_t* out) {
    if (heads <= 0 || h.dq != int64_t(heads) * B_HD) fail(E_INVALID, "attention_bi: q width must be heads x 64");
    if (t < 0 || h.tpad < t || h.tpad % B_KT != 0) fail(E_INVALID, "attention_bi: padded rows must cover t");
    if (window < 0) fail(E_INVALID, "attention_bi: negative window");
    if (!h.q16 || !h.k16 || !h.vt || !h.meta || !out) fail(E_INVALID, "attention_bi: missing buffer");
    if (h.tpad * B_HD * 2 >= 0x7fff0000LL) fail(E_INVALID, "attention_bi: head arrays of 2 GiB or more");
    if (t == 0) return;
    BiArgs a{h, heads, t, (t + B_ROWS - 1) / B_ROWS, window, out};
    const int64_t items = int64_t(heads) * a.nqb;
    attention_bi_kernel<<<dim3(unsigned((items + 7) / 8 * 8)), dim3(B_T), 0, s>>>(a);
    OMG_HIP(hipGetLastError());
}

#define OMG_NV_SWITCH(nv, CALL)                       \
    switch (nv) {                                     \
        case 1: { constexpr int NV = 1; CALL; } break; \
        case 2: { constexpr int NV = 2; CALL; } break; \
        case 3: { constexpr int NV = 3; CALL; } break; \
        case 4: { constexpr int NV = 4; CALL; } break; \
        case 5: { constexpr int NV = 5; CALL; } break; \
        case 6: { constexpr int NV = 6; CALL; } break; \
        case 7: { constexpr int NV = 7; CALL; } break; \
        default: { constexpr int NV = 8; CALL; } break; \
    }

void launch_embed_ln(hipStream_t s, const DevWeight& E, const uint32_t* ids, int64_t t, const float* w,
                     float eps, float* x, half_t* x16) {
    const int nv = row_nv(E.cols, "embed_ln");
    if (!ids || !w || !x || !x16) fail(E_INVALID, "embed_ln: missing buffer");
    if (t <= 0) return;
    const dim3 grid(unsigned((t + 3) / 4)), block(256);
    switch (E.dtype) {
        case F16_DT: OMG_NV_SWITCH(nv, (embed_ln_kernel<F16_DT, NV><<<grid, block, 0, s>>>(E, ids, t, w, eps, x, x16))); break;
        case Q8_DT: OMG_NV_SWITCH(nv, (embed_ln_kernel<Q8_DT, NV><<<grid, block, 0, s>>>(E, ids, t, w, eps, x, x16))); break;
        default: OMG_NV_SWITCH(nv, (embed_ln_kernel<Q4_DT, NV><<<grid, block, 0, s>>>(E, ids, t, w, eps, x, x16))); break;
    }
    OMG_HIP(hipGetLastError());
}

void launch_add_ln(hipStream_t s, float* x, const float* a, const float* rb, const float* w, const float* b,
                   float eps, int64_t t, int64_t d, half_t* h16) {
    const int nv = row_nv(d, "add_ln");
    if (!x || !a || !w || !h16) fail(E_INVALID, "add_ln: missing buffer");
    if (t <= 0) return;
    const dim3 grid(unsigned((t + 3) / 4)), block(256);
    OMG_NV_SWITCH(nv, (add_ln_kernel<NV><<<grid, block, 0, s>>>(x, a, rb, w, b, eps, t, d, h16)));
    OMG_HIP(hipGetLastError());
}

void launch_add_ln_final(hipStream_t s, float* x, const float* a, const float* wf, const float* temb,
                         const uint32_t* qtypes, const float* w1, const float* b1, float eps, int64_t t, int64_t d,
                         half_t* h16) {
    const int nv = row_nv(d, "add_ln_final");
    if (!x || !a || !wf || (temb && !qtypes) || (w1 && !h16)) fail(E_INVALID, "add_ln_final: missing buffer");
    if (t <= 0) return;
    const dim3 grid(unsigned((t + 3) / 4)), block(256);
    OMG_NV_SWITCH(nv, (add_ln_final_kernel<NV><<<grid, block, 0, s>>>(x, a, wf, temb, qtypes, w1, b1, eps, t, d, h16)));
    OMG_HIP(hipGetLastError());
}

void launch_gather_rows(hipStream_t s, const float* x, const float* a, const float* bias, const int32_t* rows,
                        int64_t n, int64_t d, float* out) {
    if (d <= 0 || d % 4 != 0) fail(E_INVALID, "gather_rows: row width must be a multiple of 4");
    if (a && !bias) fail(E_INVALID, "gather_rows: bias required with a");
    if (n <= 0) return;
    gather_rows_kernel<<<dim3(unsigned((n + 3) / 4)), dim3(256), 0, s>>>(x, a, bias, rows, n, d, out);
    OMG_HIP(hipGetLastError());
}

}  // namespace omg
