// Row-wise kernels of the forward: embedding gather + first norm, the fused
// residual norms, q/k preparation with the f16 K/V cache write, the
// readout (final norm at the wanted rows, label / vocabulary logits) and
// the K/V <-> state-row conversions.  One wave64 per row; reductions are
// wave-level shuffles, no LDS round trips.
#include <cmath>
#include <mutex>
#include <string>

#include "common.h"
#include "kern_common.h"

namespace omg {

// ------------------------------------------------------------ embedding

// embed.wgsl:15-48 + the layer-0 input norm (rmsnorm.wgsl:41-61), one wave
// per token.  The stored row is deq(E[id]) * sqrt(d) in f32: the decode is
// exact, so the one product rounds exactly like reference.rs:186.
template <int DT>
__global__ __launch_bounds__(256) void embed_norm_kernel(DevWeight E, const uint32_t* __restrict__ ids,
                                                         int64_t t, float escale,
                                                         const float* __restrict__ w, float eps,
                                                         float* __restrict__ x, half_t* __restrict__ hn) {
    const int wave = int(threadIdx.x) / WAVE, lane = int(threadIdx.x) % WAVE;
    const int64_t row = int64_t(blockIdx.x) * 4 + wave;
    if (row >= t) return;
    const int64_t d = E.cols;
    const int64_t id = ids[row];
    float ss = 0.0f;
    for (int64_t q = lane; q < d / 4; q += WAVE) {
        float v[4];
        load4_f32<DT>(E, id, 4 * q, v);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[i] = v[i] * escale;
            ss += v[i] * v[i];
        }
        *reinterpret_cast<float4*>(x + row * d + 4 * q) = make_float4(v[0], v[1], v[2], v[3]);
    }
    const float inv = 1.0f / sqrtf(wave_sum(ss) / float(d) + eps);
    for (int64_t q = lane; q < d / 4; q += WAVE) {
        const float4 v = *reinterpret_cast<const float4*>(x + row * d + 4 * q);
        const float4 g = *reinterpret_cast<const float4*>(w + 4 * q);
        half4 o = {half_t(v.x * inv * g.x), half_t(v.y * inv * g.y), half_t(v.z * inv * g.z),
                   half_t(v.w * inv * g.w)};
        *reinterpret_cast<half4*>(hn + row * d + 4 * q) = o;
    }
}

void launch_embed_norm(hipStream_t s, const DevWeight& E, const uint32_t* ids, int64_t t,
                       float embed_scale, const float* w, float eps, float* x, half_t* hn) {
    if (t <= 0) return;
    if (E.cols % 32 != 0) fail(E_INVALID, "embed: width must be a multiple of 32");
    const dim3 grid(unsigned((t + 3) / 4)), block(256);
    switch (E.dtype) {
        case F16_DT: embed_norm_kernel<F16_DT><<<grid, block, 0, s>>>(E, ids, t, embed_scale, w, eps, x, hn); break;
        case Q8_DT: embed_norm_kernel<Q8_DT><<<grid, block, 0, s>>>(E, ids, t, embed_scale, w, eps, x, hn); break;
        default: embed_norm_kernel<Q4_DT><<<grid, block, 0, s>>>(E, ids, t, embed_scale, w, eps, x, hn); break;
    }
    OMG_HIP(hipGetLastError());
}

// -------------------------------------------------------- residual norm

// rmsnorm.wgsl:41-68 in residual mode with the fused second norm: the
// post-attention / post-feedforward norm of `a` is added into the stream x,
// then the norm that reads x next writes its f16 input hn.  W waves per row
// (1 up to 512 wide, 2 up to 1,536, 4 above: a function of the width, so
// a row's sums do not depend on the pass), the row in registers: lane l of
// the row's wave s holds float4 q = 64 (s + W j) + l, NV of them.  A row's
// sums of squares are each wave's wave_sum, added in wave order.
// `a` may come in parts (the K pieces of a split product): part z at
// a + z * part_stride.  Consecutive runs of `group` parts are added in
// order into one sum each, and those sums in order into the total:
//   ((p0 + p1) + ...) + ((p_G + p_G+1) + ...) + ...
// which is what a product that adds each run in its registers and writes
// one part per run gives with group 1 — the same bits either way.  The
// parts are loaded RP at a time (RP: the part count rounded up to a power
// of two, at most 24 / NV), the first round together with the row and the
// norm weights, before the first reduction.
template <int NV, int RP, int W>
__global__ __launch_bounds__(256) void residual_norm_kernel(const float* __restrict__ a,
                                                            const float* __restrict__ w1,
                                                            float* __restrict__ x,
                                                            const float* __restrict__ w2,
                                                            half_t* __restrict__ hn, int64_t t,
                                                            int64_t d, float eps, float scale, int parts,
                                                            int64_t part_stride, int group) {
    // Every product and sum rounds on its own: no instance may fuse a
    // multiply into an add where another does not (the x and hn of a row
    // must not depend on which instance produced them).
#pragma clang fp contract(off)
    const int wave = int(threadIdx.x) / WAVE, lane = int(threadIdx.x) % WAVE;
    const int64_t row = int64_t(blockIdx.x) * (4 / W) + wave / W;
    const int sub = wave % W;
    __shared__ float red[2][4];  // per-wave sums of squares (W > 1)
    // Rows past the end still reach the barriers (W > 1); they load and
    // store nothing.
    const bool live = row < t;
    if (W == 1 && !live) return;
    const int64_t nq = live ? d / 4 : 0;
    auto col = [&](int j) { return int64_t(WAVE) * (sub + W * j) + lane; };  // this lane's float4 j
    const float* ar = a + row * d;
    float* xr = x + row * d;
    float4 av[NV], gs[NV], xv[NV], g1[NV], g2[NV];
    float4 pv[RP][NV];
    auto load_round = [&](int z0) {
#pragma unroll
        for (int u = 0; u < RP; ++u)
#pragma unroll
            for (int j = 0; j < NV; ++j) {
                const int64_t q = col(j);
                if (z0 + u < parts && q < nq) pv[u][j] = *reinterpret_cast<const float4*>(ar + (z0 + u) * part_stride + 4 * q);
            }
    };
    load_round(0);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int64_t q = col(j);
        if (q < nq) {
            xv[j] = *reinterpret_cast<const float4*>(xr + 4 * q);
            g1[j] = *reinterpret_cast<const float4*>(w1 + 4 * q);
            if (w2) g2[j] = *reinterpret_cast<const float4*>(w2 + 4 * q);
        }
    }
    // gi: position inside the current run; si: runs finished so far.
    int gi = 0, si = 0;
    for (int z0 = 0; z0 < parts; z0 += RP) {
        if (z0 > 0) load_round(z0);
#pragma unroll
        for (int u = 0; u < RP; ++u) {
            if (z0 + u >= parts) break;
#pragma unroll
            for (int j = 0; j < NV; ++j) {
                if (col(j) >= nq) continue;
                const float4 b = pv[u][j];
                if (si == 0) {  // the first run sums straight into the total
                    if (gi == 0)
                        av[j] = b;
                    else
                        av[j].x += b.x, av[j].y += b.y, av[j].z += b.z, av[j].w += b.w;
                } else {
                    if (gi == 0)
                        gs[j] = b;
                    else
                        gs[j].x += b.x, gs[j].y += b.y, gs[j].z += b.z, gs[j].w += b.w;
                    if (gi + 1 == group) {
                        const float4 c = gs[j];
                        av[j].x += c.x, av[j].y += c.y, av[j].z += c.z, av[j].w += c.w;
                    }
                }
            }
            if (++gi == group) {
                gi = 0;
                ++si;
            }
        }
    }
    // The row's sum of squares: this wave's, then (W > 1) the row's waves'
    // in order through LDS.
    auto row_sum = [&](float v, int k) {
        v = wave_sum(v);
        if constexpr (W > 1) {
            if (lane == 0) red[k][wave] = v;
            __syncthreads();
            const int w0 = wave - sub;
            v = red[k][w0];
#pragma unroll
            for (int s = 1; s < W; ++s) v += red[k][w0 + s];
        }
        return v;
    };
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j)
        if (col(j) < nq) {
            const float4 v = av[j];
            ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
        }
    const float inv = 1.0f / sqrtf(row_sum(ss, 0) / float(d) + eps);
    float ss2 = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int64_t q = col(j);
        if (q < nq) {
            const float4 v = av[j], g = g1[j];
            float4 o = xv[j];
            o.x = (v.x * inv * g.x + o.x) * scale;
            o.y = (v.y * inv * g.y + o.y) * scale;
            o.z = (v.z * inv * g.z + o.z) * scale;
            o.w = (v.w * inv * g.w + o.w) * scale;
            *reinterpret_cast<float4*>(xr + 4 * q) = o;
            ss2 += o.x * o.x + o.y * o.y + o.z * o.z + o.w * o.w;
            xv[j] = o;
        }
    }
    if (!w2) {
        if (!hn) return;
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int64_t q = col(j);
            if (q < nq) {
                const float4 v = xv[j];
                *reinterpret_cast<half4*>(hn + row * d + 4 * q) =
                    half4{f16_rounded(v.x), f16_rounded(v.y), f16_rounded(v.z), f16_rounded(v.w)};
            }
        }
        return;
    }
    const float inv2 = 1.0f / sqrtf(row_sum(ss2, 1) / float(d) + eps);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int64_t q = col(j);
        if (q < nq) {
            const float4 v = xv[j], g = g2[j];
            half4 o = {f16_rounded(v.x * inv2 * g.x), f16_rounded(v.y * inv2 * g.y), f16_rounded(v.z * inv2 * g.z),
                       f16_rounded(v.w * inv2 * g.w)};
            *reinterpret_cast<half4*>(hn + row * d + 4 * q) = o;
        }
    }
}

// Waves per row: a function of the width alone.
// At most three float4 per lane up to 3,072 wide, so up to eight parts load
// in one round.
static int rn_waves(int64_t d) { return d <= 512 ? 1 : (d <= 1536 ? 2 : 4); }

// Parts loaded per round: the part count rounded up to a power of two, up
// to 24 float4 per lane.
static int rn_round(int nv, int parts) {
    int r = 1;
    while (r < parts && r < 8 && 2 * r * nv <= 24) r *= 2;
    return r;
}

void launch_residual_norm(hipStream_t s, const float* a, const float* w1, float* x, const float* w2,
                          half_t* hn, int64_t t, int64_t d, float eps, float scale, int parts,
                          int64_t part_stride, int group) {
    if (t <= 0) return;
    if (d % 4 != 0) fail(E_INVALID, "residual_norm: width must be a multiple of 4");
    if (parts < 1 || group < 1 || parts % group != 0 || (parts > 1 && (part_stride < t * d || part_stride % 4)))
        fail(E_INVALID, "residual_norm: split-K partials");
    if (d > 4096) fail(E_INVALID, "residual_norm: width above 4096");
    const int w = rn_waves(d);
    const int nv = int((d / 4 + WAVE * w - 1) / (WAVE * w));  // float4 per lane
    const dim3 grid(unsigned((t + 4 / w - 1) / (4 / w))), block(256);
    const int rp = rn_round(nv, parts);
#define OMG_RN(N, R, W)                                                                                          \
    case (N * 16 + R) * 8 + W:                                                                                  \
        residual_norm_kernel<N, R, W><<<grid, block, 0, s>>>(a, w1, x, w2, hn, t, d, eps, scale, parts,          \
                                                             part_stride, group);                                \
        break;
#define OMG_RNR(N, W) OMG_RN(N, 1, W) OMG_RN(N, 2, W) OMG_RN(N, 4, W) OMG_RN(N, 8, W)
    // one to three float4 per lane on one, two or four waves; four on four
    // from 3,076 wide
    switch ((nv * 16 + rp) * 8 + w) {
        OMG_RNR(1, 1) OMG_RNR(2, 1) OMG_RNR(3, 1) OMG_RNR(2, 2) OMG_RNR(3, 2) OMG_RNR(1, 4) OMG_RNR(2, 4)
        OMG_RNR(3, 4) OMG_RN(4, 1, 4) OMG_RN(4, 2, 4) OMG_RN(4, 4, 4)
        OMG_RN(4, 1, 2) OMG_RN(4, 2, 2) OMG_RN(4, 4, 2) OMG_RN(5, 1, 2) OMG_RN(5, 2, 2) OMG_RN(5, 4, 2)
        OMG_RN(6, 1, 2) OMG_RN(6, 2, 2) OMG_RN(6, 4, 2)
        default: fail(E_INVALID, "residual_norm: unsupported shape");
    }
#undef OMG_RNR
#undef OMG_RN
    OMG_HIP(hipGetLastError());
}

// ------------------------------------------------- per-layer inputs

// pl_combine.wgsl: per (token, layer) slice of P elements of
// proj = f16(x) . pl_model_proj^T (in place in `pl`),
//   pl = (rmsnorm(proj / sqrt(d)) * w + f16(table[id, slice]) * sqrt(P)) / sqrt(2).
// One wave per slice holding it in registers (NV float4 per lane).
template <int DT, int NV>
__global__ __launch_bounds__(256) void pl_combine_kernel(DevWeight table, const uint32_t* __restrict__ ids,
                                                         const float* __restrict__ w, float* __restrict__ pl,
                                                         int64_t t, int64_t P, int64_t layers, float eps,
                                                         float proj_scale, float emb_scale, float out_scale) {
    const int wave = int(threadIdx.x) / WAVE, lane = int(threadIdx.x) % WAVE;
    const int64_t slice = int64_t(blockIdx.x) * 4 + wave;  // token * layers + layer
    if (slice >= t * layers) return;
    const int64_t tok = slice / layers;
    const int64_t nq = P / 4;
    float* row = pl + slice * P;
    float4 v[NV];
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int64_t q = lane + j * WAVE;
        if (q < nq) {
            v[j] = *reinterpret_cast<const float4*>(row + 4 * q);
            v[j].x *= proj_scale, v[j].y *= proj_scale, v[j].z *= proj_scale, v[j].w *= proj_scale;
            ss += v[j].x * v[j].x + v[j].y * v[j].y + v[j].z * v[j].z + v[j].w * v[j].w;
        }
    }
    const float inv = 1.0f / sqrtf(wave_sum(ss) / float(P) + eps);
    const int64_t col0 = (slice - tok * layers) * P;
    const int64_t id = ids[tok];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int64_t q = lane + j * WAVE;
        if (q < nq) {
            float e[4];
            load4_f32<DT>(table, id, col0 + 4 * q, e);
            const float4 g = *reinterpret_cast<const float4*>(w + 4 * q);
            const float vv[4] = {v[j].x, v[j].y, v[j].z, v[j].w}, gg[4] = {g.x, g.y, g.z, g.w};
            float o[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) o[i] = (vv[i] * inv * gg[i] + float(half_t(e[i])) * emb_scale) * out_scale;
            *reinterpret_cast<float4*>(row + 4 * q) = make_float4(o[0], o[1], o[2], o[3]);
        }
    }
}

void launch_pl_combine(hipStream_t s, const DevWeight& table, const uint32_t* ids, const float* w, float* pl,
                       int64_t t, int64_t P, int64_t layers, float eps, float proj_scale, float emb_scale,
                       float out_scale) {
    if (t <= 0) return;
    if (P % 4 != 0 || P > 1024) fail(E_INVALID, "pl_combine: per-layer width must be a multiple of 4, at most 1024");
    if (table.cols != P * layers) fail(E_INVALID, "pl_combine: table width must be per-layer width x layers");
    const int nv = int((P / 4 + WAVE - 1) / WAVE);
    const dim3 grid(unsigned((t * layers + 3) / 4)), block(256);
#define OMG_PLC(D, N) \
    pl_combine_kernel<D, N><<<grid, block, 0, s>>>(table, ids, w, pl, t, P, layers, eps, proj_scale, emb_scale, out_scale)
#define OMG_PLC_NV(D)                      \
    switch (nv) {                          \
        case 1: OMG_PLC(D, 1); break;      \
        case 2: OMG_PLC(D, 2); break;      \
        default: OMG_PLC(D, 4); break;     \
    }
    switch (table.dtype) {
        case F16_DT: OMG_PLC_NV(F16_DT) break;
        case Q8_DT: OMG_PLC_NV(Q8_DT) break;
        default: OMG_PLC_NV(Q4_DT) break;
    }
#undef OMG_PLC_NV
#undef OMG_PLC
    OMG_HIP(hipGetLastError());
}

// pl_gate.wgsl: out[t][j] = f16(gelu_tanh(g[t][j]) * pl[t][layer * P + j]).
__global__ __launch_bounds__(256) void pl_gate_kernel(const float* __restrict__ g, const float* __restrict__ pl,
                                                      half_t* __restrict__ out, int64_t t, int64_t P,
                                                      int64_t pl_stride, int64_t layer) {
    const int64_t i = (int64_t(blockIdx.x) * 256 + threadIdx.x) * 4;
    if (i >= t * P) return;
    const int64_t tok = i / P, j = i - tok * P;
    const float4 gv = *reinterpret_cast<const float4*>(g + i);
    const float4 pv = *reinterpret_cast<const float4*>(pl + tok * pl_stride + layer * P + j);
    auto gelu = [](float x) { return 0.5f * x * (1.0f + tanhf(0.7978845608f * (x + 0.044715f * x * x * x))); };
    *reinterpret_cast<half4*>(out + i) =
        half4{half_t(gelu(gv.x) * pv.x), half_t(gelu(gv.y) * pv.y), half_t(gelu(gv.z) * pv.z), half_t(gelu(gv.w) * pv.w)};
}

void launch_pl_gate(hipStream_t s, const float* g, const float* pl, half_t* out, int64_t t, int64_t P, int64_t layers,
                    int64_t layer) {
    if (t <= 0) return;
    if (P % 4 != 0 || layer < 0 || layer >= layers) fail(E_INVALID, "pl_gate: shape");
    const int64_t n4 = t * P / 4;
    pl_gate_kernel<<<dim3(unsigned((n4 + 255) / 256)), dim3(256), 0, s>>>(g, pl, out, t, P, P * layers, layer);
    OMG_HIP(hipGetLastError());
}

// out[i] = f16(x[i]), n % 4 == 0.
__global__ __launch_bounds__(256) void to_f16_kernel(const float* __restrict__ x, half_t* __restrict__ out, int64_t n) {
    const int64_t i = (int64_t(blockIdx.x) * 256 + threadIdx.x) * 4;
    if (i >= n) return;
    const float4 v = *reinterpret_cast<const float4*>(x + i);
    *reinterpret_cast<half4*>(out + i) = half4{half_t(v.x), half_t(v.y), half_t(v.z), half_t(v.w)};
}

void launch_to_f16(hipStream_t s, const float* x, half_t* out, int64_t n) {
    if (n <= 0) return;
    if (n % 4 != 0) fail(E_INVALID, "to_f16: count must be a multiple of 4");
    to_f16_kernel<<<dim3(unsigned((n / 4 + 255) / 256)), dim3(256), 0, s>>>(x, out, n);
    OMG_HIP(hipGetLastError());
}

// -------------------------------------------------------------- qk prep

// qk_prep.wgsl:66-114 in two kinds of blocks of one launch.
//
// The first vblocks blocks own one (64-row V^T cache tile, kv head) each:
// wave w normalises the tile's rows 16w..16w+15 (when v_norm) and stores
// them as f16 rows in LDS; then thread c owns head dimension c and writes
// that dimension's 64 key columns (vt_col order) as eight 16-byte chunks,
// so every 128-byte row of the tile is written whole from one block.  A
// tile only partly inside this pass's rows is read first and its other
// keys' columns are written back unchanged (no other block of the launch
// touches them).
//
// The remaining blocks hold one wave per (token, q or k head slot): the
// head row is normed, rotated with the position's (cos, sin) and stored
// f16.  Head row element e = lane * EPL + i, so the RoPE partner e +- HD/2
// sits in lane ^ 32.
template <int HD>
__global__ __launch_bounds__(256) void qk_prep_kernel(QkArgs a, int64_t vblocks, int qk_slots) {
    constexpr int EPL = HD / WAVE;   // elements per lane: 4 (hd 256) or 8 (hd 512)
    constexpr int NQ = EPL / 4;      // float4 per lane
    constexpr int HALF = HD / 2;
    constexpr int DPT = HD / 256;    // V^T dimensions per thread
    static_assert(HD == 256 || HD == 512, "qk_prep: head_dim 256 or 512");
    const int wave = int(threadIdx.x) / WAVE, lane = int(threadIdx.x) % WAVE;
    const int e0 = lane * EPL;
    const int H = a.heads, KV = a.kv_heads;
    if (int64_t(blockIdx.x) < vblocks) {
        __shared__ half_t tile_rows[64][HD];
        const int64_t tile = a.base / 64 + int64_t(blockIdx.x) / KV;
        const int head = int(int64_t(blockIdx.x) % KV);
        const int64_t r0 = tile * 64;
        const int64_t lo = r0 > a.base ? r0 : a.base;
        const int64_t hi = r0 + 64 < a.base + a.t ? r0 + 64 : a.base + a.t;
        const bool whole = lo == r0 && hi == r0 + 64;
        // The destination's current contents first (a tile only partly in
        // this pass keeps its other keys' columns), then all 16 rows of the
        // wave, so every load is in flight before the first use.
        uint4 kept[DPT][8];
        if (!whole) {
#pragma unroll
            for (int dd = 0; dd < DPT; ++dd) {
                const int dim = int(threadIdx.x) + 256 * dd;
                const half_t* dst = a.vt + ((int64_t(head) * (a.cap_pad / 64) + tile) * HD + dim) * 64;
#pragma unroll
                for (int c = 0; c < 8; ++c) kept[dd][c] = reinterpret_cast<const uint4*>(dst)[c];
            }
        }
        const float* src = a.qkv + int64_t(H + KV + head) * HD + e0;
        float4 v[16][NQ];
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const int64_t row = r0 + 16 * wave + k;
#pragma unroll
            for (int q = 0; q < NQ; ++q)
                v[k][q] = row >= lo && row < hi
                              ? *reinterpret_cast<const float4*>(src + (row - a.base) * a.qkv_stride + 4 * q)
                              : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            float inv = 1.0f;
            if (a.v_norm) {
                float ss = 0.0f;
#pragma unroll
                for (int q = 0; q < NQ; ++q)
                    ss += v[k][q].x * v[k][q].x + v[k][q].y * v[k][q].y + v[k][q].z * v[k][q].z + v[k][q].w * v[k][q].w;
                inv = 1.0f / sqrtf(wave_sum(ss) / float(HD) + a.eps);
            }
#pragma unroll
            for (int q = 0; q < NQ; ++q) {
                half4 h = {half_t(v[k][q].x * inv), half_t(v[k][q].y * inv), half_t(v[k][q].z * inv),
                           half_t(v[k][q].w * inv)};
                *reinterpret_cast<half4*>(&tile_rows[16 * wave + k][e0 + 4 * q]) = h;
            }
        }
        __syncthreads();
#pragma unroll
        for (int dd = 0; dd < DPT; ++dd) {
            const int dim = int(threadIdx.x) + 256 * dd;
            half_t* dst = a.vt + ((int64_t(head) * (a.cap_pad / 64) + tile) * HD + dim) * 64;
            // Chunk (half hf, group m) holds keys 32hf + 4m + 0..3, then 32hf + 16 + 4m + 0..3.
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                const int hf = c / 4, m = c % 4;
                uint32_t h[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int key = 32 * hf + 16 * (j / 4) + 4 * m + j % 4;
                    h[j] = __builtin_bit_cast(uint16_t, tile_rows[key][dim]);
                    if (!whole && (r0 + key < lo || r0 + key >= hi)) {
                        const uint4 kc = kept[dd][c];
                        const uint32_t w = j / 2 == 0 ? kc.x : j / 2 == 1 ? kc.y : j / 2 == 2 ? kc.z : kc.w;
                        h[j] = (w >> (16 * (j % 2))) & 0xffffu;
                    }
                }
                const uint4 u = {h[0] | h[1] << 16, h[2] | h[3] << 16, h[4] | h[5] << 16, h[6] | h[7] << 16};
                reinterpret_cast<uint4*>(dst)[c] = u;
            }
        }
        return;
    }
    const int64_t id = (int64_t(blockIdx.x) - vblocks) * 4 + wave;
    if (id >= a.t * qk_slots) return;
    const int64_t tok = id / qk_slots;
    const int slot = int(id - tok * qk_slots);
    const int64_t row = a.base + tok;
    const bool is_q = slot < H;
    const int head = is_q ? slot : slot - H;
    int pos = a.meta[4 * row];
    pos = pos < 0 ? 0 : (pos >= a.rope_rows ? int(a.rope_rows - 1) : pos);
    const float* vsrc = a.qkv + tok * a.qkv_stride + int64_t(slot) * HD + e0;
    const float* wsrc = (is_q ? a.q_norm : a.k_norm) + e0;
    const int d0 = e0 % HALF;
    // (cos, sin) pairs of the lane's EPL dimensions: 2 * EPL floats.
    const float4* rt = reinterpret_cast<const float4*>(a.rope + int64_t(pos) * HALF + d0);
    float v[EPL], w[EPL], cs[EPL], sn[EPL];
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
        const float4 v4 = *reinterpret_cast<const float4*>(vsrc + 4 * q);
        const float4 w4 = *reinterpret_cast<const float4*>(wsrc + 4 * q);
        const float4 r01 = rt[2 * q], r23 = rt[2 * q + 1];
        v[4 * q] = v4.x, v[4 * q + 1] = v4.y, v[4 * q + 2] = v4.z, v[4 * q + 3] = v4.w;
        w[4 * q] = w4.x, w[4 * q + 1] = w4.y, w[4 * q + 2] = w4.z, w[4 * q + 3] = w4.w;
        cs[4 * q] = r01.x, cs[4 * q + 1] = r01.z, cs[4 * q + 2] = r23.x, cs[4 * q + 3] = r23.z;
        sn[4 * q] = r01.y, sn[4 * q + 1] = r01.w, sn[4 * q + 2] = r23.y, sn[4 * q + 3] = r23.w;
    }
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < EPL; ++i) ss += v[i] * v[i];
    const float inv = 1.0f / sqrtf(wave_sum(ss) / float(HD) + a.eps);
    float o[EPL];
#pragma unroll
    for (int i = 0; i < EPL; ++i) {
        const float y = v[i] * inv * w[i];
        const float partner = __shfl_xor(y, 32, WAVE);
        if (d0 + i < a.rope_dims / 2)
            o[i] = e0 < HALF ? y * cs[i] - partner * sn[i] : y * cs[i] + partner * sn[i];
        else
            o[i] = y;
    }
    half_t* dst = is_q ? a.q16 + (tok * H + head) * HD + e0 : a.kc + (int64_t(head) * a.cap_pad + row) * HD + e0;
    const float sc = is_q ? a.q_scale : 1.0f;
#pragma unroll
    for (int q = 0; q < NQ; ++q)
        *reinterpret_cast<half4*>(dst + 4 * q) = half4{half_t(o[4 * q] * sc), half_t(o[4 * q + 1] * sc),
                                                       half_t(o[4 * q + 2] * sc), half_t(o[4 * q + 3] * sc)};
}

void launch_qk_prep(hipStream_t s, const QkArgs& a) {
    if (a.t <= 0) return;
    if (a.base + a.t > a.cap_pad || a.cap_pad % 64) fail(E_INVALID, "qk_prep: cache rows out of range");
    if (a.hd != 256 && a.hd != 512) fail(E_INVALID, "qk_prep: head_dim must be 256 or 512");
    if (a.rope_rows <= 0 || a.rope_dims > a.hd) fail(E_INVALID, "qk_prep: rope table");
    const int qk_slots = a.heads + (a.has_kv ? a.kv_heads : 0);
    const int64_t tiles = a.has_kv ? (a.base + a.t + 63) / 64 - a.base / 64 : 0;
    const int64_t vblocks = tiles * a.kv_heads;
    const int64_t blocks = vblocks + (a.t * qk_slots + 3) / 4;
    if (a.hd == 512)
        qk_prep_kernel<512><<<dim3(unsigned(blocks)), dim3(256), 0, s>>>(a, vblocks, qk_slots);
    else
        qk_prep_kernel<256><<<dim3(unsigned(blocks)), dim3(256), 0, s>>>(a, vblocks, qk_slots);
    OMG_HIP(hipGetLastError());
}

__global__ __launch_bounds__(256) void rope_table_kernel(const float* inv_freq, int64_t rows, int64_t half,
                                                         float2* out) {
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= rows * half) return;
    const int64_t p = i / half, dd = i - p * half;
    const float ang = float(p) * inv_freq[dd];
    out[i] = make_float2(cosf(ang), sinf(ang));
}

void launch_rope_table(hipStream_t s, const float* inv_freq, int64_t rows, int64_t half, float2* out) {
    if (rows <= 0 || half <= 0) fail(E_INVALID, "rope table: empty");
    if (rows >= (int64_t(1) << 24)) fail(E_INVALID, "rope table: positions must stay below 2^24");
    rope_table_kernel<<<dim3(unsigned((rows * half + 255) / 256)), dim3(256), 0, s>>>(inv_freq, rows, half, out);
    OMG_HIP(hipGetLastError());
}

// -------------------------------------------------------------- readout

// The last layer's fused norm (engine.rs:1752-1758) applied at the wanted
// rows only: rows[i] = rmsnorm(x[wanted[i]]) * w in f32.
__global__ __launch_bounds__(256) void final_rows_kernel(const float* __restrict__ x,
                                                         const int32_t* __restrict__ wanted, int64_t n,
                                                         int64_t d, const float* __restrict__ w,
                                                         float eps, float* __restrict__ rows) {
    const int wave = int(threadIdx.x) / WAVE, lane = int(threadIdx.x) % WAVE;
    const int64_t i = int64_t(blockIdx.x) * 4 + wave;
    if (i >= n) return;
    const float* xr = x + (wanted ? int64_t(wanted[i]) : i) * d;  // no list: row i
    float ss = 0.0f;
    for (int64_t q = lane; q < d / 4; q += WAVE) {
        const float4 v = *reinterpret_cast<const float4*>(xr + 4 * q);
        ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
    }
    const float inv = 1.0f / sqrtf(wave_sum(ss) / float(d) + eps);
    for (int64_t q = lane; q < d / 4; q += WAVE) {
        const float4 v = *reinterpret_cast<const float4*>(xr + 4 * q);
        const float4 g = *reinterpret_cast<const float4*>(w + 4 * q);
        *reinterpret_cast<float4*>(rows + i * d + 4 * q) =
            make_float4(v.x * inv * g.x, v.y * inv * g.y, v.z * inv * g.z, v.w * inv * g.w);
    }
}

void launch_final_rows(hipStream_t s, const float* x, const int32_t* wanted, int64_t n, int64_t d,
                       const float* w, float eps, float* rows) {
    if (n <= 0) return;
    final_rows_kernel<<<dim3(unsigned((n + 3) / 4)), dim3(256), 0, s>>>(x, wanted, n, d, w, eps, rows);
    OMG_HIP(hipGetLastError());
}

// Rows rows[i] - r0 (i < n) of an f16 matrix of width wa, an f32 matrix of
// width wx and (p non-null) wp f32 columns from column po of an f32 matrix
// of row stride ps, copied to rows i of aw, xw and pw: one workgroup per
// row, 16 bytes per thread and step.
__global__ __launch_bounds__(256) void gather_out_kernel(const half_t* __restrict__ a, int64_t wa,
                                                         const float* __restrict__ x, int64_t wx,
                                                         const float* __restrict__ p, int64_t ps, int64_t po,
                                                         int64_t wp, const int32_t* __restrict__ rows, int64_t r0,
                                                         half_t* __restrict__ aw, float* __restrict__ xw,
                                                         float* __restrict__ pw) {
    const int64_t i = blockIdx.x, r = int64_t(rows[i]) - r0;
    const uint4* as = reinterpret_cast<const uint4*>(a + r * wa);
    uint4* ad = reinterpret_cast<uint4*>(aw + i * wa);
    for (int64_t q = threadIdx.x; q < wa / 8; q += blockDim.x) ad[q] = as[q];
    const float4* xs = reinterpret_cast<const float4*>(x + r * wx);
    float4* xd = reinterpret_cast<float4*>(xw + i * wx);
    for (int64_t q = threadIdx.x; q < wx / 4; q += blockDim.x) xd[q] = xs[q];
    if (p) {
        const float4* ps4 = reinterpret_cast<const float4*>(p + r * ps + po);
        float4* pd = reinterpret_cast<float4*>(pw + i * wp);
        for (int64_t q = threadIdx.x; q < wp / 4; q += blockDim.x) pd[q] = ps4[q];
    }
}

void launch_gather_out(hipStream_t s, const half_t* a, int64_t wa, const float* x, int64_t wx, const int32_t* rows,
                       int64_t r0, int64_t n, half_t* aw, float* xw, const float* p, int64_t ps, int64_t po,
                       int64_t wp, float* pw) {
    if (n <= 0) return;
    if (wa % 8 != 0 || wx % 4 != 0 || (p && (wp % 4 != 0 || ps % 4 != 0 || po % 4 != 0 || !pw)))
        fail(E_INVALID, "gather_out: widths must be multiples of 8 (f16) and 4 (f32)");
    gather_out_kernel<<<dim3(unsigned(n)), dim3(256), 0, s>>>(a, wa, x, wx, p, ps, po, wp, rows, r0, aw, xw, pw);
    OMG_HIP(hipGetLastError());
}

// logits.wgsl:38-79's product, rows . deq(E[col])^T in f32 (no f16
// rounding on this path, as in the reference), on v_mfma_f32_16x16x4_f32.
// A workgroup owns 64 output columns (vocabulary rows of E, or the label
// ids in `cols`), 16 per wave, and up to LG_R = 16 readout rows at a time:
// D[col][row] = sum_k E[col][k] x[row][k] with A = the decoded weights
// (lane l: column l % 16) and B = the rows from LDS.  Inside a 32-element
// block the K order is permuted alike in both operands: MFMA step s of
// lane group G = l / 16 takes element 8 G + s, so a lane decodes one Q4
// word (one Q8 pair, 16 bytes of f16) per block.  A column's sums do not
// depend on which columns share its wave: full rows, label columns and the
// log-sum-exp path give bit-equal logits.  With `part`, every workgroup
// also writes each row's (max, sum of exp(z - max)) over its 64 columns.
constexpr int LG_R = 16;     // readout rows per pass over K
constexpr int LG_KC = 512;   // K elements of the rows staged in LDS at once

// Elements 8 g .. 8 g + 7 of block b of column `col`, f32.
template <int DT>
__device__ inline void logit_octet(const DevWeight& E, int64_t col, int64_t b, int g, float w[8]) {
    const int64_t K = E.cols;
    if constexpr (DT == Q4_DT) {
        const float d = half_bits_to_f32(E.scales[col * E.sld + b]);
        const uint32_t word = static_cast<const uint32_t*>(E.data)[(col * (K / 32) + b) * 4 + g];
#pragma unroll
        for (int p = 0; p < 8; ++p) w[p] = q4_elem_f32(word, p, d);
    } else if constexpr (DT == Q8_DT) {
        const float d = half_bits_to_f32(E.scales[col * E.sld + b]);
        const uint2 u = *reinterpret_cast<const uint2*>(static_cast<const uint8_t*>(E.data) + col * K + b * 32 + 8 * g);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            w[k] = float(int8_t(u.x >> (8 * k))) * d;
            w[4 + k] = float(int8_t(u.y >> (8 * k))) * d;
        }
    } else {
        const uint4 u = *reinterpret_cast<const uint4*>(static_cast<const half_t*>(E.data) + col * K + b * 32 + 8 * g);
        const uint32_t words[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const half2v h = as_half2(words[k]);
            w[2 * k] = float(h.x);
            w[2 * k + 1] = float(h.y);
        }
    }
}

template <int DT>
__global__ __launch_bounds__(256) void logits_kernel(DevWeight E, const float* __restrict__ rows, int64_t nrows,
                                                     const uint32_t* __restrict__ cols, int64_t ncols, float softcap,
                                                     float* __restrict__ out, float2* __restrict__ part) {
    __shared__ __attribute__((aligned(16))) float xs[LG_R][LG_KC];
    __shared__ float red[4][LG_R][2];
    const int tid = int(threadIdx.x), lane = tid % WAVE;
    const int wave = __builtin_amdgcn_readfirstlane(tid / WAVE);
    const int lr = lane % 16, G = lane / 16;
    // A operand: column wave * 16 + lr of the workgroup's 64
    const int64_t ja = int64_t(blockIdx.x) * 64 + wave * 16 + lr;
    const int64_t col = ja < ncols ? (cols ? int64_t(cols[ja]) : ja) : 0;  // idle columns read row 0, dropped
    // D: columns wave * 16 + 4 G + r, row lr
    const int64_t jd = int64_t(blockIdx.x) * 64 + wave * 16 + 4 * G;
    const int64_t K = E.cols;
    for (int64_t r0 = 0; r0 < nrows; r0 += LG_R) {
        const int nr = int(nrows - r0 < LG_R ? nrows - r0 : LG_R);
        floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int64_t k0 = 0; k0 < K; k0 += LG_KC) {
            const int kc = int(K - k0 < LG_KC ? K - k0 : LG_KC);
            __syncthreads();  // the previous chunk's reads are done
            for (int i = tid; i < LG_R * (kc / 4); i += 256) {
                const int r = i / (kc / 4), c4 = i % (kc / 4);
                const float4 v = r < nr ? *reinterpret_cast<const float4*>(rows + (r0 + r) * K + k0 + 4 * c4)
                                        : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                *reinterpret_cast<float4*>(&xs[r][4 * c4]) = v;
            }
            __syncthreads();
            for (int bl = 0; bl < kc / 32; ++bl) {
                float w[8];
                logit_octet<DT>(E, col, k0 / 32 + bl, G, w);
                const float4 x0 = *reinterpret_cast<const float4*>(&xs[lr][bl * 32 + 8 * G]);
                const float4 x1 = *reinterpret_cast<const float4*>(&xs[lr][bl * 32 + 8 * G + 4]);
                const float x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
                for (int st = 0; st < 8; ++st) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(w[st], x[st], acc, 0, 0, 0);
            }
        }
        // lane: row lr, columns jd .. jd + 3
        const bool row_ok = lr < nr;
        float z[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            z[r] = acc[r];
            if (softcap > 0.0f) z[r] = softcap * tanhf(z[r] / softcap);
        }
        if (row_ok) {
            float* dst = out + (r0 + lr) * ncols + jd;
            // (rows of a width that is not a multiple of 4 start off the
            // 16-byte grid: those go out as single floats)
            if (jd + 3 < ncols && (reinterpret_cast<uintptr_t>(dst) & 15) == 0) {
                *reinterpret_cast<float4*>(dst) = make_float4(z[0], z[1], z[2], z[3]);
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (jd + r < ncols) dst[r] = z[r];
            }
        }
        if (part) {
            // per row: max and sum of exp over the workgroup's 64 columns,
            // lanes (row, G) then waves in a fixed order
            float m = -INFINITY;
#pragma unroll
            for (int r = 0; r < 4; ++r) m = fmaxf(m, jd + r < ncols ? z[r] : -INFINITY);
            m = max_lanes_16_32(m);
            if (G == 0) red[wave][lr][0] = m;
            __syncthreads();
            m = fmaxf(fmaxf(red[0][lr][0], red[1][lr][0]), fmaxf(red[2][lr][0], red[3][lr][0]));
            float e = 0.0f;
#pragma unroll
            for (int r = 0; r < 4; ++r) e += jd + r < ncols ? expf(z[r] - m) : 0.0f;
            e = sum_lanes_16_32(e);
            if (G == 0) red[wave][lr][1] = e;
            __syncthreads();
            if (wave == 0 && G == 0 && row_ok)
                part[int64_t(blockIdx.x) * nrows + r0 + lr] =
                    make_float2(m, ((red[0][lr][1] + red[1][lr][1]) + red[2][lr][1]) + red[3][lr][1]);
        }
    }
}

void launch_logits(hipStream_t s, const DevWeight& E, const float* rows, int64_t nrows, const uint32_t* cols,
                   int64_t ncols, float softcap, float* out, float2* part) {
    if (nrows <= 0 || ncols <= 0) return;
    if (E.cols % 32 != 0) fail(E_INVALID, "logits: width must be a multiple of 32");
    if (reinterpret_cast<uintptr_t>(rows) % 16 != 0 || reinterpret_cast<uintptr_t>(out) % 4 != 0 ||
        reinterpret_cast<uintptr_t>(part) % 8 != 0)
        fail(E_INVALID, "logits: rows must be 16-byte aligned, the output 4-byte and the partials 8-byte aligned");
    const dim3 grid(unsigned((ncols + WAVE - 1) / WAVE)), block(256);
    switch (E.dtype) {
        case F16_DT: logits_kernel<F16_DT><<<grid, block, 0, s>>>(E, rows, nrows, cols, ncols, softcap, out, part); break;
        case Q8_DT: logits_kernel<Q8_DT><<<grid, block, 0, s>>>(E, rows, nrows, cols, ncols, softcap, out, part); break;
        default: logits_kernel<Q4_DT><<<grid, block, 0, s>>>(E, rows, nrows, cols, ncols, softcap, out, part); break;
    }
    OMG_HIP(hipGetLastError());
}

int64_t logits_blocks(int64_t ncols) { return (ncols + WAVE - 1) / WAVE; }

// Readout::distribution's inputs per row (readout.rs:124-146): the label
// columns of a full logits row and the row's log-sum-exp, from the logits
// kernel's per-workgroup (max, sum of exp) pairs: M = max of the maxima,
// lse = M + log(sum_b s_b exp(m_b - M)), in f32 (the reference sums the
// row in f64 on the host; over 25,000 terms the two agree to a few 1e-7
// relative).  One workgroup per row, the pairs summed in a fixed order.
// A label id outside the vocabulary reads nothing and gives NaN (the
// engine refuses such ids on the host; device-resident ids of the
// kernel-level entry point are not checked before the launch).
__global__ __launch_bounds__(256) void label_lse_kernel(const float* __restrict__ logits, int64_t vocab,
                                                        const float2* __restrict__ part, int64_t nblocks,
                                                        int64_t nrows, const uint32_t* __restrict__ labels,
                                                        int64_t nlabels, float* __restrict__ out) {
    __shared__ float red[256 / WAVE];
    const int64_t r = blockIdx.x;
    const int tid = int(threadIdx.x), wave = tid / WAVE, lane = tid % WAVE;
    float m = -INFINITY;
    for (int64_t b = tid; b < nblocks; b += 256) m = fmaxf(m, part[b * nrows + r].x);
    m = wave_max(m);
    if (lane == 0) red[wave] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    float sum = 0.0f;
    for (int64_t b = tid; b < nblocks; b += 256) {
        const float2 p = part[b * nrows + r];
        sum += p.y * expf(p.x - m);
    }
    sum = wave_sum(sum);
    if (lane == 0) red[wave] = sum;
    __syncthreads();
    const float* row = logits + r * vocab;
    float* o = out + r * (nlabels + 1);
    for (int64_t i = tid; i < nlabels; i += 256) {
        const uint32_t c = labels[i];
        o[i] = int64_t(c) < vocab ? row[c] : __builtin_nanf("");
    }
    if (tid == 0) o[nlabels] = m + logf((red[0] + red[1]) + (red[2] + red[3]));
}

void launch_label_lse(hipStream_t s, const float* logits, int64_t nrows, int64_t vocab, const float2* part,
                      int64_t nblocks, const uint32_t* labels, int64_t nlabels, float* out) {
    if (nrows <= 0) return;
    if (vocab <= 0 || nlabels <= 0 || nblocks <= 0) fail(E_INVALID, "label_lse: empty row or no labels");
    label_lse_kernel<<<dim3(unsigned(nrows)), dim3(256), 0, s>>>(logits, vocab, part, nblocks, nrows, labels,
                                                                 nlabels, out);
    OMG_HIP(hipGetLastError());
}

// ------------------------------------------------------ pointer readout

// readout.rs:30-36 (PointerHead::project) for the rows that have a map: one
// workgroup per row, the row in LDS, each wave one output at a time (its
// weight row read once, coalesced, and summed across the wave).
__global__ __launch_bounds__(256) void pointer_project_kernel(const float* __restrict__ rows, int64_t d,
                                                              const float* __restrict__ w,
                                                              const float* __restrict__ b, int64_t dp,
                                                              const int32_t* __restrict__ mat,
                                                              float* __restrict__ proj) {
    extern __shared__ float h[];
    const int64_t r = blockIdx.x;
    const int m = mat[r];
    if (m < 0) return;
    const int wave = int(threadIdx.x) / WAVE, lane = int(threadIdx.x) % WAVE;
    for (int64_t i = threadIdx.x; i < d; i += blockDim.x) h[i] = rows[r * d + i];
    __syncthreads();
    const float* W = w + int64_t(m) * dp * d;
    for (int64_t o = wave; o < dp; o += blockDim.x / WAVE) {
        float acc = 0.0f;
        for (int64_t i = lane; i < d; i += WAVE) acc += W[o * d + i] * h[i];
        acc = wave_sum(acc);
        if (lane == 0) proj[r * dp + o] = acc + b[int64_t(m) * dp + o];
    }
}

// readout.rs:37-44 (PointerHead::logits): one wave per (option, decide) pair.
__global__ __launch_bounds__(256) void pointer_logits_kernel(const float* __restrict__ proj, int64_t dp,
                                                             const int2* __restrict__ pairs, int64_t npairs,
                                                             float scale, float* __restrict__ out) {
    const int64_t i = int64_t(blockIdx.x) * (blockDim.x / WAVE) + int(threadIdx.x) / WAVE;
    if (i >= npairs) return;
    const int lane = int(threadIdx.x) % WAVE;
    const int2 pr = pairs[i];
    const float* k = proj + int64_t(pr.x) * dp;
    const float* q = proj + int64_t(pr.y) * dp;
    float acc = 0.0f;
    for (int64_t j = lane; j < dp; j += WAVE) acc += k[j] * q[j];
    acc = wave_sum(acc);
    if (lane == 0) out[i] = acc * scale;
}

void launch_pointer(hipStream_t s, const float* rows, int64_t nrows, int64_t d, const float* w, const float* b,
                    int64_t dp, const int32_t* mat, float* proj, const int2* pairs, int64_t npairs, float* out) {
    if (nrows <= 0) return;
    if (d <= 0 || d > 16384 || dp <= 0) fail(E_INVALID, "pointer: width out of range");
    pointer_project_kernel<<<dim3(unsigned(nrows)), dim3(256), size_t(d) * 4, s>>>(rows, d, w, b, dp, mat, proj);
    OMG_HIP(hipGetLastError());
    if (npairs <= 0) return;
    const float scale = 1.0f / std::sqrt(float(dp));
    pointer_logits_kernel<<<dim3(unsigned((npairs + 3) / 4)), dim3(256), 0, s>>>(proj, dp, pairs, npairs, scale, out);
    OMG_HIP(hipGetLastError());
}

// ------------------------------------------- readout without allocation

// Scratch of launch_label_readout_noalloc: the full logits rows, then the
// logits kernel's (max, sum of exp) pairs.  A file-scope device array, so
// every GPU the library runs on holds its own copy (16 MiB) until the
// process ends; calls that overlap on one GPU share it and race.  Nothing
// in it needs to start at zero: both parts are written whole before they
// are read.
constexpr int64_t READOUT_SCRATCH_FLOATS = int64_t(4) << 20;
static __device__ __align__(256) float scratch[READOUT_SCRATCH_FLOATS];

// The array's device address on the current GPU, looked up once per device
// (in host code `scratch` names a host-side stand-in, not device memory).
static float* readout_scratch() {
    int dev = 0;
    OMG_HIP(hipGetDevice(&dev));
    constexpr int MAX_DEV = 64;
    if (dev < 0 || dev >= MAX_DEV) fail(E_DEVICE, "label_readout_noalloc: device index out of range");
    static std::mutex mu;
    static float* ptr[MAX_DEV] = {};
    std::lock_guard<std::mutex> lock(mu);
    if (!ptr[dev]) {
        void* p = nullptr;
        OMG_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (!p) fail(E_DEVICE, "label_readout_noalloc: no device address for the scratch array");
        ptr[dev] = static_cast<float*>(p);
    }
    return ptr[dev];
}

int64_t label_readout_scratch_floats() { return READOUT_SCRATCH_FLOATS; }

void launch_label_readout_noalloc(hipStream_t s, const DevWeight& E, const float* rows, int64_t nrows,
                                  const uint32_t* labels, int64_t nlabels, float softcap, float* out) {
    if (nrows <= 0 || nlabels <= 0) fail(E_INVALID, "label readout: no rows or no labels");
    const int64_t vocab = E.rows, nb = logits_blocks(vocab);
    const int64_t nlog = (nrows * vocab + 1) / 2 * 2;  // float2 partials on an 8-byte boundary
    if (nlog + 2 * nb * nrows > READOUT_SCRATCH_FLOATS)
        fail(E_CAPACITY, "label_readout_noalloc: " + std::to_string(nrows) + " rows x " + std::to_string(vocab) +
                             " logits exceed the " + std::to_string(READOUT_SCRATCH_FLOATS) + "-float scratch");
    float* base = readout_scratch();
    float2* part = reinterpret_cast<float2*>(base + nlog);
    launch_logits(s, E, rows, nrows, nullptr, vocab, softcap, base, part);
    launch_label_lse(s, base, nrows, vocab, part, nb, labels, nlabels, out);
}

// ---------------------------------------------------------- state rows

// engine.rs:499-502: a state row is every K head then every V head of one
// token, f16.  The cache keeps K row-major and V in 64-row transposed tiles.
__global__ void kv_gather_kernel(const half_t* __restrict__ kc, const half_t* __restrict__ vt,
                                 int64_t cap_pad, int kvh, int hd, int64_t row0, int64_t rows,
                                 half_t* __restrict__ out) {
    const int64_t width = int64_t(2) * kvh * hd;
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= rows * width) return;
    const int64_t r = i / width, c = i % width, row = row0 + r;
    const int64_t g = (c / hd) % kvh, e = c % hd;
    if (c < int64_t(kvh) * hd)
        out[i] = kc[(g * cap_pad + row) * hd + e];
    else
        out[i] = vt[((g * (cap_pad / 64) + row / 64) * hd + e) * 64 + vt_col(row)];
}

__global__ void kv_scatter_kernel(half_t* __restrict__ kc, half_t* __restrict__ vt, int64_t cap_pad,
                                  int kvh, int hd, int64_t row0, int64_t rows,
                                  const half_t* __restrict__ in) {
    const int64_t width = int64_t(2) * kvh * hd;
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= rows * width) return;
    const int64_t r = i / width, c = i % width, row = row0 + r;
    const int64_t g = (c / hd) % kvh, e = c % hd;
    if (c < int64_t(kvh) * hd)
        kc[(g * cap_pad + row) * hd + e] = in[i];
    else
        vt[((g * (cap_pad / 64) + row / 64) * hd + e) * 64 + vt_col(row)] = in[i];
}

void launch_kv_gather(hipStream_t s, const half_t* kc, const half_t* vt, int64_t cap_pad, int kv_heads,
                      int hd, int64_t row0, int64_t rows, half_t* out) {
    if (rows <= 0) return;
    if (row0 < 0 || row0 + rows > cap_pad) fail(E_INVALID, "kv_gather: rows out of range");
    const int64_t n = rows * 2 * kv_heads * hd;
    kv_gather_kernel<<<dim3(unsigned((n + 255) / 256)), dim3(256), 0, s>>>(kc, vt, cap_pad, kv_heads, hd,
                                                                          row0, rows, out);
    OMG_HIP(hipGetLastError());
}

void launch_kv_scatter(hipStream_t s, half_t* kc, half_t* vt, int64_t cap_pad, int kv_heads, int hd,
                       int64_t row0, int64_t rows, const half_t* in) {
    if (rows <= 0) return;
    if (row0 < 0 || row0 + rows > cap_pad) fail(E_INVALID, "kv_scatter: rows out of range");
    const int64_t n = rows * 2 * kv_heads * hd;
    kv_scatter_kernel<<<dim3(unsigned((n + 255) / 256)), dim3(256), 0, s>>>(kc, vt, cap_pad, kv_heads, hd,
                                                                           row0, rows, in);
    OMG_HIP(hipGetLastError());
}

// --------------------------------------------------------------- repack

void repack_q4(const uint8_t* src, uint8_t* dst, int64_t n) {
    for (int64_t b = 0; b < n / 32; ++b) {
        const uint8_t* in = src + 16 * b;
        uint8_t q[32];
        for (int j = 0; j < 16; ++j) {
            q[j] = in[j] & 0xf;
            q[j + 16] = in[j] >> 4;
        }
        for (int w = 0; w < 4; ++w) {
            uint32_t word = 0;
            for (int p = 0; p < 8; ++p) {
                const int sh = (p & 1) ? 16 + 4 * (p >> 1) : 4 * (p >> 1);
                word |= uint32_t(q[8 * w + p]) << sh;
            }
            std::memcpy(dst + 16 * b + 4 * w, &word, 4);
        }
    }
}

}  // namespace omg
