// Block-causal GQA attention over the f16 K/V cache (attention.wgsl's job):
// a query sees a key iff both are in the same group of the pass, the key is
// in the group's prefix or the query's own branch, at or before the
// query's position and, on sliding layers, less than `window` positions
// back (attention.wgsl:70-76).  Online softmax in f32, flash style.
//
// Work split: a work item is one query tile (64 rows = (64 / hpg) tokens x
// the hpg query heads sharing one KV head, 16 rows per wave) and a range of
// 64-key tiles; the host builds the item lists from the pass's metadata
// (AttnWork).  On global layers the key range is cut at fixed multiples of
// `chunk` tiles and the per-chunk partial results are merged in key order
// by attention_merge; on sliding layers one item covers the whole range.
// Because chunk boundaries are absolute cache rows and a tile that a query
// cannot see leaves its state exactly unchanged, each query's arithmetic
// is the same whichever tokens share its tile: rows over a resident prefix
// are bit-equal to a full pass.
//
// Per item: K and V tiles are double-buffered in LDS; the next tile's
// global loads are issued into registers before the current tile's MFMAs
// and stored after them, one barrier per tile.  A wave that sees no key of
// a tile skips it; a wave that sees every key of it skips the masking.
//
// Both products run on v_mfma_f32_16x16x32_f16 arranged so that no operand
// needs a register transpose:
//   S^T[key][q] = K[key][:] . Q[q][:]   (A = K rows from LDS, B = Q from
//                 registers): lane l holds S[q = l%16][keys 16j + 4(l/16) + r];
//   O^T[c][q]  += V^T[c][key] . P^T[key][q]  (A = V^T from the cache's
//                 transposed tiles, B = the lane's own probabilities).
// A lane owns one query row for the softmax statistics and the output, so
// the running max and sum need only the 4 lanes of that row.
#include <climits>
#include <string>

#include "common.h"
#include "kern_common.h"

namespace omg {

constexpr int A_KT = 64;  // keys per tile
constexpr int A_THREADS = 256;
constexpr int A_ROWS = 64;  // query rows per tile

__device__ inline bool visible(int qp, int qs, int kp, int ks, int window) {
    const bool same_group = ((ks ^ qs) >> 12) == 0;
    return same_group && ((ks & 0xfff) == 0 || ks == qs) && kp <= qp &&
           (window == 0 || unsigned(qp - kp) < unsigned(window));
}

// LDS of one work item.  K and V^T tiles are stored without padding; the
// 16-byte chunks of each row are XOR-swizzled so that the MFMA operand reads
// (16 lanes on 16 consecutive rows at one logical chunk) hit 16 distinct
// bank groups:
//   K   [64 keys][HD]:  physical chunk = logical ^ (row & 15)  (32-chunk rows)
//   V^T [HD][64 keys]:  physical chunk = logical ^ ((row >> 1) & 7)  (8-chunk rows)
template <int HD>
struct AttnSmem {
    half_t k[2][A_KT * HD];
    half_t v[2][HD * A_KT];
    int kpos[2][A_KT];
    int kseq[2][A_KT];
    int qpos[A_ROWS];
    int qseq[A_ROWS];
};

typedef __attribute__((address_space(3))) void* lds_void_ptr;
typedef __attribute__((address_space(1))) void* global_void_ptr;

// Issue this wave's share of one K/V tile as direct global -> LDS loads
// (global_load_lds_dwordx4: lane i of an instruction writes 16 bytes at LDS
// base + 16 i).  Every lane picks the global chunk that belongs at its LDS
// slot, which is how the swizzle is applied.
template <int HD>
__device__ __attribute__((always_inline)) inline void dma_tile(AttnSmem<HD>& sm, int buf, const half_t* kt,
                                                               const half_t* vt, int wave, int lane) {
    constexpr int KROW = HD / 8;                     // 16 B chunks per K row
    constexpr int KINS = A_KT * HD / 8 / WAVE / 4;   // instructions per wave for K
    constexpr int VINS = HD * A_KT / 8 / WAVE / 4;
#pragma unroll
    for (int i = 0; i < KINS; ++i) {
        const int blk = wave * KINS + i;            // 1 KB block of the tile
        const int slot = blk * WAVE + lane;         // physical chunk index in the tile
        const int row = slot / KROW, pc = slot % KROW;
        const int lc = pc ^ (row & 15);
        __builtin_amdgcn_global_load_lds((global_void_ptr)(kt + row * HD + lc * 8),
                                         (lds_void_ptr)(sm.k[buf] + blk * WAVE * 8), 16, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < VINS; ++i) {
        const int blk = wave * VINS + i;
        const int slot = blk * WAVE + lane;
        const int row = slot / (A_KT / 8), pc = slot % (A_KT / 8);
        const int lc = pc ^ ((row >> 1) & 7);
        __builtin_amdgcn_global_load_lds((global_void_ptr)(vt + row * A_KT + lc * 8),
                                         (lds_void_ptr)(sm.v[buf] + blk * WAVE * 8), 16, 0, 0);
    }
}

template <int HD>
__global__ __launch_bounds__(A_THREADS) void attention_kernel(AttnArgs a, const int4* __restrict__ items) {
    using SM = AttnSmem<HD>;
    constexpr int DS = HD / 32;  // MFMA steps over the head dim
    constexpr int CT = HD / 16;  // 16-wide output column tiles
    constexpr float LOG2E = 1.4426950408889634f;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem_raw[];
    SM& sm = *reinterpret_cast<SM*>(smem_raw);

    const int4 item = items[blockIdx.x];
    const int qtile = item.x, tb = item.y, te = item.z, slot = item.w;
    const int tid = int(threadIdx.x), wave = tid / WAVE, lane = tid % WAVE;
    const int H = a.heads, hpg = a.heads / a.kv_heads, tpw = 16 / hpg, tpb = 4 * tpw;
    const int g = int(blockIdx.y);
    const int64_t tok0 = int64_t(qtile) * tpb;
    const int lr = lane % 16, G = lane / 16;
    const int64_t tq = tok0 + wave * tpw + lr / hpg;
    const int head = g * hpg + lr % hpg;
    const bool valid = tq < a.t;
    const int64_t kend = a.base + a.t;  // cache rows holding keys

    if (tid < tpb) {
        const int64_t tk = tok0 + tid;
        if (tk < a.t) {
            const int4 m = reinterpret_cast<const int4*>(a.meta)[a.base + tk];
            sm.qpos[tid] = m.x;
            sm.qseq[tid] = m.y;
        } else {
            sm.qpos[tid] = -1;  // sees nothing: every key position is >= 0
            sm.qseq[tid] = -2;
        }
    }
    int qp = -1, qsq = -2;
    if (valid) {
        const int4 m = reinterpret_cast<const int4*>(a.meta)[a.base + tq];
        qp = m.x;
        qsq = m.y;
    }

    half8 qf[DS];
#pragma unroll
    for (int s = 0; s < DS; ++s)
        qf[s] = valid ? *reinterpret_cast<const half8*>(a.q16 + (tq * H + head) * HD + s * 32 + G * 8) : half8{};
    floatx4 o[CT];
#pragma unroll
    for (int c = 0; c < CT; ++c) o[c] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    float m_run = -INFINITY, l_run = 0.0f;

    const half_t* kbase = a.kc + int64_t(g) * a.cap_pad * HD;
    const half_t* vbase = a.vt + int64_t(g) * (a.cap_pad / 64) * HD * 64;
    // Key metadata of the next tile travels in registers (threads < 64).
    int2 km = make_int2(INT_MAX, -3);
    auto key_meta = [&](int tile) {
        const int64_t row = int64_t(tile) * A_KT + tid;
        km = make_int2(INT_MAX, -3);
        if (tid < A_KT && row < kend) {
            const int4 m = reinterpret_cast<const int4*>(a.meta)[row];
            km = make_int2(m.x, m.y);
        }
    };
    if (tb < te) {
        dma_tile<HD>(sm, 0, kbase + int64_t(tb) * A_KT * HD, vbase + int64_t(tb) * HD * A_KT, wave, lane);
        key_meta(tb);
    }
    for (int tile = tb; tile < te; ++tile) {
        const int cur = (tile - tb) & 1;
        // This wave's loads of `tile` are the only ones outstanding.
        __builtin_amdgcn_s_waitcnt(0);
        if (tid < A_KT) {
            sm.kpos[cur][tid] = km.x;
            sm.kseq[cur][tid] = km.y;
        }
        // Every wave's part of `tile` has landed, and every wave is done
        // with the other buffer (tile - 1), which the next loads overwrite.
        __syncthreads();
        if (tile + 1 < te) {
            dma_tile<HD>(sm, cur ^ 1, kbase + int64_t(tile + 1) * A_KT * HD, vbase + int64_t(tile + 1) * HD * A_KT,
                         wave, lane);
            key_meta(tile + 1);
        }
        // Which of this tile's keys the wave's queries see.
        bool any = false, all = true;
        {
            const int kp = sm.kpos[cur][lane], ks = sm.kseq[cur][lane];
            for (int u = 0; u < tpw; ++u) {
                const bool v = visible(sm.qpos[wave * tpw + u], sm.qseq[wave * tpw + u], kp, ks, a.window);
                any |= v;
                all &= v;
            }
        }
        if (__ballot(any) != 0ull) {
            const bool full = __ballot(!all) == 0ull;
            const half_t* K = sm.k[cur];
            floatx4 sacc[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                sacc[j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int s = 0; s < DS; ++s) {
                    const int pc = (s * 4 + G) ^ lr;  // row & 15 == lr
                    const half8 kf = *reinterpret_cast<const half8*>(K + (j * 16 + lr) * HD + pc * 8);
                    sacc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf[s], sacc[j], 0, 0, 0);
                }
            }
            float mt = -INFINITY;
            if (full) {
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        sacc[j][r] *= LOG2E;
                        mt = fmaxf(mt, sacc[j][r]);
                    }
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int4 kp4 = *reinterpret_cast<const int4*>(sm.kpos[cur] + j * 16 + G * 4);
                    const int4 ks4 = *reinterpret_cast<const int4*>(sm.kseq[cur] + j * 16 + G * 4);
                    const int kpv[4] = {kp4.x, kp4.y, kp4.z, kp4.w};
                    const int ksv[4] = {ks4.x, ks4.y, ks4.z, ks4.w};
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float sv =
                            visible(qp, qsq, kpv[r], ksv[r], a.window) ? sacc[j][r] * LOG2E : -INFINITY;
                        sacc[j][r] = sv;
                        mt = fmaxf(mt, sv);
                    }
                }
            }
            mt = fmaxf(mt, __shfl_xor(mt, 16, WAVE));
            mt = fmaxf(mt, __shfl_xor(mt, 32, WAVE));
            const float m_new = fmaxf(m_run, mt);
            float alpha = 1.0f;
            half8 pb[2];
            float psum = 0.0f;
            if (m_new == -INFINITY) {
                pb[0] = half8{};
                pb[1] = half8{};
            } else {
                alpha = exp2f(m_run - m_new);
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const half_t p = half_t(exp2f(sacc[j][r] - m_new));
                        psum += float(p);
                        pb[j / 2][(j % 2) * 4 + r] = p;
                    }
            }
            l_run = l_run * alpha + psum;
            m_run = m_new;
            if (__ballot(alpha != 1.0f) != 0ull) {
#pragma unroll
                for (int c = 0; c < CT; ++c) o[c] *= alpha;
            }
            const half_t* V = sm.v[cur];
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
                for (int c = 0; c < CT; ++c) {
                    const int row = c * 16 + lr, sw = (row >> 1) & 7;
                    const half_t* vr = V + row * A_KT + (G & 1) * 4;
                    const half4 lo = *reinterpret_cast<const half4*>(vr + (((tt * 4 + (G >> 1)) ^ sw) * 8));
                    const half4 hi = *reinterpret_cast<const half4*>(vr + (((tt * 4 + 2 + (G >> 1)) ^ sw) * 8));
                    const half8 vf = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
                    o[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pb[tt], o[c], 0, 0, 0);
                }
            }
        }
    }

    float l = l_run + __shfl_xor(l_run, 16, WAVE);
    l += __shfl_xor(l, 32, WAVE);
    const int row = wave * 16 + lr;
    if (slot >= 0) {
        // Partial result of this chunk: unnormalised O (f32), max and sum.
        float* op = a.part_o + (int64_t(slot) * A_ROWS + row) * HD + G * 4;
#pragma unroll
        for (int c = 0; c < CT; ++c) *reinterpret_cast<floatx4*>(op + c * 16) = o[c];
        if (G == 0) {
            a.part_ml[(int64_t(slot) * A_ROWS + row) * 2] = m_run;
            a.part_ml[(int64_t(slot) * A_ROWS + row) * 2 + 1] = l;
        }
        return;
    }
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    if (valid) {
        half_t* dst = a.out + (tq * H + head) * HD + G * 4;
#pragma unroll
        for (int c = 0; c < CT; ++c) {
            const half4 v = {half_t(o[c][0] * inv), half_t(o[c][1] * inv), half_t(o[c][2] * inv),
                             half_t(o[c][3] * inv)};
            *reinterpret_cast<half4*>(dst + c * 16) = v;
        }
    }
}

// Merge the chunk partials of one query tile in key order:
// out = sum_c O_c 2^(m_c - M) / sum_c l_c 2^(m_c - M), M = max_c m_c, over
// the chunks the row saw anything in.  A row with one such chunk gets
// exactly O / l, as if its tile had not been split.
template <int HD>
__global__ __launch_bounds__(256) void attention_merge_kernel(AttnArgs a, const int4* __restrict__ merges) {
    const int4 mg = merges[blockIdx.x];
    const int qtile = mg.x, slot0 = mg.y, n = mg.z;
    const int row = int(threadIdx.x) / 4, quarter = int(threadIdx.x) % 4;
    const int hpg = a.heads / a.kv_heads, tpw = 16 / hpg, tpb = 4 * tpw;
    const int wave = row / 16, lr = row % 16;
    const int64_t tq = int64_t(qtile) * tpb + wave * tpw + lr / hpg;
    const int head = int(blockIdx.y) * hpg + lr % hpg;
    if (tq >= a.t) return;
    float M = -INFINITY;
    for (int c = 0; c < n; ++c) M = fmaxf(M, a.part_ml[(int64_t(slot0 + c) * A_ROWS + row) * 2]);
    constexpr int W = HD / 4;
    float acc[W];
#pragma unroll
    for (int i = 0; i < W; ++i) acc[i] = 0.0f;
    float L = 0.0f;
    for (int c = 0; c < n; ++c) {
        const int64_t base = int64_t(slot0 + c) * A_ROWS + row;
        const float m = a.part_ml[base * 2];
        if (m == -INFINITY) continue;
        const float w = exp2f(m - M);
        L += a.part_ml[base * 2 + 1] * w;
        const float* op = a.part_o + base * HD + quarter * W;
#pragma unroll
        for (int i = 0; i < W; i += 4) {
            const float4 v = *reinterpret_cast<const float4*>(op + i);
            acc[i] += v.x * w;
            acc[i + 1] += v.y * w;
            acc[i + 2] += v.z * w;
            acc[i + 3] += v.w * w;
        }
    }
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    half_t* dst = a.out + (tq * a.heads + head) * HD + quarter * W;
#pragma unroll
    for (int i = 0; i < W; i += 4) {
        const half4 v = {half_t(acc[i] * inv), half_t(acc[i + 1] * inv), half_t(acc[i + 2] * inv),
                         half_t(acc[i + 3] * inv)};
        *reinterpret_cast<half4*>(dst + i) = v;
    }
}

void attention_work(const int32_t* meta, int64_t t, int heads, int kv_heads, int window, int chunk,
                    AttnWork& w) {
    w.items.clear();
    w.merges.clear();
    const int hpg = heads / kv_heads, tpb = 4 * (16 / hpg);
    int slot = 0;
    for (int64_t q0 = 0, qt = 0; q0 < t; q0 += tpb, ++qt) {
        int64_t lo = INT64_MAX, hi = 0;
        for (int64_t i = q0; i < t && i < q0 + tpb; ++i) {
            const int32_t* m = meta + 4 * i;
            const int64_t l = int64_t(m[2]) + (window > 0 ? std::max<int64_t>(0, int64_t(m[0]) - window + 1) : 0);
            lo = std::min(lo, l);
            hi = std::max(hi, int64_t(m[3]));
        }
        const int t0 = int(lo / A_KT), t1 = int((hi + A_KT - 1) / A_KT);
        if (chunk <= 0 || t1 - t0 <= 0 || (t0 / chunk) == ((t1 - 1) / chunk)) {
            w.items.push_back({int(qt), t0, t1, -1});
            continue;
        }
        const int first = slot;
        for (int c = t0 / chunk; c <= (t1 - 1) / chunk; ++c) {
            w.items.push_back({int(qt), std::max(t0, c * chunk), std::min(t1, (c + 1) * chunk), slot++});
        }
        w.merges.push_back({int(qt), first, slot - first, 0});
    }
    w.slots = slot;
}

void launch_attention(hipStream_t s, const AttnArgs& a, const int4* items, int64_t nitems, const int4* merges,
                      int64_t nmerges) {
    if (a.t <= 0 || nitems <= 0) return;
    if (a.hd != 256) fail(E_INVALID, "attention: head_dim must be 256");
    if (a.kv_heads <= 0 || a.heads % a.kv_heads) fail(E_INVALID, "attention: heads / kv_heads");
    const int hpg = a.heads / a.kv_heads;
    if (16 % hpg) fail(E_INVALID, "attention: query heads per KV head must divide 16");
    if (a.cap_pad % A_KT || a.base + a.t > a.cap_pad) fail(E_INVALID, "attention: cache rows out of range");
    if (a.window < 0) fail(E_INVALID, "attention: negative window");
    const size_t smem = sizeof(AttnSmem<256>);
    static bool attr_set = false;
    if (!attr_set) {
        OMG_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&attention_kernel<256>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, int(smem)));
        attr_set = true;
    }
    attention_kernel<256><<<dim3(unsigned(nitems), unsigned(a.kv_heads)), dim3(A_THREADS), smem, s>>>(a, items);
    OMG_HIP(hipGetLastError());
    if (nmerges > 0) {
        attention_merge_kernel<256><<<dim3(unsigned(nmerges), unsigned(a.kv_heads)), dim3(256), 0, s>>>(a, merges);
        OMG_HIP(hipGetLastError());
    }
}

}  // namespace omg
