// Block-causal GQA attention over the f16 K/V cache (attention.wgsl's job):
// a query sees a key iff both are in the same group of the pass, the key is
// in the group's prefix or the query's own branch, at or before the
// query's position and, on sliding layers, less than `window` positions
// back (attention.wgsl:70-76).  Online softmax in f32, flash style.
//
// Work split: a workgroup of 4 wave64s owns 64 query rows of one KV head;
// each wave owns 16 rows = (16 / hpg) tokens x the hpg query heads sharing
// that KV head, so every K/V tile the workgroup stages in LDS is used by
// 64 rows.  Keys stream 64 at a time from the range the workgroup's tokens
// can see: from their group's first cache row (raised by the window on
// sliding layers) to the last of their own rows.  A wave that sees no key
// of a tile skips it.
//
// Both products run on v_mfma_f32_16x16x32_f16 and are arranged so that no
// operand needs a transpose in registers:
//   S^T[key][q] = K[key][:] . Q[q][:]   (A = K rows from LDS, B = Q from
//                 registers): lane l holds S[q = l%16][keys 16j + 4(l/16) + r];
//   O^T[c][q]  += V^T[c][key] . P^T[key][q]  (A = V^T from the cache's
//                 transposed tiles, B = the lane's own probabilities).
// A lane therefore owns one query row for the softmax statistics and the
// output, and the running max / sum need only the 4 lanes of that row.
#include <climits>
#include <string>

#include "common.h"
#include "kern_common.h"

namespace omg {

constexpr int A_KT = 64;  // keys per tile
constexpr int A_THREADS = 256;

__device__ inline bool visible(int qp, int qs, int kp, int ks, int window) {
    const bool same_group = ((ks ^ qs) >> 12) == 0;
    return same_group && ((ks & 0xfff) == 0 || ks == qs) && kp <= qp &&
           (window == 0 || unsigned(qp - kp) < unsigned(window));
}

template <int HD>
__global__ __launch_bounds__(A_THREADS) void attention_kernel(AttnArgs a) {
    constexpr int KLD = HD + 8;    // K tile row stride (halfs)
    constexpr int VLD = A_KT + 8;  // V^T tile row stride (halfs)
    constexpr int DS = HD / 32;    // MFMA steps over the head dim
    constexpr int CT = HD / 16;    // 16-wide output column tiles
    constexpr float LOG2E = 1.4426950408889634f;
    __shared__ __attribute__((aligned(16))) half_t Ks[A_KT * KLD];
    __shared__ __attribute__((aligned(16))) half_t Vs[HD * VLD];
    __shared__ __attribute__((aligned(16))) int kpos[A_KT];
    __shared__ __attribute__((aligned(16))) int kseq[A_KT];
    __shared__ int qpos_s[64], qseq_s[64];
    __shared__ int s_lo, s_hi;

    const int tid = int(threadIdx.x), wave = tid / WAVE, lane = tid % WAVE;
    const int H = a.heads, hpg = a.heads / a.kv_heads, tpw = 16 / hpg, tpb = 4 * tpw;
    const int g = int(blockIdx.y);
    const int64_t tok0 = int64_t(blockIdx.x) * tpb;
    const int lr = lane % 16, G = lane / 16;
    const int64_t tq = tok0 + wave * tpw + lr / hpg;
    const int head = g * hpg + lr % hpg;
    const bool valid = tq < a.t;
    const int64_t kend = a.base + a.t;  // cache rows holding keys

    if (tid == 0) {
        s_lo = INT_MAX;
        s_hi = 0;
    }
    if (tid < tpb) {
        const int64_t tk = tok0 + tid;
        if (tk < a.t) {
            const int4 m = reinterpret_cast<const int4*>(a.meta)[a.base + tk];
            qpos_s[tid] = m.x;
            qseq_s[tid] = m.y;
        } else {
            qpos_s[tid] = -1;  // sees nothing: every key position is >= 0
            qseq_s[tid] = -2;
        }
    }
    __syncthreads();
    int qp = -1, qsq = -2;
    if (valid) {
        const int4 m = reinterpret_cast<const int4*>(a.meta)[a.base + tq];
        qp = m.x;
        qsq = m.y;
        // Prefix key rows are row_lo + position, and every visible key lies
        // at or after the first in-window prefix row.
        const int lo = m.z + (a.window > 0 ? max(0, qp - a.window + 1) : 0);
        atomicMin(&s_lo, lo);
        atomicMax(&s_hi, m.w);
    }
    __syncthreads();
    const int64_t klo = s_lo, khi = s_hi;

    half8 qf[DS];
#pragma unroll
    for (int s = 0; s < DS; ++s) {
        if (valid)
            qf[s] = *reinterpret_cast<const half8*>(a.q16 + (tq * H + head) * HD + s * 32 + G * 8);
        else
            qf[s] = half8{};
    }
    floatx4 o[CT];
#pragma unroll
    for (int c = 0; c < CT; ++c) o[c] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    float m_run = -INFINITY, l_run = 0.0f;

    const half_t* kbase = a.kc + int64_t(g) * a.cap_pad * HD;
    const half_t* vbase = a.vt + int64_t(g) * (a.cap_pad / 64) * HD * 64;
    for (int64_t kt0 = (klo / A_KT) * A_KT; kt0 < khi; kt0 += A_KT) {
        {
            const uint4* src = reinterpret_cast<const uint4*>(kbase + kt0 * HD);
            for (int c = tid; c < A_KT * HD / 8; c += A_THREADS) {
                const int r = c / (HD / 8), cc = c % (HD / 8);
                *reinterpret_cast<uint4*>(Ks + r * KLD + cc * 8) = src[c];
            }
            const uint4* vsrc = reinterpret_cast<const uint4*>(vbase + (kt0 / A_KT) * HD * A_KT);
            for (int c = tid; c < HD * A_KT / 8; c += A_THREADS) {
                const int r = c / (A_KT / 8), cc = c % (A_KT / 8);
                *reinterpret_cast<uint4*>(Vs + r * VLD + cc * 8) = vsrc[c];
            }
            if (tid < A_KT) {
                const int64_t row = kt0 + tid;
                if (row < kend) {
                    const int4 m = reinterpret_cast<const int4*>(a.meta)[row];
                    kpos[tid] = m.x;
                    kseq[tid] = m.y;
                } else {
                    kpos[tid] = INT_MAX;
                    kseq[tid] = -3;
                }
            }
        }
        __syncthreads();
        bool any = false;
        {
            const int kp = kpos[lane], ks = kseq[lane];
            for (int u = 0; u < tpw; ++u)
                any |= visible(qpos_s[wave * tpw + u], qseq_s[wave * tpw + u], kp, ks, a.window);
        }
        if (__ballot(any) != 0ull) {
            floatx4 sacc[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                sacc[j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int s = 0; s < DS; ++s) {
                    const half8 kf = *reinterpret_cast<const half8*>(Ks + (j * 16 + lr) * KLD + s * 32 + G * 8);
                    sacc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf[s], sacc[j], 0, 0, 0);
                }
            }
            float mt = -INFINITY;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int4 kp4 = *reinterpret_cast<const int4*>(kpos + j * 16 + G * 4);
                const int4 ks4 = *reinterpret_cast<const int4*>(kseq + j * 16 + G * 4);
                const int kpv[4] = {kp4.x, kp4.y, kp4.z, kp4.w};
                const int ksv[4] = {ks4.x, ks4.y, ks4.z, ks4.w};
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float sv = visible(qp, qsq, kpv[r], ksv[r], a.window) ? sacc[j][r] * LOG2E : -INFINITY;
                    sacc[j][r] = sv;
                    mt = fmaxf(mt, sv);
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
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
                for (int c = 0; c < CT; ++c) {
                    const half_t* vr = Vs + (c * 16 + lr) * VLD + tt * 32 + G * 4;
                    const half4 lo = *reinterpret_cast<const half4*>(vr);
                    const half4 hi = *reinterpret_cast<const half4*>(vr + 16);
                    const half8 vf = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
                    o[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pb[tt], o[c], 0, 0, 0);
                }
            }
        }
        __syncthreads();
    }

    float l = l_run + __shfl_xor(l_run, 16, WAVE);
    l += __shfl_xor(l, 32, WAVE);
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

void launch_attention(hipStream_t s, const AttnArgs& a) {
    if (a.t <= 0) return;
    if (a.hd != 256) fail(E_INVALID, "attention: head_dim must be 256");
    if (a.kv_heads <= 0 || a.heads % a.kv_heads) fail(E_INVALID, "attention: heads / kv_heads");
    const int hpg = a.heads / a.kv_heads;
    if (16 % hpg) fail(E_INVALID, "attention: query heads per KV head must divide 16");
    if (a.cap_pad % A_KT || a.base + a.t > a.cap_pad) fail(E_INVALID, "attention: cache rows out of range");
    if (a.window < 0) fail(E_INVALID, "attention: negative window");
    const int tpb = 4 * (16 / hpg);
    const dim3 grid(unsigned((a.t + tpb - 1) / tpb), unsigned(a.kv_heads));
    attention_kernel<256><<<grid, dim3(A_THREADS), 0, s>>>(a);
    OMG_HIP(hipGetLastError());
}

}  // namespace omg
