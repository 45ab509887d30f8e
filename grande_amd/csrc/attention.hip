// Block-causal GQA attention over the f16 K/V cache (attention.wgsl's job):
// a query sees a key iff both are in the same group of the pass, the key is
// in the group's prefix or the query's own branch, at or before the
// query's position and, on sliding layers, less than `window` positions
// back (attention.wgsl:70-76).  Online softmax in f32, flash style.
//
// Work split: a work item is one query tile (A_ROWS rows = A_ROWS / hpg
// tokens x the hpg query heads sharing one KV head; each wave holds A_QB
// blocks of 16 rows, and every K / V fragment read from LDS feeds the
// MFMAs of all of them) and a range of 32-key tiles; the host builds the item lists from the pass's metadata
// (AttnWork).  A tile's key range is cut at fixed multiples of `chunk`
// tiles (sliding layers: 256 keys; global layers: 384 keys or more) and the
// per-chunk partial results are merged in key order by attention_merge.
// Because chunk boundaries are absolute cache rows and a tile that a query
// cannot see leaves its state exactly unchanged, each query's arithmetic
// is the same whichever tokens share its tile: rows over a resident prefix
// are bit-equal to a full pass.
//
// Per item: K and V^T tiles are double-buffered in LDS, loaded by LDS DMA
// one tile ahead (issued once the current tile's fragments are in
// registers); one barrier per tile.  A wave that sees no key of a tile
// skips it; a wave that sees every key of it skips the masking.  Masks are
// per-token 64-bit ballots over the tile's keys.
//
// Both products run on v_mfma_f32_16x16x32_f16 arranged so that no operand
// needs a register transpose:
//   S^T[key][q] = K[key][:] . Q[q][:]   (A = K rows from LDS, B = Q from
//                 registers): lane l holds S[q = l%16][keys 16j + 4(l/16) + r];
//   O^T[c][q]  += V^T[c][key] . P^T[key][q]  (A = V^T from the cache's
//                 transposed tiles, B = the lane's own probabilities).
// The cache stores V^T tile columns in the order of vt_col, so the eight
// keys a lane holds probabilities for are one contiguous 16-byte read.  A
// lane owns one query row for the softmax statistics and the output, so the
// running max and sum need only the 4 lanes of that row.
#include <algorithm>
#include <climits>
#include <string>
#include <type_traits>

#include "common.h"
#include "kern_common.h"

namespace omg {

// Geometry: A_KT keys per K/V tile, NW waves of A_QB 16-row query blocks
// per work item: A_NW (4) in long passes, 2 in short ones, where twice the
// items fill more of the chip (a row's sums do not depend on NW, see
// attention_work).
constexpr int A_KT = 32;
constexpr int A_NW = 4;  // the most waves per item (buffers are sized for it)
// One block per wave measured faster than two on MI355X (two need about 270
// registers per lane: one wave per SIMD).
constexpr int A_QB = 1;  // 16-row query blocks per wave
constexpr int A_ROWS = A_NW * 16 * A_QB;  // query rows per work item, at most
constexpr int A_KB = A_KT / 16;    // 16-key MFMA blocks per tile
constexpr int A_TT = A_KT / 32;    // 32-key MFMA steps of the O product per tile
static_assert(A_KT == 32 || A_KT == 64, "key tile");

int attention_key_tile() { return A_KT; }
int attention_rows() { return A_ROWS; }

// V^T tile rows hold A_KT keys (A_KT / 8 chunks of 16 B); the chunk swizzle
// spreads the rows a 16-byte fragment read serves at once over distinct
// banks.  Measured on the 32-key tiles (rocprofv3 SQ_LDS_BANK_CONFLICT /
// SQ_LDS_IDX_ACTIVE, C2 cold pass): (row >> 2) & 3 left 33.5% of the LDS
// cycles in bank conflicts, (row >> 1) & 3 7.3% (attention 19.6 -> 19.0 us);
// row & 3 and (row ^ (row >> 2)) & 3 no better than the first.
__device__ inline int vt_swz(int row) { return A_KT == 64 ? ((row >> 1) & 7) : ((row >> 1) & 3); }


// LDS of one work item.  K and V^T tiles are stored without padding; the
// 16-byte chunks of each row are XOR-swizzled so that the MFMA operand reads
// (16 lanes on 16 consecutive rows at one logical chunk) hit distinct banks:
//   K   [64 keys][HD]:  physical chunk = logical ^ (row & 15)  (32-chunk rows)
//   V^T [HD][A_KT keys]:  physical chunk = logical ^ vt_swz(row)
// Head dims above 256 split the output columns over HD / 256 workgroups
// (blockIdx.z), each holding the full K tile and its 256 rows of V^T.
template <int HD>
constexpr int attn_col_splits() { return HD / 256; }

template <int HD>
struct AttnSmem {
    half_t k[2][A_KT * HD];
    half_t v[2][(HD / attn_col_splits<HD>()) * A_KT];
};

typedef __attribute__((address_space(3))) void* lds_void_ptr;

constexpr int RSRC_RAW = 0x00020000;  // raw (untyped) 32-bit buffer

__device__ inline __amdgpu_buffer_rsrc_t attn_rsrc(const void* base, int64_t bytes) {
    const int n = bytes > 0x7fffffff ? 0x7fffffff : int(bytes);
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, n, RSRC_RAW);
}

// Geometry of one K/V tile's DMA: buffer loads to LDS (lane i of an
// instruction writes 16 bytes at LDS base + 16 i) where every lane picks
// the global chunk that belongs at its LDS slot, which is how the swizzle
// is applied.  The lane offsets are the same for every tile (the compiler
// keeps them out of the loop); the tile's position rides in the scalar
// offset.
template <int HD, int NW>
struct TileDma {
    static constexpr int KROW = HD / 8;                     // 16 B chunks per K row
    static constexpr int KINS = A_KT * HD / 8 / WAVE / NW;  // instructions per wave for K
    static constexpr int VINS = (HD / attn_col_splits<HD>()) * A_KT / 8 / WAVE / NW;
};

// exp2(s log2(e) - m) for a whole-number m (as the integer mi), as
// 2^frac(x) * 2^(floor(x) - m) with x = s log2(e): the fraction and the
// exponent depend on the score alone, so a probability taken against
// another whole-number max differs by an exact power of two, and so does
// its f16 rounding (above f16's subnormals).  With MASKED, scores may be
// -inf (masked keys) and give 0; without, every score is finite.
template <bool MASKED>
__device__ inline float prob(float s, int mi) {
    constexpr float LOG2E = 1.4426950408889634f;
    float x = s * LOG2E;
    if constexpr (MASKED) x = fmaxf(x, -16384.0f);
    int xi;  // floor(x) as an integer in one instruction
    asm("v_cvt_flr_i32_f32 %0, %1" : "=v"(xi) : "v"(x));
    return __builtin_amdgcn_ldexpf(__builtin_amdgcn_exp2f(__builtin_amdgcn_fractf(x)), xi - mi);
}

// One work item per workgroup: NW * 16 query rows (TPW tokens x HPG heads
// per wave in QB blocks of 16 rows, NW waves) against key tiles [tb, te)
// of the KV head blockIdx.y, output columns [256 z, 256 z + 256) for
// z = blockIdx.z when HD > 256.
template <int HD, int HPG, int NW>
__global__ __launch_bounds__(NW * 64) void attention_kernel(AttnArgs a, const int4* __restrict__ items) {
    constexpr int ROWS = NW * 16 * A_QB;  // query rows of the item
    using SM = AttnSmem<HD>;
    constexpr int DS = HD / 32;  // MFMA steps over the head dim
    constexpr int KG = DS < 8 ? DS : 8;  // K fragments in registers at once (per 16-key block)
    constexpr int NCS = attn_col_splits<HD>();
    constexpr int VD = HD / NCS;  // output columns of this workgroup
    constexpr int CT = VD / 16;   // 16-wide output column tiles
    constexpr int QB = A_QB, TPQ = 16 / HPG;  // tokens per 16-row block
    constexpr int TPW = QB * TPQ, TPB = NW * TPW;
    constexpr float LOG2E = 1.4426950408889634f;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem_raw[];
    SM& sm = *reinterpret_cast<SM*>(smem_raw);

    const int4 item = items[blockIdx.x];
    const int qtile = item.x, tb = item.y, te = item.z, slot = item.w;
    if (qtile < 0) return;  // padding of the launch order
    const int tid = int(threadIdx.x), lane = tid % WAVE;
    const int wave = __builtin_amdgcn_readfirstlane(tid / WAVE);
    const int H = a.heads;
    const int g = int(blockIdx.y);
    const int ch = NCS > 1 ? int(blockIdx.z) : 0;  // output column split
    const int64_t tok0 = int64_t(qtile) * TPB + wave * TPW;
    const int lr = lane % 16, G = lane / 16;
    const int u_lane = lr / HPG;  // the lane's token within each block
    const int head = g * HPG + lr % HPG;
    const int4* meta = reinterpret_cast<const int4*>(a.meta);
    const int4* qmeta = a.qmeta ? reinterpret_cast<const int4*>(a.qmeta) : meta + a.base;  // the queries' rows
    const int64_t kend = a.kend > 0 ? a.kend : a.base + a.t;                                 // keys before this row

    const half_t* kbase = a.kc + int64_t(g) * a.cap_pad * HD;
    const half_t* vbase = a.vt + int64_t(g) * (a.cap_pad / 64) * HD * 64;
    using TD = TileDma<HD, NW>;
    const int64_t cache_bytes = a.cap_pad * HD * 2;
    // Issue this wave's share of key tile `tile` into buffer `buf`.
    auto issue = [&](int tile, int buf) {
        const int k0 = tile * A_KT;
#pragma unroll
        for (int i = 0; i < TD::KINS; ++i) {
            const int slot = (wave * TD::KINS + i) * WAVE + lane;  // physical chunk index in the tile
            const int row = slot / TD::KROW, pc = slot % TD::KROW;
            const uint32_t o = uint32_t((row * HD + (pc ^ (row & 15)) * 8) * 2);
            const __amdgpu_buffer_rsrc_t r = attn_rsrc(kbase, cache_bytes);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_ptr)(sm.k[buf] + (wave * TD::KINS + i) * WAVE * 8),
                                                     16, o, k0 * HD * 2, 0, 0);
        }
        // First element of the tile's V^T columns (rows of this column split).
        const int vtile = (k0 / 64) * HD * 64 + k0 % 64 + ch * VD * 64;
#pragma unroll
        for (int i = 0; i < TD::VINS; ++i) {
            const int slot = (wave * TD::VINS + i) * WAVE + lane;
            const int row = slot / (A_KT / 8), pc = slot % (A_KT / 8);
            const uint32_t o = uint32_t((row * 64 + (pc ^ vt_swz(row)) * 8) * 2);
            const __amdgpu_buffer_rsrc_t r = attn_rsrc(vbase, cache_bytes);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_ptr)(sm.v[buf] + (wave * TD::VINS + i) * WAVE * 8),
                                                     16, o, vtile * 2, 0, 0);
        }
    };
    // The query fragments go out first, then the first tile, then the
    // tokens' metadata (whose wait then holds up nothing else).  Block b
    // holds tokens tok0 + b * TPQ .. (lane: token tok0 + b * TPQ + u_lane);
    // rows past the pass lie beyond the buffer's range and read as zeros.
    half8 qf[QB][DS];
    {
        const __amdgpu_buffer_rsrc_t qr = attn_rsrc(a.q16, a.t * H * HD * 2);
#pragma unroll
        for (int b = 0; b < QB; ++b) {
            const int64_t tq = tok0 + b * TPQ + u_lane;
            const int64_t qe = tq < a.t ? (tq * H + head) * HD + G * 8 : a.t * H * HD;  // in halves
            const uint32_t qo = uint32_t(qe > 0x3fffffff ? 0x3fffffff : qe) * 2;
#pragma unroll
            for (int s = 0; s < DS; ++s)
                qf[b][s] = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(qr, qo + s * 64, 0, 0));
        }
    }
    // Key metadata (one key per lane) travels in registers one tile ahead;
    // rows past the cache's valid range read as never visible.
    int4 km_next = make_int4(0, 0, 0, 0);
    if (tb < te) {
        issue(tb, 0);
        km_next = meta[tb * A_KT + lane % A_KT];
    }

    // Positions and sequence ids of the wave's tokens, wave-uniform.
    int qpos[TPW], qseq[TPW];
#pragma unroll
    for (int u = 0; u < TPW; ++u) {
        int4 m = make_int4(-1, -2, 0, 0);  // past the pass: sees nothing (positions are >= 0)
        if (tok0 + u < a.t) m = qmeta[tok0 + u];
        qpos[u] = __builtin_amdgcn_readfirstlane(m.x);
        qseq[u] = __builtin_amdgcn_readfirstlane(m.y);
    }

    floatx4 o[QB][CT];
#pragma unroll
    for (int b = 0; b < QB; ++b)
#pragma unroll
        for (int c = 0; c < CT; ++c) o[b][c] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    float m_run[QB], l_run[QB];
#pragma unroll
    for (int b = 0; b < QB; ++b) {
        m_run[b] = -INFINITY;
        l_run[b] = 0.0f;
    }

    for (int tile = tb; tile < te; ++tile) {
        const int cur = (tile - tb) & 1;
        // This wave's loads of `tile` are the only ones outstanding.
        __builtin_amdgcn_s_waitcnt(0);
        // Every wave's part of `tile` has landed, and every wave is done
        // with the other buffer (tile - 1), which the next loads overwrite.
        __syncthreads();
        // The keys' metadata of this tile arrived in registers with the
        // previous tile; the next tile's K / V and metadata go out now.
        const int4 km = km_next;
        if (tile + 1 < te) {
            issue(tile + 1, cur ^ 1);
            km_next = meta[(tile + 1) * A_KT + lane % A_KT];
        }

        // The tile's K fragments are read KG steps at a time (at HD 256 all
        // at once: their LDS latency hides behind the mask ballots), then
        // the QK products run with the accumulation chains interleaved.
        const half_t* K = sm.k[cur];
        half8 kf[A_KB][KG];
        auto load_kf = [&](int sg) {
#pragma unroll
            for (int j = 0; j < A_KB; ++j)
#pragma unroll
                for (int s = 0; s < KG; ++s) {
                    const int pc = ((sg * KG + s) * 4 + G) ^ lr;  // row & 15 == lr
                    kf[j][s] = *reinterpret_cast<const half8*>(K + (j * 16 + lr) * HD + pc * 8);
                }
        };
        load_kf(0);
        __builtin_amdgcn_sched_barrier(0);

        // Which keys of the tile each of the wave's tokens sees: lane = key.
        // Rows at or past the pass's end are never visible (their stale
        // metadata may look valid).
        // Each condition of `visible` is one lane ballot (a vector compare
        // into a scalar mask); the masks combine in scalar code.
        constexpr uint64_t KEYS = A_KT == 64 ? ~0ull : 0xffffffffull;
        const uint64_t ok = __ballot(int64_t(tile) * A_KT + (lane % A_KT) < kend) & KEYS;
        const uint64_t prefix_keys = __ballot((km.y & 0xfff) == 0);
        const int kgroup = km.y >> 12;
        const unsigned reach = a.window > 0 ? unsigned(a.window) : 0x7fffffffu;
        uint64_t vis[TPW];
        uint64_t any = 0, all = KEYS;
#pragma unroll
        for (int u = 0; u < TPW; ++u) {
            // (reach = window, or 2^31 - 1 on global layers: then the test
            // only repeats kp <= qp)
            const uint64_t m = ok & __ballot(kgroup == (qseq[u] >> 12)) &
                               (prefix_keys | __ballot(km.y == qseq[u])) & __ballot(km.x <= qpos[u]) &
                               __ballot(unsigned(qpos[u] - km.x) < reach);
            vis[u] = m;
            any |= m;
            all &= m;
        }
        if (any == 0ull) continue;
        const bool full = all == KEYS;

        // S^T blocks: every K fragment feeds the MFMAs of all QB blocks.
        floatx4 sacc[QB][A_KB];
#pragma unroll
        for (int b = 0; b < QB; ++b)
#pragma unroll
            for (int j = 0; j < A_KB; ++j) sacc[b][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int sg = 0; sg < DS / KG; ++sg) {
            if (sg > 0) load_kf(sg);
#pragma unroll
            for (int s = 0; s < KG; ++s)
#pragma unroll
                for (int j = 0; j < A_KB; ++j)
#pragma unroll
                    for (int b = 0; b < QB; ++b)
                        sacc[b][j] =
                            __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[j][s], qf[b][sg * KG + s], sacc[b][j], 0, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);

        // The V^T fragments go out before the softmax, whose arithmetic then
        // hides their latency.
        const half_t* V = sm.v[cur];
        half8 vf[A_TT][CT];
#pragma unroll
        for (int tt = 0; tt < A_TT; ++tt)
#pragma unroll
            for (int c = 0; c < CT; ++c) {
                const int row = c * 16 + lr;
                vf[tt][c] = *reinterpret_cast<const half8*>(V + row * A_KT + (((tt * 4 + G) ^ vt_swz(row)) * 8));
            }
        __builtin_amdgcn_sched_barrier(0);

        half8 pb[QB][A_TT];
        bool any_rescale = false;
        float alpha[QB];
#pragma unroll
        for (int b = 0; b < QB; ++b) {
            // Scores stay in natural units; the max is scaled to log2 units
            // once (scaling by LOG2E > 0 commutes with the max) and each
            // exponent is one fma(s, LOG2E, -m).
            float mt = -INFINITY;
            if (full) {
#pragma unroll
                for (int j = 0; j < A_KB; ++j)
#pragma unroll
                    for (int r = 0; r < 4; ++r) mt = fmaxf(mt, sacc[b][j][r]);
            } else {
                // The lane's 16 keys are bits 16j + 4G + r of its token's mask.
                uint64_t mk = vis[b * TPQ];
#pragma unroll
                for (int u = 1; u < TPQ; ++u) mk = u_lane == u ? vis[b * TPQ + u] : mk;
                uint32_t bits = 0;
#pragma unroll
                for (int j = 0; j < A_KB; ++j) bits |= uint32_t((mk >> (16 * j + 4 * G)) & 0xfu) << (4 * j);
#pragma unroll
                for (int j = 0; j < A_KB; ++j)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float sv = (bits >> (4 * j + r)) & 1u ? sacc[b][j][r] : -INFINITY;
                        sacc[b][j][r] = sv;
                        mt = fmaxf(mt, sv);
                    }
            }
            mt = max_lanes_16_32(mt) * LOG2E;
            // Lazy rescaling: the running max moves only when the tile's max
            // exceeds it by more than TAU (log2 units), so most tiles skip
            // the rescale of O; probabilities then reach at most 2^TAU, which
            // f16 holds with the same relative precision.  A row that has
            // seen nothing yet keeps m = -inf; exponents are taken against 0
            // then, which gives exactly 0 for every -inf score.
            // The max is kept at whole powers of two (ceil in log2 units):
            // wherever the row's keys fall into tiles, its probabilities
            // differ only by exact powers of two, which scale through the
            // f16 rounding of P, the sums and the rescales without changing
            // a bit, so a row's result does not depend on where its group
            // sits in the cache (beyond f32 summation order).
            constexpr float TAU = 8.0f;
            const bool grow = mt > m_run[b] + TAU;
            const float m_new = grow ? ceilf(mt) : m_run[b];
            const float m_use = m_new == -INFINITY ? 0.0f : m_new;
            alpha[b] = grow ? __builtin_amdgcn_exp2f(m_run[b] - m_use) : 1.0f;
            // A row that had seen nothing still holds O = 0: no rescale.
            any_rescale = any_rescale || (grow && m_run[b] != -INFINITY);
            const int mi = int(m_use);
            float psum = 0.0f;
            auto probs = [&](auto masked) {
                constexpr bool MK = decltype(masked)::value;
#pragma unroll
                for (int j = 0; j < A_KB; ++j) {
                    half2v pr[2];
#pragma unroll
                    for (int r = 0; r < 4; r += 2) {
                        pr[r / 2] = half2v{half_t(prob<MK>(sacc[b][j][r], mi)), half_t(prob<MK>(sacc[b][j][r + 1], mi))};
                        psum = __builtin_amdgcn_fdot2(pr[r / 2], half2v{half_t(1.0f), half_t(1.0f)}, psum, false);
                    }
                    pb[b][j / 2][(j % 2) * 4 + 0] = pr[0].x;
                    pb[b][j / 2][(j % 2) * 4 + 1] = pr[0].y;
                    pb[b][j / 2][(j % 2) * 4 + 2] = pr[1].x;
                    pb[b][j / 2][(j % 2) * 4 + 3] = pr[1].y;
                }
            };
            if (full)
                probs(std::false_type{});
            else
                probs(std::true_type{});
            l_run[b] = l_run[b] * alpha[b] + psum;
            m_run[b] = m_new;
        }
        if (__ballot(any_rescale) != 0ull) {
#pragma unroll
            for (int b = 0; b < QB; ++b)
#pragma unroll
                for (int c = 0; c < CT; ++c) o[b][c] *= alpha[b];
        }
        // O^T blocks: every V^T fragment feeds the MFMAs of all QB blocks.
#pragma unroll
        for (int tt = 0; tt < A_TT; ++tt)
#pragma unroll
            for (int c = 0; c < CT; ++c)
#pragma unroll
                for (int b = 0; b < QB; ++b)
                    o[b][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf[tt][c], pb[b][tt], o[b][c], 0, 0, 0);
    }

    // The output goes out through LDS: each wave stages a 16-row block row
    // by row (rows padded by 16 bytes), then writes each row's VD columns
    // as whole 16-byte chunks, two rows per store instruction (lanes 0-31
    // one row, 32-63 the next), instead of 32-byte pieces of 16 rows.  The
    // K / V buffers hold the staging: every wave is past its last read of
    // them, and no tile load is in flight after the loop.
    static_assert(VD == 256, "32 lanes per staged row");
    constexpr int SROW = VD + 8;  // staged row, halves
    static_assert(NW * 16 * SROW * 2 <= int(sizeof(SM)), "staging fits the tile buffers");
    __syncthreads();
    half_t* stage = reinterpret_cast<half_t*>(smem_raw) + wave * 16 * SROW;
#pragma unroll
    for (int b = 0; b < QB; ++b) {
        float l = l_run[b] + __shfl_xor(l_run[b], 16, WAVE);
        l += __shfl_xor(l, 32, WAVE);
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
        // O / l rounded to f16; a split item's partial is rounded exactly
        // as an unsplit tile's output.
#pragma unroll
        for (int c = 0; c < CT; ++c)
            *reinterpret_cast<half4*>(stage + lr * SROW + c * 16 + G * 4) =
                half4{half_t(o[b][c][0] * inv), half_t(o[b][c][1] * inv), half_t(o[b][c][2] * inv),
                      half_t(o[b][c][3] * inv)};
        const int row0 = (wave * QB + b) * 16;  // the block's first row of the item
        // A slot holds A_ROWS rows per KV head whatever the item's width:
        // row ranges of one pass that run at once on their own streams take
        // disjoint slot numbers, and items of 2 and 4 waves may meet there.
        const int64_t prow0 = (int64_t(slot) * a.kv_heads + g) * A_ROWS + row0;
        if (slot >= 0 && G == 0 && ch == 0) {
            // the chunk's max and sum
            a.part_ml[(prow0 + lr) * 2] = m_run[b];
            a.part_ml[(prow0 + lr) * 2 + 1] = l;
        }
        const int cc = (lane % 32) * 8;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int r = 2 * i + lane / 32;
            const half8 v = *reinterpret_cast<const half8*>(stage + r * SROW + cc);
            if (slot >= 0) {
                *reinterpret_cast<half8*>(a.part_o + (prow0 + r) * HD + ch * VD + cc) = v;
            } else {
                const int64_t tq = tok0 + b * TPQ + r / HPG;
                if (tq < a.t)
                    *reinterpret_cast<half8*>(a.out + (tq * H + g * HPG + r % HPG) * HD + ch * VD + cc) = v;
            }
        }
    }
}

// Merge the chunk partials of one query tile in key order: with O_c the
// chunk's normalised output (f16), m_c its max and l_c its sum,
// out = sum_c O_c l_c 2^(m_c - M) / sum_c l_c 2^(m_c - M), M = max_c m_c,
// over the chunks the row saw anything in.  A row with one such chunk gets
// that chunk's f16 output unchanged, exactly what an unsplit tile writes.
// One wave per row (four rows per workgroup); lane l owns columns
// 256 q + 4l .. 256 q + 4l + 3 (q < HD / 256), so every 256 columns of a
// partial row are one contiguous 512-byte wave load.
// The statistics and partial rows of up to MAXC chunks are loaded together
// (one round trip after the merge record).
template <int HD, int NW>
__global__ __launch_bounds__(256) void attention_merge_kernel(AttnArgs a, const int4* __restrict__ merges) {
    constexpr int ROWS = NW * 16 * A_QB;  // query rows of a work item
    static_assert(HD == 256 || HD == 512, "half4 column groups per lane");
    constexpr int NQ = HD / 256;
    constexpr int MAXC = 8;  // chunks loaded per round
    const int4 mg = merges[blockIdx.x / (ROWS / 4)];
    const int qtile = mg.x, slot0 = mg.y, n = mg.z;
    const int g = int(blockIdx.y);
    const int wave = int(threadIdx.x) / WAVE, lane = int(threadIdx.x) % WAVE;
    const int row = int(blockIdx.x % (ROWS / 4)) * 4 + wave;
    // Row r of a work item: 16-row block r / 16 (wave-major), 16 / hpg tokens
    // per block, the lane's token (r % 16) / hpg within it.
    const int hpg = a.heads / a.kv_heads, tpq = 16 / hpg, tpb = NW * A_QB * tpq;
    const int64_t tq = int64_t(qtile) * tpb + (row / 16) * tpq + (row % 16) / hpg;
    if (tq >= a.t) return;
    const int head = g * hpg + (row % 16) % hpg;
    auto base = [&](int c) { return (int64_t(slot0 + c) * a.kv_heads + g) * A_ROWS + row; };  // slot stride A_ROWS
    // Running merge over rounds of MAXC chunks (one round for n <= MAXC):
    // (M, L, acc) rescaled when a later round raises the max.
    float M = -INFINITY, L = 0.0f;
    float4 acc[NQ];
    half4 only[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
        acc[q] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        only[q] = half4{};
    }
    int seen = 0;
    for (int c0 = 0; c0 < n; c0 += MAXC) {
        half4 v[MAXC][NQ];
        float2 ml[MAXC];
#pragma unroll
        for (int c = 0; c < MAXC; ++c) {
            if (c0 + c < n) {
                ml[c] = *reinterpret_cast<const float2*>(a.part_ml + base(c0 + c) * 2);
#pragma unroll
                for (int q = 0; q < NQ; ++q)
                    v[c][q] = *reinterpret_cast<const half4*>(a.part_o + base(c0 + c) * HD + q * 256 + lane * 4);
            } else {
                ml[c] = make_float2(-INFINITY, 0.0f);
            }
        }
        float Mr = M;
#pragma unroll
        for (int c = 0; c < MAXC; ++c) Mr = fmaxf(Mr, ml[c].x);
        if (Mr == -INFINITY) continue;
        const float r = M == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(M - Mr);
        L *= r;
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
            acc[q].x *= r;
            acc[q].y *= r;
            acc[q].z *= r;
            acc[q].w *= r;
        }
        M = Mr;
#pragma unroll
        for (int c = 0; c < MAXC; ++c) {
            if (ml[c].x == -INFINITY) continue;
            ++seen;
            const float w = ml[c].y * __builtin_amdgcn_exp2f(ml[c].x - M);
            L += w;
#pragma unroll
            for (int q = 0; q < NQ; ++q) {
                only[q] = v[c][q];
                acc[q].x += float(v[c][q].x) * w;
                acc[q].y += float(v[c][q].y) * w;
                acc[q].z += float(v[c][q].z) * w;
                acc[q].w += float(v[c][q].w) * w;
            }
        }
    }
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
        const half4 o = seen == 1 ? only[q]
                                  : half4{half_t(acc[q].x * inv), half_t(acc[q].y * inv), half_t(acc[q].z * inv),
                                          half_t(acc[q].w * inv)};
        *reinterpret_cast<half4*>(a.out + (tq * a.heads + head) * HD + q * 256 + lane * 4) = o;
    }
}

void attention_work(const int32_t* meta, int64_t t, int heads, int kv_heads, int window, int chunk, int nw,
                    AttnWork& w) {
    w.items.clear();
    w.merges.clear();
    if (nw != 2 && nw != A_NW) fail(E_INVALID, "attention_work: waves per item must be 2 or 4");
    const int hpg = heads / kv_heads, tpb = nw * A_QB * (16 / hpg);
    w.nw = nw;
    w.aligned = true;
    int slot = 0;
    // A query tile's key range, one span per group among its tokens (in
    // key order: groups are laid out one after another).  Padding rows
    // between groups are left out of the ranges: they see nothing or other
    // padding rows, and their outputs are never read.
    struct Span {
        int64_t row_lo, lo, hi;
    };
    std::vector<Span> spans;
    std::vector<int4> pieces;
    for (int64_t q0 = 0, qt = 0; q0 < t; q0 += tpb, ++qt) {
        spans.clear();
        for (int64_t i = q0; i < t && i < q0 + tpb; ++i) {
            const int32_t* m = meta + 4 * i;
            if (m[1] < 0) continue;
            const int64_t l = int64_t(m[2]) + (window > 0 ? std::max<int64_t>(0, int64_t(m[0]) - window + 1) : 0);
            if (spans.empty() || spans.back().row_lo != m[2]) spans.push_back({m[2], l, m[3]});
            spans.back().lo = std::min(spans.back().lo, l);
            spans.back().hi = std::max(spans.back().hi, int64_t(m[3]));
        }
        if (spans.empty()) {
            // Padding only: an empty key range writes zeros (finite values
            // keep the padding rows' K / V finite, so the exact zeros that
            // masked keys contribute stay zero).
            w.items.push_back({int(qt), 0, 0, -1});
            continue;
        }
        // Chunk boundaries count from each group's first key row when every
        // group of the tile starts on a key tile (the engine aligns them),
        // so a group's partials are the same wherever it sits in the cache;
        // otherwise from cache row 0 over the tile's whole range.
        bool aligned = true;
        for (const Span& sp : spans) aligned = aligned && sp.row_lo % A_KT == 0;
        w.aligned = w.aligned && aligned;
        if (!aligned) {
            int64_t lo = INT64_MAX, hi = 0;
            for (const Span& sp : spans) {
                lo = std::min(lo, sp.lo);
                hi = std::max(hi, sp.hi);
            }
            spans.assign(1, Span{0, lo, hi});
        }
        pieces.clear();
        for (const Span& sp : spans) {
            const int org = int(sp.row_lo / A_KT);
            const int t0 = int(sp.lo / A_KT), t1 = int((sp.hi + A_KT - 1) / A_KT);
            if (t1 <= t0) continue;
            if (chunk <= 0) {
                pieces.push_back({int(qt), t0, t1, 0});
                continue;
            }
            for (int c = (t0 - org) / chunk; c <= (t1 - 1 - org) / chunk; ++c)
                pieces.push_back({int(qt), std::max(t0, org + c * chunk), std::min(t1, org + (c + 1) * chunk), 0});
        }
        if (pieces.size() == 1) {
            w.items.push_back({int(qt), pieces[0].y, pieces[0].z, -1});
            continue;
        }
        if (pieces.empty()) continue;
        const int first = slot;
        for (int4 pc : pieces) w.items.push_back({pc.x, pc.y, pc.z, slot++});
        w.merges.push_back({int(qt), first, slot - first, 0});
    }
    w.slots = slot;
    // Launch order.  Workgroup b runs on XCD b % 8, and each XCD has its
    // own L2: XCD x gets the x-th of eight contiguous runs of query tiles
    // (cut at equal work, a tile counting one and an item's start about
    // two and a half, its first loads' latency), so the key tiles its
    // items read are mostly the same few and stay in its L2.  Inside a
    // run, longest items first: the dispatcher places one workgroup per CU
    // before it doubles up, so the long items each start on a CU of their
    // own.  Runs are padded to one length with no-op items (query tile -1),
    // which keeps b % 8 the XCD for every blockIdx.y too.  (The result does
    // not depend on the order.)
    constexpr int NXCD = 8;
    constexpr double START = 2.5;
    double total = 0.0;
    for (const int4& it : w.items) total += START + (it.z - it.y);
    std::vector<std::vector<int4>> runs(NXCD);
    double acc = 0.0;
    for (const int4& it : w.items) {
        const double wgt = START + (it.z - it.y);
        const int x = std::min(NXCD - 1, int((acc + 0.5 * wgt) * NXCD / total));
        runs[size_t(x)].push_back(it);
        acc += wgt;
    }
    size_t len = 0;
    for (auto& r : runs) {
        std::stable_sort(r.begin(), r.end(), [](const int4& x, const int4& y) { return x.z - x.y > y.z - y.y; });
        len = std::max(len, r.size());
    }
    w.items.assign(len * NXCD, int4{-1, 0, 0, -1});
    for (int x = 0; x < NXCD; ++x)
        for (size_t i = 0; i < runs[size_t(x)].size(); ++i) w.items[i * NXCD + size_t(x)] = runs[size_t(x)][i];
}

template <int HD, int HPG, int NW>
static void run_attention_nw(hipStream_t s, const AttnArgs& a, const int4* items, int64_t nitems, size_t smem) {
    static bool attr_set = false;  // once per instantiation (per process)
    if (!attr_set) {
        OMG_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&attention_kernel<HD, HPG, NW>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, int(smem)));
        attr_set = true;
    }
    attention_kernel<HD, HPG, NW><<<dim3(unsigned(nitems), unsigned(a.kv_heads), unsigned(attn_col_splits<HD>())),
                                    dim3(NW * 64), smem, s>>>(a, items);
    OMG_HIP(hipGetLastError());
}

template <int HD, int HPG>
static void run_attention(hipStream_t s, const AttnArgs& a, const int4* items, int64_t nitems, size_t smem, int nw) {
    if (nw == 2)
        run_attention_nw<HD, HPG, 2>(s, a, items, nitems, smem);
    else
        run_attention_nw<HD, HPG, A_NW>(s, a, items, nitems, smem);
}

void launch_attention(hipStream_t s, const AttnArgs& a, const int4* items, int64_t nitems, int nw) {
    if (a.t <= 0 || nitems <= 0) return;
    if (nw != 2 && nw != A_NW) fail(E_INVALID, "attention: waves per item must be 2 or 4");
    if (a.hd != 256 && a.hd != 512) fail(E_INVALID, "attention: head_dim must be 256 or 512");
    if (a.kv_heads <= 0 || a.heads % a.kv_heads) fail(E_INVALID, "attention: heads / kv_heads");
    const int hpg = a.heads / a.kv_heads;
    if (16 % hpg) fail(E_INVALID, "attention: query heads per KV head must divide 16");
    if (a.cap_pad % 64 || a.base + a.t > a.cap_pad || a.kend > a.cap_pad)
        fail(E_INVALID, "attention: cache rows out of range");
    if (a.window < 0) fail(E_INVALID, "attention: negative window");
    // the query rows are read through a buffer resource (32-bit byte offsets)
    if (a.t * a.heads * a.hd * 2 > 0x7fffffff) fail(E_INVALID, "attention: query rows past 2 GiB");
    if (a.hd == 512) {
        const size_t smem = sizeof(AttnSmem<512>);
        switch (hpg) {
            case 1: run_attention<512, 1>(s, a, items, nitems, smem, nw); break;
            case 2: run_attention<512, 2>(s, a, items, nitems, smem, nw); break;
            case 4: run_attention<512, 4>(s, a, items, nitems, smem, nw); break;
            case 8: run_attention<512, 8>(s, a, items, nitems, smem, nw); break;
            default: run_attention<512, 16>(s, a, items, nitems, smem, nw); break;
        }
        return;
    }
    const size_t smem = sizeof(AttnSmem<256>);
    switch (hpg) {
        case 1: run_attention<256, 1>(s, a, items, nitems, smem, nw); break;
        case 2: run_attention<256, 2>(s, a, items, nitems, smem, nw); break;
        case 4: run_attention<256, 4>(s, a, items, nitems, smem, nw); break;
        case 8: run_attention<256, 8>(s, a, items, nitems, smem, nw); break;
        default: run_attention<256, 16>(s, a, items, nitems, smem, nw); break;
    }
}

void launch_attention_merge(hipStream_t s, const AttnArgs& a, const int4* merges, int64_t nmerges, int nw) {
    if (a.t <= 0 || nmerges <= 0) return;
    if (nw != 2 && nw != A_NW) fail(E_INVALID, "attention_merge: waves per item must be 2 or 4");
    const dim3 grid(unsigned(nmerges * (nw * 16 * A_QB / 4)), unsigned(a.kv_heads));
    if (a.hd != 512 && a.hd != 256) fail(E_INVALID, "attention_merge: head_dim must be 256 or 512");
    if (a.hd == 512 && nw == 2)
        attention_merge_kernel<512, 2><<<grid, dim3(256), 0, s>>>(a, merges);
    else if (a.hd == 512)
        attention_merge_kernel<512, A_NW><<<grid, dim3(256), 0, s>>>(a, merges);
    else if (nw == 2)
        attention_merge_kernel<256, 2><<<grid, dim3(256), 0, s>>>(a, merges);
    else
        attention_merge_kernel<256, A_NW><<<grid, dim3(256), 0, s>>>(a, merges);
    OMG_HIP(hipGetLastError());
}

}  // namespace omg
