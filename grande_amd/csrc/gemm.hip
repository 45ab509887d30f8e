// Dequant-fused MFMA GEMMs for the linear layers (matmul.wgsl and
// matmul_gated.wgsl's job): Y[M,N] = f16(X)[M,K] . deq(W)[N,K]^T with f32
// accumulation on v_mfma_f32_16x16x32_f16.
//
// One workgroup = 4 wave64s in a 2x2 grid over a BM x BN output tile.  K
// streams through LDS 64 at a time (two 32-element quant blocks): the X
// tile is copied as f16, the weight tile is decoded once per workgroup
// from Q4_0 / Q8_0 codes to f16 (the reference's rounding point,
// shaders/weight.wgsl:40-54) and then read by every row tile of the
// workgroup.  Two LDS buffers; the next stage's global loads are in flight
// while the current stage's MFMAs run.
//
// MFMA operand layout used throughout (16x16x32 f16): lane l supplies
// A[l % 16][8*(l/16) .. +8) and B[8*(l/16) .. +8)[l % 16]; the f32 result
// D[4*(l/16) + r][l % 16] lands in element r of the lane's float4.
#include <string>

#include "common.h"
#include "kern_common.h"

namespace omg {

constexpr int G_BK = 64;         // k per LDS stage
constexpr int G_LDS = G_BK + 8;  // halfs per LDS row: a 16 B pad
constexpr int G_THREADS = 256;

template <int QUANT>
struct BWords {
    static constexpr int N = QUANT == Q4_DT ? 1 : (QUANT == Q8_DT ? 2 : 4);  // uint4 per 32-element block
};

// One thread's share of a stage between the global loads and the LDS stores.
template <int QUANT, int BM, int BNW>
struct Stage {
    static constexpr int A_CHUNKS = BM * (G_BK / 8) / G_THREADS;
    static constexpr int B_TASKS = (BNW * 2 + G_THREADS - 1) / G_THREADS;
    uint4 a[A_CHUNKS];
    uint4 b[B_TASKS][BWords<QUANT>::N];
    uint16_t sc[B_TASKS];
};

struct GemmArgs {
    const half_t* x;
    int64_t ldx, m;
    DevWeight w0, w1;  // w1: the up projection of the gated kernel
    void* y;
    int64_t ldy;
};

template <int QUANT, int BM, int BN, bool GATED>
__device__ inline void load_stage(Stage<QUANT, BM, (GATED ? 2 * BN : BN)>& st, const GemmArgs& g,
                                  int64_t m0, int64_t n0, int64_t k0, int tid) {
    constexpr int BNW = GATED ? 2 * BN : BN;
    using S = Stage<QUANT, BM, BNW>;
    const int64_t M = g.m, K = g.w0.cols, N = g.w0.rows;
#pragma unroll
    for (int c = 0; c < S::A_CHUNKS; ++c) {
        const int idx = tid + c * G_THREADS;
        const int r = idx / (G_BK / 8), cc = idx % (G_BK / 8);
        const int64_t m = m0 + r, k = k0 + cc * 8;
        st.a[c] = (m < M && k < K) ? *reinterpret_cast<const uint4*>(g.x + m * g.ldx + k) : make_uint4(0, 0, 0, 0);
    }
    const int64_t KB = K / 32;
#pragma unroll
    for (int t = 0; t < S::B_TASKS; ++t) {
        const int idx = tid + t * G_THREADS;
        const int nl = idx / 2, blk = idx % 2;
        const bool up = GATED && nl >= BN;
        const DevWeight& w = up ? g.w1 : g.w0;
        const int64_t n = n0 + (GATED ? nl % BN : nl);
        const int64_t kb = k0 / 32 + blk;
        const bool ok = idx < BNW * 2 && n < N && kb < KB;
#pragma unroll
        for (int q = 0; q < BWords<QUANT>::N; ++q) st.b[t][q] = make_uint4(0, 0, 0, 0);
        st.sc[t] = 0;
        if (ok) {
            if constexpr (QUANT == Q4_DT) {
                st.b[t][0] = reinterpret_cast<const uint4*>(w.data)[n * KB + kb];
            } else if constexpr (QUANT == Q8_DT) {
                const uint4* p = reinterpret_cast<const uint4*>(static_cast<const uint8_t*>(w.data) + n * K + kb * 32);
                st.b[t][0] = p[0];
                st.b[t][1] = p[1];
            } else {
                const uint4* p = reinterpret_cast<const uint4*>(static_cast<const half_t*>(w.data) + n * K + kb * 32);
#pragma unroll
                for (int q = 0; q < 4; ++q) st.b[t][q] = p[q];
            }
            if constexpr (QUANT != F16_DT) st.sc[t] = w.scales[n * KB + kb];
        }
    }
}

template <int QUANT, int BM, int BNW>
__device__ inline void store_stage(const Stage<QUANT, BM, BNW>& st, half_t* As, half_t* Bs, int tid) {
    using S = Stage<QUANT, BM, BNW>;
#pragma unroll
    for (int c = 0; c < S::A_CHUNKS; ++c) {
        const int idx = tid + c * G_THREADS;
        const int r = idx / (G_BK / 8), cc = idx % (G_BK / 8);
        *reinterpret_cast<uint4*>(As + r * G_LDS + cc * 8) = st.a[c];
    }
#pragma unroll
    for (int t = 0; t < S::B_TASKS; ++t) {
        const int idx = tid + t * G_THREADS;
        if (idx >= BNW * 2) break;
        const int nl = idx / 2, blk = idx % 2;
        half8* dst = reinterpret_cast<half8*>(Bs + nl * G_LDS + blk * 32);
        if constexpr (QUANT == Q4_DT) {
            const half_t d = __builtin_bit_cast(half_t, st.sc[t]);
            const half2v dd = {d, d};
            const uint4 u = st.b[t][0];
            dst[0] = dq4_word(u.x, dd);
            dst[1] = dq4_word(u.y, dd);
            dst[2] = dq4_word(u.z, dd);
            dst[3] = dq4_word(u.w, dd);
        } else if constexpr (QUANT == Q8_DT) {
            const half_t d = __builtin_bit_cast(half_t, st.sc[t]);
            dst[0] = dq8_words(st.b[t][0].x, st.b[t][0].y, d);
            dst[1] = dq8_words(st.b[t][0].z, st.b[t][0].w, d);
            dst[2] = dq8_words(st.b[t][1].x, st.b[t][1].y, d);
            dst[3] = dq8_words(st.b[t][1].z, st.b[t][1].w, d);
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) reinterpret_cast<uint4*>(dst)[q] = st.b[t][q];
        }
    }
}

// matmul_gated.wgsl:126-134: tanh GELU with the argument clamped to +-15.
__device__ inline float gelu_tanh(float x) {
    float z = 0.7978845608028654f * (x + 0.044715f * x * x * x);
    z = fminf(15.0f, fmaxf(-15.0f, z));
    return 0.5f * x * (1.0f + tanhf(z));
}

template <int QUANT, int BM, int BN, bool GATED>
__global__ __launch_bounds__(G_THREADS) void gemm_kernel(GemmArgs g) {
    constexpr int BNW = GATED ? 2 * BN : BN;
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int MI = WM / 16, NI = WN / 16;
    constexpr int NJ = GATED ? 2 * NI : NI;
    __shared__ __attribute__((aligned(16))) half_t smem[2 * (BM + BNW) * G_LDS];
    // Buffer b: A tile at smem + b * BM * G_LDS, B tile after both A tiles.
    auto a_tile = [&](int b) { return smem + b * BM * G_LDS; };
    auto b_tile = [&](int b) { return smem + 2 * BM * G_LDS + b * BNW * G_LDS; };

    const int tid = int(threadIdx.x);
    const int wave = tid / WAVE, lane = tid % WAVE;
    const int wm = wave / 2, wn = wave % 2;
    const int64_t n0 = int64_t(blockIdx.x) * BN, m0 = int64_t(blockIdx.y) * BM;
    const int64_t K = g.w0.cols;
    const int nk = int((K + G_BK - 1) / G_BK);

    floatx4 acc[MI][NJ];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j) acc[i][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

    Stage<QUANT, BM, BNW> st;
    load_stage<QUANT, BM, BN, GATED>(st, g, m0, n0, 0, tid);
    store_stage<QUANT, BM, BNW>(st, a_tile(0), b_tile(0), tid);
    __syncthreads();

    const int lr = lane % 16, lk = (lane / 16) * 8;
    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < nk) load_stage<QUANT, BM, BN, GATED>(st, g, m0, n0, int64_t(kt + 1) * G_BK, tid);
        const half_t* A = a_tile(cur);
        const half_t* B = b_tile(cur);
#pragma unroll
        for (int ks = 0; ks < G_BK / 32; ++ks) {
            half8 af[MI], bf[NJ];
#pragma unroll
            for (int i = 0; i < MI; ++i)
                af[i] = *reinterpret_cast<const half8*>(A + (wm * WM + i * 16 + lr) * G_LDS + ks * 32 + lk);
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                const int brow = (GATED && j >= NI) ? BN + wn * WN + (j - NI) * 16 : wn * WN + j * 16;
                bf[j] = *reinterpret_cast<const half8*>(B + (brow + lr) * G_LDS + ks * 32 + lk);
            }
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int j = 0; j < NJ; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) store_stage<QUANT, BM, BNW>(st, a_tile(cur ^ 1), b_tile(cur ^ 1), tid);
        __syncthreads();
    }

    const int64_t N = g.w0.rows;
#pragma unroll
    for (int i = 0; i < MI; ++i) {
#pragma unroll
        for (int j = 0; j < NI; ++j) {
            const int64_t n = n0 + wn * WN + j * 16 + lr;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t m = m0 + wm * WM + i * 16 + (lane / 16) * 4 + r;
                if (m >= g.m || n >= N) continue;
                if constexpr (GATED) {
                    const float v = gelu_tanh(acc[i][j][r]) * acc[i][j + NI][r];
                    static_cast<half_t*>(g.y)[m * g.ldy + n] = half_t(v);
                } else {
                    static_cast<float*>(g.y)[m * g.ldy + n] = acc[i][j][r];
                }
            }
        }
    }
}

template <int QUANT, int BM, int BN, bool GATED>
static void run(hipStream_t s, const GemmArgs& g) {
    const int64_t N = g.w0.rows;
    const dim3 grid(unsigned((N + BN - 1) / BN), unsigned((g.m + BM - 1) / BM));
    gemm_kernel<QUANT, BM, BN, GATED><<<grid, dim3(G_THREADS), 0, s>>>(g);
    OMG_HIP(hipGetLastError());
}

// Tile choice: the largest tile that still gives about one workgroup per CU
// (256 CUs); small M falls back to 64 x 64 (gated: 64 x 32).
template <int QUANT, bool GATED>
static void dispatch(hipStream_t s, const GemmArgs& g) {
    const int64_t N = g.w0.rows, M = g.m;
    auto tiles = [&](int64_t bm, int64_t bn) { return ((M + bm - 1) / bm) * ((N + bn - 1) / bn); };
    if (!GATED) {
        if (tiles(128, 128) >= 240) return run<QUANT, 128, 128, false>(s, g);
        if (tiles(64, 128) >= 240) return run<QUANT, 64, 128, false>(s, g);
        return run<QUANT, 64, 64, false>(s, g);
    }
    if (tiles(128, 64) >= 240) return run<QUANT, 128, 64, GATED>(s, g);
    if (tiles(64, 64) >= 240) return run<QUANT, 64, 64, GATED>(s, g);
    return run<QUANT, 64, 32, GATED>(s, g);
}

static void check(const half_t* x, int64_t ldx, const DevWeight& w, int64_t ldy, int64_t m) {
    if (m < 0) fail(E_INVALID, "gemm: negative M");
    if (w.cols % 32 != 0) fail(E_INVALID, "gemm: K must be a multiple of 32");
    if (ldx < w.cols || ldx % 8 != 0) fail(E_INVALID, "gemm: X row stride must be >= K and a multiple of 8");
    if (reinterpret_cast<uintptr_t>(x) % 16 != 0 || reinterpret_cast<uintptr_t>(w.data) % 16 != 0)
        fail(E_INVALID, "gemm: operands must be 16-byte aligned");
    if (ldy < w.rows) fail(E_INVALID, "gemm: Y row stride must be >= N");
    if (w.dtype != F16_DT && !w.scales) fail(E_INVALID, "gemm: quantized weight without scales");
}

void launch_gemm(hipStream_t s, const half_t* x, int64_t ldx, const DevWeight& w, float* y, int64_t ldy,
                 int64_t m) {
    check(x, ldx, w, ldy, m);
    if (m == 0) return;
    const GemmArgs g{x, ldx, m, w, w, y, ldy};
    switch (w.dtype) {
        case F16_DT: return dispatch<F16_DT, false>(s, g);
        case Q8_DT: return dispatch<Q8_DT, false>(s, g);
        default: return dispatch<Q4_DT, false>(s, g);
    }
}

void launch_gemm_geglu(hipStream_t s, const half_t* x, int64_t ldx, const DevWeight& wg,
                       const DevWeight& wu, half_t* act, int64_t ldact, int64_t m) {
    check(x, ldx, wg, ldact, m);
    if (wu.rows != wg.rows || wu.cols != wg.cols || wu.dtype != wg.dtype)
        fail(E_INVALID, "gemm_geglu: gate and up must share shape and storage type");
    if (m == 0) return;
    const GemmArgs g{x, ldx, m, wg, wu, act, ldact};
    switch (wg.dtype) {
        case F16_DT: return dispatch<F16_DT, true>(s, g);
        case Q8_DT: return dispatch<Q8_DT, true>(s, g);
        default: return dispatch<Q4_DT, true>(s, g);
    }
}

}  // namespace omg
