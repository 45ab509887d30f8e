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
// D[4*(l/16) + r][l % 16] lands in element r of the lane's float4.  The
// weight tile is the A operand and the activation tile the B operand, so
// D = (X W^T)^T and a lane ends up with four consecutive output columns of
// one row: the epilogue stores them as one vector.
//
// Global loads are buffer loads on per-tile resources: rows past M or N
// read as zero in hardware, and the K tail is sent out of range the same
// way, so the loads carry no branches.
#include <string>

#include "common.h"
#include "kern_common.h"

namespace omg {

constexpr int G_BK = 64;         // k per LDS stage
constexpr int G_LDS = G_BK + 8;  // halfs per LDS row: a 16 B pad
constexpr int G_THREADS = 256;

// One thread's share of a stage between the global loads and the LDS stores.
// The weight tile is decoded in tasks of one quant block (32 elements), or
// of half a block when whole blocks would leave threads idle, so that every
// thread decodes the same amount.
template <int QUANT, int BM, int BNW>
struct Stage {
    static constexpr int A_CHUNKS = BM * (G_BK / 8) / G_THREADS;
    static constexpr int SPLIT = BNW * 2 < G_THREADS ? 2 : 1;                // tasks per block
    static constexpr int B_TASKS = (BNW * 2 * SPLIT + G_THREADS - 1) / G_THREADS;
    static constexpr int B_WORDS = (QUANT == Q4_DT ? 4 : (QUANT == Q8_DT ? 8 : 16)) / SPLIT;  // u32 per task
    uint4 a[A_CHUNKS];
    uint32_t b[B_TASKS][B_WORDS];
    uint16_t sc[B_TASKS];
};

struct GemmArgs {
    const half_t* x;
    int64_t ldx, m;
    DevWeight w0, w1;  // w1: the up projection of the gated kernel
    void* y;
    int64_t ldy;
};

// Buffer resources of one workgroup's tiles.
struct TileRes {
    __amdgpu_buffer_rsrc_t x, w0, w1, s0, s1;
};

constexpr int RSRC_FLAGS = 0x00020000;  // raw (untyped) 32-bit buffer

__device__ inline __amdgpu_buffer_rsrc_t rsrc(const void* base, int64_t bytes) {
    const int64_t n = bytes < 0 ? 0 : (bytes > 0x7fffffff ? 0x7fffffff : bytes);
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, int(n), RSRC_FLAGS);
}

template <int QUANT, int BM, int BN, bool GATED>
__device__ inline TileRes tile_res(const GemmArgs& g, int64_t m0, int64_t n0) {
    const int64_t M = g.m, K = g.w0.cols, N = g.w0.rows, KB = K / 32;
    const int64_t rows_m = M - m0 < BM ? M - m0 : BM;
    const int64_t rows_n = N - n0 < BN ? N - n0 : BN;
    TileRes r;
    r.x = rsrc(g.x + m0 * g.ldx, rows_m * g.ldx * 2);
    const int64_t wrow = QUANT == Q4_DT ? KB * 16 : (QUANT == Q8_DT ? K : 2 * K);  // bytes per weight row
    r.w0 = rsrc(static_cast<const uint8_t*>(g.w0.data) + n0 * wrow, rows_n * wrow);
    r.w1 = rsrc(static_cast<const uint8_t*>(g.w1.data) + n0 * wrow, rows_n * wrow);
    r.s0 = rsrc(g.w0.scales ? g.w0.scales + n0 * KB : nullptr, g.w0.scales ? rows_n * KB * 2 : 0);
    r.s1 = rsrc(g.w1.scales ? g.w1.scales + n0 * KB : nullptr, g.w1.scales ? rows_n * KB * 2 : 0);
    return r;
}

__device__ inline uint4 bload16(__amdgpu_buffer_rsrc_t r, int off) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

constexpr int OOB = 0x7ffffff0;  // an offset past every resource

template <int QUANT, int BM, int BN, bool GATED>
__device__ inline void load_stage(Stage<QUANT, BM, (GATED ? 2 * BN : BN)>& st, const TileRes& tr,
                                  const GemmArgs& g, int64_t k0, int tid) {
    constexpr int BNW = GATED ? 2 * BN : BN;
    using S = Stage<QUANT, BM, BNW>;
    const int64_t K = g.w0.cols, KB = K / 32;
#pragma unroll
    for (int c = 0; c < S::A_CHUNKS; ++c) {
        const int idx = tid + c * G_THREADS;
        const int r = idx / (G_BK / 8), cc = idx % (G_BK / 8);
        const int64_t k = k0 + cc * 8;
        st.a[c] = bload16(tr.x, k < K ? int((r * g.ldx + k) * 2) : OOB);
    }
#pragma unroll
    for (int t = 0; t < S::B_TASKS; ++t) {
        constexpr int SP = S::SPLIT, W = S::B_WORDS;
        const int idx = tid + t * G_THREADS;
        const int nl = idx / (2 * SP), blk = (idx / SP) % 2, part = idx % SP;
        const bool up = GATED && nl >= BN;
        const __amdgpu_buffer_rsrc_t wr = up ? tr.w1 : tr.w0;
        const __amdgpu_buffer_rsrc_t sr = up ? tr.s1 : tr.s0;
        const int64_t n = GATED ? nl % BN : nl;  // row within the tile
        const int64_t kb = k0 / 32 + blk;
        const bool ok = idx < BNW * 2 * SP && kb < KB;
        // Byte offset of this task's payload within the tile's weight rows.
        const int64_t base = QUANT == Q4_DT ? (n * KB + kb) * 16 : (QUANT == Q8_DT ? n * K + kb * 32 : (n * K + kb * 32) * 2);
        const int off = ok ? int(base + part * W * 4) : OOB;
        if constexpr (W == 2) {
            const uint2 u = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(wr, off, 0, 0));
            st.b[t][0] = u.x;
            st.b[t][1] = u.y;
        } else {
#pragma unroll
            for (int q = 0; q < W / 4; ++q) {
                const uint4 u = bload16(wr, ok ? off + 16 * q : OOB);
                st.b[t][4 * q] = u.x;
                st.b[t][4 * q + 1] = u.y;
                st.b[t][4 * q + 2] = u.z;
                st.b[t][4 * q + 3] = u.w;
            }
        }
        if constexpr (QUANT != F16_DT)
            st.sc[t] = uint16_t(__builtin_amdgcn_raw_buffer_load_b16(sr, ok ? int((n * KB + kb) * 2) : OOB, 0, 0));
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
        constexpr int SP = S::SPLIT, W = S::B_WORDS;
        const int idx = tid + t * G_THREADS;
        if (idx >= BNW * 2 * SP) break;
        const int nl = idx / (2 * SP), blk = (idx / SP) % 2, part = idx % SP;
        half8* dst = reinterpret_cast<half8*>(Bs + nl * G_LDS + blk * 32 + part * (32 / SP));
        if constexpr (QUANT == Q4_DT) {
            const half_t d = __builtin_bit_cast(half_t, st.sc[t]);
            const half2v dd = {d, d};
#pragma unroll
            for (int q = 0; q < W; ++q) dst[q] = dq4_word(st.b[t][q], dd);
        } else if constexpr (QUANT == Q8_DT) {
            const half_t d = __builtin_bit_cast(half_t, st.sc[t]);
#pragma unroll
            for (int q = 0; q < W / 2; ++q) dst[q] = dq8_words(st.b[t][2 * q], st.b[t][2 * q + 1], d);
        } else {
#pragma unroll
            for (int q = 0; q < W / 4; ++q)
                reinterpret_cast<uint4*>(dst)[q] =
                    make_uint4(st.b[t][4 * q], st.b[t][4 * q + 1], st.b[t][4 * q + 2], st.b[t][4 * q + 3]);
        }
    }
}

// matmul_gated.wgsl:126-134: tanh GELU with the argument clamped to +-15,
// through the identity 0.5 (1 + tanh z) = 1 / (1 + e^(-2z)) evaluated with
// the hardware exp2 and reciprocal.
__device__ inline float gelu_tanh(float x) {
    float z = 0.7978845608028654f * (x + 0.044715f * x * x * x);
    z = fminf(15.0f, fmaxf(-15.0f, z));
    const float e = __builtin_amdgcn_exp2f(z * -2.8853900817779268f);  // e^(-2z)
    return x * __builtin_amdgcn_rcpf(1.0f + e);
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
    // Workgroups are dispatched round-robin over the 8 XCDs (each with its
    // own L2): workgroup b runs on XCD b % 8.  Give each XCD a contiguous run
    // of tiles, row-tile major, so the activation rows it reads stay in its
    // L2 while it sweeps the (small) weight matrix.
    const int ntn = int((g.w0.rows + BN - 1) / BN);
    const int ntiles = ntn * int((g.m + BM - 1) / BM);
    const int per_xcd = int(gridDim.x) / 8;
    const int tile = (int(blockIdx.x) % 8) * per_xcd + int(blockIdx.x) / 8;
    if (tile >= ntiles) return;
    const int64_t n0 = int64_t(tile % ntn) * BN, m0 = int64_t(tile / ntn) * BM;
    const int64_t K = g.w0.cols;
    const int nk = int((K + G_BK - 1) / G_BK);

    floatx4 acc[MI][NJ];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j) acc[i][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

    const TileRes tr = tile_res<QUANT, BM, BN, GATED>(g, m0, n0);
    Stage<QUANT, BM, BNW> st;
    load_stage<QUANT, BM, BN, GATED>(st, tr, g, 0, tid);
    store_stage<QUANT, BM, BNW>(st, a_tile(0), b_tile(0), tid);
    __syncthreads();

    const int lr = lane % 16, lk = (lane / 16) * 8;
    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < nk) load_stage<QUANT, BM, BN, GATED>(st, tr, g, int64_t(kt + 1) * G_BK, tid);
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
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bf[j], af[i], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) store_stage<QUANT, BM, BNW>(st, a_tile(cur ^ 1), b_tile(cur ^ 1), tid);
        __syncthreads();
    }

    // Lane (lr, G) holds columns 4G..4G+3 of row lr of each 16 x 16 tile.
    const int64_t N = g.w0.rows;
#pragma unroll
    for (int i = 0; i < MI; ++i) {
        const int64_t m = m0 + wm * WM + i * 16 + lr;
        if (m >= g.m) continue;
#pragma unroll
        for (int j = 0; j < NI; ++j) {
            const int64_t n = n0 + wn * WN + j * 16 + (lane / 16) * 4;
            float v[4];
#pragma unroll
            for (int r = 0; r < 4; ++r)
                v[r] = GATED ? gelu_tanh(acc[i][j][r]) * acc[i][j + (GATED ? NI : 0)][r] : acc[i][j][r];
            if (n + 3 < N) {
                if constexpr (GATED) {
                    *reinterpret_cast<half4*>(static_cast<half_t*>(g.y) + m * g.ldy + n) =
                        half4{half_t(v[0]), half_t(v[1]), half_t(v[2]), half_t(v[3])};
                } else {
                    *reinterpret_cast<float4*>(static_cast<float*>(g.y) + m * g.ldy + n) =
                        make_float4(v[0], v[1], v[2], v[3]);
                }
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    if (n + r >= N) break;
                    if constexpr (GATED)
                        static_cast<half_t*>(g.y)[m * g.ldy + n + r] = half_t(v[r]);
                    else
                        static_cast<float*>(g.y)[m * g.ldy + n + r] = v[r];
                }
            }
        }
    }
}

template <int QUANT, int BM, int BN, bool GATED>
static void run(hipStream_t s, const GemmArgs& g) {
    const int64_t N = g.w0.rows;
    const int64_t tiles = ((N + BN - 1) / BN) * ((g.m + BM - 1) / BM);
    const dim3 grid(unsigned((tiles + 7) / 8 * 8));
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
    if (ldy % 4 != 0) fail(E_INVALID, "gemm: Y row stride must be a multiple of 4");
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
