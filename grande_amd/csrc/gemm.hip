// Dequant-fused MFMA GEMMs for the linear layers (matmul.wgsl and
// matmul_gated.wgsl's job): Y[M,N] = f16(X)[M,K] . deq(W)[N,K]^T with f32
// accumulation on v_mfma_f32_16x16x32_f16.
//
// Row-owner tiles: NW wave64s per workgroup over a BM x BN output tile,
// BM = 16 * MI activation rows.  Each wave owns 16 * NJ weight rows (gated:
// NJ / 2 row blocks of the gate matrix and the same rows of the up matrix)
// across all BM rows, so every weight row is decoded by exactly one wave,
// straight from its codes into MFMA operand registers.  K advances 64 at a
// time ("stages").  Data path of one stage:
//
//   global --LDS DMA--> ring slot (NS slots): X tile f16 [BM][64], raw
//       weight codes (Q4: [rows][2 blocks][16 B], Q8: [rows][64 B], F16:
//       [rows][64] f16) and one dword of two block scales per weight row;
//   ring slot --ds_read--> X fragments (b128) and this wave's codes and
//       scales --decode in registers--> weight fragments --> MFMA.
//
// The DMA (buffer_load ... lds, 16 B or 4 B per lane) keeps NS - 1 stages
// in flight with no registers held for them; the stage's K offset rides in
// the instruction's scalar offset, so the per-lane offsets are fixed for
// the whole loop.  One barrier per stage.  The ring alone sets the LDS
// footprint, so several workgroups share a CU.  The decode rounds
// (q - 8) * d (or q * d) to f16 once, the reference's f16 rounding point
// (shaders/weight.wgsl:40-54).
//
// X and f16 weight tiles are 128 B per row with the 16 B chunk c of row r
// stored at c ^ ((r >> 1) & 7), so the 16 rows x 4 chunks of one fragment
// read hit distinct banks.
//
// MFMA operand layout (16x16x32 f16): lane l supplies A[l % 16][8*(l/16)..+8)
// and B[8*(l/16)..+8)[l % 16]; the f32 result D[4*(l/16) + r][l % 16] lands
// in element r of the lane's float4.  The weight fragment is the A operand
// and the activation fragment the B operand, so D = (X W^T)^T and each lane
// ends up with four consecutive output columns of one row: the epilogue
// stores them as one vector.
//
// Bounds: every global read is a buffer load on a per-tile resource, so rows
// past M or N read as zero in hardware; in the K tail (K % 64 == 32) the X
// lanes and weight lanes past K are sent out of range by their lane offset
// (a zero activation times a zero weight).
#include <string>
#include <utility>

#include "common.h"
#include "kern_common.h"

namespace omg {

constexpr int G_BK = 64;  // k per stage
constexpr int G_ROW = G_BK * 2;  // bytes per LDS tile row
constexpr uint32_t OOB = 0x7ffffff0u;  // an offset past every resource

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Epilogues: what a tile does with its f32 accumulators.
//   EPI_F32        y[m][n] = acc (f32)
//   EPI_GELU_TANH  y[m][n] = f16(gelu_tanh(acc_gate) * acc_up)  (gated)
//   EPI_GELU_ERF   y[m][n] = f16(gelu_erf(acc_gate) * acc_up)   (gated)
//   EPI_RELU_F16   y[m][n] = f16(max(acc + bias[n], 0))
//   EPI_QKV        the fused [q | k | v] projection of a bidirectional
//                  encoder, scattered per head as f16 (see QkvHeads)
//   EPI_QKPREP     the decoder's [q | k | v] projection with qk_prep's
//                  work (per-head RMS norm, RoPE, query scale; q as f16
//                  rows, k and V^T into the f16 cache), head_dim 256
constexpr int EPI_F32 = 0, EPI_GELU_TANH = 1, EPI_GELU_ERF = 2, EPI_RELU_F16 = 3, EPI_QKV = 4, EPI_QKPREP = 5;

struct GemmArgs {
    const half_t* x;
    int64_t ldx, m;
    DevWeight w0, w1;  // w1: the up projection of the gated kernel
    void* y;
    int64_t ldy;
    const uint16_t* bias;  // f16 per output column (EPI_RELU_F16; EPI_QKV, may be null)
    QkvHeads qkv;          // EPI_QKV
    QkArgs qk;             // EPI_QKPREP (its qkv / qkv_stride unused)
    // Split K (EPI_F32): blockIdx.y = split z sums K range
    // [z K / ksplit, (z + 1) K / ksplit) into y + z * part_stride.
    int ksplit = 1;
    int64_t part_stride = 0;
    // gemm32_kernel EPI_F32 with FOLD: K pieces of kfold stages counted
    // from the split's first stage; see launch_gemm_splitk.
    int kfold = 0;
    // gemm32_kernel: row tiles start at BM * i - mshift (0 <= mshift < BM)
    int64_t mshift = 0;
};

constexpr int RSRC_FLAGS = 0x00020000;  // raw (untyped) 32-bit buffer

__device__ inline __amdgpu_buffer_rsrc_t rsrc(const void* base, int64_t bytes) {
    const int64_t n = bytes < 0 ? 0 : (bytes > 0x7fffffff ? 0x7fffffff : bytes);
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, int(n), RSRC_FLAGS);
}

__device__ inline int swz(int r) { return (r >> 1) & 7; }

// s_waitcnt vmcnt(N) with the other counters left alone (gfx9 encoding:
// vmcnt in bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
template <int N>
__device__ inline void wait_vm() {
    static_assert(N >= 0 && N <= 63, "vmcnt");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// LDS operations done (s_waitcnt lgkmcnt(0), other counters left alone),
// then the workgroup barrier, between compiler fences for memory.  Written
// with builtins rather than inline assembly so that the compiler's own
// wait-count tracking knows the LDS counter is clear afterwards.
__device__ inline void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// matmul_gated.wgsl:117-129: exact GELU, 0.5 x (1 + erf(x / sqrt 2)), with
// erf from Abramowitz & Stegun 7.1.26 (|error| < 1.5e-7), the form the
// reference evaluates.
__device__ inline float gelu_erf(float x) {
    const float z = x * 0.7071067811865476f;
    const float a = fabsf(z);
    const float t = __builtin_amdgcn_rcpf(1.0f + 0.3275911f * a);
    const float poly = ((((1.061405429f * t - 1.453152027f) * t + 1.421413741f) * t - 0.284496736f) * t +
                        0.254829592f) * t;
    const float e = __builtin_amdgcn_exp2f(-a * a * 1.4426950408889634f);  // e^(-a^2)
    const float y = 1.0f - poly * e;
    return 0.5f * x * (1.0f + (z < 0.0f ? -y : y));
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

template <int QUANT, int MI, int NJ, int EPI, int NS, int NW_ = 4, int WM_ = 1>
struct Cfg {
    static constexpr bool GATED = EPI == EPI_GELU_TANH || EPI == EPI_GELU_ERF;
    static constexpr int NW = NW_, T = NW * WAVE;
    static constexpr int WM = WM_, WN = NW / WM;       // waves along M and along N
    static constexpr int BM = 16 * MI * WM;
    static constexpr int WR = 16 * NJ;                 // weight rows per wave
    static constexpr int BNW = WN * WR;                // weight rows per tile
    static constexpr int BN = GATED ? BNW / 2 : BNW;   // output columns per tile
    static constexpr int X_CH = BM * 8, X_I = (X_CH + T - 1) / T;  // padded lanes go out of range
    static constexpr int W_CPR = QUANT == Q4_DT ? 2 : (QUANT == Q8_DT ? 4 : 8);
    static constexpr int W_CH = BNW * W_CPR, W_I = (W_CH + T - 1) / T;
    static constexpr int S_I = QUANT == F16_DT ? 0 : (BNW + T - 1) / T;
    static constexpr int C = X_I + W_I + S_I;  // DMA instructions per wave per stage
    static constexpr int X_BYTES = X_I * T * 16, W_BYTES = W_I * T * 16, S_BYTES = S_I * T * 4;
    static constexpr int STAGE = X_BYTES + W_BYTES + S_BYTES;
    static constexpr int LDS = NS * STAGE;
    static_assert(LDS <= 160 * 1024, "ring larger than the LDS");
    static_assert(!GATED || NJ % 2 == 0, "gated tiles pair gate and up row blocks");
    static_assert(BN % 64 == 0 || !GATED, "a scale DMA instruction must stay in one matrix");
    static_assert(NS >= 2, "ring needs >= 2 slots");
    static_assert(NW % WM == 0, "waves split evenly over M");
    static_assert(C <= 63, "vmcnt range");
    static_assert(EPI != EPI_QKV || WR == 64, "the Q/K/V epilogue gives each wave one 64-wide head");
};

template <int QUANT, int MI, int NJ, int EPI, int NS, int NW_, int WM_>
__global__ __launch_bounds__(NW_ * WAVE) void gemm_kernel(GemmArgs g) {
    using P = Cfg<QUANT, MI, NJ, EPI, NS, NW_, WM_>;
    constexpr bool GATED = P::GATED;
    constexpr int NW = P::NW, BM = P::BM, BN = P::BN, WR = P::WR;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int tid = int(threadIdx.x), lane = tid % WAVE;
    const int wave = __builtin_amdgcn_readfirstlane(tid / WAVE);
    // The wave's place in the tile: activation row blocks wm * MI .. + MI,
    // weight rows of block column wn.
    const int wn = wave % P::WN, wm = wave / P::WN;

    // Workgroups are dispatched round-robin over the 8 XCDs (each with its
    // own L2): workgroup b runs on XCD b % 8.  Give each XCD a contiguous run
    // of tiles, row-tile major, so the activation rows it reads stay in its
    // L2 while it sweeps the (small) weight matrix.
    const int64_t N = g.w0.rows, K = g.w0.cols, KB = K / 32, M = g.m;
    const int ntn = int((N + BN - 1) / BN);
    const int ntiles = ntn * int((M + BM - 1) / BM);
    const int per_xcd = int(gridDim.x) / 8;
    const int tile = (int(blockIdx.x) % 8) * per_xcd + int(blockIdx.x) / 8;
    if (tile >= ntiles) return;
    const int64_t n0 = int64_t(tile % ntn) * BN, m0 = int64_t(tile / ntn) * BM;
    const int kbeg = int(blockIdx.y) * int(K / g.ksplit);  // this split's K range (multiples of G_BK)
    const int nk = int((K / g.ksplit + G_BK - 1) / G_BK);
    const int K32 = int(K);
    const int64_t rows_m = M - m0 < BM ? M - m0 : BM;
    const int64_t rows_n = N - n0 < BN ? N - n0 : BN;

    const int64_t wrow = QUANT == Q4_DT ? KB * 16 : (QUANT == Q8_DT ? K : 2 * K);
    const uint8_t* const wbase0 = static_cast<const uint8_t*>(g.w0.data) + n0 * wrow;
    const uint8_t* const wbase1 = static_cast<const uint8_t*>(g.w1.data) + n0 * wrow;
    const uint16_t* const sbase0 = g.w0.scales ? g.w0.scales + n0 * g.w0.sld : nullptr;
    const uint16_t* const sbase1 = g.w1.scales ? g.w1.scales + n0 * g.w1.sld : nullptr;
    const int64_t sbytes = g.w0.scales ? rows_n * g.w0.sld * 2 : 0;

    uint32_t xoff[P::X_I];
    int xcol[P::X_I];
#pragma unroll
    for (int i = 0; i < P::X_I; ++i) {
        const int slot = (i * NW + wave) * WAVE + lane;
        const int r = slot / 8, lc = (slot % 8) ^ swz(r);
        xcol[i] = lc * 8;
        xoff[i] = slot < P::X_CH ? uint32_t((r * g.ldx + lc * 8) * 2) : OOB;
    }
    uint32_t woff[P::W_I], wtail[P::W_I];  // wtail: the lane's offset in the K-tail stage
    bool wup[P::W_I];
#pragma unroll
    for (int i = 0; i < P::W_I; ++i) {
        const int blk = i * NW + wave;
        const int slot = blk * WAVE + lane;
        const int rw = slot / P::W_CPR, c = slot % P::W_CPR;
        wup[i] = GATED && blk * WAVE / P::W_CPR >= BN;
        const int n = GATED && rw >= BN ? rw - BN : rw;
        uint32_t o;
        bool past;  // chunk past K when only the stage's first 32 k exist
        if constexpr (QUANT == Q4_DT) {
            o = uint32_t((n * KB + c) * 16);
            past = c >= 1;
        } else if constexpr (QUANT == Q8_DT) {
            o = uint32_t(n * K + c * 16);
            past = c >= 2;
        } else {
            const int lc = c ^ swz(rw);
            o = uint32_t((n * K + lc * 8) * 2);
            past = lc >= 4;
        }
        woff[i] = slot < P::W_CH ? o : OOB;
        wtail[i] = slot < P::W_CH && !past ? o : OOB;
    }
    uint32_t soff[P::S_I > 0 ? P::S_I : 1];
    bool sup[P::S_I > 0 ? P::S_I : 1];
#pragma unroll
    for (int i = 0; i < P::S_I; ++i) {
        const int rw = (i * NW + wave) * WAVE + lane;  // one scale dword per weight row
        sup[i] = GATED && (i * NW + wave) * WAVE >= BN;
        const int n = GATED && rw >= BN ? rw - BN : rw;
        soff[i] = rw < P::BNW ? uint32_t(n * g.w0.sld * 2) : OOB;
    }

    // Issue stage s's DMA into its ring slot.  The stage's K offset rides in
    // the scalar offset, so the lane offsets stay fixed; only the K-tail
    // stage (K % 64 == 32) masks X lanes per lane.  Stages past the end
    // repeat the last one (in range, never consumed), so every wave always
    // issues P::C instructions per stage and the resources do not change.
    auto slot_base = [&](int s) { return smem + (unsigned(s) % unsigned(NS)) * P::STAGE; };
    const int last = nk - 1;
    const int64_t xbytes = rows_m * g.ldx * 2;
    const bool ktail = (K32 & (G_BK - 1)) != 0;
    auto issue = [&](int s) {
        uint8_t* base = slot_base(s);
        const int k0 = __builtin_amdgcn_readfirstlane(kbeg + (s < last ? s : last) * G_BK);
        // (Range checks cover the lane offset only: a row's offset plus the
        // stage offset stays inside the row, and rows past M are out of
        // range by their lane offset.  Each resource is a named value built
        // at its use: passed inline, or held across branches, it is not
        // accepted by the host-side compile of this kernel.)
        const bool tail = ktail && k0 + G_BK > K32;
#pragma unroll
        for (int i = 0; i < P::X_I; ++i) {
            const uint32_t o = tail && xcol[i] >= K32 - k0 ? OOB : xoff[i];
            const __amdgpu_buffer_rsrc_t r = rsrc(g.x + m0 * g.ldx, xbytes);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)(base + (i * NW + wave) * WAVE * 16), 16, o,
                                                     k0 * 2, 0, 0);
        }
        // (So in the K-tail stage the weight lanes past K are masked by
        // offset as well.)
        const int wstep = QUANT == Q4_DT ? k0 / 2 : (QUANT == Q8_DT ? k0 : k0 * 2);
#pragma unroll
        for (int i = 0; i < P::W_I; ++i) {
            const uint32_t o = tail ? wtail[i] : woff[i];
            const __amdgpu_buffer_rsrc_t r = rsrc(wup[i] ? wbase1 : wbase0, rows_n * wrow);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)(base + P::X_BYTES + (i * NW + wave) * WAVE * 16),
                                                     16, o, wstep, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < P::S_I; ++i) {
            const __amdgpu_buffer_rsrc_t r = rsrc(sup[i] ? sbase1 : sbase0, sbytes);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                r, (lds_ptr_t)(base + P::X_BYTES + P::W_BYTES + (i * NW + wave) * WAVE * 4), 4, soff[i], k0 / 16, 0, 0);
        }
    };

    // Tile-local weight row of this wave's row block j.
    auto wrow_of = [&](int j) {
        if constexpr (GATED)
            return j < NJ / 2 ? wn * (WR / 2) + 16 * j : BN + wn * (WR / 2) + 16 * (j - NJ / 2);
        else
            return wn * WR + 16 * j;
    };

    floatx4 acc[MI][NJ];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j) acc[i][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

    const int lr = lane % 16, lg = lane / 16;
    int foff[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) foff[ks] = lr * G_ROW + (((ks * 4 + lg) ^ swz(lr)) * 16);

#pragma unroll
    for (int s = 0; s < NS - 1; ++s) issue(s);

    for (int kt = 0; kt < nk; ++kt) {
        // This wave's DMA of stage kt landed, then everyone's; everyone is
        // done reading stage kt - 1, whose slot the next DMA reuses.
        wait_vm<(NS - 2) * P::C>();
        lds_barrier();
        issue(kt + NS - 1);
        const uint8_t* X = slot_base(kt);
        const uint8_t* Wr = X + P::X_BYTES;
        const uint8_t* S = Wr + P::W_BYTES;
        // Every LDS read of the stage goes out first (X fragments, this
        // wave's codes and scales), so their latencies overlap; then the
        // decode and the MFMAs.
        half8 xf[2][MI];
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int i = 0; i < MI; ++i)
                xf[ks][i] = *reinterpret_cast<const half8*>(X + (wm * MI + i) * 16 * G_ROW + foff[ks]);
        uint32_t sc[NJ];
        uint2 code[2][NJ];  // Q4: .x only; Q8: both words
        half8 wf16[2][NJ];
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int rw = wrow_of(j) + lr;
            if constexpr (QUANT != F16_DT) sc[j] = *reinterpret_cast<const uint32_t*>(S + rw * 4);
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                if constexpr (QUANT == F16_DT)
                    wf16[ks][j] = *reinterpret_cast<const half8*>(Wr + wrow_of(j) * G_ROW + foff[ks]);
                else if constexpr (QUANT == Q4_DT)
                    code[ks][j].x = *reinterpret_cast<const uint32_t*>(Wr + rw * 32 + ks * 16 + lg * 4);
                else
                    code[ks][j] = *reinterpret_cast<const uint2*>(Wr + rw * 64 + ks * 32 + lg * 8);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            half8 wf[NJ];
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                if constexpr (QUANT == F16_DT) {
                    wf[j] = wf16[ks][j];
                } else {
                    const half_t d = __builtin_bit_cast(half_t, uint16_t(sc[j] >> (16 * ks)));
                    if constexpr (QUANT == Q4_DT)
                        wf[j] = dq4_word(code[ks][j].x, half2v{d, d});
                    else
                        wf[j] = dq8_words(code[ks][j].x, code[ks][j].y, half2v{d, d});
                }
            }
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int j = 0; j < NJ; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wf[j], xf[ks][i], acc[i][j], 0, 0, 0);
        }
    }
    wait_vm<0>();

    // Epilogue: lane (lr, lg) holds output columns 4 lg..4 lg + 3 of row lr
    // of each 16 x 16 block.
    if constexpr (EPI == EPI_QKV) {
        // The wave's 64 columns are one head of q, k or v (the q width and
        // the tile edges are multiples of 64).  RoPE pairs dims (c, c + 32),
        // which sit in blocks j and j + 2 of the same lane.
        const QkvHeads& o = g.qkv;
        const int64_t c0 = n0 + wn * WR;
        if (c0 >= N) return;
        const int sec = int(c0 / o.dq);
        const int64_t head = (c0 % o.dq) / 64;
        float bias[NJ][4];
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                bias[j][r] = g.bias ? float(__builtin_bit_cast(half_t, g.bias[c0 + 16 * j + 4 * lg + r])) : 0.0f;
#pragma unroll
        for (int i = 0; i < MI; ++i) {
            const int64_t m = m0 + (wm * MI + i) * 16 + lr;
            if (m >= M) continue;
            float v[NJ][4];
#pragma unroll
            for (int j = 0; j < NJ; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) v[j][r] = acc[i][j][r] + bias[j][r];
            if (sec < 2 && o.rope) {
                // rope_bi.wgsl:30-49: a' = a cos - b sin, b' = b cos + a sin.
                const float2* rp = o.rope + int64_t(o.meta[4 * m]) * 32;
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float2 cs = rp[16 * j + 4 * lg + r];
                        const float a = v[j][r], b = v[j + 2][r];
                        v[j][r] = a * cs.x - b * cs.y;
                        v[j + 2][r] = b * cs.x + a * cs.y;
                    }
            }
            if (sec < 2) {
                const float sc = sec == 0 ? o.qscale : 1.0f;
                half_t* dst = (sec == 0 ? o.q16 : o.k16) + (head * o.tpad + m) * 64;
#pragma unroll
                for (int j = 0; j < NJ; ++j)
                    *reinterpret_cast<half4*>(dst + 16 * j + 4 * lg) =
                        half4{half_t(v[j][0] * sc), half_t(v[j][1] * sc), half_t(v[j][2] * sc), half_t(v[j][3] * sc)};
            } else {
                half_t* dst = o.vt + (head * (o.tpad / 32) + m / 32) * (64 * 32) + vt_col32(int(m % 32));
#pragma unroll
                for (int j = 0; j < NJ; ++j)
#pragma unroll
                    for (int r = 0; r < 4; ++r) dst[(16 * j + 4 * lg + r) * 32] = half_t(v[j][r]);
            }
        }
        return;
    }
    constexpr int NO = GATED ? NJ / 2 : NJ;
    const int64_t nw0 = n0 + (GATED ? wn * (WR / 2) : wn * WR);
    float cbias[EPI == EPI_RELU_F16 ? NO : 1][4];
    if constexpr (EPI == EPI_RELU_F16) {
#pragma unroll
        for (int j = 0; j < NO; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t n = nw0 + j * 16 + lg * 4 + r;
                cbias[j][r] = n < N ? float(__builtin_bit_cast(half_t, g.bias[n])) : 0.0f;
            }
    }
#pragma unroll
    for (int i = 0; i < MI; ++i) {
        const int64_t m = m0 + (wm * MI + i) * 16 + lr;
        if (m >= M) continue;
#pragma unroll
        for (int j = 0; j < NO; ++j) {
            const int64_t n = nw0 + j * 16 + lg * 4;
            float v[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                if constexpr (EPI == EPI_GELU_TANH)
                    v[r] = gelu_tanh(acc[i][j][r]) * acc[i][j + NJ / 2][r];
                else if constexpr (EPI == EPI_GELU_ERF)
                    v[r] = gelu_erf(acc[i][j][r]) * acc[i][j + NJ / 2][r];
                else if constexpr (EPI == EPI_RELU_F16)
                    v[r] = fmaxf(acc[i][j][r] + cbias[j][r], 0.0f);
                else
                    v[r] = acc[i][j][r];
            }
            constexpr bool F16_OUT = EPI != EPI_F32;
            if (n + 3 < N) {
                if constexpr (F16_OUT) {
                    *reinterpret_cast<half4*>(static_cast<half_t*>(g.y) + m * g.ldy + n) =
                        half4{half_t(v[0]), half_t(v[1]), half_t(v[2]), half_t(v[3])};
                } else {
                    *reinterpret_cast<float4*>(static_cast<float*>(g.y) + int64_t(blockIdx.y) * g.part_stride +
                                               m * g.ldy + n) =
                        make_float4(v[0], v[1], v[2], v[3]);
                }
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    if (n + r >= N) break;
                    if constexpr (F16_OUT)
                        static_cast<half_t*>(g.y)[m * g.ldy + n + r] = half_t(v[r]);
                    else
                        static_cast<float*>(g.y)[int64_t(blockIdx.y) * g.part_stride + m * g.ldy + n + r] = v[r];
                }
            }
        }
    }
}

// ------------------------------------------------------ 32x32x16 tiles

// The decoder's products (f32 out and the gated GeGLU) on
// v_mfma_f32_32x32x16_f16, which issues at full rate on gfx950 with one or
// two accumulation chains per wave (16x16x32 needs about sixteen).  Row-
// owner scheme: each wave owns 32 * NJ weight rows across all BM = 32 * MI
// activation rows, so its weights are private to it and go straight from
// their stage tiles (kernels.h) into registers: per stage and row block
// one coalesced 16-byte-per-lane load of the packet (lane 32 h + r gets
// row r's four k-steps of half h) and one 4-byte load of the row's block
// scales.  Only the activation tile, which every wave reads, goes through
// LDS.  Per 64-wide K stage, four 16-wide steps: lane l supplies A = the
// decoded weight word of row l % 32 at k 16 s + 8 (l / 32) (one Q4 word,
// two Q8 words or 16 bytes of f16), B = X row l % 32 of each activation
// block at the same k (one 16-byte LDS read), and holds D for activation
// row l % 32 at weight rows 8 j + 4 (l / 32) + i: four consecutive output
// columns per j, stored as one vector.  The K order (stage, step) does not
// depend on the tile shape, so every dispatch gives every output element
// the same sums: rows of a pass are the same whatever else it holds.
//
// Pipeline, iteration kt (stage kt):
//   wait for stage kt + 1's X DMA (this wave's), barrier (everyone's; and
//       everyone has finished reading the ring slot of stage kt - 1);
//   DMA stage kt + NS - 1's X tile into that slot;
//   read stage kt + 1's X fragments from LDS into registers;
//   decode + MFMA stage kt (X fragments read one iteration earlier,
//       weights loaded NS - 1 iterations earlier);
//   load stage kt + NS - 1's weights into the register slot just used.
// Every wave issues the same memory instructions in every iteration (past
// the end they read empty resources), so the wait counts are constants.
template <int QUANT, int MI, int NJ, int EPI, int NS, int NW_ = 4, bool PAIR_ = false>
struct Cfg32 {
    static constexpr bool GATED = EPI == EPI_GELU_TANH || EPI == EPI_GELU_ERF;
    // PAIR: a gated tile whose waves hold one matrix each, the first half
    // the gate blocks and the second half the matching up blocks; the gate
    // sums go through LDS to the up waves, which finish the tile.
    static constexpr bool PAIR = PAIR_;
    static constexpr int NW = NW_, T = NW * WAVE;
    static constexpr int BM = 32 * MI;
    static constexpr int WR = 32 * NJ;                 // weight rows per wave
    static constexpr int BNW = NW * WR;                // weight rows per tile
    static constexpr int BN = GATED ? BNW / 2 : BNW;   // output columns per tile
    static constexpr int PM = BN / 32;                 // row blocks per matrix
    static constexpr int PK = tile_packet_bytes(QUANT);
    static constexpr int CL = PK / 1024;               // 16-byte code loads per row block and stage
    static constexpr int X_CH = BM * 8, X_I = (X_CH + T - 1) / T;
    static constexpr int WL = NJ * (CL + (QUANT == F16_DT ? 0 : 1));  // weight loads per wave and stage
    static constexpr int C = X_I + WL;                 // memory instructions per wave and stage
    static constexpr int R = NS - 1;                   // weight register slots
    static constexpr int U = R % 2 == 0 ? R : 2 * R;   // loop unroll: X fragments alternate two sets
    static constexpr int X_BYTES = X_I * T * 16;
    // EPI_QKPREP stages the f32 tile [BM][256] (rows padded to 260
    // floats), eight partial sums of squares and a scale per row in LDS
    // after the K loop.
    static constexpr int QK_TS = 260;
    static constexpr int QK_LDS = EPI == EPI_QKPREP ? BM * (QK_TS + 17) * 4 : 0;  // + [BM][16] sums, [BM] scales
    static constexpr int PAIR_LDS = PAIR ? (NW / 2) * MI * NJ * 16 * WAVE * 4 : 0;  // the gate waves' sums
    static constexpr int EPI_LDS = QK_LDS > PAIR_LDS ? QK_LDS : PAIR_LDS;           // LDS after the K loop
    static constexpr int LDS = NS * X_BYTES > EPI_LDS ? NS * X_BYTES : EPI_LDS;
    static_assert(EPI != EPI_QKPREP || (BN == 256 && (NW == 4 || NW == 8)),
                  "the q/k/v epilogue: one 256-wide head on four or eight waves");
    static_assert(LDS <= 160 * 1024, "ring larger than the LDS");
    static_assert(!PAIR || (GATED && NW % 2 == 0), "paired tiles: gated, gate and up waves in pairs");
    static_assert(!GATED || PAIR || NJ % 2 == 0, "gated tiles pair gate and up row blocks");
    static_assert(NS >= 3, "ring needs >= 3 slots: one read into registers, one landing, one in flight");
    static_assert(WL + (NS - 2) * C <= 63, "vmcnt range");
};

template <class F, size_t... I>
__device__ inline bool run_phases(F& f, std::index_sequence<I...>) {
    return (f(std::integral_constant<int, int(I)>{}) && ...);
}

// XR (resident X): the workgroup's whole X tile (BM rows x its K range)
// lands in LDS in the prologue, one slot per stage, and the K loop runs
// with no barrier and no X wait (the weights are each wave's own).  Same
// MFMA sequence, same sums; chosen per launch when the tile fits.
template <int QUANT, int MI, int NJ, int EPI, int NS, int NW_, bool FOLD, bool XR, bool PAIR>
__global__ __launch_bounds__(NW_ * WAVE) void gemm32_kernel(GemmArgs g) {
    using P = Cfg32<QUANT, MI, NJ, EPI, NS, NW_, PAIR>;
    static_assert(!FOLD || EPI == EPI_F32, "K chunks: f32 products only");
    constexpr bool GATED = P::GATED;
    constexpr int NW = P::NW, BM = P::BM, BN = P::BN, WR = P::WR, PK = P::PK, PM = P::PM, R = P::R;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int tid = int(threadIdx.x), lane = tid % WAVE;
    const int wave = __builtin_amdgcn_readfirstlane(tid / WAVE);

    // XCD-aware tile order (see gemm_kernel).  Row tiles start at
    // BM * i - mshift (mshift < BM: the first tile is short), so a caller
    // can align the tiles to its own row grid.
    const int64_t N = g.w0.rows, K = g.w0.cols, M = g.m;
    const int ntn = int((N + BN - 1) / BN);
    const int ntiles = ntn * int((M + g.mshift + BM - 1) / BM);
    const int per_xcd = int(gridDim.x) / 8;
    const int tile = (int(blockIdx.x) % 8) * per_xcd + int(blockIdx.x) / 8;
    if (tile >= ntiles) return;
    const int64_t n0 = int64_t(tile % ntn) * BN, m0 = int64_t(tile / ntn) * BM - g.mshift;
    const int kbeg = int(blockIdx.y) * int(K / g.ksplit);
    const int nk = int((K / g.ksplit + G_BK - 1) / G_BK);
    const int K32 = int(K);
    auto row_ok = [&](int64_t r) { return m0 + r >= 0 && m0 + r < M; };  // tile row r is a row of the pass

    // X lanes: row m0 + r of the whole matrix (rows before 0 or from M on
    // are out of range, so they read as zeros).
    uint32_t xoff[P::X_I];
    int xcol[P::X_I];
#pragma unroll
    for (int i = 0; i < P::X_I; ++i) {
        const int slot = (i * NW + wave) * WAVE + lane;
        const int r = slot / 8, lc = (slot % 8) ^ swz(r);
        xcol[i] = lc * 8;
        xoff[i] = slot < P::X_CH && row_ok(r) ? uint32_t(((m0 + r) * g.ldx + lc * 8) * 2) : OOB;
    }

    // This wave's row blocks: j < NJ / 2 of the gate matrix and the rest of
    // the up matrix when gated (PAIR: all NJ of the gate matrix in the
    // first half of the waves, of the up matrix in the second, wave w and
    // w + NW / 2 on the same blocks).  Block j's packet of stage st sits at
    // st * PK + bj * stages * PK from the matrix's first block of the tile.
    const int64_t stages = g.w0.stages, rblocks = (N + 31) / 32, rb0 = n0 / 32;
    const int64_t live_blocks = rblocks - rb0;  // > 0: the tile starts inside N
    const int pw = PAIR ? wave % (NW / 2) : wave;  // the wave's place among the waves of its matrix
    auto mat_of = [&](int j) { return PAIR ? (wave >= NW / 2 ? 1 : 0) : (GATED && j >= NJ / 2 ? 1 : 0); };
    auto blk_of = [&](int j) {
        return PAIR ? pw * NJ + j : (GATED ? wave * (NJ / 2) + (j % (NJ / 2)) : wave * NJ + j);
    };
    uint32_t coff[NJ], scoff[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        coff[j] = blk_of(j) < live_blocks ? uint32_t(blk_of(j) * stages * PK + lane * (PK / 64)) : OOB;
        scoff[j] = blk_of(j) < live_blocks ? uint32_t(blk_of(j) * stages * TILE_SCALE_BYTES + (lane % 32) * 4) : OOB;
    }

    // Stages past the end repeat the last one (in range, never consumed),
    // so the resources and lane offsets stay the same for every stage and
    // only the scalar stage offset moves.
    auto slot_base = [&](int s) { return smem + (XR ? unsigned(s) : unsigned(s) % unsigned(NS)) * P::X_BYTES; };
    const int last = nk - 1;
    const int64_t xbytes = M * g.ldx * 2;
    const bool ktail = (K32 & (G_BK - 1)) != 0;  // K % 64 == 32: the last stage masks lanes
    // X tile of stage s into its ring slot.
    auto issue_x = [&](int s) {
        uint8_t* base = slot_base(s);
        const int k0 = __builtin_amdgcn_readfirstlane(kbeg + (s < last ? s : last) * G_BK);  // a scalar offset
        const bool tail = ktail && k0 + G_BK > K32;
#pragma unroll
        for (int i = 0; i < P::X_I; ++i) {
            const uint32_t o = tail && xcol[i] >= K32 - k0 ? OOB : xoff[i];
            const __amdgpu_buffer_rsrc_t r = rsrc(g.x, xbytes);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)(base + (i * NW + wave) * WAVE * 16), 16, o,
                                                     k0 * 2, 0, 0);
        }
    };

    // A stage's weights in registers.
    struct WRegs {
        uint4 code[NJ][P::CL];
        uint32_t sc[NJ];
    };
    const int st0 = kbeg / G_BK;  // this split's first stage
    auto issue_w = [&](int s, WRegs& w) {
        const int st = __builtin_amdgcn_readfirstlane(st0 + (s < last ? s : last));
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const DevWeight& wt = mat_of(j) ? g.w1 : g.w0;
            const __amdgpu_buffer_rsrc_t r = rsrc(wt.tiles + rb0 * stages * PK, live_blocks * stages * PK);
#pragma unroll
            for (int c = 0; c < P::CL; ++c)
                w.code[j][c] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                                             r, coff[j] + 16 * c, st * PK, 0));
            if constexpr (QUANT != F16_DT) {
                const __amdgpu_buffer_rsrc_t rs = rsrc(wt.tscales + rb0 * stages * TILE_SCALE_BYTES,
                                                       live_blocks * stages * TILE_SCALE_BYTES);
                w.sc[j] = __builtin_amdgcn_raw_buffer_load_b32(rs, scoff[j], st * TILE_SCALE_BYTES, 0);
            }
        }
    };

    floatx16 acc[MI][NJ];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j) acc[i][j] = floatx16{};
    // FOLD: the products of each K piece (g.kfold stages) accumulate from
    // zero in acc and the piece sums are added into tot in K order — the
    // sums of a pass that runs every piece in a workgroup of its own and
    // adds the partials in order (the residual norm's runs).
    floatx16 tot[FOLD ? MI : 1][FOLD ? NJ : 1];
    int kleft = g.kfold;  // stages left in the current piece (FOLD)
    bool folded = false;
    auto fold = [&] {
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                tot[i][j] = folded ? tot[i][j] + acc[i][j] : acc[i][j];
                acc[i][j] = floatx16{};
            }
        folded = true;
    };

    const int lr = lane % 32, lh = lane / 32;
    int foff[4];  // the lane's X fragment offset within a 32-row block, per k-step
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) foff[ks] = lr * G_ROW + (((2 * ks + lh) ^ swz(lr)) * 16);

    struct XRegs {
        half8 x[4][MI];
    };
    auto read_x = [&](int s, XRegs& f) {
        const uint8_t* X = slot_base(s);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
#pragma unroll
            for (int i = 0; i < MI; ++i) f.x[ks][i] = *reinterpret_cast<const half8*>(X + i * 32 * G_ROW + foff[ks]);
    };
    auto compute = [&](const XRegs& f, const WRegs& w) {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            half8 wf[NJ];
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                if constexpr (QUANT == F16_DT) {
                    wf[j] = __builtin_bit_cast(half8, w.code[j][ks]);
                } else {
                    // k-steps 0, 1 are the stage's first block, 2, 3 its second
                    const half_t d = __builtin_bit_cast(half_t, uint16_t(w.sc[j] >> (16 * (ks / 2))));
                    if constexpr (QUANT == Q4_DT) {
                        const uint4 u = w.code[j][0];
                        const uint32_t word = ks == 0 ? u.x : ks == 1 ? u.y : ks == 2 ? u.z : u.w;
                        wf[j] = dq4_word(word, half2v{d, d});
                    } else {
                        const uint4 u = w.code[j][ks / 2];
                        wf[j] = ks % 2 == 0 ? dq8_words(u.x, u.y, half2v{d, d}) : dq8_words(u.z, u.w, half2v{d, d});
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int j = 0; j < NJ; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wf[j], f.x[ks][i], acc[i][j], 0, 0, 0);
        }
    };

    // EPI_QKPREP, q and k heads: the rope rows of the rows this thread
    // finishes (RP rows per pass of the workgroup, row p * RP + tid / 32),
    // loaded now so their latency hides behind the K loop.
    constexpr int QK_RP = NW * WAVE / 32;  // rows per pass: 32 threads per row
    constexpr int QK_PASSES = EPI == EPI_QKPREP ? BM / QK_RP : 1;
    int qpos[QK_PASSES];
    if constexpr (EPI == EPI_QKPREP) {
        const QkArgs& a = g.qk;
        const bool qk_head = n0 / 256 < a.heads + a.kv_heads;
#pragma unroll
        for (int p = 0; p < QK_PASSES; ++p) {
            // Every thread loads the position of a row of the pass (its own
            // row, clamped into the pass), so the loads go out back to back
            // with no branch between them; rows outside the pass and the v
            // head take position 0.
            const int r = p * QK_RP + tid / 32;
            const int64_t m = m0 + r < 0 ? 0 : (m0 + r < M ? m0 + r : M - 1);
            const int pos = a.meta[4 * (a.base + m)];
            qpos[p] = qk_head && row_ok(r) ? (pos < 0 ? 0 : (pos >= a.rope_rows ? int(a.rope_rows - 1) : pos)) : 0;
        }
    }

    WRegs wr[R];
    XRegs xa, xb;
    int kt = 0;
    if constexpr (XR) {
        // Prologue: every stage's X, then weight stages 0 .. R - 1; all of
        // it landed (everyone's X: one barrier), then stage 0's fragments.
        for (int s = 0; s < nk; ++s) issue_x(s);
#pragma unroll
        for (int s = 0; s < R; ++s) issue_w(s, wr[s]);
        wait_vm<0>();
        lds_barrier();
        read_x(0, xa);
        auto xstep = [&](auto phase) {
            constexpr int PH = decltype(phase)::value;
            XRegs& cur = PH % 2 == 0 ? xa : xb;
            XRegs& nxt = PH % 2 == 0 ? xb : xa;
            // Stage kt's weights (issued R iterations ago) landed: at most
            // the R - 1 later stages' loads are still out.
            wait_vm<(R - 1) * P::WL>();
            if (kt + 1 < nk) read_x(kt + 1, nxt);
            compute(cur, wr[PH % R]);
            issue_w(kt + R, wr[PH % R]);
            if constexpr (FOLD) {
                if (--kleft == 0 || kt + 1 == nk) {
                    kleft = g.kfold;
                    fold();
                }
            }
            return ++kt < nk;
        };
        while (run_phases(xstep, std::make_index_sequence<P::U>{})) {
        }
    }
    // Prologue: stages 0 .. NS - 2 in the same order as the loop issues
    // them (X, then weights), then stage 0's X fragments.
    if constexpr (!XR) {
#pragma unroll
    for (int s = 0; s < R; ++s) {
        issue_x(s);
        issue_w(s, wr[s]);
    }
    wait_vm<P::WL + (NS - 2) * P::C>();
    lds_barrier();
    read_x(0, xa);
    }
    auto step = [&](auto phase) {
        constexpr int PH = decltype(phase)::value;
        XRegs& cur = PH % 2 == 0 ? xa : xb;
        XRegs& nxt = PH % 2 == 0 ? xb : xa;
        // Stage kt + 1's X landed: after it this wave issued its weights
        // and NS - 3 whole stages.
        wait_vm<P::WL + (NS - 3) * P::C>();
        lds_barrier();
        issue_x(kt + NS - 1);
        if (kt + 1 < nk) read_x(kt + 1, nxt);
        compute(cur, wr[PH % R]);
        issue_w(kt + NS - 1, wr[PH % R]);
        if constexpr (FOLD) {
            if (--kleft == 0 || kt + 1 == nk) {
                kleft = g.kfold;
                fold();
            }
        }
        return ++kt < nk;
    };
    if constexpr (!XR) {
        while (run_phases(step, std::make_index_sequence<P::U>{})) {
        }
    }
    wait_vm<0>();
    if constexpr (FOLD) {
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int j = 0; j < NJ; ++j) acc[i][j] = tot[i][j];
    }

    if constexpr (EPI == EPI_QKPREP) {
        // Every multiply-add that rounds once is an explicit fmaf and every
        // f16 comes from an f32 value (nothing for the compiler to fuse in
        // one tile shape and not another): a row's outputs are the same
        // bits from the four-wave and the eight-wave tile.
        // qk_prep.wgsl:66-114 on the tile's rows, without cross-lane
        // traffic: each lane's sums of squares over its 16 accumulators of
        // a row in each 32-column block go to LDS with the f32 tile (the
        // ring is free: every DMA landed, every read done); a row's RMS is
        // the sum of its sixteen partials (block, lane half) in a fixed
        // order, whichever wave held which block.  q and k heads: 32 threads per row,
        // thread c holding head dimensions 4c..4c+3 and their RoPE partners
        // 128 + 4c..: RMS norm with the head's weight, RoPE, query scale,
        // f16 q rows or k cache rows.  v head: (optional) RMS norm, then
        // the V^T tiles of the cache in whole 16-byte chunks of 8 keys, 8
        // lanes per 128-byte dimension row (the caller aligns the row tiles
        // to 32 cache rows, so every chunk belongs to one tile; at the
        // pass's edges a chunk keeps the cache's other keys).
        constexpr int HD = 256, TS = P::QK_TS, HALF = HD / 2;
        const QkArgs& a = g.qk;
        float* T = reinterpret_cast<float*>(smem);
        float* ssp = T + BM * TS;  // [BM][16] partial sums of squares
        lds_barrier();
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                float ss = 0.0f;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    *reinterpret_cast<float4*>(T + (i * 32 + lr) * TS + wave * WR + j * 32 + 8 * q + 4 * lh) =
                        make_float4(acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]);
#pragma unroll
                    for (int r = 0; r < 4; ++r) ss = fmaf(acc[i][j][4 * q + r], acc[i][j][4 * q + r], ss);
                }
                ssp[(i * 32 + lr) * 16 + 2 * (wave * NJ + j) + lh] = ss;
            }
        const int slot = int(n0 / HD);
        const int H = a.heads, KV = a.kv_heads;
        const bool is_v = slot >= H + KV;
        const int c = tid % 32, d0 = 4 * c;
        // The rope pairs of every pass now, while the tile is staged.
        float4 r01[QK_PASSES], r23[QK_PASSES];
        if (!is_v) {
#pragma unroll
            for (int p = 0; p < QK_PASSES; ++p) {
                const float4* rt = reinterpret_cast<const float4*>(a.rope + int64_t(qpos[p]) * HALF + d0);
                r01[p] = rt[0];
                r23[p] = rt[1];
            }
        }
        lds_barrier();
        // Each row's scale once, from the sum of its sixteen partials in
        // order; the passes below read it.
        float* rinv = ssp + BM * 16;  // [BM] row scales
        if (tid < BM) {
            float ss = 0.0f;
#pragma unroll
            for (int k = 0; k < 16; ++k) ss += ssp[tid * 16 + k];
            rinv[tid] = 1.0f / sqrtf(ss / float(HD) + a.eps);
        }
        lds_barrier();
        if (!is_v) {
            const bool is_q = slot < H;
            const int head = is_q ? slot : slot - H;
            const float* wn = is_q ? a.q_norm : a.k_norm;
            const float4 wl = *reinterpret_cast<const float4*>(wn + d0), wh = *reinterpret_cast<const float4*>(wn + HALF + d0);
            const float w_lo[4] = {wl.x, wl.y, wl.z, wl.w}, w_hi[4] = {wh.x, wh.y, wh.z, wh.w};
            const float sc = is_q ? a.q_scale : 1.0f;
            const int rot = int(a.rope_dims / 2);
#pragma unroll
            for (int p = 0; p < QK_PASSES; ++p) {
                const int r = p * QK_RP + tid / 32;
                if (!row_ok(r)) continue;
                const float inv = rinv[r];
                const float4 vl = *reinterpret_cast<const float4*>(T + r * TS + d0);
                const float4 vh = *reinterpret_cast<const float4*>(T + r * TS + HALF + d0);
                const float v_lo[4] = {vl.x, vl.y, vl.z, vl.w}, v_hi[4] = {vh.x, vh.y, vh.z, vh.w};
                const float cs[4] = {r01[p].x, r01[p].z, r23[p].x, r23[p].z};
                const float sn[4] = {r01[p].y, r01[p].w, r23[p].y, r23[p].w};
                float o_lo[4], o_hi[4];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const float y0 = v_lo[k] * inv * w_lo[k], y1 = v_hi[k] * inv * w_hi[k];
                    if (d0 + k < rot) {
                        o_lo[k] = fmaf(y0, cs[k], -(y1 * sn[k]));
                        o_hi[k] = fmaf(y1, cs[k], y0 * sn[k]);
                    } else {
                        o_lo[k] = y0;
                        o_hi[k] = y1;
                    }
                }
                const int64_t tok = m0 + r, row = a.base + tok;
                half_t* dst = is_q ? a.q16 + (tok * H + head) * HD : a.kc + (int64_t(head) * a.cap_pad + row) * HD;
                *reinterpret_cast<half4*>(dst + d0) =
                    half4{f16_rounded(o_lo[0] * sc), f16_rounded(o_lo[1] * sc), f16_rounded(o_lo[2] * sc),
                          f16_rounded(o_lo[3] * sc)};
                *reinterpret_cast<half4*>(dst + HALF + d0) =
                    half4{f16_rounded(o_hi[0] * sc), f16_rounded(o_hi[1] * sc), f16_rounded(o_hi[2] * sc),
                          f16_rounded(o_hi[3] * sc)};
            }
            return;
        }
        // V head: per 32-key half of the tile, item (dim, chunk cc) for
        // 256 dims x 4 chunks; chunk 4 hf + cc of a 64-key cache tile holds
        // keys 32 hf + 4 cc + {0..3, 16..19} (vt_col).
        const int head = slot - H - KV;
#pragma unroll
        for (int hh = 0; hh < BM / 32; ++hh) {
            const int64_t kh = a.base + m0 + 32 * hh;  // first cache row of this half (a multiple of 32)
            if (m0 + 32 * hh + 32 <= 0 || m0 + 32 * hh >= M) continue;
            const int64_t t0 = kh / 64 * 64;
            const int hf = int((kh % 64) / 32);
#pragma unroll
            for (int u = 0; u < 1024 / (NW * WAVE); ++u) {
                const int item = tid + NW * WAVE * u;
                const int dim = item / 4, cc = item % 4;
                half_t* dst = a.vt + ((int64_t(head) * (a.cap_pad / 64) + t0 / 64) * HD + dim) * 64 + 8 * (4 * hf + cc);
                half_t h[8];
                bool all = true;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int r = 32 * hh + 4 * cc + 16 * (e / 4) + e % 4;  // tile row of key e
                    const bool in = row_ok(r);
                    all = all && in;
                    const float v = T[r * TS + dim];
                    h[e] = f16_rounded(a.v_norm ? v * rinv[r] : v);
                }
                if (!all) {
                    // a pass edge: the chunk's other keys keep the cache's values
                    const half8 old = *reinterpret_cast<const half8*>(dst);
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const int r = 32 * hh + 4 * cc + 16 * (e / 4) + e % 4;
                        if (!row_ok(r)) h[e] = old[e];
                    }
                }
                *reinterpret_cast<half8*>(dst) = half8{h[0], h[1], h[2], h[3], h[4], h[5], h[6], h[7]};
            }
        }
        return;
    }

    // PAIR: the gate waves' sums to the up waves, element for element (the
    // same lane layout), through LDS that every wave has finished with.
    floatx16 gsum[PAIR ? MI : 1][PAIR ? NJ : 1];
    if constexpr (PAIR) {
        float* E = reinterpret_cast<float*>(smem);
        lds_barrier();
        if (wave < NW / 2) {
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int j = 0; j < NJ; ++j)
#pragma unroll
                    for (int e = 0; e < 16; ++e) E[(((pw * MI + i) * NJ + j) * 16 + e) * WAVE + lane] = acc[i][j][e];
        }
        lds_barrier();
        if (wave < NW / 2) return;
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int j = 0; j < NJ; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) gsum[i][j][e] = E[(((pw * MI + i) * NJ + j) * 16 + e) * WAVE + lane];
    }

    // Epilogue: lane (lr, lh) holds, for activation row lr of block i,
    // output columns 8 q + 4 lh + 0..3 of weight block j (q = 0..3).
    constexpr int NO = GATED && !PAIR ? NJ / 2 : NJ;
    const int64_t nw0 = n0 + (PAIR ? pw * WR : GATED ? wave * (WR / 2) : wave * WR);
#pragma unroll
    for (int i = 0; i < MI; ++i) {
        const int64_t m = m0 + i * 32 + lr;
        if (m < 0 || m >= M) continue;
#pragma unroll
        for (int j = 0; j < NO; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int64_t n = nw0 + j * 32 + 8 * q + 4 * lh;
                float v[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    if constexpr (PAIR && EPI == EPI_GELU_TANH)
                        v[r] = gelu_tanh(gsum[i][j][4 * q + r]) * acc[i][j][4 * q + r];
                    else if constexpr (PAIR)
                        v[r] = gelu_erf(gsum[i][j][4 * q + r]) * acc[i][j][4 * q + r];
                    else if constexpr (EPI == EPI_GELU_TANH)
                        v[r] = gelu_tanh(acc[i][j][4 * q + r]) * acc[i][j + NJ / 2][4 * q + r];
                    else if constexpr (EPI == EPI_GELU_ERF)
                        v[r] = gelu_erf(acc[i][j][4 * q + r]) * acc[i][j + NJ / 2][4 * q + r];
                    else
                        v[r] = acc[i][j][4 * q + r];
                }
                if (n + 3 < N) {
                    // f16 from the f32 value in every tile shape (no fused
                    // multiply-convert in one instance and not another)
                    if constexpr (GATED)
                        *reinterpret_cast<half4*>(static_cast<half_t*>(g.y) + m * g.ldy + n) =
                            half4{f16_rounded(v[0]), f16_rounded(v[1]), f16_rounded(v[2]), f16_rounded(v[3])};
                    else
                        *reinterpret_cast<float4*>(static_cast<float*>(g.y) + int64_t(blockIdx.y) * g.part_stride +
                                                   m * g.ldy + n) = make_float4(v[0], v[1], v[2], v[3]);
                } else {
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        if (n + r >= N) break;
                        if constexpr (GATED)
                            static_cast<half_t*>(g.y)[m * g.ldy + n + r] = f16_rounded(v[r]);
                        else
                            static_cast<float*>(g.y)[int64_t(blockIdx.y) * g.part_stride + m * g.ldy + n + r] = v[r];
                    }
                }
            }
    }
}

// Resident X tiles up to this many bytes of LDS (one workgroup per CU
// above half of it).
constexpr int XR_MAX_LDS = 96 * 1024;

template <int QUANT, int MI, int NJ, int EPI, int NS, int NW = 4, bool FOLD = false, bool PAIR = false>
static void run32(hipStream_t s, const GemmArgs& g) {
    using P = Cfg32<QUANT, MI, NJ, EPI, NS, NW, PAIR>;
    for (const DevWeight* w : {&g.w0, &g.w1})
        if (!w->tiles || w->stages != (w->cols + G_BK - 1) / G_BK || (QUANT != F16_DT && !w->tscales))
            fail(E_INVALID, "gemm: weight without stage tiles");
    static bool lds_set = false;
    if (!lds_set) {
        OMG_HIP(hipFuncSetAttribute(
            reinterpret_cast<const void*>(&gemm32_kernel<QUANT, MI, NJ, EPI, NS, NW, FOLD, false, PAIR>),
            hipFuncAttributeMaxDynamicSharedMemorySize, P::LDS));
        OMG_HIP(hipFuncSetAttribute(
            reinterpret_cast<const void*>(&gemm32_kernel<QUANT, MI, NJ, EPI, NS, NW, FOLD, true, PAIR>),
            hipFuncAttributeMaxDynamicSharedMemorySize, XR_MAX_LDS > P::EPI_LDS ? XR_MAX_LDS : P::EPI_LDS));
        lds_set = true;
    }
    const int64_t N = g.w0.rows;
    if (g.mshift < 0 || g.mshift >= P::BM) fail(E_INVALID, "gemm: row tile shift out of range");
    const int64_t tiles = ((N + P::BN - 1) / P::BN) * ((g.m + g.mshift + P::BM - 1) / P::BM);
    const dim3 grid(unsigned((tiles + 7) / 8 * 8), unsigned(g.ksplit));
    const int64_t nk = (g.w0.cols / g.ksplit + G_BK - 1) / G_BK;
    const int64_t xr_lds = nk * P::X_BYTES;
    if (xr_lds <= XR_MAX_LDS) {
        const int lds = int(xr_lds > P::EPI_LDS ? xr_lds : P::EPI_LDS);
        gemm32_kernel<QUANT, MI, NJ, EPI, NS, NW, FOLD, true, PAIR><<<grid, dim3(P::T), lds, s>>>(g);
    } else {
        gemm32_kernel<QUANT, MI, NJ, EPI, NS, NW, FOLD, false, PAIR><<<grid, dim3(P::T), P::LDS, s>>>(g);
    }
    OMG_HIP(hipGetLastError());
}

template <int QUANT, int MI, int NJ, int EPI, int NS, int NW = 4, int WM = 1>
static void run(hipStream_t s, const GemmArgs& g) {
    using P = Cfg<QUANT, MI, NJ, EPI, NS, NW, WM>;
    static bool lds_set = false;
    if (!lds_set) {
        OMG_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_kernel<QUANT, MI, NJ, EPI, NS, NW, WM>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, P::LDS));
        lds_set = true;
    }
    const int64_t N = g.w0.rows;
    const int64_t tiles = ((N + P::BN - 1) / P::BN) * ((g.m + P::BM - 1) / P::BM);
    const dim3 grid(unsigned((tiles + 7) / 8 * 8), unsigned(g.ksplit));
    gemm_kernel<QUANT, MI, NJ, EPI, NS, NW, WM><<<grid, dim3(P::T), P::LDS, s>>>(g);
    OMG_HIP(hipGetLastError());
}

// Tile choice, measured on MI355X (tiles are activation rows x weight rows).
// f32 products (gemm32_kernel, 32x32x16, four waves; whole-pass A/B on the
// 270M model and an isolated sweep with rotating weight sets): 32 x 128
// for short passes (M <= 512), 64 x 128, 96 x 128 when K is split (twice
// the tiles), 128 x 128 for long passes (M >= 8192, the encoder's
// 49,152-token batches).  The other epilogues (gemm_kernel, 16x16x32):
//   bias+ReLU: short passes 32 x 32 on two waves; 64 x 64 (96 x 64 from
//   N = 768) for N <= 1280; 128 x 64, 96 x 128 for K >= 4096; 192 x 128
//   for long passes.  Q/K/V head scatter (64 weight rows per wave): 32 x
//   256 short, 96 x 256 otherwise.
//   Gated: 160 x 128 weight rows (64 output columns; a 2,384-token pass
//   of the 270M model is 480 tiles, at most two per CU, where 128-row
//   tiles made 608 and left 96 CUs a third) with three ring slots (two:
//   the whole pass 0.8% slower, though the product's own event time is
//   0.4 µs shorter), 128 x 256 with three slots
//   for very wide layers, 192 x 128 for long passes, 64 x 128 for short
//   (four slots from K 1,024).
// One template per product type for every M: rows do not depend on M.
template <int QUANT, int EPI>
static void dispatch(hipStream_t s, const GemmArgs& g) {
    const int64_t N = g.w0.rows, K = g.w0.cols, M = g.m;
    if constexpr (EPI == EPI_QKV) {
        if (M <= 512) return run<QUANT, 2, 4, EPI, 4, 4>(s, g);
        return run<QUANT, 6, 4, EPI, 2, 4>(s, g);
    } else if constexpr (EPI == EPI_RELU_F16) {
        if (M <= 512) return run<QUANT, 2, 1, EPI, 4, 2>(s, g);
        if (M >= 8192) return run<QUANT, 12, 2, EPI, 2, 4>(s, g);
        if (N <= 1280) {
            if (N > 768) return run<QUANT, 6, 1, EPI, 4, 4>(s, g);
            return run<QUANT, 4, 1, EPI, 4, 4>(s, g);
        }
        if (K >= 4096) return run<QUANT, 6, 2, EPI, 2, 4>(s, g);
        return run<QUANT, 8, 1, EPI, 2, 4>(s, g);
    } else if constexpr (EPI == EPI_QKPREP) {
        // One head on eight waves of one 32-row weight block each (half the
        // decode per wave and K stage of the four-wave tile): short passes,
        // and long ones whose 64-row X tile stays resident (K <= 768; the
        // 270M model's cold q/k/v 15.9 -> 13.3 us, its cold pass -3.2%); at
        // K 2,560 (the 4B model) eight waves through the ring were slower
        // (396 -> 522 us a launch) than four of two blocks each.
        if (M <= 512) return run32<QUANT, 1, 1, EPI, 4, 8>(s, g);
        if (K <= 768) return run32<QUANT, 2, 1, EPI, 4, 8>(s, g);
        return run32<QUANT, 2, 2, EPI, 4, 4>(s, g);
    } else if constexpr (EPI == EPI_F32) {
        // 32x32x16 tiles (gemm32_kernel) for every M: the same sums per element
        if (g.kfold > 0) {  // K pieces added in registers (up to 96-row tiles: the totals fit)
            if (M <= 512) return run32<QUANT, 1, 1, EPI, 4, 4, true>(s, g);
            return run32<QUANT, 3, 1, EPI, 4, 4, true>(s, g);
        }
        if (M <= 512) return run32<QUANT, 1, 1, EPI, 4, 4>(s, g);
        if (M >= 8192) return run32<QUANT, 4, 1, EPI, 3, 4>(s, g);
        if (g.ksplit > 1) return run32<QUANT, 3, 1, EPI, 4, 4>(s, g);  // split K: twice the tiles
        return run32<QUANT, 2, 1, EPI, 4, 4>(s, g);
    } else {
        if constexpr (EPI == EPI_GELU_TANH) {
            // The decoder's gated products on the 32x32x16 kernel, weights
            // in registers: 96 x 128 outputs, 32 x 128 for short passes
            // (same box against the 16x16x32 kernel below: the 270M
            // model's cold gate/up 20.7 -> 20.2 us, warm 9.7 -> 9.0 us; the
            // 4B model's cold gate/up 1,890 -> 1,565 us, its cold pass
            // -4.8%, warm -5.4%; E2B's warm pass -8.5%).  Ring slots: three
            // for long passes (270M cold pass -0.5%), four for short ones
            // (three: the flushed one-branch passes 1-5% slower); 128-row
            // or 64-column tiles and five slots were 3-10% slower.
            // Branch-sized passes (M <= 64) pair the waves (a gate and an
            // up wave per 32 columns: half the decode per wave and stage;
            // flushed one-branch passes, same box, against 32 x 128 on
            // four waves of gate and up each: the 270M model's gate/up
            // 9.2 -> 7.4 us and pass 1.064 -> 1.027 ms, the 4B model's
            // 23.9 -> 21.4 us and 3.60 -> 3.50 ms).  With X resident (K
            // <= 1,024) nine slots of weights (four: 7.9 us); through the
            // ring 64 rows on four waves, four slots (32 rows on two: 21.8
            // us; five to nine slots 26-29 us).
            if (M <= 64) {
                if (K <= 1024) return run32<QUANT, 1, 1, EPI, 9, 2, false, true>(s, g);
                return run32<QUANT, 2, 1, EPI, 4, 4, false, true>(s, g);
            }
            if (M <= 512) return run32<QUANT, 1, 2, EPI, 4, 4>(s, g);
            return run32<QUANT, 3, 2, EPI, 3, 4>(s, g);
        }
        // Short passes: four ring slots from K 1,024 (two are better at
        // K 640).  The ring depth does not change any sum.
        if (M <= 512) {
            if (K >= 1024) return run<QUANT, 4, 2, EPI, 4, 4>(s, g);
            return run<QUANT, 4, 2, EPI, 2, 4>(s, g);
        }
        if (N >= 8192) return run<QUANT, 8, 4, EPI, 3, 4>(s, g);
        if (M >= 8192) return run<QUANT, 12, 2, EPI, 2, 4>(s, g);
        return run<QUANT, 10, 2, EPI, 3, 4>(s, g);
    }
}

template <int EPI>
static void dispatch_dtype(hipStream_t s, const GemmArgs& g) {
    switch (g.w0.dtype) {
        case F16_DT: return dispatch<F16_DT, EPI>(s, g);
        case Q8_DT: return dispatch<Q8_DT, EPI>(s, g);
        default: return dispatch<Q4_DT, EPI>(s, g);
    }
}

static void check(const half_t* x, int64_t ldx, const DevWeight& w, int64_t ldy, int64_t m) {
    if (m < 0) fail(E_INVALID, "gemm: negative M");
    if (w.cols % 32 != 0) fail(E_INVALID, "gemm: K must be a multiple of 32");
    if (ldx < w.cols || ldx % 8 != 0) fail(E_INVALID, "gemm: X row stride must be >= K and a multiple of 8");
    if (reinterpret_cast<uintptr_t>(x) % 16 != 0 || reinterpret_cast<uintptr_t>(w.data) % 16 != 0)
        fail(E_INVALID, "gemm: operands must be 16-byte aligned");
    if (ldy < w.rows) fail(E_INVALID, "gemm: Y row stride must be >= N");
    if (ldy % 4 != 0) fail(E_INVALID, "gemm: Y row stride must be a multiple of 4");
    if (w.dtype != F16_DT && (!w.scales || w.sld < (w.cols / 32 + 1) / 2 * 2))
        fail(E_INVALID, "gemm: quantized weight without padded scales");
    // Buffer offsets are 32-bit.
    if (m * ldx * 2 >= 0x7fff0000LL || w.rows * w.cols * 2 >= 0x7fff0000LL)
        fail(E_INVALID, "gemm: operand of 2 GiB or more");
}

void launch_gemm(hipStream_t s, const half_t* x, int64_t ldx, const DevWeight& w, float* y, int64_t ldy,
                 int64_t m) {
    check(x, ldx, w, ldy, m);
    if (m == 0) return;
    dispatch_dtype<EPI_F32>(s, GemmArgs{x, ldx, m, w, w, y, ldy, nullptr, {}});
}

void launch_gemm_splitk(hipStream_t s, const half_t* x, int64_t ldx, const DevWeight& w, float* y, int64_t ldy,
                       int64_t m, int parts, int64_t part_stride, int kfold) {
    check(x, ldx, w, ldy, m);
    if (parts < 1 || (parts > 1 && w.cols % (int64_t(G_BK) * parts) != 0))
        fail(E_INVALID, "gemm_splitk: K must split into parts of whole 64-wide stages");
    if (kfold < 0) fail(E_INVALID, "gemm_splitk: negative K piece length");
    if (parts > 1 && part_stride < m * ldy) fail(E_INVALID, "gemm_splitk: partial outputs overlap");
    if (m == 0) return;
    GemmArgs g{x, ldx, m, w, w, y, ldy, nullptr, {}};
    g.ksplit = parts;
    g.part_stride = part_stride;
    g.kfold = kfold;
    dispatch_dtype<EPI_F32>(s, g);
}

void launch_gemm_geglu(hipStream_t s, const half_t* x, int64_t ldx, const DevWeight& wg,
                       const DevWeight& wu, half_t* act, int64_t ldact, int64_t m, bool erf) {
    check(x, ldx, wg, ldact, m);
    if (wu.rows != wg.rows || wu.cols != wg.cols || wu.dtype != wg.dtype || wu.sld != wg.sld)
        fail(E_INVALID, "gemm_geglu: gate and up must share shape and storage type");
    if (m == 0) return;
    const GemmArgs g{x, ldx, m, wg, wu, act, ldact, nullptr, {}};
    if (erf) return dispatch_dtype<EPI_GELU_ERF>(s, g);
    dispatch_dtype<EPI_GELU_TANH>(s, g);
}

void launch_gemm_bias_relu(hipStream_t s, const half_t* x, int64_t ldx, const DevWeight& w,
                           const uint16_t* bias, half_t* y, int64_t ldy, int64_t m) {
    check(x, ldx, w, ldy, m);
    if (!bias) fail(E_INVALID, "gemm_bias_relu: bias required");
    if (m == 0) return;
    dispatch_dtype<EPI_RELU_F16>(s, GemmArgs{x, ldx, m, w, w, y, ldy, bias, {}});
}

void launch_gemm_qkprep(hipStream_t s, const half_t* x, int64_t ldx, const DevWeight& w, const QkArgs& a, int64_t m) {
    check(x, ldx, w, w.rows, m);
    const int64_t slots = a.heads + (a.has_kv ? 2 * a.kv_heads : 0);
    if (a.hd != 256 || a.heads <= 0 || a.kv_heads <= 0 || w.rows != slots * 256)
        fail(E_INVALID, "gemm_qkprep: head_dim 256 and N = (heads + 2 kv_heads) x 256 (heads x 256 without K/V)");
    if (a.base < 0 || a.base + m > a.cap_pad || a.cap_pad % 64) fail(E_INVALID, "gemm_qkprep: cache rows out of range");
    if (a.rope_rows <= 0 || a.rope_dims > a.hd || !a.rope || !a.meta || !a.q_norm || !a.q16)
        fail(E_INVALID, "gemm_qkprep: rope table, row meta, q norm and q output required");
    if (a.has_kv && (!a.k_norm || !a.kc || !a.vt)) fail(E_INVALID, "gemm_qkprep: K/V layer without k norm or cache");
    if (m == 0) return;
    GemmArgs g{x, ldx, m, w, w, nullptr, 0, nullptr, {}};
    g.qk = a;
    g.mshift = a.base % 32;  // row tiles on the cache's 32-row grid: whole V^T chunks per tile
    dispatch_dtype<EPI_QKPREP>(s, g);
}

void launch_gemm_qkv_heads(hipStream_t s, const half_t* x, int64_t ldx, const DevWeight& w,
                           const uint16_t* bias, const QkvHeads& o, int64_t m) {
    check(x, ldx, w, w.rows, m);
    if (o.dq <= 0 || o.dq % 64 != 0 || w.rows != 3 * o.dq)
        fail(E_INVALID, "gemm_qkv_heads: N must be 3 x the q width, a multiple of 64");
    if (o.tpad < m || o.tpad % 32 != 0) fail(E_INVALID, "gemm_qkv_heads: padded rows must cover M, multiple of 32");
    if (!o.q16 || !o.k16 || !o.vt || (o.rope && !o.meta)) fail(E_INVALID, "gemm_qkv_heads: missing output");
    if (m == 0) return;
    dispatch_dtype<EPI_QKV>(s, GemmArgs{x, ldx, m, w, w, nullptr, 0, bias, o});
}

}  // namespace omg
