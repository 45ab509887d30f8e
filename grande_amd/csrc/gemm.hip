// Dequant-fused MFMA GEMMs for the linear layers (matmul.wgsl and
// matmul_gated.wgsl's job): Y[M,N] = f16(X)[M,K] . deq(W)[N,K]^T with f32
// accumulation on v_mfma_f32_16x16x32_f16.
//
// One workgroup = WGM x 2 wave64s over a BM x BN output tile (8 waves for
// the large tiles, so two waves share each SIMD); K advances 64 at a time
// ("stages").  Data path of one stage:
//
//   global --LDS DMA--> ring slot (NS slots): X tile f16 [BM][64], raw weight
//       codes (Q4: [BNW][2 blocks][16 B], Q8: [BNW][64 B]) and the two block
//       scales of every weight row;
//   ring slot --decode (all threads, one stage ahead)--> f16 weight tile
//       [BNW][64] (two buffers);
//   X tile + f16 weight tile --ds_read_b128--> MFMA.
//
// The DMA (buffer_load ... lds, 16 B or 4 B per lane) keeps NS - 2 stages of
// loads in flight beyond the one being decoded, with no registers held for
// them; the weight is decoded once per workgroup and stage (the reference's
// f16 rounding point, shaders/weight.wgsl:40-54) and read by all BM rows.
// F16 weights skip the decode: their tile is DMA'd straight into the ring.
// One barrier per stage; the decode's arithmetic is interleaved with the
// stage's MFMAs.
//
// X and f16-weight tiles are 128 B per row with the 16 B chunk c of row r
// stored at c ^ ((r >> 1) & 7), so the 16 rows x 4 chunks of one fragment
// read hit distinct banks.
//
// MFMA operand layout (16x16x32 f16): lane l supplies A[l % 16][8*(l/16)..+8)
// and B[8*(l/16)..+8)[l % 16]; the f32 result D[4*(l/16) + r][l % 16] lands
// in element r of the lane's float4.  The weight tile is the A operand and
// the activation tile the B operand, so D = (X W^T)^T and each lane ends up
// with four consecutive output columns of one row: the epilogue stores them
// as one vector.
//
// Bounds: every global read is a buffer load on a per-tile resource, so rows
// past M or N read as zero in hardware; the K tail (K % 64 == 32) is sent
// out of range for X and decoded as zero for W.
#include <string>

#include "common.h"
#include "kern_common.h"

namespace omg {

constexpr int G_BK = 64;  // k per stage
constexpr int G_ROW = G_BK * 2;  // bytes per LDS tile row
constexpr uint32_t OOB = 0x7ffffff0u;  // an offset past every resource
// VALU instructions scheduled after each MFMA of the main loop (0: leave
// the order to the compiler).
constexpr int G_SCHED = 4;

typedef __attribute__((address_space(3))) void* lds_ptr_t;

template <int QUANT, int BM, int BN, bool GATED, int NS, int WGM>
struct Cfg {
    // WGM x 2 waves; wave (wm, wn) computes rows wm * WM.. and columns wn * BN / 2..
    static constexpr int NW = WGM * 2, T = NW * WAVE, WM = BM / WGM;
    static constexpr int BNW = GATED ? 2 * BN : BN;  // weight rows per tile
    static constexpr int MI = WM / 16, NI = BN / 32, NJ = GATED ? 2 * NI : NI;
    // 16-byte chunks per stage and DMA instructions per wave per stage.
    static constexpr int X_CH = BM * 8;
    static constexpr int X_I = X_CH / T;
    static constexpr int W_CPR = QUANT == Q4_DT ? 2 : (QUANT == Q8_DT ? 4 : 8);  // chunks per weight row
    static constexpr int W_CH = BNW * W_CPR;
    static constexpr int W_I = (W_CH + T - 1) / T;
    // Scales: one dword (two f16) per weight row, gate and up rows apart.
    static constexpr int S_HALF = QUANT == F16_DT ? 0 : BN;  // rows per matrix
    static constexpr int S_I = QUANT == F16_DT ? 0 : (S_HALF + T - 1) / T;
    static constexpr int S_MATS = GATED ? 2 : 1;
    static constexpr int C = X_I + W_I + S_I * S_MATS;  // DMA instructions per wave per stage
    static constexpr int X_BYTES = BM * G_ROW;
    static constexpr int W_BYTES = W_I * T * 16;
    static constexpr int S_BYTES = S_I * T * 4;  // per matrix
    static constexpr int STAGE = X_BYTES + W_BYTES + S_MATS * S_BYTES;
    static constexpr int W16_BYTES = QUANT == F16_DT ? 0 : BNW * G_ROW;
    static constexpr int LDS = NS * STAGE + 2 * W16_BYTES;
    // Decode work per thread and stage: one 16 B f16 chunk (8 weights) each.
    static constexpr int DQ = BNW * 8 / T;
    static_assert(WM % 16 == 0 && BN % 32 == 0, "tile sizes");
    static_assert(X_CH % T == 0, "X tile must split evenly over the waves");
    static_assert(QUANT != F16_DT || W_CH % T == 0, "f16 weight tile must split evenly");
    static_assert(QUANT == F16_DT || (BNW * 8) % T == 0, "decode must split evenly");
    static_assert(NS >= 3, "ring needs >= 3 slots");
    static_assert(C <= 63, "vmcnt range");
};

struct GemmArgs {
    const half_t* x;
    int64_t ldx, m;
    DevWeight w0, w1;  // w1: the up projection of the gated kernel
    void* y;
    int64_t ldy;
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

// LDS writes done, then the workgroup barrier; a compiler fence for memory.
__device__ inline void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// matmul_gated.wgsl:126-134: tanh GELU with the argument clamped to +-15,
// through the identity 0.5 (1 + tanh z) = 1 / (1 + e^(-2z)) evaluated with
// the hardware exp2 and reciprocal.
__device__ inline float gelu_tanh(float x) {
    float z = 0.7978845608028654f * (x + 0.044715f * x * x * x);
    z = fminf(15.0f, fmaxf(-15.0f, z));
    const float e = __builtin_amdgcn_exp2f(z * -2.8853900817779268f);  // e^(-2z)
    return x * __builtin_amdgcn_rcpf(1.0f + e);
}

template <int QUANT, int BM, int BN, bool GATED, int NS, int WGM>
__global__ __launch_bounds__(WGM * 2 * WAVE) void gemm_kernel(GemmArgs g) {
    using P = Cfg<QUANT, BM, BN, GATED, NS, WGM>;
    constexpr int NW = P::NW;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int tid = int(threadIdx.x), lane = tid % WAVE;
    const int wave = __builtin_amdgcn_readfirstlane(tid / WAVE);
    const int wm = wave / 2, wn = wave % 2;  // wave grid WGM x 2

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
    const int nk = int((K + G_BK - 1) / G_BK);
    const int K32 = int(K), KB32 = int(KB);
    const int64_t rows_m = M - m0 < BM ? M - m0 : BM;
    const int64_t rows_n = N - n0 < BN ? N - n0 : BN;

    // ---- per-tile buffer resources and per-lane DMA offsets (stage 0)
    const __amdgpu_buffer_rsrc_t rx = rsrc(g.x + m0 * g.ldx, rows_m * g.ldx * 2);
    const int64_t wrow = QUANT == Q4_DT ? KB * 16 : (QUANT == Q8_DT ? K : 2 * K);  // bytes per weight row
    const uint8_t* const wbase0 = static_cast<const uint8_t*>(g.w0.data) + n0 * wrow;
    const uint8_t* const wbase1 = static_cast<const uint8_t*>(g.w1.data) + n0 * wrow;
    const uint16_t* const sbase0 = g.w0.scales ? g.w0.scales + n0 * g.w0.sld : nullptr;
    const uint16_t* const sbase1 = g.w1.scales ? g.w1.scales + n0 * g.w1.sld : nullptr;
    const int64_t sbytes = g.w0.scales ? rows_n * g.w0.sld * 2 : 0;

    // X chunk of this lane in instruction i: LDS slot (i * 4 + wave) * 64 + lane.
    uint32_t xoff[P::X_I];
    int xcol[P::X_I];
#pragma unroll
    for (int i = 0; i < P::X_I; ++i) {
        const int slot = (i * NW + wave) * WAVE + lane;
        const int r = slot / 8, lc = (slot % 8) ^ swz(r);
        xcol[i] = lc * 8;
        xoff[i] = uint32_t((r * g.ldx + lc * 8) * 2);
    }
    uint32_t woff[P::W_I];
    bool wup[P::W_I];
#pragma unroll
    for (int i = 0; i < P::W_I; ++i) {
        const int blk = i * NW + wave;  // wave-uniform
        const int slot = blk * WAVE + lane;
        const int rw = slot / P::W_CPR, c = slot % P::W_CPR;
        wup[i] = GATED && blk * WAVE / P::W_CPR >= BN;  // whole instruction on one matrix
        const int n = GATED && rw >= BN ? rw - BN : rw;
        uint32_t o;
        if constexpr (QUANT == Q4_DT) {
            o = uint32_t((n * KB + c) * 16);
        } else if constexpr (QUANT == Q8_DT) {
            o = uint32_t(n * K + c * 16);
        } else {
            const int lc = c ^ swz(rw);
            o = uint32_t((n * K + lc * 8) * 2);
        }
        woff[i] = slot < P::W_CH ? o : OOB;
    }
    uint32_t soff[P::S_I > 0 ? P::S_I : 1];
#pragma unroll
    for (int i = 0; i < P::S_I; ++i) {
        const int slot = (i * NW + wave) * WAVE + lane;  // weight row within one matrix
        soff[i] = slot < BN ? uint32_t(slot * g.w0.sld * 2) : OOB;
    }

    auto slot_base = [&](int s) { return smem + (s % NS) * P::STAGE; };

    // Issue stage s's DMA into its ring slot (all lanes OOB past the end, so
    // every wave always issues P::C instructions per stage).
    auto issue = [&](int s) {
        uint8_t* base = slot_base(s);
        const bool live = s < nk;
        const int k0 = s * G_BK;
        const int kk = live ? K32 : 0;  // past the end: every lane out of range
#pragma unroll
        for (int i = 0; i < P::X_I; ++i) {
            const uint32_t o = k0 + xcol[i] < kk ? xoff[i] + uint32_t(k0 * 2) : OOB;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rx, (lds_ptr_t)(base + (i * NW + wave) * WAVE * 16), 16, o, 0, 0, 0);
        }
        const uint32_t wstep = QUANT == Q4_DT ? uint32_t(k0 / 2) : (QUANT == Q8_DT ? uint32_t(k0) : uint32_t(k0 * 2));
#pragma unroll
        for (int i = 0; i < P::W_I; ++i) {
            const uint32_t o = live ? woff[i] + wstep : OOB;
            // (A select between two buffer resources is not accepted by
            // the host-side compile of this kernel; select the base.)
            const __amdgpu_buffer_rsrc_t rw = rsrc(wup[i] ? wbase1 : wbase0, rows_n * wrow);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rw, (lds_ptr_t)(base + P::X_BYTES + (i * NW + wave) * WAVE * 16), 16, o, 0, 0, 0);
        }
#pragma unroll
        for (int mat = 0; mat < P::S_MATS * (P::S_I > 0 ? 1 : 0); ++mat) {
#pragma unroll
            for (int i = 0; i < P::S_I; ++i) {
                const uint32_t o = live ? soff[i] + uint32_t(k0 / 16) : OOB;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    rsrc(mat ? sbase1 : sbase0, sbytes),
                    (lds_ptr_t)(base + P::X_BYTES + P::W_BYTES + mat * P::S_BYTES + (i * NW + wave) * WAVE * 4),
                    4, o, 0, 0, 0);
            }
        }
    };

    // Decode stage s (raw codes in its ring slot) into f16 tile buffer s & 1,
    // in two halves: the LDS reads of the codes and scales, issued early,
    // and per 16 B chunk the arithmetic and the LDS write, spread between
    // the MFMAs of the current stage.
    struct Raw {
        uint2 code[P::DQ];
        half2v dd[P::DQ];  // the block scale, twice
    };
    auto decode_read = [&](int s, Raw& r) {
        if constexpr (QUANT != F16_DT) {
            const uint8_t* base = slot_base(s);
            const uint8_t* raw = base + P::X_BYTES;
            const uint8_t* sc = base + P::X_BYTES + P::W_BYTES;
            const int kb0 = s * 2;
#pragma unroll
            for (int q = 0; q < P::DQ; ++q) {
                const int w = tid + q * P::T;  // 16 B output chunk: row w / 8, k chunk w % 8
                const int rw = w / 8, lc = w % 8, blk = lc / 4;
                const int srow = GATED && rw >= BN ? P::S_BYTES + (rw - BN) * 4 : rw * 4;
                half_t d = *reinterpret_cast<const half_t*>(sc + srow + blk * 2);
                // K tail: codes past K are garbage but finite ((q - 8) or an
                // int8), so a zero scale zeroes them.
                if (kb0 + blk >= KB32) d = half_t(0.0f);
                r.dd[q] = half2v{d, d};
                if constexpr (QUANT == Q4_DT)
                    r.code[q].x = *reinterpret_cast<const uint32_t*>(raw + rw * 32 + blk * 16 + (lc % 4) * 4);
                else
                    r.code[q] = *reinterpret_cast<const uint2*>(raw + rw * 64 + lc * 8);
            }
        }
    };
    auto decode_write = [&](int s, const Raw& r, int q) {
        if constexpr (QUANT != F16_DT) {
            uint8_t* dst = smem + NS * P::STAGE + (s & 1) * P::W16_BYTES;
            const int w = tid + q * P::T;
            const int rw = w / 8, lc = w % 8;
            half8 v;
            if constexpr (QUANT == Q4_DT)
                v = dq4_word(r.code[q].x, r.dd[q]);
            else
                v = dq8_words(r.code[q].x, r.code[q].y, r.dd[q]);
            *reinterpret_cast<half8*>(dst + rw * G_ROW + ((lc ^ swz(rw)) * 16)) = v;
        }
    };
    auto decode = [&](int s) {
        Raw r;
        decode_read(s, r);
#pragma unroll
        for (int q = 0; q < P::DQ; ++q) decode_write(s, r, q);
    };

    floatx4 acc[P::MI][P::NJ];
#pragma unroll
    for (int i = 0; i < P::MI; ++i)
#pragma unroll
        for (int j = 0; j < P::NJ; ++j) acc[i][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

    // Per-lane LDS byte offsets of the fragment reads (row l % 16 of a
    // 16-row block, chunk ks * 4 + l / 16, swizzled; blocks start at
    // multiples of 16 so the swizzle depends on l % 16 only).
    const int lr = lane % 16;
    int foff[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) foff[ks] = lr * G_ROW + (((ks * 4 + lane / 16) ^ swz(lr)) * 16);

    // ---- prologue: stages 0 .. NS-2 in flight, stage 0 decoded
#pragma unroll
    for (int s = 0; s < NS - 1; ++s) issue(s);
    wait_vm<(NS - 2) * P::C>();
    lds_barrier();
    decode(0);

    for (int kt = 0; kt < nk; ++kt) {
        // stage kt + 1 landed (this wave's DMA), then everyone's, and
        // everyone is done with stage kt - 1 (its slot and f16 buffer)
        wait_vm<(NS - 3) * P::C>();
        lds_barrier();
        issue(kt + NS - 1);

        // Past the last stage the decode below turns the zeros of an
        // out-of-range DMA into a buffer nobody reads; unconditional keeps
        // the loop simple.
        Raw raw;
        decode_read(kt + 1, raw);
        const uint8_t* X = slot_base(kt);
        const uint8_t* W = QUANT == F16_DT ? slot_base(kt) + P::X_BYTES
                                           : smem + NS * P::STAGE + (kt & 1) * P::W16_BYTES;
        half8 af[2][P::MI], bf[2][P::NJ];
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
            for (int i = 0; i < P::MI; ++i)
                af[ks][i] = *reinterpret_cast<const half8*>(X + (wm * P::WM + i * 16) * G_ROW + foff[ks]);
#pragma unroll
            for (int j = 0; j < P::NJ; ++j) {
                const int brow = (GATED && j >= P::NI) ? BN + wn * (BN / 2) + (j - P::NI) * 16 : wn * (BN / 2) + j * 16;
                bf[ks][j] = *reinterpret_cast<const half8*>(W + brow * G_ROW + foff[ks]);
            }
        }
        constexpr int NMF = P::MI * P::NJ * 2;
        constexpr int PER = P::DQ > 0 ? (NMF / P::DQ > 0 ? NMF / P::DQ : 1) : NMF + 1;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int i = 0; i < P::MI; ++i)
#pragma unroll
                for (int j = 0; j < P::NJ; ++j) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bf[ks][j], af[ks][i], acc[i][j], 0, 0, 0);
                    const int m = (ks * P::MI + i) * P::NJ + j + 1;
                    if (m % PER == 0 && m / PER <= P::DQ) decode_write(kt + 1, raw, m / PER - 1);
                }
        if constexpr (G_SCHED > 0) {
            // Issue order for the stage: the DMA, every LDS read (fragments
            // and raw codes), then the MFMAs with the decode's VALU work in
            // their shadow, then the decode's LDS writes.
            constexpr int NDSR = (P::MI + P::NJ) * 2 + (QUANT == F16_DT ? 0 : 2 * P::DQ);
            __builtin_amdgcn_sched_group_barrier(0x020, P::C, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, NDSR, 0);
#pragma unroll
            for (int q = 0; q < NMF; ++q) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, G_SCHED, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x200, P::DQ, 0);
        }
    }
    wait_vm<0>();  // the trailing (out-of-range) DMA before the workgroup ends

    // ---- epilogue: lane (lr, G) holds columns 4G..4G+3 of row lr of each 16 x 16 tile.
#pragma unroll
    for (int i = 0; i < P::MI; ++i) {
        const int64_t m = m0 + wm * P::WM + i * 16 + lr;
        if (m >= M) continue;
#pragma unroll
        for (int j = 0; j < P::NI; ++j) {
            const int64_t n = n0 + wn * (BN / 2) + j * 16 + (lane / 16) * 4;
            float v[4];
#pragma unroll
            for (int r = 0; r < 4; ++r)
                v[r] = GATED ? gelu_tanh(acc[i][j][r]) * acc[i][j + (GATED ? P::NI : 0)][r] : acc[i][j][r];
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

template <int QUANT, int BM, int BN, bool GATED, int NS, int WGM = 2>
static void run(hipStream_t s, const GemmArgs& g) {
    using P = Cfg<QUANT, BM, BN, GATED, NS, WGM>;
    static bool lds_set = false;  // once per instantiation (per process)
    if (!lds_set) {
        OMG_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_kernel<QUANT, BM, BN, GATED, NS, WGM>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, P::LDS));
        lds_set = true;
    }
    const int64_t N = g.w0.rows;
    const int64_t tiles = ((N + BN - 1) / BN) * ((g.m + BM - 1) / BM);
    const dim3 grid(unsigned((tiles + 7) / 8 * 8));
    gemm_kernel<QUANT, BM, BN, GATED, NS, WGM><<<grid, dim3(P::T), P::LDS, s>>>(g);
    OMG_HIP(hipGetLastError());
}

// Tile choice (measured on MI355X over the 270M / 1B decoder shapes):
// 128 x 128 (128 x 64 gated) tiles with 8 waves while they still give about
// 160+ workgroups; smaller tiles for the short branch-only passes.
template <int QUANT, bool GATED>
static void dispatch(hipStream_t s, const GemmArgs& g) {
    const int64_t N = g.w0.rows, M = g.m;
    auto tiles = [&](int64_t bm, int64_t bn) { return ((M + bm - 1) / bm) * ((N + bn - 1) / bn); };
    if constexpr (!GATED) {
        if (tiles(128, 128) >= 160) return run<QUANT, 128, 128, false, 4, 4>(s, g);
        if (tiles(128, 64) >= 160) return run<QUANT, 128, 64, false, 4, 4>(s, g);
        if (tiles(64, 64) >= 128) return run<QUANT, 64, 64, false, 4, 4>(s, g);
        return run<QUANT, 32, 32, false, 8, 2>(s, g);
    } else {
        if (tiles(128, 64) >= 160) return run<QUANT, 128, 64, true, 4, 4>(s, g);
        if (tiles(128, 32) >= 160) return run<QUANT, 128, 32, true, 4, 4>(s, g);
        return run<QUANT, 64, 32, true, 4, 4>(s, g);
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
    if (m * ldx * 2 > 0x7fffffffLL || w.rows * w.cols * 2 > 0x7fffffffLL)
        fail(E_INVALID, "gemm: operand larger than 2 GiB");
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
    if (wu.rows != wg.rows || wu.cols != wg.cols || wu.dtype != wg.dtype || wu.sld != wg.sld)
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
