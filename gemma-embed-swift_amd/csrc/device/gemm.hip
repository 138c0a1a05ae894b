// Q8_0 GEMM on gfx950 MFMA: activations fp16, weights Q8_0 repacked into int8 quant and fp16
// scale planes, dequantised to fp16 while staged into LDS, v_mfma_f32_32x32x16_f16 with fp32
// accumulation. Replaces the reference's gemm_q8_* Metal kernels (Shaders/GEMM.metal:72-165,
// 218-355), which widen Q8_0 to fp32 in threadgroup memory for fp32 8x8 simdgroup MMA.
#include <cstring>

#include "common.hpp"
#include "kernels.hpp"

namespace ge {

// ============================================================================ Q8_0 GEMM
//
// Y[M][N] = X[M][K] * W[N][K]^T. A workgroup computes a BM x BN tile with WM x WN waves, each
// wave a (BM / WM) x (BN / WN) sub-tile of 32 x 32 MFMA accumulators. K advances in stages of
// BK (a multiple of the 32-wide Q8_0 block): the stage after the current one is loaded from
// global memory into registers while the current one is multiplied from LDS, then dequantised
// and stored into the other LDS buffer, one barrier per stage. LDS rows are padded by 8 halves
// so the 16-byte fragment reads of 16 consecutive lanes fall in distinct banks.
//
// Tile order is XCD-aware: workgroups are dealt to the 8 XCDs round robin, so workgroup b runs
// on XCD b % 8; tile (b % 8) * (T / 8) + b / 8 gives each XCD a contiguous, M-major run of tiles,
// whose A row blocks and whole weight matrix stay in that XCD's L2.

__device__ __forceinline__ half8_t dequant8(uint32_t a, uint32_t b, _Float16 d) {
    half8_t r;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        r[j] = _Float16(int8_t((a >> (8 * j)) & 0xff)) * d;
        r[4 + j] = _Float16(int8_t((b >> (8 * j)) & 0xff)) * d;
    }
    return r;
}

template <int BM, int BN, int BK, int WM, int WN, int EPI>
__global__ __launch_bounds__(WM* WN * 64) void gemm_q8_kernel(const uint16_t* __restrict__ X,
                                                               const int8_t* __restrict__ Wq,
                                                               const uint16_t* __restrict__ Ws, void* __restrict__ Y,
                                                               int M, int N, int K, float out_scale, int tiles_n,
                                                               int tiles) {
    constexpr int NT = WM * WN * 64;
    constexpr int LDK = BK + 8;
    constexpr int TM = BM / WM, TN = BN / WN, FM = TM / 32, FN = TN / 32;
    constexpr int ACH = BM * BK / 8;   // 16-byte A chunks per stage (8 halves)
    constexpr int BCH = BN * BK / 16;  // 16-byte B chunks per stage (16 int8)
    constexpr int AL = ACH / NT, BL = BCH / NT;
    static_assert(ACH % NT == 0 && BCH % NT == 0, "staging must divide evenly");
    static_assert(BK % 32 == 0 && TM % 32 == 0 && TN % 32 == 0, "tile shape");
    __shared__ __attribute__((aligned(16))) _Float16 As[2][BM * LDK];
    __shared__ __attribute__((aligned(16))) _Float16 Bs[2][BN * LDK];

    const int b = blockIdx.x;
    const int full = tiles / 8 * 8;
    const int tile = b < full ? (b % 8) * (full / 8) + b / 8 : b;
    const int m0 = (tile / tiles_n) * BM, n0 = (tile % tiles_n) * BN;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int KB = K / BK, KQ = K / 32;

    // Global sources of this thread's staging chunks. Rows past M or N are clamped to the last
    // row: their products land only in outputs that are never stored.
    const uint16_t* ap[AL];
#pragma unroll
    for (int i = 0; i < AL; i++) {
        const int c = tid + i * NT, r = c / (BK / 8), col = (c % (BK / 8)) * 8;
        ap[i] = X + (size_t)min(m0 + r, M - 1) * K + col;
    }
    const int8_t* bp[BL];
    const uint16_t* sp[BL];
#pragma unroll
    for (int i = 0; i < BL; i++) {
        const int c = tid + i * NT, r = c / (BK / 16), col = (c % (BK / 16)) * 16;
        const int rr = min(n0 + r, N - 1);
        bp[i] = Wq + (size_t)rr * K + col;
        sp[i] = Ws + (size_t)rr * KQ + col / 32;
    }

    // Two register slots: stage kb + 2 loads into one while stage kb + 1, loaded a full stage
    // earlier, drains from the other into LDS, so each load has two stages of MFMA work to land.
    u32x4 ra0[AL], rb0[BL], ra1[AL], rb1[BL];
    uint16_t rs0[BL], rs1[BL];
#define GEMM_LOAD(RA, RB, RS, kb)                                                           \
    do {                                                                                    \
        _Pragma("unroll") for (int i = 0; i < AL; i++) RA[i] =                              \
            *reinterpret_cast<const u32x4*>(ap[i] + (kb) * BK);                             \
        _Pragma("unroll") for (int i = 0; i < BL; i++) {                                    \
            RB[i] = *reinterpret_cast<const u32x4*>(bp[i] + (kb) * BK);                     \
            RS[i] = sp[i][(kb) * (BK / 32)];                                                \
        }                                                                                   \
    } while (0)
    // int8 and the fp16 scale are exact in fp16, so q * d rounds once.
#define GEMM_STORE(RA, RB, RS, buf)                                                         \
    do {                                                                                    \
        _Pragma("unroll") for (int i = 0; i < AL; i++) {                                    \
            const int c = tid + i * NT, r = c / (BK / 8), col = (c % (BK / 8)) * 8;         \
            *reinterpret_cast<u32x4*>(&As[buf][r * LDK + col]) = RA[i];                     \
        }                                                                                   \
        _Pragma("unroll") for (int i = 0; i < BL; i++) {                                    \
            const int c = tid + i * NT, r = c / (BK / 16), col = (c % (BK / 16)) * 16;      \
            const _Float16 d = __builtin_bit_cast(_Float16, RS[i]);                         \
            *reinterpret_cast<half8_t*>(&Bs[buf][r * LDK + col]) = dequant8(RB[i][0], RB[i][1], d);     \
            *reinterpret_cast<half8_t*>(&Bs[buf][r * LDK + col + 8]) = dequant8(RB[i][2], RB[i][3], d); \
        }                                                                                   \
    } while (0)

    float16_t acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

    const int wm = wave / WN, wn = wave % WN;
    const int fr = lane & 31, fk = (lane >> 5) * 8;
#define GEMM_MMA_STAGE(buf)                                                                          \
    do {                                                                                             \
        const _Float16* as = &As[buf][(wm * TM + fr) * LDK + fk];                                    \
        const _Float16* bs = &Bs[buf][(wn * TN + fr) * LDK + fk];                                    \
        _Pragma("unroll") for (int ks = 0; ks < BK / 16; ks++) {                                     \
            half8_t af[FM], bf[FN];                                                                  \
            _Pragma("unroll") for (int i = 0; i < FM; i++) af[i] =                                   \
                *reinterpret_cast<const half8_t*>(as + i * 32 * LDK + ks * 16);                      \
            _Pragma("unroll") for (int j = 0; j < FN; j++) bf[j] =                                   \
                *reinterpret_cast<const half8_t*>(bs + j * 32 * LDK + ks * 16);                      \
            _Pragma("unroll") for (int i = 0; i < FM; i++)                                           \
                _Pragma("unroll") for (int j = 0; j < FN; j++) acc[i][j] =                           \
                    __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);        \
        }                                                                                            \
    } while (0)

    // KB is even (checked by the launcher). Stage s lives in register slot s % 2 and LDS buffer s % 2.
    GEMM_LOAD(ra0, rb0, rs0, 0);
    GEMM_LOAD(ra1, rb1, rs1, 1);
    GEMM_STORE(ra0, rb0, rs0, 0);
    __syncthreads();
    // Loads past the last stage re-read the last stage (in bounds, never stored), which keeps
    // every load unconditional so the register slots stay in registers.
    for (int kb = 0; kb < KB; kb += 2) {
        GEMM_LOAD(ra0, rb0, rs0, min(kb + 2, KB - 1));
        GEMM_MMA_STAGE(0);
        GEMM_STORE(ra1, rb1, rs1, 1);
        __syncthreads();
        GEMM_LOAD(ra1, rb1, rs1, min(kb + 3, KB - 1));
        GEMM_MMA_STAGE(1);
        if (kb + 2 < KB) GEMM_STORE(ra0, rb0, rs0, 0);
        __syncthreads();
    }
#undef GEMM_LOAD
#undef GEMM_STORE
#undef GEMM_MMA_STAGE

    // Accumulator layout of a 32x32 MFMA tile: register r of lane l holds
    // row (r / 4) * 8 + (l / 32) * 4 + r % 4, column l % 32.
    const int rbase = m0 + wm * TM + (lane >> 5) * 4;
    if constexpr (EPI == kEpiGeglu) {
        // Weight rows come in 32-row gate/up pairs: tile column pair (2p, 2p + 1) of the wave is
        // (gate, up) for output column (n0 + wn * TN) / 2 + p * 32 + lane % 32.
        static_assert(FN % 2 == 0, "geglu pairs tiles");
        const int F = N / 2;
        _Float16* act = static_cast<_Float16*>(Y);
#pragma unroll
        for (int p = 0; p < FN / 2; p++) {
            const int gcol = n0 + wn * TN + p * 64;
            if (gcol >= N) continue;
            const int col = gcol / 2 + (lane & 31);
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int row = rbase + i * 32 + (r >> 2) * 8 + (r & 3);
                    if (row < M)
                        act[(size_t)row * F + col] = _Float16(gelu_tanh(acc[i][2 * p][r]) * acc[i][2 * p + 1][r] * out_scale);
                }
        }
    } else {
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int j = 0; j < FN; j++) {
                const int col = n0 + wn * TN + j * 32 + (lane & 31);
                if (col >= N) continue;
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int row = rbase + i * 32 + (r >> 2) * 8 + (r & 3);
                    if (row >= M) continue;
                    if (EPI == kEpiF32)
                        static_cast<float*>(Y)[(size_t)row * N + col] = acc[i][j][r] * out_scale;
                    else
                        static_cast<_Float16*>(Y)[(size_t)row * N + col] = _Float16(acc[i][j][r] * out_scale);
                }
            }
    }
}

void q8_fragment_order(const int8_t* q, const uint16_t* s, int rows, int cols, int8_t* fq, uint16_t* fs) {
    const int KQ = cols / 32;
    for (int j = 0; j < rows / 32; j++)
        for (int b = 0; b < KQ; b++) {
            int8_t* chunk = fq + ((size_t)j * KQ + b) * 1024;
            for (int l = 0; l < 64; l++) {
                const int8_t* row = q + (size_t)(32 * j + l % 32) * cols + 32 * b + 8 * (l / 32);
                std::memcpy(chunk + l * 16, row, 8);
                std::memcpy(chunk + l * 16 + 8, row + 16, 8);
            }
            for (int r = 0; r < 32; r++) fs[((size_t)j * KQ + b) * 32 + r] = s[(size_t)(32 * j + r) * KQ + b];
        }
}

// ============================================================================ Q8_0 GEMM, weights in fragment order
//
// The same product with the weights read straight from global memory (L2-resident: a layer's
// matrices are at most a few MB) into registers in fragment order: one coalesced 16-byte load
// per lane brings a lane its B fragments for the two k-steps of one Q8_0 block, dequantised in
// registers. Only the activations go through LDS. Waves split N, so no weight element is
// dequantised twice inside a workgroup. K advances 64 (two Q8_0 blocks) per stage; both operands
// are loaded two stages ahead into a pair of register slots (the loop runs stages in pairs so
// every slot index is a compile-time constant).
template <int BM, int BN, int WM, int WN, int EPI>
__global__ __launch_bounds__(WM* WN * 64) void gemm_q8f_kernel(const uint16_t* __restrict__ X,
                                                                const int8_t* __restrict__ Fq,
                                                                const uint16_t* __restrict__ Fs, void* __restrict__ Y,
                                                                int M, int N, int K, float out_scale, int tiles_n,
                                                                int tiles) {
    constexpr int BK = 64, NT = WM * WN * 64, LDK = BK + 8;
    constexpr int TM = BM / WM, TN = BN / WN, FM = TM / 32, FN = TN / 32;
    constexpr int ACH = BM * BK / 8, AL = ACH / NT;
    static_assert(ACH % NT == 0 && TM % 32 == 0 && TN % 32 == 0, "tile shape");
    __shared__ __attribute__((aligned(16))) _Float16 As[2][BM * LDK];

    const int b = blockIdx.x;
    const int full = tiles / 8 * 8;
    const int tile = b < full ? (b % 8) * (full / 8) + b / 8 : b;
    const int m0 = (tile / tiles_n) * BM, n0 = (tile % tiles_n) * BN;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int KB = K / BK, KQ = K / 32;
    const int wm = wave / WN, wn = wave % WN;

    const uint16_t* ap[AL];
#pragma unroll
    for (int i = 0; i < AL; i++) {
        const int c = tid + i * NT, r = c / (BK / 8), col = (c % (BK / 8)) * 8;
        ap[i] = X + (size_t)min(m0 + r, M - 1) * K + col;
    }
    // This wave's 32-row weight blocks (clamped past N: their outputs are never stored).
    const u32x4* fp[FN];
    const uint16_t* fsp[FN];
#pragma unroll
    for (int j = 0; j < FN; j++) {
        const int jg = min((n0 + wn * TN) / 32 + j, N / 32 - 1);
        fp[j] = reinterpret_cast<const u32x4*>(Fq + (size_t)jg * KQ * 1024) + lane;
        fsp[j] = Fs + (size_t)jg * KQ * 32 + (lane & 31);
    }

    u32x4 ra0[AL], ra1[AL], rb0[FN][2], rb1[FN][2];
    uint16_t rs0[FN][2], rs1[FN][2];
#define GQ_LOAD_A(RA, kb)                                                                                \
    do {                                                                                                 \
        _Pragma("unroll") for (int i = 0; i < AL; i++) RA[i] = *reinterpret_cast<const u32x4*>(ap[i] + (kb) * BK); \
    } while (0)
#define GQ_LOAD_B(RB, RS, kb)                                                                            \
    do {                                                                                                 \
        _Pragma("unroll") for (int j = 0; j < FN; j++) _Pragma("unroll") for (int h = 0; h < 2; h++) {   \
            RB[j][h] = fp[j][(size_t)(2 * (kb) + h) * 64];                                               \
            RS[j][h] = fsp[j][(size_t)(2 * (kb) + h) * 32];                                              \
        }                                                                                                \
    } while (0)
#define GQ_STORE_A(RA, buf)                                                                              \
    do {                                                                                                 \
        _Pragma("unroll") for (int i = 0; i < AL; i++) {                                                 \
            const int c = tid + i * NT, r = c / (BK / 8), col = (c % (BK / 8)) * 8;                      \
            *reinterpret_cast<u32x4*>(&As[buf][r * LDK + col]) = RA[i];                                  \
        }                                                                                                \
    } while (0)
    // k-step ks of the stage: Q8_0 block ks / 2, first or second 8-byte half of the lane's chunk.
#define GQ_MMA(buf, RB, RS)                                                                              \
    do {                                                                                                 \
        const _Float16* as = &As[buf][(wm * TM + (lane & 31)) * LDK + (lane >> 5) * 8];                  \
        _Pragma("unroll") for (int ks = 0; ks < BK / 16; ks++) {                                         \
            half8_t af[FM], bf[FN];                                                                      \
            _Pragma("unroll") for (int i = 0; i < FM; i++) af[i] =                                       \
                *reinterpret_cast<const half8_t*>(as + i * 32 * LDK + ks * 16);                          \
            _Pragma("unroll") for (int j = 0; j < FN; j++) {                                             \
                const u32x4 w = RB[j][ks >> 1];                                                          \
                const _Float16 d = __builtin_bit_cast(_Float16, RS[j][ks >> 1]);                         \
                bf[j] = (ks & 1) ? dequant8(w[2], w[3], d) : dequant8(w[0], w[1], d);                    \
            }                                                                                            \
            _Pragma("unroll") for (int i = 0; i < FM; i++)                                               \
                _Pragma("unroll") for (int j = 0; j < FN; j++) acc[i][j] =                               \
                    __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);            \
        }                                                                                                \
    } while (0)

    float16_t acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

    // KB is even (checked by the launcher). Stage s uses slot s % 2 and LDS buffer s % 2; loads
    // past the last stage re-read the last stage (in bounds, never used).
    GQ_LOAD_A(ra0, 0);
    GQ_LOAD_B(rb0, rs0, 0);
    GQ_LOAD_A(ra1, 1);
    GQ_LOAD_B(rb1, rs1, 1);
    GQ_STORE_A(ra0, 0);
    __syncthreads();
    for (int kb = 0; kb < KB; kb += 2) {
        GQ_LOAD_A(ra0, min(kb + 2, KB - 1));
        GQ_MMA(0, rb0, rs0);
        GQ_LOAD_B(rb0, rs0, min(kb + 2, KB - 1));
        GQ_STORE_A(ra1, 1);
        __syncthreads();
        GQ_LOAD_A(ra1, min(kb + 3, KB - 1));
        GQ_MMA(1, rb1, rs1);
        GQ_LOAD_B(rb1, rs1, min(kb + 3, KB - 1));
        if (kb + 2 < KB) GQ_STORE_A(ra0, 0);
        __syncthreads();
    }
#undef GQ_LOAD_A
#undef GQ_LOAD_B
#undef GQ_STORE_A
#undef GQ_MMA

    const int rbase = m0 + wm * TM + (lane >> 5) * 4;
    if constexpr (EPI == kEpiGeglu) {
        static_assert(FN % 2 == 0, "geglu pairs tiles");
        const int F = N / 2;
        _Float16* act = static_cast<_Float16*>(Y);
#pragma unroll
        for (int p = 0; p < FN / 2; p++) {
            const int gcol = n0 + wn * TN + p * 64;
            if (gcol >= N) continue;
            const int col = gcol / 2 + (lane & 31);
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int row = rbase + i * 32 + (r >> 2) * 8 + (r & 3);
                    if (row < M)
                        act[(size_t)row * F + col] = _Float16(gelu_tanh(acc[i][2 * p][r]) * acc[i][2 * p + 1][r] * out_scale);
                }
        }
    } else {
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int j = 0; j < FN; j++) {
                const int col = n0 + wn * TN + j * 32 + (lane & 31);
                if (col >= N) continue;
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int row = rbase + i * 32 + (r >> 2) * 8 + (r & 3);
                    if (row >= M) continue;
                    if (EPI == kEpiF32)
                        static_cast<float*>(Y)[(size_t)row * N + col] = acc[i][j][r] * out_scale;
                    else
                        static_cast<_Float16*>(Y)[(size_t)row * N + col] = _Float16(acc[i][j][r] * out_scale);
                }
            }
    }
}

template <int BM, int BN, int WM, int WN>
hipError_t gemm_q8f_launch(hipStream_t s, const Q8Dev& w, const uint16_t* x, int M, void* y, GemmEpilogue epi,
                           float out_scale) {
    const int N = w.rows, K = w.cols;
    if (K % 128 != 0 || N % 32 != 0 || !w.fq || !w.fs) return hipErrorInvalidValue;
    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN, tiles = tiles_m * tiles_n;
    const dim3 grid(tiles), block(WM * WN * 64);
    switch (epi) {
    case kEpiF32: launch_kernel(gemm_q8f_kernel<BM, BN, WM, WN, kEpiF32>, grid, block, 0, s, x, w.fq, w.fs, y, M, N, K, out_scale, tiles_n, tiles); break;
    case kEpiF16: launch_kernel(gemm_q8f_kernel<BM, BN, WM, WN, kEpiF16>, grid, block, 0, s, x, w.fq, w.fs, y, M, N, K, out_scale, tiles_n, tiles); break;
    case kEpiGeglu:
        if constexpr ((BN / WN / 32) % 2 == 0)
            launch_kernel(gemm_q8f_kernel<BM, BN, WM, WN, kEpiGeglu>, grid, block, 0, s, x, w.fq, w.fs, y, M, N, K, out_scale, tiles_n, tiles);
        else
            return hipErrorInvalidValue;
        break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

void q8_dequant_fragment_order(const int8_t* q, const uint16_t* s, int rows, int cols, uint16_t* fh) {
    const int KQ = cols / 32, KT = cols / 16;
    for (int j = 0; j < rows / 32; j++)
        for (int t = 0; t < KT; t++) {
            uint16_t* chunk = fh + ((size_t)j * KT + t) * 512;
            for (int l = 0; l < 64; l++) {
                const int row = 32 * j + l % 32, k0 = 16 * t + 8 * (l / 32);
                for (int e = 0; e < 8; e++) {
                    const int k = k0 + e;
                    const _Float16 d = __builtin_bit_cast(_Float16, s[(size_t)row * KQ + k / 32]);
                    // fp32 holds q * d exactly; one rounding to fp16, as dequant8 does on the device.
                    const float v = float(q[(size_t)row * cols + k]) * float(d);
                    chunk[l * 8 + e] = __builtin_bit_cast(uint16_t, _Float16(v));
                }
            }
        }
}

// ============================================================================ GEMM, dequantised weights in fragment order
//
// The Q8_0 weights are dequantised once at upload (fp16 of q * d, the value the in-kernel
// dequantisation produces) and laid out so that one coalesced 16-byte load per lane is that
// lane's B fragment for one 16-wide k-step. Waves split N and stream their fragments straight
// from L2 into registers; only the activations go through LDS. The MFMA loop then carries no
// conversion work: per k-step a wave issues FM LDS reads, FN global loads and FM x FN MFMAs.
// K advances 64 per stage; both operands are loaded two stages ahead into a pair of register
// slots (stages run in pairs so slot indices are compile-time constants).
template <int BM, int BN, int WM, int WN, int EPI>
__global__ __launch_bounds__(WM* WN * 64) void gemm_h_kernel(const uint16_t* __restrict__ X,
                                                              const uint16_t* __restrict__ Fh, void* __restrict__ Y,
                                                              int M, int N, int K, float out_scale, int tiles_n,
                                                              int tiles) {
    constexpr int BK = 64, KS = BK / 16, NT = WM * WN * 64, LDK = BK + 8;
    constexpr int TM = BM / WM, TN = BN / WN, FM = TM / 32, FN = TN / 32;
    constexpr int ACH = BM * BK / 8, AL = ACH / NT;
    static_assert(ACH % NT == 0 && TM % 32 == 0 && TN % 32 == 0, "tile shape");
    __shared__ __attribute__((aligned(16))) _Float16 As[2][BM * LDK];

    const int b = blockIdx.x;
    const int full = tiles / 8 * 8;
    const int tile = b < full ? (b % 8) * (full / 8) + b / 8 : b;
    const int m0 = (tile / tiles_n) * BM, n0 = (tile % tiles_n) * BN;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int KB = K / BK, KT = K / 16;
    const int wm = wave / WN, wn = wave % WN;

    const uint16_t* ap[AL];
#pragma unroll
    for (int i = 0; i < AL; i++) {
        const int c = tid + i * NT, r = c / (BK / 8), col = (c % (BK / 8)) * 8;
        ap[i] = X + (size_t)min(m0 + r, M - 1) * K + col;
    }
    const u32x4* fp[FN];
#pragma unroll
    for (int j = 0; j < FN; j++) {
        const int jg = min((n0 + wn * TN) / 32 + j, N / 32 - 1);
        fp[j] = reinterpret_cast<const u32x4*>(Fh + (size_t)jg * KT * 512) + lane;
    }

    u32x4 ra0[AL], ra1[AL], rb0[FN][KS], rb1[FN][KS];
#define GH_LOAD_A(RA, kb)                                                                                \
    do {                                                                                                 \
        _Pragma("unroll") for (int i = 0; i < AL; i++) RA[i] = *reinterpret_cast<const u32x4*>(ap[i] + (kb) * BK); \
    } while (0)
#define GH_LOAD_B(RB, kb)                                                                                \
    do {                                                                                                 \
        _Pragma("unroll") for (int j = 0; j < FN; j++) _Pragma("unroll") for (int t = 0; t < KS; t++)  \
            RB[j][t] = fp[j][(size_t)((kb) * KS + t) * 64];                                              \
    } while (0)
#define GH_STORE_A(RA, buf)                                                                              \
    do {                                                                                                 \
        _Pragma("unroll") for (int i = 0; i < AL; i++) {                                                 \
            const int c = tid + i * NT, r = c / (BK / 8), col = (c % (BK / 8)) * 8;                      \
            *reinterpret_cast<u32x4*>(&As[buf][r * LDK + col]) = RA[i];                                  \
        }                                                                                                \
    } while (0)
#define GH_MMA(buf, RB)                                                                                  \
    do {                                                                                                 \
        const _Float16* as = &As[buf][(wm * TM + (lane & 31)) * LDK + (lane >> 5) * 8];                  \
        _Pragma("unroll") for (int ks = 0; ks < KS; ks++) {                                              \
            half8_t af[FM];                                                                              \
            _Pragma("unroll") for (int i = 0; i < FM; i++) af[i] =                                       \
                *reinterpret_cast<const half8_t*>(as + i * 32 * LDK + ks * 16);                          \
            _Pragma("unroll") for (int i = 0; i < FM; i++)                                               \
                _Pragma("unroll") for (int j = 0; j < FN; j++) acc[i][j] =                               \
                    __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], __builtin_bit_cast(half8_t, RB[j][ks]), \
                                                           acc[i][j], 0, 0, 0);                          \
        }                                                                                                \
    } while (0)

    float16_t acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

    // Two register slots: stage kb + 2 loads into one while stage kb + 1, loaded a stage earlier,
    // is in the other; loads past the last stage re-read it (in bounds, never used).
    GH_LOAD_A(ra0, 0);
    GH_LOAD_B(rb0, 0);
    GH_LOAD_A(ra1, 1);
    GH_LOAD_B(rb1, 1);
    GH_STORE_A(ra0, 0);
    __syncthreads();
    for (int kb = 0; kb < KB; kb += 2) {
        GH_LOAD_A(ra0, min(kb + 2, KB - 1));
        GH_MMA(0, rb0);
        GH_LOAD_B(rb0, min(kb + 2, KB - 1));
        GH_STORE_A(ra1, 1);
        __syncthreads();
        GH_LOAD_A(ra1, min(kb + 3, KB - 1));
        GH_MMA(1, rb1);
        GH_LOAD_B(rb1, min(kb + 3, KB - 1));
        if (kb + 2 < KB) GH_STORE_A(ra0, 0);
        __syncthreads();
    }
#undef GH_LOAD_A
#undef GH_LOAD_B
#undef GH_STORE_A
#undef GH_MMA

    const int rbase = m0 + wm * TM + (lane >> 5) * 4;
    if constexpr (EPI == kEpiGeglu) {
        static_assert(FN % 2 == 0, "geglu pairs tiles");
        const int F = N / 2;
        _Float16* act = static_cast<_Float16*>(Y);
#pragma unroll
        for (int p = 0; p < FN / 2; p++) {
            const int gcol = n0 + wn * TN + p * 64;
            if (gcol >= N) continue;
            const int col = gcol / 2 + (lane & 31);
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int row = rbase + i * 32 + (r >> 2) * 8 + (r & 3);
                    if (row < M)
                        act[(size_t)row * F + col] = _Float16(gelu_tanh(acc[i][2 * p][r]) * acc[i][2 * p + 1][r] * out_scale);
                }
        }
    } else {
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int j = 0; j < FN; j++) {
                const int col = n0 + wn * TN + j * 32 + (lane & 31);
                if (col >= N) continue;
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int row = rbase + i * 32 + (r >> 2) * 8 + (r & 3);
                    if (row >= M) continue;
                    if (EPI == kEpiF32)
                        static_cast<float*>(Y)[(size_t)row * N + col] = acc[i][j][r] * out_scale;
                    else
                        static_cast<_Float16*>(Y)[(size_t)row * N + col] = _Float16(acc[i][j][r] * out_scale);
                }
            }
    }
}

template <int BM, int BN, int WM, int WN>
hipError_t gemm_h_launch(hipStream_t s, const Q8Dev& w, const uint16_t* x, int M, void* y, GemmEpilogue epi,
                         float out_scale) {
    const int N = w.rows, K = w.cols;
    if (K % 128 != 0 || N % 32 != 0 || !w.fh) return hipErrorInvalidValue;
    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN, tiles = tiles_m * tiles_n;
    const dim3 grid(tiles), block(WM * WN * 64);
    switch (epi) {
    case kEpiF32: launch_kernel(gemm_h_kernel<BM, BN, WM, WN, kEpiF32>, grid, block, 0, s, x, w.fh, y, M, N, K, out_scale, tiles_n, tiles); break;
    case kEpiF16: launch_kernel(gemm_h_kernel<BM, BN, WM, WN, kEpiF16>, grid, block, 0, s, x, w.fh, y, M, N, K, out_scale, tiles_n, tiles); break;
    case kEpiGeglu:
        if constexpr ((BN / WN / 32) % 2 == 0)
            launch_kernel(gemm_h_kernel<BM, BN, WM, WN, kEpiGeglu>, grid, block, 0, s, x, w.fh, y, M, N, K, out_scale, tiles_n, tiles);
        else
            return hipErrorInvalidValue;
        break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// One thread per lane fragment: 8 halves of Q8Dev::fh from the row-major planes.
__global__ __launch_bounds__(256) void q8_fragments_kernel(const int8_t* __restrict__ q, const uint16_t* __restrict__ s,
                                                           int cols, size_t n_frag, u32x4* __restrict__ fh) {
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= n_frag) return;
    const int KT = cols / 16, l = int(idx % 64);
    const size_t chunk = idx / 64;
    const int t = int(chunk % KT), j = int(chunk / KT);
    const int row = 32 * j + l % 32, k0 = 16 * t + 8 * (l / 32);
    const uint32_t* src = reinterpret_cast<const uint32_t*>(q + (size_t)row * cols + k0);
    const _Float16 d = __builtin_bit_cast(_Float16, s[(size_t)row * (cols / 32) + k0 / 32]);
    fh[idx] = __builtin_bit_cast(u32x4, dequant8(src[0], src[1], d));
}

hipError_t launch_q8_fragments(hipStream_t s, const Q8Dev& w, uint16_t* fh) {
    if (!w.q || !w.s || !fh || w.rows <= 0 || w.rows % 32 || w.cols <= 0 || w.cols % 32) return hipErrorInvalidValue;
    const size_t n_frag = (size_t)w.rows / 32 * (w.cols / 16) * 64;
    launch_kernel(q8_fragments_kernel, dim3(unsigned((n_frag + 255) / 256)), dim3(256), 0, s, w.q, w.s, w.cols, n_frag,
                  reinterpret_cast<u32x4*>(fh));
    return hipGetLastError();
}

template <int BM, int BN, int BK, int WM, int WN>
hipError_t gemm_q8_launch(hipStream_t s, const Q8Dev& w, const uint16_t* x, int M, void* y, GemmEpilogue epi,
                          float out_scale) {
    const int N = w.rows, K = w.cols;
    if (K % (2 * BK) != 0) return hipErrorInvalidValue;  // the K loop runs stages in pairs
    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN, tiles = tiles_m * tiles_n;
    const dim3 grid(tiles), block(WM * WN * 64);
    switch (epi) {
    case kEpiF32: launch_kernel(gemm_q8_kernel<BM, BN, BK, WM, WN, kEpiF32>, grid, block, 0, s, x, w.q, w.s, y, M, N, K, out_scale, tiles_n, tiles); break;
    case kEpiF16: launch_kernel(gemm_q8_kernel<BM, BN, BK, WM, WN, kEpiF16>, grid, block, 0, s, x, w.q, w.s, y, M, N, K, out_scale, tiles_n, tiles); break;
    case kEpiGeglu: launch_kernel(gemm_q8_kernel<BM, BN, BK, WM, WN, kEpiGeglu>, grid, block, 0, s, x, w.q, w.s, y, M, N, K, out_scale, tiles_n, tiles); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_gemm_q8(hipStream_t s, const Q8Dev& w, const uint16_t* x, int M, void* y, GemmEpilogue epi,
                          float out_scale) {
    const int N = w.rows, K = w.cols;
    if (M < 0 || N <= 0 || K <= 0 || K % 32 != 0 || N % 64 != 0 || !w.q || !w.s || !x || !y) return hipErrorInvalidValue;
    if (M == 0) return hipSuccess;
    if (w.fh && K % 128 == 0) {
        if (epi == kEpiGeglu) return gemm_h_launch<64, 256, 1, 4>(s, w, x, M, y, epi, out_scale);
        return gemm_h_launch<128, 128, 1, 4>(s, w, x, M, y, epi, out_scale);
    }
    if (K % 128 == 0) return gemm_q8_launch<128, 128, 64, 2, 2>(s, w, x, M, y, epi, out_scale);
    if (K % 64 == 0) return gemm_q8_launch<128, 128, 32, 2, 2>(s, w, x, M, y, epi, out_scale);
    return hipErrorInvalidValue;
}

}  // namespace ge
