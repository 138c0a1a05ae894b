// Q8_0 GEMM on gfx950 MFMA: y = x * W^T with x fp16 activations and W a Q8_0 matrix that was
// dequantised once, at upload, into fp16 in MFMA fragment order (Q8Dev::fh); v_mfma_f32_32x32x16_f16
// with fp32 accumulation. Replaces the reference's gemm_q8_* Metal kernels
// (Shaders/GEMM.metal:72-165, 218-355), which widen Q8_0 to fp32 in threadgroup memory for fp32
// 8x8 simdgroup MMA on every call.
#include "common.hpp"
#include "kernels.hpp"

namespace ge {

__device__ __forceinline__ half8_t dequant8(uint32_t a, uint32_t b, _Float16 d) {
    half8_t r;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        r[j] = _Float16(int8_t((a >> (8 * j)) & 0xff)) * d;
        r[4 + j] = _Float16(int8_t((b >> (8 * j)) & 0xff)) * d;
    }
    return r;
}

// Stores a wave's FM x FN accumulator tiles; row0, cbase: the wave's first row and column.
// GUARD false: the caller has checked that every row and column is inside Y.
template <int FM, int FN, int EPI, bool GUARD>
__device__ __forceinline__ void gemm_store_tile_impl(const float16_t (&acc)[FM][FN], void* __restrict__ Y, int M, int N,
                                                     int row0, int cbase, int lane, float out_scale) {
    const int rbase = row0 + (lane >> 5) * 4;
    if constexpr (EPI == kEpiGeglu) {
        static_assert(FN % 2 == 0, "geglu pairs tiles");
        const int F = N / 2;
        _Float16* act = static_cast<_Float16*>(Y);
#pragma unroll
        for (int p = 0; p < FN / 2; p++) {
            const int gcol = cbase + p * 64;
            if (GUARD && gcol >= N) continue;
            _Float16* dst = act + gcol / 2 + (lane & 31);
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int row = rbase + i * 32 + (r >> 2) * 8 + (r & 3);
                    if (!GUARD || row < M)
                        dst[(size_t)row * F] = _Float16(gelu_tanh(acc[i][2 * p][r]) * acc[i][2 * p + 1][r] * out_scale);
                }
        }
    } else {
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int j = 0; j < FN; j++) {
                const int col = cbase + j * 32 + (lane & 31);
                if (GUARD && col >= N) continue;
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int row = rbase + i * 32 + (r >> 2) * 8 + (r & 3);
                    if (GUARD && row >= M) continue;
                    if constexpr (EPI == kEpiF32)
                        static_cast<float*>(Y)[(size_t)row * N + col] = acc[i][j][r] * out_scale;
                    else
                        static_cast<_Float16*>(Y)[(size_t)row * N + col] = _Float16(acc[i][j][r] * out_scale);
                }
            }
    }
}

template <int FM, int FN, int EPI>
__device__ __forceinline__ void gemm_store_tile(const float16_t (&acc)[FM][FN], void* __restrict__ Y, int M, int N,
                                                int row0, int cbase, int lane, float out_scale) {
    if (row0 + FM * 32 <= M && cbase + FN * 32 <= N)
        gemm_store_tile_impl<FM, FN, EPI, false>(acc, Y, M, N, row0, cbase, lane, out_scale);
    else
        gemm_store_tile_impl<FM, FN, EPI, true>(acc, Y, M, N, row0, cbase, lane, out_scale);
}

// ============================================================================ GEMM
//
// Y[M][N] = X[M][K] * W[N][K]^T. A workgroup computes a BM x BN tile with WM x WN waves, each wave
// a (BM / WM) x (BN / WN) block of 32 x 32 MFMA accumulators. Both operands move from global memory into LDS with global_load_lds_dwordx4: each lane's 16
// bytes land at (wave's LDS base) + 16 * lane, and no register holds them on the way. A stage is
// BK columns of K: the activation tile (BM rows, row-major in global memory) and the weight tile
// (BN rows, Q8Dev::fh fragment order, so each of its 1 KB chunks is one contiguous copy). ST stages
// rotate through LDS: while stage s is multiplied, stages s + 1 .. s + ST - 1 are in flight.
//
// Activation chunks hold 1024 / (2 BK) rows of BK halves. The 16-byte slot of logical column
// group g of row r sits at slot g ^ swz(r), which spreads the 32-row fragment reads of one
// k-step over all 64 banks (16 lanes, 16 consecutive rows, are served per cycle); the swizzle is
// applied by choosing each lane's source address.
//
// Tile order is XCD-aware: workgroups are dealt to the 8 XCDs round robin, so workgroup b runs
// on XCD b % 8; tile (b % 8) * (T / 8) + b / 8 gives each XCD a contiguous, M-major run of tiles,
// whose activation row blocks and the weight matrix stay in that XCD's L2.
// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding: vmcnt in bits 3:0
// and 15:14; expcnt and lgkmcnt at their maxima).
template <int BK>
struct DTile {
    static constexpr int RB = 2 * BK;          // bytes per activation row in LDS
    static constexpr int RPC = 1024 / RB;      // rows per 1 KB chunk
    static constexpr int SPR = BK / 8;         // 16-byte slots per row
    static constexpr int RSH = 256 / RB;       // rows covering the 256 bytes of the 64 banks
    __device__ static constexpr int swz(int r) { return (r / RSH) % SPR; }
    // byte offset of (row r, column group g) inside the activation tile
    __device__ static constexpr int a_off(int r, int g) { return (r / RPC) * 1024 + (r % RPC) * RB + ((g ^ swz(r)) * 16); }
};

template <int BM, int BN, int WM, int WN, int BK, int ST>
constexpr int gemm_d_lds_bytes() { return ST * (BM + BN) * BK * 2; }

template <int BM, int BN, int WM, int WN, int BK, int ST, int EPI>
__global__ __launch_bounds__(WM* WN * 64) void gemm_d_kernel(const uint16_t* __restrict__ X,
                                                              const uint16_t* __restrict__ Fh, void* __restrict__ Y,
                                                              int M, int N, int K, float out_scale, int tiles_n,
                                                              int tiles) {
    using T = DTile<BK>;
    constexpr int NW = WM * WN, KS = BK / 16;
    constexpr int TM = BM / WM, TN = BN / WN, FM = TM / 32, FN = TN / 32;
    constexpr int ACH = BM * BK / 512, BCH = BN * BK / 512;  // 1 KB chunks per stage
    constexpr int AW = ACH / NW, BW = BCH / NW;               // chunks per wave per stage
    constexpr int A_BYTES = BM * BK * 2, STAGE = (BM + BN) * BK * 2;
    static_assert(ACH % NW == 0 && BCH % NW == 0 && TM % 32 == 0 && TN % 32 == 0, "tile shape");
    extern __shared__ __attribute__((aligned(1024))) unsigned char lds[];

    const int b = blockIdx.x;
    const int full = tiles / 8 * 8;
    const int tile = b < full ? (b % 8) * (full / 8) + b / 8 : b;
    const int m0 = (tile / tiles_n) * BM, n0 = (tile % tiles_n) * BN;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int KB = K / BK, KT = K / 16;
    const int wm = wave / WN, wn = wave % WN;

    // Source of this lane's 16 bytes for each of the wave's chunks, at stage 0.
    const uint16_t* asrc[AW];
#pragma unroll
    for (int i = 0; i < AW; i++) {
        const int c = wave * AW + i, r = c * T::RPC + lane / T::SPR, slot = lane % T::SPR;
        asrc[i] = X + (size_t)min(m0 + r, M - 1) * K + (slot ^ T::swz(r)) * 8;
    }
    const uint16_t* bsrc[BW];
#pragma unroll
    for (int i = 0; i < BW; i++) {
        const int c = wave * BW + i, jb = c / KS, t = c % KS;
        const int jg = min(n0 / 32 + jb, N / 32 - 1);
        bsrc[i] = Fh + ((size_t)jg * KT + t) * 512 + lane * 8;
    }

#define GD_ISSUE(stage, buf)                                                                               \
    do {                                                                                                   \
        unsigned char* base_ = lds + (buf) * STAGE;                                                        \
        _Pragma("unroll") for (int i = 0; i < AW; i++)                                                     \
            lds_copy16(asrc[i] + (size_t)(stage) * BK, base_ + (wave * AW + i) * 1024);                    \
        _Pragma("unroll") for (int i = 0; i < BW; i++)                                                     \
            lds_copy16(bsrc[i] + (size_t)(stage) * KS * 512, base_ + A_BYTES + (wave * BW + i) * 1024);    \
    } while (0)

    float16_t acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

#pragma unroll
    for (int s = 0; s < ST - 1; s++)
        if (s < KB) GD_ISSUE(s, s);

    const int arow = wm * TM + (lane & 31), half = lane >> 5;
    // Fragment registers are double-buffered: the reads of k-step ks + 1 are issued before the
    // MFMAs of k-step ks. The stage boundary (wait for the next stage's copies, barrier) sits
    // before the last k-step's MFMAs, so reading the next stage's first fragments overlaps them.
    half8_t af[2][FM], bf[2][FN];
#define GD_FRAGS(p, buf, ks)                                                                                  \
    do {                                                                                                      \
        const unsigned char* ab_ = lds + (buf) * STAGE;                                                       \
        _Pragma("unroll") for (int i = 0; i < FM; i++) af[p][i] =                                             \
            *reinterpret_cast<const half8_t*>(ab_ + T::a_off(arow + i * 32, 2 * (ks) + half));                \
        _Pragma("unroll") for (int j = 0; j < FN; j++) bf[p][j] =                                             \
            *reinterpret_cast<const half8_t*>(ab_ + A_BYTES + ((wn * FN + j) * KS + (ks)) * 1024 + lane * 16); \
    } while (0)
#define GD_STAGE_WAIT(kb)                                                                                     \
    do {                                                                                                      \
        if ((kb) + ST - 2 < KB)                                                                               \
            wait_vmcnt<(ST - 2) * (AW + BW)>();                                                               \
        else                                                                                                  \
            wait_vmcnt<0>();                                                                                  \
        wait_lgkmcnt0();                                                                                      \
        workgroup_barrier();                                                                                  \
    } while (0)

    // Stage kb's copies have landed once at most (ST - 2) later stages' copies are outstanding;
    // the barrier then covers every wave's copies. Waiting for this wave's LDS reads first makes
    // the barrier also mean that every read of the buffer the next copies overwrite is done.
    GD_STAGE_WAIT(0);
    GD_FRAGS(0, 0, 0);
    int buf = 0;
    for (int kb = 0; kb < KB; kb++) {
        if (kb + ST - 1 < KB) GD_ISSUE(kb + ST - 1, (buf + ST - 1) % ST);
        const int next = buf + 1 == ST ? 0 : buf + 1;
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            const int p = ks & 1;
            if (ks + 1 < KS) {
                GD_FRAGS(p ^ 1, buf, ks + 1);
            } else if (kb + 1 < KB) {
                GD_STAGE_WAIT(kb + 1);
                GD_FRAGS(p ^ 1, next, 0);
            }
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int j = 0; j < FN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[p][i], bf[p][j], acc[i][j], 0, 0, 0);
        }
        buf = next;
    }
#undef GD_FRAGS
#undef GD_STAGE_WAIT
#undef GD_ISSUE
    gemm_store_tile<FM, FN, EPI>(acc, Y, M, N, m0 + wm * TM, n0 + wn * TN, lane, out_scale);
}

template <typename... KArgs>
hipError_t set_lds_limit(void (*kernel)(KArgs...), int bytes) {
    return hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
}

template <int BM, int BN, int WM, int WN, int BK, int ST>
hipError_t gemm_d_launch(hipStream_t s, const Q8Dev& w, const uint16_t* x, int M, void* y, GemmEpilogue epi,
                         float out_scale) {
    const int N = w.rows, K = w.cols;
    constexpr int FN = BN / WN / 32;
    if (K % BK != 0 || N % 32 != 0 || !w.fh) return hipErrorInvalidValue;
    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN, tiles = tiles_m * tiles_n;
    const dim3 grid(tiles), block(WM * WN * 64);
    constexpr uint32_t lds = gemm_d_lds_bytes<BM, BN, WM, WN, BK, ST>();
#define GD_LAUNCH(E) launch_kernel(gemm_d_kernel<BM, BN, WM, WN, BK, ST, E>, grid, block, lds, s, x, w.fh, y, M, N, K, out_scale, tiles_n, tiles)
    if (lds > 65536) {
        hipError_t e = hipSuccess;
        switch (epi) {
        case kEpiF32: e = set_lds_limit(gemm_d_kernel<BM, BN, WM, WN, BK, ST, kEpiF32>, lds); break;
        case kEpiF16: e = set_lds_limit(gemm_d_kernel<BM, BN, WM, WN, BK, ST, kEpiF16>, lds); break;
        case kEpiGeglu:
            if constexpr (FN % 2 == 0) e = set_lds_limit(gemm_d_kernel<BM, BN, WM, WN, BK, ST, kEpiGeglu>, lds);
            break;
        default: break;
        }
        if (e != hipSuccess) return e;
    }
    switch (epi) {
    case kEpiF32: GD_LAUNCH(kEpiF32); break;
    case kEpiF16: GD_LAUNCH(kEpiF16); break;
    case kEpiGeglu:
        if constexpr (FN % 2 == 0)
            GD_LAUNCH(kEpiGeglu);
        else
            return hipErrorInvalidValue;
        break;
    default: return hipErrorInvalidValue;
    }
#undef GD_LAUNCH
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

hipError_t launch_gemm_q8(hipStream_t s, const Q8Dev& w, const uint16_t* x, int M, void* y, GemmEpilogue epi,
                          float out_scale) {
    const int N = w.rows, K = w.cols;
    if (M < 0 || N <= 0 || K <= 0 || K % 32 != 0 || N % 64 != 0 || !w.fh || !x || !y) return hipErrorInvalidValue;
    if (M == 0) return hipSuccess;
    // 128 x 128 tiles, 2 x 2 waves of 64 x 64, K in stages of 32, three stages in LDS (48 KB):
    // the fastest of the tile sweep on every projection shape of the encoder (M = 16384).
    return gemm_d_launch<128, 128, 2, 2, 32, 3>(s, w, x, M, y, epi, out_scale);
}

}  // namespace ge
