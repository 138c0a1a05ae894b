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
// a (BM / WM) x (BN / WN) block of 32 x 32 MFMA accumulators. Both operands move from global
// memory into LDS with buffer_load_dwordx4 ... lds: each lane's 16 bytes land at (wave's LDS
// base) + 16 * lane and no register holds them on the way. (The global_load_lds form of the same
// copy is a FLAT instruction, which makes the compiler treat every LDS wait after it as a full
// lgkmcnt(0); the buffer form leaves the fragment reads their partial waits.) A stage is BK
// columns of K: the activation tile (BM rows, row-major in global memory) and the weight tile (BN
// rows, Q8Dev::fh fragment order, so each of its 1 KB chunks is one contiguous copy). ST stages
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

template <int BM, int BN, int BK, int ST>
constexpr int gemm_lds_bytes() { return ST * (BM + BN) * BK * 2; }

// Buffer resource over [p, p + bytes): raw (untyped) dword access, no swizzle; reads past the
// end return zero.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, bytes, 0x00020000);
}

// buffer_load_dwordx4 ... lds: lane l's 16 bytes at byte offset voff + soff of r land at
// lds_base + 16 l (lds_base is wave-uniform). The copy counts against vmcnt like a load.
__device__ __forceinline__ void lds_copy16(__amdgpu_buffer_rsrc_t r, void* lds_base, uint32_t voff, uint32_t soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds_base, 16, voff, soff, 0, 0);
}

template <int BM, int BN, int WM, int WN, int BK, int ST, int EPI>
__global__ __launch_bounds__(WM* WN * 64) void gemm_kernel(const uint16_t* __restrict__ X,
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
    static_assert(KS % 2 == 0, "fragment buffers alternate per k-step and restart at each stage");
    extern __shared__ __attribute__((aligned(1024))) unsigned char lds[];

    const int b = blockIdx.x;
    const int full = tiles / 8 * 8;
    const int tile = b < full ? (b % 8) * (full / 8) + b / 8 : b;
    const int m0 = (tile / tiles_n) * BM, n0 = (tile % tiles_n) * BN;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int KB = K / BK, KT = K / 16;
    const int wm = wave / WN, wn = wave % WN;
    // The epilogue's kernel arguments into SGPRs before the main loop: a scalar load still in
    // flight there would turn every LDS wait of the loop into a full lgkmcnt(0).
    asm volatile("" ::"s"(Y), "s"(out_scale), "s"(M), "s"(N));

    // Byte offset of this lane's 16 bytes for each of the wave's chunks, at stage 0; a stage
    // adds BK * 2 bytes (activations) or KS KB (weights) through the scalar offset.
    const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(X, uint32_t(M) * uint32_t(K) * 2u);
    const __amdgpu_buffer_rsrc_t fr = buffer_rsrc(Fh, uint32_t(N) * uint32_t(K) * 2u);
    uint32_t aoff[AW], boff[BW];
#pragma unroll
    for (int i = 0; i < AW; i++) {
        const int c = wave * AW + i, r = c * T::RPC + lane / T::SPR, slot = lane % T::SPR;
        aoff[i] = uint32_t(((size_t)min(m0 + r, M - 1) * K + (slot ^ T::swz(r)) * 8) * 2);
    }
#pragma unroll
    for (int i = 0; i < BW; i++) {
        const int c = wave * BW + i, jb = c / KS, t = c % KS;
        const int jg = min(n0 / 32 + jb, N / 32 - 1);
        boff[i] = uint32_t((((size_t)jg * KT + t) * 512 + lane * 8) * 2);
    }
#define G_ISSUE(stage, buf)                                                                               \
    do {                                                                                                  \
        unsigned char* base_ = lds + (buf) * STAGE;                                                       \
        _Pragma("unroll") for (int i = 0; i < AW; i++)                                                    \
            lds_copy16(xr, base_ + (wave * AW + i) * 1024, aoff[i], (stage) * BK * 2);                    \
        _Pragma("unroll") for (int i = 0; i < BW; i++)                                                    \
            lds_copy16(fr, base_ + A_BYTES + (wave * BW + i) * 1024, boff[i], (stage) * KS * 1024);       \
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
        if (s < KB) G_ISSUE(s, s);

    const int arow = wm * TM + (lane & 31), half = lane >> 5;
    // Fragment registers are double-buffered: the reads of k-step ks + 1 are issued before the
    // MFMAs of k-step ks. The stage boundary (wait for the next stage's copies, barrier) sits
    // before the last k-step's MFMAs, so reading the next stage's first fragments overlaps them.
    // The scheduling barriers keep the compiler from sinking those reads below the MFMAs.
    half8_t af[2][FM], bf[2][FN];
#define G_FRAGS(p, buf, ks)                                                                                   \
    do {                                                                                                      \
        const unsigned char* ab_ = lds + (buf) * STAGE;                                                       \
        _Pragma("unroll") for (int i = 0; i < FM; i++) af[p][i] =                                             \
            *reinterpret_cast<const half8_t*>(ab_ + T::a_off(arow + i * 32, 2 * (ks) + half));                \
        _Pragma("unroll") for (int j = 0; j < FN; j++) bf[p][j] =                                             \
            *reinterpret_cast<const half8_t*>(ab_ + A_BYTES + ((wn * FN + j) * KS + (ks)) * 1024 + lane * 16); \
    } while (0)
    // One stage. ISSUE: copy stage kb + ST - 1; VMW: copies this wave may leave in flight when
    // stage kb + 1 must have landed (at most ST - 2 later stages); LAST: no next stage. The
    // barrier after waiting for this wave's copies and LDS reads covers every wave's, so it also
    // means every read of the buffer the next copies overwrite is done. ISSUE and LAST are
    // literals, so the loop below has no branch that merges a path without the stage wait into
    // the MFMAs (which would make the compiler wait for the next stage's fragment reads there).
#define G_STAGE(ISSUE, VMW, LAST)                                                                             \
    do {                                                                                                      \
        if (ISSUE) G_ISSUE(kb + ST - 1, (buf + ST - 1) % ST);                                                 \
        const int next = buf + 1 == ST ? 0 : buf + 1;                                                         \
        _Pragma("unroll") for (int ks = 0; ks < KS; ks++) {                                                   \
            const int p = ks & 1;                                                                             \
            if (ks + 1 < KS) {                                                                                \
                G_FRAGS(p ^ 1, buf, ks + 1);                                                                  \
            } else if (!(LAST)) {                                                                             \
                wait_vmcnt<VMW>();                                                                            \
                wait_lgkmcnt0();                                                                              \
                workgroup_barrier();                                                                          \
                G_FRAGS(p ^ 1, next, 0);                                                                      \
            }                                                                                                 \
            __builtin_amdgcn_sched_barrier(0);                                                                \
            _Pragma("unroll") for (int i = 0; i < FM; i++) _Pragma("unroll") for (int j = 0; j < FN; j++)      \
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[p][i], bf[p][j], acc[i][j], 0, 0, 0);    \
            __builtin_amdgcn_sched_barrier(0);                                                                \
        }                                                                                                     \
        buf = next;                                                                                           \
    } while (0)

    if (ST - 2 < KB)
        wait_vmcnt<(ST - 2) * (AW + BW)>();
    else
        wait_vmcnt<0>();
    wait_lgkmcnt0();
    workgroup_barrier();
    G_FRAGS(0, 0, 0);
    int buf = 0, kb = 0;
    for (; kb + ST - 1 < KB; kb++) G_STAGE(1, (ST - 2) * (AW + BW), 0);
    for (; kb < KB - 1; kb++) G_STAGE(0, 0, 0);
    G_STAGE(0, 0, 1);
#undef G_STAGE
#undef G_FRAGS
#undef G_ISSUE
    gemm_store_tile<FM, FN, EPI>(acc, Y, M, N, m0 + wm * TM, n0 + wn * TN, lane, out_scale);
}

template <typename... KArgs>
hipError_t set_lds_limit(void (*kernel)(KArgs...), int bytes) {
    return hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
}

// The tile shapes the forward uses (M = 16384 tokens, from the tile sweep over the encoder's
// projections): 128 x 256 tiles of 2 x 4 waves, K in stages of 32, three stages in LDS (72 KB,
// two workgroups per CU) for the wide projections (QKV, gate/up); 256 x 256 tiles of 4 x 4 waves,
// K in stages of 64, two stages (128 KB) for the 768-wide ones (attention output, down).
struct GemmWide {
    static constexpr int BM = 128, BN = 256, WM = 2, WN = 4, BK = 32, ST = 3;
};
struct GemmSquare {
    static constexpr int BM = 256, BN = 256, WM = 4, WN = 4, BK = 64, ST = 2;
};

template <class C, int EPI>
constexpr auto gemm_kernel_of() { return gemm_kernel<C::BM, C::BN, C::WM, C::WN, C::BK, C::ST, EPI>; }

template <class C>
hipError_t gemm_configure_shape() {
    constexpr int lds = gemm_lds_bytes<C::BM, C::BN, C::BK, C::ST>();
    static_assert(lds <= 160 * 1024, "LDS");
    if constexpr (lds <= 65536) return hipSuccess;
    hipError_t e = set_lds_limit(gemm_kernel_of<C, kEpiF32>(), lds);
    if (e == hipSuccess) e = set_lds_limit(gemm_kernel_of<C, kEpiF16>(), lds);
    if (e == hipSuccess) e = set_lds_limit(gemm_kernel_of<C, kEpiGeglu>(), lds);
    return e;
}

hipError_t gemm_configure() {
    hipError_t e = gemm_configure_shape<GemmWide>();
    if (e == hipSuccess) e = gemm_configure_shape<GemmSquare>();
    return e;
}

template <class C>
hipError_t gemm_launch(hipStream_t s, const Q8Dev& w, const uint16_t* x, int M, void* y, GemmEpilogue epi,
                       float out_scale) {
    const int N = w.rows, K = w.cols;
    const int tiles_m = (M + C::BM - 1) / C::BM, tiles_n = (N + C::BN - 1) / C::BN, tiles = tiles_m * tiles_n;
    const dim3 grid(tiles), block(C::WM * C::WN * 64);
    constexpr uint32_t lds = gemm_lds_bytes<C::BM, C::BN, C::BK, C::ST>();
    switch (epi) {
    case kEpiF32:
        launch_kernel(gemm_kernel_of<C, kEpiF32>(), grid, block, lds, s, x, w.fh, y, M, N, K, out_scale, tiles_n, tiles);
        break;
    case kEpiF16:
        launch_kernel(gemm_kernel_of<C, kEpiF16>(), grid, block, lds, s, x, w.fh, y, M, N, K, out_scale, tiles_n, tiles);
        break;
    case kEpiGeglu:
        launch_kernel(gemm_kernel_of<C, kEpiGeglu>(), grid, block, lds, s, x, w.fh, y, M, N, K, out_scale, tiles_n,
                      tiles);
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

hipError_t launch_gemm_q8(hipStream_t s, const Q8Dev& w, const uint16_t* x, int M, void* y, GemmEpilogue epi,
                          float out_scale) {
    const int N = w.rows, K = w.cols;
    if (M < 0 || N <= 0 || K <= 0 || K % 32 != 0 || N % 64 != 0 || !w.fh || !x || !y) return hipErrorInvalidValue;
    // The buffer resources address the operands with 32-bit byte offsets.
    if ((uint64_t)M * K * 2 >= (1ull << 32) || (uint64_t)N * K * 2 >= (1ull << 32)) return hipErrorInvalidValue;
    if (M == 0) return hipSuccess;
    if (N <= 1024 && K % GemmSquare::BK == 0) return gemm_launch<GemmSquare>(s, w, x, M, y, epi, out_scale);
    return gemm_launch<GemmWide>(s, w, x, M, y, epi, out_scale);
}

}  // namespace ge
