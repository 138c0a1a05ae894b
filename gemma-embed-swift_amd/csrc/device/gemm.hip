// Q8_0 GEMM on gfx950 MFMA: y = x * W^T with x fp16 activations and W a Q8_0 matrix that was
// dequantised once, at upload, into fp16 in MFMA fragment order (Q8Dev::fh); v_mfma_f32_32x32x16_f16
// with fp32 accumulation. Replaces the reference's gemm_q8_* Metal kernels
// (Shaders/GEMM.metal:72-165, 218-355), which widen Q8_0 to fp32 in threadgroup memory for fp32
// 8x8 simdgroup MMA on every call.
#include "common.hpp"
#include "kernels.hpp"

#include <atomic>
#include <type_traits>

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
                                                     int row0, int cbase, int lane, float out_scale,
                                                     const GemmEpiArgs& ea) {
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
                float bias = 0.0f;
                _Float16* hdst = nullptr;
                size_t hstride = 0;
                if constexpr (EPI == kEpiGeluBias || EPI == kEpiHeads) bias = ea.bias[col];
                if constexpr (EPI == kEpiHeads) {
                    // column -> (part, head, e) of the head-padded outputs
                    const int g = col / ea.hd, e = col - g * ea.hd, part = g / ea.heads, head = g - part * ea.heads;
                    hdst = reinterpret_cast<_Float16*>(ea.dst[part]) + head * ea.hp + e;
                    hstride = size_t(ea.heads) * ea.hp;
                }
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int row = rbase + i * 32 + (r >> 2) * 8 + (r & 3);
                    if (GUARD && row >= M) continue;
                    if constexpr (EPI == kEpiF32)
                        static_cast<float*>(Y)[(size_t)row * N + col] = acc[i][j][r] * out_scale;
                    else if constexpr (EPI == kEpiGeluBias)
                        static_cast<_Float16*>(Y)[(size_t)row * N + col] = _Float16(gelu_tanh(acc[i][j][r] + bias) * out_scale);
                    else if constexpr (EPI == kEpiHeads)
                        hdst[(size_t)row * hstride] = _Float16((acc[i][j][r] + bias) * out_scale);
                    else
                        static_cast<_Float16*>(Y)[(size_t)row * N + col] = _Float16(acc[i][j][r] * out_scale);
                }
            }
    }
}

template <int FM, int FN, int EPI>
__device__ __forceinline__ void gemm_store_tile(const float16_t (&acc)[FM][FN], void* __restrict__ Y, int M, int N,
                                                int row0, int cbase, int lane, float out_scale, const GemmEpiArgs& ea) {
    if (row0 + FM * 32 <= M && cbase + FN * 32 <= N)
        gemm_store_tile_impl<FM, FN, EPI, false>(acc, Y, M, N, row0, cbase, lane, out_scale, ea);
    else
        gemm_store_tile_impl<FM, FN, EPI, true>(acc, Y, M, N, row0, cbase, lane, out_scale, ea);
}

// ============================================================================ GEMM
//
// Y[M][N] = X[M][K] * W[N][K]^T. A workgroup computes a BM x BN tile with WM x WN waves, each wave
// a (BM / WM) x (BN / WN) block of 32 x 32 MFMA accumulators. Both operands move from global
// memory into LDS with buffer_load_dwordx4 ... lds (lds_copy16): each lane's 16 bytes land at
// (wave's LDS base) + 16 * lane and no register holds them on the way. A stage is BK
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

// A tile shape: BM x BN tile, WM x WN waves, K in stages of BK, ST stages in LDS.
template <int BM_, int BN_, int WM_, int WN_, int BK_, int ST_>
struct GemmCfg {
    static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_, BK = BK_, ST = ST_;
    static constexpr int NW = WM * WN, NT = NW * 64, KS = BK / 16;
    static constexpr int TM = BM / WM, TN = BN / WN, FM = TM / 32, FN = TN / 32;
    static constexpr int ACH = BM * BK / 512, BCH = BN * BK / 512;  // 1 KB chunks per stage
    static constexpr int AW = ACH / NW, BW = BCH / NW;               // chunks per wave per stage
    static constexpr int A_BYTES = BM * BK * 2, STAGE = (BM + BN) * BK * 2, LDS = ST * STAGE;
    static_assert(ACH % NW == 0 && BCH % NW == 0 && TM % 32 == 0 && TN % 32 == 0, "tile shape");
    static_assert(KS % 2 == 0, "fragment buffers alternate per k-step and restart at each stage");
    static_assert(LDS <= 160 * 1024, "LDS");
};

// The tile shapes the forward uses (M = 16384 tokens, from the tile sweep over the encoder's
// projections): 128 x 256 tiles of 2 x 4 waves, K in stages of 32, three stages in LDS (72 KB,
// two workgroups per CU) for the wide projections (QKV, gate/up); 256 x 256 tiles of 4 x 4 waves,
// K in stages of 64, two stages (128 KB) for the 768-wide ones (attention output, down).
using GemmWide = GemmCfg<128, 256, 2, 4, 32, 3>;
using GemmSquare = GemmCfg<256, 256, 4, 4, 64, 2>;
using GemmSmall = GemmCfg<128, 128, 2, 2, 64, 2>;
// 256 x 192 tiles of 4 x 2 waves of 64 x 96 (three column fragments, so no GeGLU pairs), K in
// stages of 64, two stages (112 KB): the 768-wide projections over many rows (768 = 4 x 192:
// 256 tiles at 16384 rows, one per CU).
using GemmNarrow = GemmCfg<256, 192, 4, 2, 64, 2>;

// The half-width tile of GemmWide: the same 8 waves as 4 x 2 blocks of 32 x 64 (so GeGLU pairs
// stay in one wave) over 128 x 128. A launch whose tiles leave a last partial round of at most a
// quarter of the workgroup slots (two per CU) runs those last tiles as twice as many half tiles:
// the CUs the partial round would leave idle take the other halves. Every output still comes from
// the same MFMA over the same k order, so the bits do not change (gate/up at 16384 rows, a quarter
// round: 65.9 -> 62.9 us; at 8192, an eighth: 39.4 -> 36.3 us). Larger partial rounds lost:
// 40.6 -> 42.5 us at 10000 rows (0.39 of a round), 54.9 -> 63.1 us at 14000 (0.93).
template <class C>
struct HalfTile {
    using type = void;
};
template <>
struct HalfTile<GemmWide> {
    using type = GemmCfg<128, 128, 4, 2, 32, 3>;
};

// Workgroup b's tile: workgroups are dealt to the 8 XCDs round robin (b runs on XCD b % 8), and
// tile (b % 8) * (T / 8) + b / 8 gives each XCD a contiguous, M-major run of tiles.
__device__ __forceinline__ int xcd_tile(int b, int tiles) {
    const int full = tiles / 8 * 8;
    return b < full ? (b % 8) * (full / 8) + b / 8 : b;
}

// The main loop: acc = X[m0 .. m0 + BM) * W[n0 .. n0 + BN)^T over all of K for this wave's
// (TM x TN) block. TR: accumulate the transposed block (operands swapped in the MFMA): register
// 4 g + e of acc[i][j] then holds row i * 32 + lane % 32, column j * 32 + g * 8 + (lane / 32) * 4 + e
// of the wave's block, instead of row i * 32 + g * 8 + (lane / 32) * 4 + e, column j * 32 + lane % 32.
// Leaves the stage buffers' reads outstanding (the caller waits before reusing LDS).
template <class C, bool TR>
__device__ __forceinline__ void gemm_mainloop(const uint16_t* __restrict__ X, const uint16_t* __restrict__ Fh, int M,
                                              int N, int K, int m0, int n0, unsigned char* lds,
                                              float16_t (&acc)[C::FM][C::FN]) {
    using T = DTile<C::BK>;
    constexpr int BK = C::BK, ST = C::ST, KS = C::KS, FM = C::FM, FN = C::FN, AW = C::AW, BW = C::BW;
    constexpr int A_BYTES = C::A_BYTES, STAGE = C::STAGE;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int KB = K / BK, KT = K / 16;
    const int wm = wave / C::WN, wn = wave % C::WN;

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

#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

#pragma unroll
    for (int s = 0; s < ST - 1; s++)
        if (s < KB) G_ISSUE(s, s);

    const int arow = wm * C::TM + (lane & 31), half = lane >> 5;
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
                acc[i][j] = TR ? __builtin_amdgcn_mfma_f32_32x32x16_f16(bf[p][j], af[p][i], acc[i][j], 0, 0, 0) \
                               : __builtin_amdgcn_mfma_f32_32x32x16_f16(af[p][i], bf[p][j], acc[i][j], 0, 0, 0); \
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
}

// Workgroups [0, n_full) take the first n_full tiles whole; with a half-tile shape (HalfTile), the
// workgroups after them take the remaining tiles' halves, two per tile (the grid is then
// n_full + 2 (tiles - n_full)).
template <class C, int EPI>
__global__ __launch_bounds__(C::NT) void gemm_kernel(const uint16_t* __restrict__ X, const uint16_t* __restrict__ Fh,
                                                      void* __restrict__ Y, int M, int N, int K, float out_scale,
                                                      int tiles_n, int n_full, GemmEpiArgs ea) {
    extern __shared__ __attribute__((aligned(1024))) unsigned char lds[];
    // The epilogue's kernel arguments into SGPRs before the main loop: a scalar load still in
    // flight there would turn every LDS wait of the loop into a full lgkmcnt(0).
    asm volatile("" ::"s"(Y), "s"(out_scale));
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    using CH = typename HalfTile<C>::type;
    if constexpr (!std::is_void_v<CH>) {
        static_assert(CH::NT == C::NT && 2 * CH::BN == C::BN && CH::BM == C::BM && CH::LDS <= C::LDS, "half tile");
        if (int(blockIdx.x) >= n_full) {
            const int hb = int(blockIdx.x) - n_full, tile = n_full + hb / 2;
            const int m0 = (tile / tiles_n) * C::BM, n0 = (tile % tiles_n) * C::BN + (hb % 2) * CH::BN;
            if (n0 >= N) return;  // the right half of a last column tile that N ends inside
            float16_t acc[CH::FM][CH::FN];
            gemm_mainloop<CH, false>(X, Fh, M, N, K, m0, n0, lds, acc);
            gemm_store_tile<CH::FM, CH::FN, EPI>(acc, Y, M, N, m0 + (wave / CH::WN) * CH::TM,
                                                 n0 + (wave % CH::WN) * CH::TN, lane, out_scale, ea);
            return;
        }
    }
    const int tile = xcd_tile(blockIdx.x, n_full);
    const int m0 = (tile / tiles_n) * C::BM, n0 = (tile % tiles_n) * C::BN;
    float16_t acc[C::FM][C::FN];
    gemm_mainloop<C, false>(X, Fh, M, N, K, m0, n0, lds, acc);
    gemm_store_tile<C::FM, C::FN, EPI>(acc, Y, M, N, m0 + (wave / C::WN) * C::TM, n0 + (wave % C::WN) * C::TN, lane,
                                       out_scale, ea);
}


// ============================================================================ skinny GEMM
//
// For short batches (a few dozen tokens) the tiled kernel has a handful of workgroups. Here each
// wave computes one block of 32 rows by 32 * NJ columns over the whole of K on its own: the
// fragments come straight from global memory into registers (activations through a buffer
// resource whose range check returns zeros past row M, weights in fragment order, 1 KB per
// fragment), SK k-steps in flight, no LDS and no barrier. The MFMA, its operand order and the
// order of the k-steps are those of the tiled kernel, so every output has the same bits there
// and here, whichever the batch size selects. TR: the transposed accumulation of the QKV kernel,
// stored as its fp16 staging (acc * out_scale, row-major [M][N]) for the separate row pass.
// SK: k-steps in flight per wave (a short batch's GEMM is bound by how fast its few waves stream
// the weights): the largest of 24, 16, 8 (16, 12, 4 for the GeGLU pairs) that divides K / 16. It
// sets only how far the loads run ahead, not the order of the MFMAs, so it does not change a bit
// of the result. One wave per workgroup, so that the waves land on as many CUs (and their L1
// and L2 request paths) as there are waves: with four per workgroup, a real-architecture
// 1 x 64-token forward took 2.48 ms, with one 1.89 ms, and 1.47 ms once the loads also ran as
// one continuous pipeline (every slot refilled right after its MFMA, no branch around a load).
constexpr int kSkinnyWaves = 1;
template <int EPI, bool TR, int NJ, int SK>
__global__ __launch_bounds__(64 * kSkinnyWaves) void gemm_skinny_kernel(const uint16_t* __restrict__ X,
                                                          const uint16_t* __restrict__ Fh, void* __restrict__ Y,
                                                          int M, int N, int K, float out_scale, GemmEpiArgs ea) {
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
    const int groups = N / (32 * NJ), items = (M + 31) / 32 * groups;
    const int item = blockIdx.x * kSkinnyWaves + wave;
    if (item >= items) return;
    const int rt = item / groups, cg = item % groups;
    const int KT = K / 16;
    // The launcher picks SK dividing K / 16 > 0; known here, the first chunk's loads stay in
    // the entry block, in slot order, instead of sinking below a loop guard.
    __builtin_assume(KT >= SK);
    asm volatile("" ::"s"(Y), "s"(out_scale));
    const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(X, uint32_t(M) * uint32_t(K) * 2u);
    const __amdgpu_buffer_rsrc_t fr = buffer_rsrc(Fh, uint32_t(N) * uint32_t(K) * 2u);
    // lane l: activation row rt * 32 + l % 32, k-step columns 8 (l / 32) .. + 8; weight fragment
    // bytes 16 l of the 1 KB chunk (jb, t)
    const uint32_t aoff = uint32_t(((rt * 32 + (lane & 31)) * K + 8 * (lane >> 5)) * 2);
    uint32_t boff[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) boff[j] = uint32_t(((cg * NJ + j) * KT * 512 + lane * 8) * 2);
    half8_t a[SK], b[SK][NJ];
    // k-step t (wave-uniform) through the scalar offset: no per-load address arithmetic
#define SK_LOAD(u, t)                                                                                   \
    do {                                                                                                \
        a[u] = __builtin_bit_cast(half8_t, __builtin_amdgcn_raw_buffer_load_b128(xr, aoff, (t) * 32, 0)); \
        _Pragma("unroll") for (int j = 0; j < NJ; j++) b[u][j] =                                        \
            __builtin_bit_cast(half8_t, __builtin_amdgcn_raw_buffer_load_b128(fr, boff[j], (t) * 1024, 0)); \
    } while (0)
    float16_t acc[1][NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[0][j][r] = 0.0f;
    // Loads issue in slot order, in the prologue and in the loop (the scheduling barriers), so
    // slot u is always the oldest load in flight when its MFMA comes: the wait before it can
    // leave the other slots' loads in flight.
#pragma unroll
    for (int u = 0; u < SK; u++) {
        SK_LOAD(u, u);
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll 1
    for (int t0 = 0; t0 < KT; t0 += SK) {
#pragma unroll
        for (int u = 0; u < SK; u++) {
#pragma unroll
            for (int j = 0; j < NJ; j++)
                acc[0][j] = TR ? __builtin_amdgcn_mfma_f32_32x32x16_f16(b[u][j], a[u], acc[0][j], 0, 0, 0)
                               : __builtin_amdgcn_mfma_f32_32x32x16_f16(a[u], b[u][j], acc[0][j], 0, 0, 0);
            // The refill of slot u after its MFMAs (the old values dead, so the new ones take the
            // same registers) and unconditional, the last chunk re-reading k-step KT - 1 (never
            // used): a load under a branch, or into a register still holding the previous value,
            // makes the compiler wait for every load in flight.
            SK_LOAD(u, min(t0 + SK + u, KT - 1));
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#undef SK_LOAD
    if constexpr (TR) {
        // register 4 g + e of acc[j]: row rt * 32 + lane % 32, column 32 (cg NJ + j) + 8 g + 4 (lane / 32) + e
        const int row = rt * 32 + (lane & 31);
        if (row < M) {
            _Float16* yrow = static_cast<_Float16*>(Y) + (size_t)row * N + 32 * cg * NJ + 4 * (lane >> 5);
#pragma unroll
            for (int j = 0; j < NJ; j++)
#pragma unroll
                for (int g = 0; g < 4; g++) {
                    half4_t h;
#pragma unroll
                    for (int e = 0; e < 4; e++) h[e] = _Float16(acc[0][j][4 * g + e] * out_scale);
                    *reinterpret_cast<half4_t*>(yrow + 32 * j + 8 * g) = h;
                }
        }
    } else {
        gemm_store_tile<1, NJ, EPI>(acc, Y, M, N, rt * 32, 32 * cg * NJ, lane, out_scale, ea);
    }
}

// ============================================================================ QKV + norms + RoPE
//
// The QKV projection with the per-head RMSNorms, NeoX RoPE and the V transpose of the attention
// input in its epilogue (the reference's separate rms_norm_rows / rope_neox kernels,
// Metal/MetalForward.swift:375-395, Shaders/Elementwise.metal). A 128 x 256 tile holds 256 / HD
// whole heads of 128 tokens. The accumulators (transposed, so a lane holds 4 consecutive columns of
// one token) are staged in LDS as fp16 qkv * scale, the rounding the unfused path stores; then
// the waves take (token, head) units of HD / 16 lanes: a lane holds 8 dims of the head and their
// 8 NeoX partners (qkv_unit below), so the rotation stays in the lane and the head's sum of
// squares is a butterfly over the unit's lanes. Normalised V rows go back into LDS for the
// transposed write, one V^T row (128 tokens) per wave instruction pair.
// One (token, head) unit of the QKV epilogue. The unit's hd/16 lanes each hold dims [k8, k8 + 8)
// (x0) and their NeoX partners [hd/2 + k8, hd/2 + k8 + 8) (x1) of the projection (fp16, scaled by
// c), and the RoPE table entries of pairs k8 .. k8 + 7 (cs: cos, sin interleaved). Returns the
// RMS-normalised values (eps already scaled by c^2), weighted and rotated when `rope` (q and k),
// plain for v. The arithmetic (explicit fused multiply-adds, no contraction beyond them) is the
// same wherever it is inlined, so the fused epilogue and the separate row pass give the same bits.
// Every lane of the unit must take part (the sum of squares is a butterfly over them).
template <int HD>
__device__ __forceinline__ void qkv_unit(const half8_t x0, const half8_t x1, const float4_t (&cs)[4], bool rope,
                                         const float* __restrict__ wnorm, int k8, float eps, half8_t& o0,
                                         half8_t& o1) {
#pragma clang fp contract(off)
    constexpr int LPR = HD / 16;
    float f0[8], f1[8], ss = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; e++) {
        f0[e] = float(x0[e]);
        f1[e] = float(x1[e]);
        ss = __builtin_fmaf(f1[e], f1[e], __builtin_fmaf(f0[e], f0[e], ss));
    }
#pragma unroll
    for (int m = LPR / 2; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, 64);
    const float inv = 1.0f / sqrtf(ss / float(HD) + eps);
    if (rope) {
        const float4_t w00 = *reinterpret_cast<const float4_t*>(wnorm + k8);
        const float4_t w01 = *reinterpret_cast<const float4_t*>(wnorm + k8 + 4);
        const float4_t w10 = *reinterpret_cast<const float4_t*>(wnorm + HD / 2 + k8);
        const float4_t w11 = *reinterpret_cast<const float4_t*>(wnorm + HD / 2 + k8 + 4);
        const float wa[8] = {w00[0], w00[1], w00[2], w00[3], w01[0], w01[1], w01[2], w01[3]};
        const float wb[8] = {w10[0], w10[1], w10[2], w10[3], w11[0], w11[1], w11[2], w11[3]};
#pragma unroll
        for (int e = 0; e < 8; e++) {
            // (a, b) = (first, second) half of pair k8 + e: a' = a c - b s, b' = a s + b c
            const float av = f0[e] * inv * wa[e], bv = f1[e] * inv * wb[e];
            const float c = cs[e / 2][2 * (e % 2)], sn = cs[e / 2][2 * (e % 2) + 1];
            o0[e] = _Float16(__builtin_fmaf(av, c, -(bv * sn)));
            o1[e] = _Float16(__builtin_fmaf(bv, c, av * sn));
        }
    } else {
#pragma unroll
        for (int e = 0; e < 8; e++) {
            o0[e] = _Float16(f0[e] * inv);
            o1[e] = _Float16(f1[e] * inv);
        }
    }
}

struct QkvStage {
    static constexpr int RB = 512;  // bytes per staged row (256 halves)
    // 16-byte chunk c of row r at chunk c ^ (r % 16): the transposed fragment writes of one
    // instruction (32 rows, one chunk) and the V^T column reads spread over the banks.
    __device__ static constexpr int off(int r, int c) { return r * RB + ((c ^ (r & 15)) << 4); }
    static constexpr int BYTES = 128 * RB;
};

template <int HD>
__global__ __launch_bounds__(GemmWide::NT) __attribute__((amdgpu_waves_per_eu(4))) void gemm_qkv_kernel(const uint16_t* __restrict__ X,
                                                                 const uint16_t* __restrict__ Fh, int M, int N, int K,
                                                                 int tiles_n, int tiles, QkvEpilogue a) {
    using C = GemmWide;
    static_assert(C::BM == 128 && C::BN == 256 && 256 % HD == 0, "heads per tile");
    static_assert(QkvStage::BYTES <= C::LDS, "staging fits the stage buffers");
    extern __shared__ __attribute__((aligned(1024))) unsigned char lds[];
    const int tile = xcd_tile(blockIdx.x, tiles);
    const int m0 = (tile / tiles_n) * C::BM, n0 = (tile % tiles_n) * C::BN;
    asm volatile("" ::"s"(a.q_norm), "s"(a.k_norm), "s"(a.positions), "s"(a.rope), "s"(a.q), "s"(a.k), "s"(a.v),
                 "s"(a.vcol), "s"(a.vt), "s"(a.scale), "s"(a.eps), "s"(a.vt_cols), "s"(a.heads), "s"(a.kv_heads));
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave / C::WN, wn = wave % C::WN;
    // Row pass over (row, head) units: a unit is one token's HD values of one head of the tile.
    // LPR lanes take a unit; lane k of them holds dims [8k, 8k + 8) and their NeoX partners
    // [HD/2 + 8k, HD/2 + 8k + 8), so the rotation needs no other lane, and its RoPE table entries
    // (pairs 8k .. 8k + 7, 64 contiguous bytes) and its q / k stores are contiguous across the
    // unit's lanes. Units u = (it * UPI + lane / LPR) * NW + wave.
    const int H = a.heads, KV = a.kv_heads, S = N / HD;
    constexpr int LPR = HD / 16, UPI = 64 / LPR, UNITS = C::BM * (256 / HD), NIT = UNITS / (UPI * C::NW);
    static_assert(NIT * UPI * C::NW == UNITS, "units per wave");
    const int k8 = (lane % LPR) * 8, ug = lane / LPR;
    // The units' positions are loaded before the main loop and their RoPE table entries right
    // after the staging writes, so neither latency is paid in the row pass.
    int upos[NIT];
#pragma unroll
    for (int it = 0; it < NIT; it++) {
        const int u = (it * UPI + ug) * C::NW + wave, t = m0 + u % C::BM;
        upos[it] = t < M ? a.positions[t] : 0;
    }
    float16_t acc[C::FM][C::FN];
    gemm_mainloop<C, true>(X, Fh, M, N, K, m0, n0, lds, acc);

    wait_lgkmcnt0();
    workgroup_barrier();  // every wave's last fragment reads are done: the stages become the tile
#pragma unroll
    for (int i = 0; i < C::FM; i++)
#pragma unroll
        for (int j = 0; j < C::FN; j++)
#pragma unroll
            for (int g = 0; g < 4; g++) {
                half4_t h;
#pragma unroll
                for (int e = 0; e < 4; e++) h[e] = _Float16(acc[i][j][4 * g + e] * a.scale);
                const int r = wm * C::TM + i * 32 + (lane & 31), c = wn * (C::TN / 8) + j * 4 + g;
                *reinterpret_cast<half4_t*>(lds + QkvStage::off(r, c) + (lane >> 5) * 8) = h;
            }
    float4_t cs[NIT][4];
#pragma unroll
    for (int it = 0; it < NIT; it++) {
        const int slot = n0 / HD + ((it * UPI + ug) * C::NW + wave) / C::BM;
        if (slot < H + KV) {
            const float* trow = a.rope + (size_t)upos[it] * HD + 2 * k8;
#pragma unroll
            for (int q = 0; q < 4; q++) cs[it][q] = *reinterpret_cast<const float4_t*>(trow + 4 * q);
        }
    }
    wait_lgkmcnt0();
    workgroup_barrier();

#pragma unroll
    for (int it = 0; it < NIT; it++) {
        const int u = (it * UPI + ug) * C::NW + wave, hh = u / C::BM, r = u % C::BM, t = m0 + r;
        const int slot = n0 / HD + hh;
        const bool valid = slot < S && t < M, isq = slot < H, isk = !isq && slot < H + KV;
        const bool isv = valid && !isq && !isk, rope = isq || isk;
        const half8_t x0 = *reinterpret_cast<const half8_t*>(lds + QkvStage::off(r, (hh * HD + k8) / 8));
        const half8_t x1 = *reinterpret_cast<const half8_t*>(lds + QkvStage::off(r, (hh * HD + HD / 2 + k8) / 8));
        half8_t o0, o1;
        qkv_unit<HD>(x0, x1, cs[it], rope, isq ? a.q_norm : a.k_norm, k8, a.eps, o0, o1);
        if (valid) {
            uint16_t* dst = isq ? a.q : (isk ? a.k : a.v);
            const int dst_heads = isq ? H : KV, dst_slot = isq ? slot : (isk ? slot - H : slot - H - KV);
            if (dst) {
                uint16_t* drow = dst + ((size_t)t * dst_heads + dst_slot) * HD;
                *reinterpret_cast<half8_t*>(drow + k8) = o0;
                *reinterpret_cast<half8_t*>(drow + HD / 2 + k8) = o1;
            }
            if (isv && a.vt) {
                *reinterpret_cast<half8_t*>(lds + QkvStage::off(r, (hh * HD + k8) / 8)) = o0;
                *reinterpret_cast<half8_t*>(lds + QkvStage::off(r, (hh * HD + HD / 2 + k8) / 8)) = o1;
            }
        }
    }
    if (!a.vt) return;
    // V^T rows: vt[(slot - H - KV) * HD + d][vcol[t]] for this tile's V heads.
    const int first_v = H + KV, tile_slot0 = n0 / HD;
    if (tile_slot0 + 256 / HD <= first_v || tile_slot0 >= S) return;  // no V head in this tile
    wait_lgkmcnt0();
    workgroup_barrier();
    const int t0 = m0 + lane, t1 = m0 + 64 + lane;
    const int vc0 = t0 < M ? a.vcol[t0] : -1, vc1 = t1 < M ? a.vcol[t1] : -1;
    for (int hh = 0; hh < 256 / HD; hh++) {
        const int sl = tile_slot0 + hh;
        if (sl < first_v || sl >= S) continue;
#pragma unroll 8
        for (int d = wave; d < HD; d += C::NW) {
            const int col = hh * HD + d;
            uint16_t* row = a.vt + (size_t)((sl - first_v) * HD + d) * a.vt_cols;
            const uint16_t v0 = *reinterpret_cast<const uint16_t*>(lds + QkvStage::off(lane, col >> 3) + (col & 7) * 2);
            const uint16_t v1 = *reinterpret_cast<const uint16_t*>(lds + QkvStage::off(64 + lane, col >> 3) + (col & 7) * 2);
            if (vc0 >= 0) row[vc0] = v0;
            if (vc1 >= 0) row[vc1] = v1;
        }
    }
}


// The QKV epilogue as its own pass over the skinny GEMM's fp16 staging [M][N] (short batches):
// the fused kernel's units and arithmetic (qkv_unit), so the same bits; units u = (token, head)
// in token-major order, hd/16 lanes each. V^T is written straight from registers.
template <int HD>
__global__ __launch_bounds__(256) void qkv_rowpass_kernel(const uint16_t* __restrict__ stage, int M, int N,
                                                          QkvEpilogue a) {
    constexpr int LPR = HD / 16, UPI = 64 / LPR;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int S = N / HD, H = a.heads, KV = a.kv_heads;
    const int gu = (blockIdx.x * 4 + wave) * UPI + lane / LPR, k8 = (lane % LPR) * 8;
    const bool live = gu < M * S;  // the same for all lanes of a unit
    const int t = live ? gu / S : 0, slot = live ? gu % S : 0;
    const bool isq = slot < H, isk = !isq && slot < H + KV, isv = !isq && !isk, rope = isq || isk;
    float4_t cs[4];
    half8_t x0 = {}, x1 = {};
    if (live) {
        if (rope) {
            const float* trow = a.rope + (size_t)a.positions[t] * HD + 2 * k8;
#pragma unroll
            for (int q = 0; q < 4; q++) cs[q] = *reinterpret_cast<const float4_t*>(trow + 4 * q);
        }
        const uint16_t* srow = stage + (size_t)t * N + slot * HD;
        x0 = *reinterpret_cast<const half8_t*>(srow + k8);
        x1 = *reinterpret_cast<const half8_t*>(srow + HD / 2 + k8);
    }
    half8_t o0, o1;
    qkv_unit<HD>(x0, x1, cs, live && rope, isq ? a.q_norm : a.k_norm, k8, a.eps, o0, o1);
    if (!live) return;
    uint16_t* dst = isq ? a.q : (isk ? a.k : a.v);
    const int dst_heads = isq ? H : KV, dst_slot = isq ? slot : (isk ? slot - H : slot - H - KV);
    if (dst) {
        uint16_t* drow = dst + ((size_t)t * dst_heads + dst_slot) * HD;
        *reinterpret_cast<half8_t*>(drow + k8) = o0;
        *reinterpret_cast<half8_t*>(drow + HD / 2 + k8) = o1;
    }
    if (isv && a.vt) {
        const int vc = a.vcol[t];
        _Float16* vt = reinterpret_cast<_Float16*>(a.vt) + (size_t)(slot - H - KV) * HD * a.vt_cols + vc;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            vt[(size_t)(k8 + e) * a.vt_cols] = o0[e];
            vt[(size_t)(HD / 2 + k8 + e) * a.vt_cols] = o1[e];
        }
    }
}

template <typename... KArgs>
hipError_t set_lds_limit(void (*kernel)(KArgs...), int bytes) {
    return hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
}

template <class C>
hipError_t gemm_configure_shape() {
    if constexpr (C::LDS <= 65536) return hipSuccess;
    hipError_t e = set_lds_limit(gemm_kernel<C, kEpiF32>, C::LDS);
    if (e == hipSuccess) e = set_lds_limit(gemm_kernel<C, kEpiF16>, C::LDS);
    if constexpr (C::FN % 2 == 0)
        if (e == hipSuccess) e = set_lds_limit(gemm_kernel<C, kEpiGeglu>, C::LDS);
    if (e == hipSuccess) e = set_lds_limit(gemm_kernel<C, kEpiGeluBias>, C::LDS);
    if (e == hipSuccess) e = set_lds_limit(gemm_kernel<C, kEpiHeads>, C::LDS);
    return e;
}

// Workgroup slots of a GemmWide launch: two workgroups per CU (contexts may be created from
// several threads; they all store the same device's count).
static std::atomic<int> g_wide_slots{512};

hipError_t gemm_configure() {
    int dev = 0, cus = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e == hipSuccess && cus > 0) g_wide_slots.store(2 * cus, std::memory_order_relaxed);
    if (e == hipSuccess) e = gemm_configure_shape<GemmWide>();
    if (e == hipSuccess) e = gemm_configure_shape<GemmSquare>();
    if (e == hipSuccess) e = gemm_configure_shape<GemmSmall>();
    if (e == hipSuccess) e = gemm_configure_shape<GemmNarrow>();
    if (e == hipSuccess) e = set_lds_limit(gemm_qkv_kernel<128>, GemmWide::LDS);
    if (e == hipSuccess) e = set_lds_limit(gemm_qkv_kernel<256>, GemmWide::LDS);
    return e;
}

template <class C>
hipError_t gemm_launch(hipStream_t s, const Q8Dev& w, const uint16_t* x, int M, void* y, GemmEpilogue epi,
                       float out_scale, const GemmEpiArgs& ea) {
    const int N = w.rows, K = w.cols;
    const int tiles_m = (M + C::BM - 1) / C::BM, tiles_n = (N + C::BN - 1) / C::BN, tiles = tiles_m * tiles_n;
    // n_full: the tiles taken whole; a last partial round of slots runs as half tiles (HalfTile)
    int n_full = tiles;
    if constexpr (!std::is_void_v<typename HalfTile<C>::type>)
        if (const int slots = g_wide_slots.load(std::memory_order_relaxed);
            tiles > slots && tiles % slots != 0 && tiles % slots <= slots / 4)
            n_full = tiles - tiles % slots;
    const dim3 grid(n_full + 2 * (tiles - n_full)), block(C::NT);
    switch (epi) {
    case kEpiF32:
        launch_kernel(gemm_kernel<C, kEpiF32>, grid, block, C::LDS, s, x, w.fh, y, M, N, K, out_scale, tiles_n, n_full, ea);
        break;
    case kEpiF16:
        launch_kernel(gemm_kernel<C, kEpiF16>, grid, block, C::LDS, s, x, w.fh, y, M, N, K, out_scale, tiles_n, n_full, ea);
        break;
    case kEpiGeglu:
        if constexpr (C::FN % 2 == 0)
            launch_kernel(gemm_kernel<C, kEpiGeglu>, grid, block, C::LDS, s, x, w.fh, y, M, N, K, out_scale, tiles_n, n_full, ea);
        else
            return hipErrorInvalidValue;  // the GeGLU epilogue pairs column fragments
        break;
    case kEpiGeluBias:
        launch_kernel(gemm_kernel<C, kEpiGeluBias>, grid, block, C::LDS, s, x, w.fh, y, M, N, K, out_scale, tiles_n, n_full, ea);
        break;
    case kEpiHeads:
        launch_kernel(gemm_kernel<C, kEpiHeads>, grid, block, C::LDS, s, x, w.fh, y, M, N, K, out_scale, tiles_n, n_full, ea);
        break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// Operand checks shared by the GEMM launchers; the buffer resources address the operands with
// 32-bit byte offsets.
static bool gemm_operands_ok(const Q8Dev& w, const void* x, int M, const void* y) {
    const int N = w.rows, K = w.cols;
    if (M < 0 || N <= 0 || K <= 0 || K % 32 != 0 || N % 64 != 0 || !w.fh || !x || !y) return false;
    return (uint64_t)M * K * 2 < (1ull << 32) && (uint64_t)N * K * 2 < (1ull << 32);
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

template <int EPI, bool TR, int NJ>
hipError_t gemm_skinny_launch(hipStream_t s, const Q8Dev& w, const uint16_t* x, int M, void* y, float out_scale,
                              const GemmEpiArgs& ea = GemmEpiArgs{}) {
    const int items = (M + 31) / 32 * (w.rows / (32 * NJ));
    const dim3 grid((items + kSkinnyWaves - 1) / kSkinnyWaves), block(64 * kSkinnyWaves);
    const int KT = w.cols / 16;
    constexpr int S0 = NJ == 1 ? 24 : 16, S1 = NJ == 1 ? 16 : 12, S2 = NJ == 1 ? 8 : 4;
    if (KT % S0 == 0)
        launch_kernel(gemm_skinny_kernel<EPI, TR, NJ, S0>, grid, block, 0, s, x, w.fh, y, M, w.rows, w.cols, out_scale, ea);
    else if (KT % S1 == 0)
        launch_kernel(gemm_skinny_kernel<EPI, TR, NJ, S1>, grid, block, 0, s, x, w.fh, y, M, w.rows, w.cols, out_scale, ea);
    else if (KT % S2 == 0)
        launch_kernel(gemm_skinny_kernel<EPI, TR, NJ, S2>, grid, block, 0, s, x, w.fh, y, M, w.rows, w.cols, out_scale, ea);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

// K / 16 must be a multiple of 8 (of 4 would do for the GeGLU pairs).
bool skinny_ok(const Q8Dev& w, int M) { return M <= kSkinnyMaxRows && w.cols % 128 == 0; }

hipError_t launch_gemm_q8(hipStream_t s, const Q8Dev& w, const uint16_t* x, int M, void* y, GemmEpilogue epi,
                          float out_scale, const GemmEpiArgs* eap) {
    const GemmEpiArgs ea = eap ? *eap : GemmEpiArgs{};
    if (epi == kEpiHeads) {
        if (!ea.bias || !ea.dst[0] || !ea.dst[1] || !ea.dst[2] || ea.hd <= 0 || ea.hp < ea.hd || ea.heads <= 0 ||
            w.rows != 3 * ea.heads * ea.hd)
            return hipErrorInvalidValue;
        y = ea.dst[0];
    } else if (epi == kEpiGeluBias && !ea.bias) {
        return hipErrorInvalidValue;
    }
    if (!gemm_operands_ok(w, x, M, y)) return hipErrorInvalidValue;
    if (M == 0) return hipSuccess;
    if (skinny_ok(w, M)) {
        switch (epi) {
        case kEpiF32: return gemm_skinny_launch<kEpiF32, false, 1>(s, w, x, M, y, out_scale);
        case kEpiF16: return gemm_skinny_launch<kEpiF16, false, 1>(s, w, x, M, y, out_scale);
        case kEpiGeglu: return gemm_skinny_launch<kEpiGeglu, false, 2>(s, w, x, M, y, out_scale);
        case kEpiGeluBias: return gemm_skinny_launch<kEpiGeluBias, false, 1>(s, w, x, M, y, out_scale, ea);
        case kEpiHeads: return gemm_skinny_launch<kEpiHeads, false, 1>(s, w, x, M, y, out_scale, ea);
        default: return hipErrorInvalidValue;
        }
    }
    // Tile shapes by projection and batch rows, from sweeps of the shapes (20 launches back to
    // back, one box). The tile shape does not change the results: every shape runs the same MFMA
    // over the same k order. The 768-wide projections (o, down): 128 x 128 tiles (K in stages of
    // 64) below 6144 rows, 128 x 256 from 6144 (the config-2 forward's four parts launch them at
    // 4096 rows each). From 12288 rows the fp16-output projections of at most 1024 outputs whose
    // width 192 divides (768: o and down) take 256 x 192 tiles: at 16384 rows o 22.6 against
    // 23.2 us (256 x 256), down 30.0 against 31.0. The image tower's 1152-wide o and down stay on
    // 128 x 256 inside the tower: with fp32 outputs 256 x 192 lost (o 72.1 against 63.2 us, down
    // 228.7 against 203.3), and with the fp16 o output the tower ran 16.03-16.04 against
    // 15.95 ms per batch (a 256 x 192 workgroup holds a whole CU, so its stores overlap no other
    // workgroup's main loop). The widest projections (the tower's QKV,
    // 3456 outputs, and MLP up, 4352) take 256 x 256 tiles: 139.1 against 151.1 us and 190.4
    // against 203.9. The 2304-wide gate/up stays on 128 x 256 (65.0 against 69.9 us).
    if (w.cols % GemmSquare::BK == 0) {
        if (M >= 12288 && w.rows <= 1024 && w.rows % GemmNarrow::BN == 0 && epi == kEpiF16)
            return gemm_launch<GemmNarrow>(s, w, x, M, y, epi, out_scale, ea);
        if (w.rows <= 1024 && M >= 12288) return gemm_launch<GemmSquare>(s, w, x, M, y, epi, out_scale, ea);
        if (w.rows <= 1024 && M < 6144) return gemm_launch<GemmSmall>(s, w, x, M, y, epi, out_scale, ea);
        if (w.rows >= 3072 && M >= 12288) return gemm_launch<GemmSquare>(s, w, x, M, y, epi, out_scale, ea);
    }
    return gemm_launch<GemmWide>(s, w, x, M, y, epi, out_scale, ea);
}

bool gemm_qkv_supported(int hd, int H, int KV) { return (hd == 128 || hd == 256) && H > 0 && KV > 0; }

hipError_t launch_gemm_qkv(hipStream_t s, const Q8Dev& w, const uint16_t* x, int M, int hd, const QkvEpilogue& e) {
    if (!gemm_operands_ok(w, x, M, e.q) || !gemm_qkv_supported(hd, e.heads, e.kv_heads) || !e.k || (!e.v && !e.vt) ||
        !e.q_norm || !e.k_norm || !e.positions || !e.rope || w.rows != (e.heads + 2 * e.kv_heads) * hd ||
        (e.vt && (!e.vcol || e.vt_cols <= 0)))
        return hipErrorInvalidValue;
    if (M == 0) return hipSuccess;
    if (e.stage && skinny_ok(w, M)) {
        // short batch: the skinny GEMM's fp16 staging, then the row pass (same bits as fused)
        hipError_t r = gemm_skinny_launch<kEpiF16, true, 1>(s, w, x, M, e.stage, e.scale);
        if (r != hipSuccess) return r;
        const int units = M * (w.rows / hd), per_block = 4 * (64 / (hd / 16));
        if (hd == 128)
            launch_kernel(qkv_rowpass_kernel<128>, dim3((units + per_block - 1) / per_block), dim3(256), 0, s, e.stage, M,
                          w.rows, e);
        else
            launch_kernel(qkv_rowpass_kernel<256>, dim3((units + per_block - 1) / per_block), dim3(256), 0, s, e.stage, M,
                          w.rows, e);
        return hipGetLastError();
    }
    using C = GemmWide;
    const int N = w.rows, K = w.cols;
    const int tiles_m = (M + C::BM - 1) / C::BM, tiles_n = (N + C::BN - 1) / C::BN, tiles = tiles_m * tiles_n;
    if (hd == 128)
        launch_kernel(gemm_qkv_kernel<128>, dim3(tiles), dim3(C::NT), C::LDS, s, x, w.fh, M, N, K, tiles_n, tiles, e);
    else
        launch_kernel(gemm_qkv_kernel<256>, dim3(tiles), dim3(C::NT), C::LDS, s, x, w.fh, M, N, K, tiles_n, tiles, e);
    return hipGetLastError();
}

}  // namespace ge
