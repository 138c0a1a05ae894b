// Q8_0 GEMM on gfx950 MFMA: activations fp16, weights Q8_0 repacked into int8 quant and fp16
// scale planes, dequantised to fp16 while staged into LDS, v_mfma_f32_32x32x16_f16 with fp32
// accumulation.
#include "common.hpp"
#include "kernels.hpp"

namespace ge {

// ============================================================================ Q8_0 GEMM
//
// Y[M][N] = X[M][K] * W[N][K]^T. Block tile 128 x 128 x 32 (one Q8_0 block along K), 4 waves
// in a 2 x 2 arrangement, each wave a 64 x 64 sub-tile of 2 x 2 MFMA 32x32x16 accumulators.
// LDS holds the fp16 A tile and the dequantised fp16 B tile, double buffered; rows are padded
// to 40 halves (80 bytes) so the 16-byte fragment reads of 16 consecutive lanes hit distinct banks.
namespace gemm {
constexpr int BM = 128, BN = 128, BK = 32, LDK = BK + 8;
}

__device__ __forceinline__ half8_t dequant8(uint32_t a, uint32_t b, _Float16 d) {
    half8_t r;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        r[j] = _Float16(int8_t((a >> (8 * j)) & 0xff)) * d;
        r[4 + j] = _Float16(int8_t((b >> (8 * j)) & 0xff)) * d;
    }
    return r;
}

template <int EPI>
__global__ __launch_bounds__(256) void gemm_q8_kernel(const uint16_t* __restrict__ X, const int8_t* __restrict__ Wq,
                                                      const uint16_t* __restrict__ Ws, void* __restrict__ Y, int M,
                                                      int N, int K, float out_scale) {
    using namespace gemm;
    __shared__ __attribute__((aligned(16))) _Float16 As[2][BM * LDK];
    __shared__ __attribute__((aligned(16))) _Float16 Bs[2][BN * LDK];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int KB = K / BK;

    // Staging: thread t owns row t / 2, columns (t % 2) * 16 .. +16 of both tiles.
    const int sr = tid >> 1, sc = (tid & 1) * 16;
    const bool a_ok = m0 + sr < M, b_ok = n0 + sr < N;
    const uint16_t* xa = X + (size_t)(a_ok ? m0 + sr : 0) * K + sc;
    const int8_t* wb = Wq + (size_t)(b_ok ? n0 + sr : 0) * K + sc;
    const uint16_t* ws = Ws + (size_t)(b_ok ? n0 + sr : 0) * KB;

    uint4 ra0, ra1, rb;
    uint16_t rs;
#define GEMM_LOAD(kb)                                                          \
    do {                                                                       \
        if (a_ok) {                                                            \
            ra0 = *reinterpret_cast<const uint4*>(xa + (kb) * BK);             \
            ra1 = *reinterpret_cast<const uint4*>(xa + (kb) * BK + 8);         \
        } else {                                                               \
            ra0 = make_uint4(0, 0, 0, 0);                                      \
            ra1 = ra0;                                                         \
        }                                                                      \
        if (b_ok) {                                                            \
            rb = *reinterpret_cast<const uint4*>(wb + (kb) * BK);              \
            rs = ws[(kb)];                                                     \
        } else {                                                               \
            rb = make_uint4(0, 0, 0, 0);                                       \
            rs = 0;                                                            \
        }                                                                      \
    } while (0)
    // int8 and the fp16 scale are exact in fp16, so q * d rounds once.
#define GEMM_STORE(buf)                                                                              \
    do {                                                                                             \
        *reinterpret_cast<uint4*>(&As[(buf)][sr * LDK + sc]) = ra0;                                  \
        *reinterpret_cast<uint4*>(&As[(buf)][sr * LDK + sc + 8]) = ra1;                              \
        const _Float16 dsc = __builtin_bit_cast(_Float16, rs);                                       \
        *reinterpret_cast<half8_t*>(&Bs[(buf)][sr * LDK + sc]) = dequant8(rb.x, rb.y, dsc);          \
        *reinterpret_cast<half8_t*>(&Bs[(buf)][sr * LDK + sc + 8]) = dequant8(rb.z, rb.w, dsc);      \
    } while (0)

    float16_t acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

    const int wm = wave >> 1, wn = wave & 1;
    const int fr = lane & 31, fk = (lane >> 5) * 8;

    GEMM_LOAD(0);
    GEMM_STORE(0);
    __syncthreads();
    for (int kb = 0; kb < KB; kb++) {
        const int buf = kb & 1;
        if (kb + 1 < KB) GEMM_LOAD(kb + 1);
        const _Float16* as = &As[buf][(wm * 64 + fr) * LDK + fk];
        const _Float16* bs = &Bs[buf][(wn * 64 + fr) * LDK + fk];
#pragma unroll
        for (int ks = 0; ks < BK / 16; ks++) {
            const half8_t a0 = *reinterpret_cast<const half8_t*>(as + ks * 16);
            const half8_t a1 = *reinterpret_cast<const half8_t*>(as + 32 * LDK + ks * 16);
            const half8_t b0 = *reinterpret_cast<const half8_t*>(bs + ks * 16);
            const half8_t b1 = *reinterpret_cast<const half8_t*>(bs + 32 * LDK + ks * 16);
            acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, b0, acc[0][0], 0, 0, 0);
            acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, b1, acc[0][1], 0, 0, 0);
            acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, b0, acc[1][0], 0, 0, 0);
            acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, b1, acc[1][1], 0, 0, 0);
        }
        if (kb + 1 < KB) GEMM_STORE(buf ^ 1);
        __syncthreads();
    }

    // Accumulator layout of a 32x32 MFMA tile: register r of lane l holds
    // row (r / 4) * 8 + (l / 32) * 4 + r % 4, column l % 32.
    const int rbase = m0 + wm * 64 + (lane >> 5) * 4;
    if (EPI == kEpiGeglu) {
        const int F = N / 2;
        const int col = (n0 + wn * 64) / 2 + (lane & 31);
        _Float16* act = static_cast<_Float16*>(Y);
#pragma unroll
        for (int mi = 0; mi < 2; mi++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int row = rbase + mi * 32 + (r >> 2) * 8 + (r & 3);
                if (row < M && n0 + wn * 64 < N)
                    act[(size_t)row * F + col] = _Float16(gelu_tanh(acc[mi][0][r]) * acc[mi][1][r] * out_scale);
            }
    } else {
#pragma unroll
        for (int mi = 0; mi < 2; mi++)
#pragma unroll
            for (int ni = 0; ni < 2; ni++) {
                const int col = n0 + wn * 64 + ni * 32 + (lane & 31);
                if (col >= N) continue;
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int row = rbase + mi * 32 + (r >> 2) * 8 + (r & 3);
                    if (row >= M) continue;
                    if (EPI == kEpiF32)
                        static_cast<float*>(Y)[(size_t)row * N + col] = acc[mi][ni][r] * out_scale;
                    else
                        static_cast<_Float16*>(Y)[(size_t)row * N + col] = _Float16(acc[mi][ni][r] * out_scale);
                }
            }
    }
}

#undef GEMM_LOAD
#undef GEMM_STORE

hipError_t launch_gemm_q8(hipStream_t s, const Q8Dev& w, const uint16_t* x, int M, void* y, GemmEpilogue epi,
                          float out_scale) {
    using namespace gemm;
    const int N = w.rows, K = w.cols;
    if (M < 0 || N <= 0 || K <= 0 || K % BK != 0 || N % 64 != 0 || !w.q || !w.s || !x || !y) return hipErrorInvalidValue;
    if (M == 0) return hipSuccess;
    dim3 grid((N + BN - 1) / BN, (M + BM - 1) / BM);
    switch (epi) {
    case kEpiF32: launch_kernel(gemm_q8_kernel<kEpiF32>, grid, 256, 0, s, x, w.q, w.s, y, M, N, K, out_scale); break;
    case kEpiF16: launch_kernel(gemm_q8_kernel<kEpiF16>, grid, 256, 0, s, x, w.q, w.s, y, M, N, K, out_scale); break;
    case kEpiGeglu: launch_kernel(gemm_q8_kernel<kEpiGeglu>, grid, 256, 0, s, x, w.q, w.s, y, M, N, K, out_scale); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}


}  // namespace ge
