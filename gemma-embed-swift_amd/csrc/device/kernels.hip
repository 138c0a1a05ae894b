// gfx950 kernels of the GemmaEmbed text-encoder forward pass.
//
// Activations: residual stream fp32, GEMM and attention operands fp16. Weights: Q8_0 repacked
// into int8 quant and fp16 scale planes, dequantised to fp16 while staged into LDS, then
// multiplied on MFMA (v_mfma_f32_32x32x16_f16) with fp32 accumulation.
#include "kernels.hpp"

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

namespace ge {

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

__device__ __forceinline__ float gelu_tanh(float x) {
    // ggml's gelu_tanh constants (reference Shaders/Common.metal:18-21, Model/Architecture.md:45).
    const float c = 0.79788456080286535587989211986876f;
    return 0.5f * x * (1.0f + tanhf(c * x * (1.0f + 0.044715f * x * x)));
}

__device__ __forceinline__ float h2f(uint16_t b) { return float(__builtin_bit_cast(_Float16, b)); }
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, _Float16(f)); }

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
    case kEpiF32: gemm_q8_kernel<kEpiF32><<<grid, 256, 0, s>>>(x, w.q, w.s, y, M, N, K, out_scale); break;
    case kEpiF16: gemm_q8_kernel<kEpiF16><<<grid, 256, 0, s>>>(x, w.q, w.s, y, M, N, K, out_scale); break;
    case kEpiGeglu: gemm_q8_kernel<kEpiGeglu><<<grid, 256, 0, s>>>(x, w.q, w.s, y, M, N, K, out_scale); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ============================================================================ embedding + norm
//
// One wave per token row; each lane owns 4 consecutive elements of every 256-wide chunk.
// x = dequant(table[id]) * scale, then h = rmsnorm(x) * w (reference Shaders/Elementwise.metal:8-35
// and :38-75; Model/CPUReference.swift:190-204, :217).
template <int CH>
__global__ __launch_bounds__(256) void embed_norm_kernel(const int8_t* __restrict__ tq, const uint16_t* __restrict__ ts,
                                                         const int32_t* __restrict__ tokens, int T, int d, float scale,
                                                         const float* __restrict__ w, float eps, float* __restrict__ x,
                                                         uint16_t* __restrict__ h) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= T) return;
    const int id = tokens[row];
    const int8_t* q = tq + (size_t)id * d;
    const uint16_t* sc = ts + (size_t)id * (d / 32);
    float v[CH][4];
    float ss = 0.0f;
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int e = c * 256 + lane * 4;
        if (e < d) {
            const uint32_t packed = *reinterpret_cast<const uint32_t*>(q + e);
            const float ds = h2f(sc[e / 32]);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                v[c][j] = ds * float(int8_t((packed >> (8 * j)) & 0xff)) * scale;
                ss += v[c][j] * v[c][j];
            }
            *reinterpret_cast<float4*>(x + (size_t)row * d + e) = make_float4(v[c][0], v[c][1], v[c][2], v[c][3]);
        }
    }
    ss = wave_sum(ss);
    const float inv = 1.0f / sqrtf(ss / float(d) + eps);
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int e = c * 256 + lane * 4;
        if (e < d) {
            half4_t o;
#pragma unroll
            for (int j = 0; j < 4; j++) o[j] = _Float16(v[c][j] * inv * w[e + j]);
            *reinterpret_cast<half4_t*>(h + (size_t)row * d + e) = o;
        }
    }
}

hipError_t launch_embed_norm(hipStream_t s, const Q8Dev& table, const int32_t* tokens, int T, float scale,
                             const float* norm_w, float eps, float* x, uint16_t* h) {
    const int d = table.cols;
    if (T < 0 || d <= 0 || d % 32 != 0 || d > 1024) return hipErrorInvalidValue;
    if (T == 0) return hipSuccess;
    const int blocks = (T + 3) / 4, CH = (d + 255) / 256;
    switch (CH) {
    case 1: embed_norm_kernel<1><<<blocks, 256, 0, s>>>(table.q, table.s, tokens, T, d, scale, norm_w, eps, x, h); break;
    case 2: embed_norm_kernel<2><<<blocks, 256, 0, s>>>(table.q, table.s, tokens, T, d, scale, norm_w, eps, x, h); break;
    case 3: embed_norm_kernel<3><<<blocks, 256, 0, s>>>(table.q, table.s, tokens, T, d, scale, norm_w, eps, x, h); break;
    default: embed_norm_kernel<4><<<blocks, 256, 0, s>>>(table.q, table.s, tokens, T, d, scale, norm_w, eps, x, h); break;
    }
    return hipGetLastError();
}

// ============================================================================ residual + norms
//
// x = (x + rmsnorm(t) * w) * out_scale, then optionally h = rmsnorm(x) * next_w in fp16: the
// post-attention / post-FFN norm, the residual add and the next block's pre-norm in one pass
// (reference Shaders/Elementwise.metal:260-354; Model/CPUReference.swift:240-245, :254-257, :269).
template <int CH>
__global__ __launch_bounds__(256) void residual_norm_kernel(float* __restrict__ x, const float* __restrict__ t,
                                                            const float* __restrict__ w, float out_scale,
                                                            const float* __restrict__ next_w, float eps, int T, int d,
                                                            uint16_t* __restrict__ h) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= T) return;
    float tv[CH][4], xv[CH][4];
    float ss = 0.0f;
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int e = c * 256 + lane * 4;
        if (e < d) {
            const float4 a = *reinterpret_cast<const float4*>(t + (size_t)row * d + e);
            tv[c][0] = a.x; tv[c][1] = a.y; tv[c][2] = a.z; tv[c][3] = a.w;
#pragma unroll
            for (int j = 0; j < 4; j++) ss += tv[c][j] * tv[c][j];
        }
    }
    ss = wave_sum(ss);
    const float inv = 1.0f / sqrtf(ss / float(d) + eps);
    float ss2 = 0.0f;
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int e = c * 256 + lane * 4;
        if (e < d) {
            float4* xp = reinterpret_cast<float4*>(x + (size_t)row * d + e);
            const float4 a = *xp;
            const float xa[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                xv[c][j] = (xa[j] + tv[c][j] * inv * w[e + j]) * out_scale;
                ss2 += xv[c][j] * xv[c][j];
            }
            *xp = make_float4(xv[c][0], xv[c][1], xv[c][2], xv[c][3]);
        }
    }
    if (!next_w) return;
    ss2 = wave_sum(ss2);
    const float inv2 = 1.0f / sqrtf(ss2 / float(d) + eps);
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int e = c * 256 + lane * 4;
        if (e < d) {
            half4_t o;
#pragma unroll
            for (int j = 0; j < 4; j++) o[j] = _Float16(xv[c][j] * inv2 * next_w[e + j]);
            *reinterpret_cast<half4_t*>(h + (size_t)row * d + e) = o;
        }
    }
}

hipError_t launch_residual_norm(hipStream_t s, float* x, const float* t, const float* w, float out_scale,
                                const float* next_w, float eps, int T, int d, uint16_t* h) {
    if (T < 0 || d <= 0 || d % 4 != 0 || d > 1024 || (next_w && !h)) return hipErrorInvalidValue;
    if (T == 0) return hipSuccess;
    const int blocks = (T + 3) / 4, CH = (d + 255) / 256;
    switch (CH) {
    case 1: residual_norm_kernel<1><<<blocks, 256, 0, s>>>(x, t, w, out_scale, next_w, eps, T, d, h); break;
    case 2: residual_norm_kernel<2><<<blocks, 256, 0, s>>>(x, t, w, out_scale, next_w, eps, T, d, h); break;
    case 3: residual_norm_kernel<3><<<blocks, 256, 0, s>>>(x, t, w, out_scale, next_w, eps, T, d, h); break;
    default: residual_norm_kernel<4><<<blocks, 256, 0, s>>>(x, t, w, out_scale, next_w, eps, T, d, h); break;
    }
    return hipGetLastError();
}

// ============================================================================ QK norm + RoPE
//
// One wave per (token, head slot) of the fused QKV projection. Lane l owns elements
// [l * C, l * C + C) of the first half of the head and their NeoX partners in the second half,
// C = hd / 128, so a rotation pair never leaves the lane (reference Shaders/Elementwise.metal:97-136;
// Model/CPUReference.swift:225-233, :98-113).
template <int HD>
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(const float* __restrict__ qkv, int T, int H, int KV,
                                                           const float* __restrict__ q_norm,
                                                           const float* __restrict__ k_norm, float eps,
                                                           const int32_t* __restrict__ positions,
                                                           const float* __restrict__ table, uint16_t* __restrict__ q,
                                                           uint16_t* __restrict__ k, uint16_t* __restrict__ v) {
    constexpr int C = HD / 128, HALF = HD / 2;
    const int slots = H + 2 * KV;
    const int item = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (item >= T * slots) return;
    const int t = item / slots, slot = item % slots;
    const float* src = qkv + (size_t)t * slots * HD + (size_t)slot * HD;
    float lo[C], hi[C];
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < C; j++) {
        lo[j] = src[lane * C + j];
        hi[j] = src[HALF + lane * C + j];
        ss += lo[j] * lo[j] + hi[j] * hi[j];
    }
    ss = wave_sum(ss);
    const float inv = 1.0f / sqrtf(ss / float(HD) + eps);
    uint16_t* dst;
    const float* w = nullptr;
    bool rope = true;
    if (slot < H) {
        dst = q + ((size_t)t * H + slot) * HD;
        w = q_norm;
    } else if (slot < H + KV) {
        dst = k + ((size_t)t * KV + (slot - H)) * HD;
        w = k_norm;
    } else {
        dst = v + ((size_t)t * KV + (slot - H - KV)) * HD;
        rope = false;
    }
    const float* cs = table + (size_t)positions[t] * HALF * 2;
#pragma unroll
    for (int j = 0; j < C; j++) {
        const int i = lane * C + j;
        float a = lo[j] * inv, b = hi[j] * inv;
        if (w) {
            a *= w[i];
            b *= w[HALF + i];
        }
        if (rope) {
            const float c = cs[2 * i], sn = cs[2 * i + 1];
            const float ra = a * c - b * sn, rb = a * sn + b * c;
            a = ra;
            b = rb;
        }
        dst[i] = f2h(a);
        dst[HALF + i] = f2h(b);
    }
}

hipError_t launch_qk_norm_rope(hipStream_t s, const float* qkv, int T, int H, int KV, int hd, const float* q_norm,
                               const float* k_norm, float eps, const int32_t* positions, const float* rope_table,
                               uint16_t* q, uint16_t* k, uint16_t* v) {
    if (T < 0 || H <= 0 || KV <= 0) return hipErrorInvalidValue;
    if (T == 0) return hipSuccess;
    const long items = (long)T * (H + 2 * KV);
    const int blocks = int((items + 3) / 4);
    switch (hd) {
    case 128: qk_norm_rope_kernel<128><<<blocks, 256, 0, s>>>(qkv, T, H, KV, q_norm, k_norm, eps, positions, rope_table, q, k, v); break;
    case 256: qk_norm_rope_kernel<256><<<blocks, 256, 0, s>>>(qkv, T, H, KV, q_norm, k_norm, eps, positions, rope_table, q, k, v); break;
    case 512: qk_norm_rope_kernel<512><<<blocks, 256, 0, s>>>(qkv, T, H, KV, q_norm, k_norm, eps, positions, rope_table, q, k, v); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ============================================================================ attention
//
// One workgroup per (work item of 32 query rows, KV head); one wave per query head of that KV
// head's group, so every K/V tile staged in LDS serves the whole group. Keys stream in blocks
// of 64 with an online softmax in fp32 (reference Shaders/Attention.metal:25-170).
//
// Both products run transposed so a query is an accumulator column, owned by lane l % 32:
//   S^T[key][query] = K[key][:] . Q[query][:]   (A = K from LDS, B = Q fragments in registers)
//   O^T[d][query]  += V^T[d][key] . P^T[key][query] (A = V^T from LDS, B = P from the S registers)
// so the softmax max / sum over keys is a reduction over a lane's own registers plus its
// partner lane l ^ 32, and the rescale by alpha is per lane. For the second product the 16
// keys of a k-step are split between the two lane halves in the order the S accumulator
// already holds them (keys 4h..4h+3 and 8+4h..8+4h+3 for half h); V^T is read in that order.
namespace attn {
constexpr int BKV = 64;
constexpr int LDV = BKV + 8;
}

template <int HD, int DS>
__global__ __launch_bounds__(256) void attention_kernel(const uint16_t* __restrict__ Qg, const uint16_t* __restrict__ Kg,
                                                        const uint16_t* __restrict__ Vg, uint16_t* __restrict__ Og,
                                                        const AttnWork* __restrict__ work, int H, int KV, int hw,
                                                        float scale) {
    using namespace attn;
    constexpr int LDK = HD + 8;
    extern __shared__ __attribute__((aligned(16))) _Float16 lds[];
    _Float16* Ks = lds;                   // [BKV][LDK]
    _Float16* Vt = lds + BKV * LDK;       // [DS][LDV]
    const AttnWork wi = work[blockIdx.x];
    const int kvh = blockIdx.y, slice = blockIdx.z;
    const int G = H / KV;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nthreads = blockDim.x;
    const int h = kvh * G + wave;
    const int len = int(wi.seq_len), q0 = int(wi.q0);
    const int qStride = H * HD, kvStride = KV * HD;
    const int d0 = slice * DS;
    const int qi = q0 + (lane & 31);
    const bool qvalid = qi < len;

    half8_t qf[HD / 16];
    {
        const _Float16* qp = reinterpret_cast<const _Float16*>(Qg) + (size_t)(wi.seq_start + qi) * qStride + h * HD + (lane >> 5) * 8;
#pragma unroll
        for (int ks = 0; ks < HD / 16; ks++) {
            if (qvalid)
                qf[ks] = *reinterpret_cast<const half8_t*>(qp + ks * 16);
            else
#pragma unroll
                for (int j = 0; j < 8; j++) qf[ks][j] = _Float16(0.0f);
        }
    }

    float16_t o[DS / 32];
#pragma unroll
    for (int i = 0; i < DS / 32; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[i][r] = 0.0f;
    float m_run = -INFINITY, l_run = 0.0f;

    int kstart = 0, kend = len;
    if (hw > 0) {
        kstart = q0 - hw > 0 ? q0 - hw : 0;
        const int hi = q0 + kAttnQueries + hw;
        kend = hi < len ? hi : len;
    }
    kstart = kstart / BKV * BKV;

    const _Float16* kbase = reinterpret_cast<const _Float16*>(Kg) + (size_t)wi.seq_start * kvStride + kvh * HD;
    const _Float16* vbase = reinterpret_cast<const _Float16*>(Vg) + (size_t)wi.seq_start * kvStride + kvh * HD + d0;

    for (int kb = kstart; kb < kend; kb += BKV) {
        __syncthreads();
        // K tile: [64 keys][HD] in 16-byte chunks.
        for (int c = tid; c < BKV * HD / 8; c += nthreads) {
            const int key = c / (HD / 8), col = (c % (HD / 8)) * 8;
            *reinterpret_cast<uint4*>(&Ks[key * LDK + col]) =
                *reinterpret_cast<const uint4*>(kbase + (size_t)(kb + key) * kvStride + col);
        }
        // V^T tile: [DS][64 keys]; a thread moves a pair of keys so each LDS write is 4 bytes.
        for (int c = tid; c < (BKV / 2) * (DS / 8); c += nthreads) {
            const int pair = c % (BKV / 2), col = (c / (BKV / 2)) * 8;
            const half8_t a = *reinterpret_cast<const half8_t*>(vbase + (size_t)(kb + 2 * pair) * kvStride + col);
            const half8_t b = *reinterpret_cast<const half8_t*>(vbase + (size_t)(kb + 2 * pair + 1) * kvStride + col);
#pragma unroll
            for (int e = 0; e < 8; e++) {
                typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
                half2_t p2;
                p2[0] = a[e];
                p2[1] = b[e];
                *reinterpret_cast<half2_t*>(&Vt[(col + e) * LDV + 2 * pair]) = p2;
            }
        }
        __syncthreads();

        float16_t s[2];
#pragma unroll
        for (int kt = 0; kt < 2; kt++) {
#pragma unroll
            for (int r = 0; r < 16; r++) s[kt][r] = 0.0f;
            const _Float16* kp = &Ks[(kt * 32 + (lane & 31)) * LDK + (lane >> 5) * 8];
#pragma unroll
            for (int ks = 0; ks < HD / 16; ks++) {
                const half8_t a = *reinterpret_cast<const half8_t*>(kp + ks * 16);
                s[kt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qf[ks], s[kt], 0, 0, 0);
            }
        }
        float bmax = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < 2; kt++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int key = kb + kt * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
                bool valid = key < len;
                if (hw > 0) valid = valid && abs(qi - key) <= hw;
                const float val = valid ? s[kt][r] * scale : -INFINITY;
                s[kt][r] = val;
                bmax = fmaxf(bmax, val);
            }
        bmax = fmaxf(bmax, __shfl_xor(bmax, 32, 64));
        const float m_new = fmaxf(m_run, bmax);
        float alpha = 1.0f, sum = 0.0f;
        if (m_new == -INFINITY) {
#pragma unroll
            for (int kt = 0; kt < 2; kt++)
#pragma unroll
                for (int r = 0; r < 16; r++) s[kt][r] = 0.0f;
        } else {
            alpha = expf(m_run - m_new);
#pragma unroll
            for (int kt = 0; kt < 2; kt++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const float p = expf(s[kt][r] - m_new);
                    s[kt][r] = p;
                    sum += p;
                }
        }
        sum += __shfl_xor(sum, 32, 64);
        l_run = l_run * alpha + sum;
        m_run = m_new;
        if (alpha != 1.0f) {
#pragma unroll
            for (int i = 0; i < DS / 32; i++)
#pragma unroll
                for (int r = 0; r < 16; r++) o[i][r] *= alpha;
        }
#pragma unroll
        for (int ks = 0; ks < BKV / 16; ks++) {
            half8_t pb;
#pragma unroll
            for (int j = 0; j < 8; j++) pb[j] = _Float16(s[ks >> 1][(ks & 1) * 8 + j]);
            const _Float16* vp = &Vt[(lane & 31) * LDV + ks * 16 + (lane >> 5) * 4];
#pragma unroll
            for (int dt = 0; dt < DS / 32; dt++) {
                const half4_t lo4 = *reinterpret_cast<const half4_t*>(vp + dt * 32 * LDV);
                const half4_t hi4 = *reinterpret_cast<const half4_t*>(vp + dt * 32 * LDV + 8);
                const half8_t a = {lo4[0], lo4[1], lo4[2], lo4[3], hi4[0], hi4[1], hi4[2], hi4[3]};
                o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pb, o[dt], 0, 0, 0);
            }
        }
    }
    if (!qvalid) return;
    const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
    _Float16* op = reinterpret_cast<_Float16*>(Og) + (size_t)(wi.seq_start + qi) * qStride + h * HD + d0 + (lane >> 5) * 4;
#pragma unroll
    for (int dt = 0; dt < DS / 32; dt++)
#pragma unroll
        for (int g = 0; g < 4; g++) {
            half4_t v4;
#pragma unroll
            for (int j = 0; j < 4; j++) v4[j] = _Float16(o[dt][g * 4 + j] * inv);
            *reinterpret_cast<half4_t*>(op + dt * 32 + g * 8) = v4;
        }
}

static size_t attention_lds_bytes(int hd, int ds) {
    return (size_t)(attn::BKV * (hd + 8) + ds * attn::LDV) * sizeof(_Float16);
}

template <int HD, int DS>
static hipError_t attention_configure() {
    return hipFuncSetAttribute(reinterpret_cast<const void*>(&attention_kernel<HD, DS>),
                               hipFuncAttributeMaxDynamicSharedMemorySize, int(attention_lds_bytes(HD, DS)));
}

hipError_t configure_kernels() {
    hipError_t e = attention_configure<128, 128>();
    if (e == hipSuccess) e = attention_configure<256, 256>();
    if (e == hipSuccess) e = attention_configure<512, 256>();
    return e;
}

template <int HD, int DS>
static hipError_t attention_dispatch(hipStream_t s, const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                     uint16_t* o, const AttnWork* work, int n_work, int H, int KV, int hw,
                                     float scale) {
    const size_t lds = attention_lds_bytes(HD, DS);
    const int G = H / KV;
    dim3 grid(n_work, KV, HD / DS);
    attention_kernel<HD, DS><<<grid, 64 * G, lds, s>>>(q, k, v, o, work, H, KV, hw, scale);
    return hipGetLastError();
}

hipError_t launch_attention(hipStream_t s, const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* o,
                            const AttnWork* work, int n_work, int H, int KV, int hd, int half_window, float scale) {
    if (n_work < 0 || H <= 0 || KV <= 0 || H % KV != 0 || H / KV > 4 || half_window < 0) return hipErrorInvalidValue;
    if (n_work == 0) return hipSuccess;
    switch (hd) {
    case 128: return attention_dispatch<128, 128>(s, q, k, v, o, work, n_work, H, KV, half_window, scale);
    case 256: return attention_dispatch<256, 256>(s, q, k, v, o, work, n_work, H, KV, half_window, scale);
    case 512: return attention_dispatch<512, 256>(s, q, k, v, o, work, n_work, H, KV, half_window, scale);
    default: return hipErrorInvalidValue;
    }
}

// ============================================================================ mean pool
//
// One workgroup per sequence; each thread sums its columns over the sequence's rows in order
// (reference Shaders/Elementwise.metal:243-256; Model/CPUReference.swift:277-282).
__global__ __launch_bounds__(256) void mean_pool_kernel(const float* __restrict__ x, const SeqRange* __restrict__ seqs,
                                                        int width, float* __restrict__ pooled) {
    const SeqRange sq = seqs[blockIdx.x];
    for (int c = threadIdx.x; c < width; c += blockDim.x) {
        float acc = 0.0f;
        for (uint32_t r = 0; r < sq.length; r++) acc += x[(size_t)(sq.start + r) * width + c];
        pooled[(size_t)blockIdx.x * width + c] = sq.length ? acc / float(sq.length) : 0.0f;
    }
}

hipError_t launch_mean_pool(hipStream_t s, const float* x, const SeqRange* seqs, int n_seqs, int width, float* pooled) {
    if (n_seqs < 0 || width <= 0) return hipErrorInvalidValue;
    if (n_seqs == 0) return hipSuccess;
    mean_pool_kernel<<<n_seqs, 256, 0, s>>>(x, seqs, width, pooled);
    return hipGetLastError();
}

// ============================================================================ conversions

__global__ void f32_to_f16_kernel(const float* __restrict__ a, uint16_t* __restrict__ b, size_t n) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) b[i] = f2h(a[i]);
}
__global__ void f16_to_f32_kernel(const uint16_t* __restrict__ a, float* __restrict__ b, size_t n) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) b[i] = h2f(a[i]);
}

hipError_t launch_f32_to_f16(hipStream_t s, const float* src, uint16_t* dst, size_t n) {
    if (n == 0) return hipSuccess;
    const size_t blocks = (n + 255) / 256;
    f32_to_f16_kernel<<<dim3(unsigned(blocks < 65536 ? blocks : 65536)), 256, 0, s>>>(src, dst, n);
    return hipGetLastError();
}
hipError_t launch_f16_to_f32(hipStream_t s, const uint16_t* src, float* dst, size_t n) {
    if (n == 0) return hipSuccess;
    const size_t blocks = (n + 255) / 256;
    f16_to_f32_kernel<<<dim3(unsigned(blocks < 65536 ? blocks : 65536)), 256, 0, s>>>(src, dst, n);
    return hipGetLastError();
}

}  // namespace ge
