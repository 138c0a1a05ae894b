// Row-wise kernels: embedding gather + norm, fused residual norms, QK norm + RoPE, mean pool,
// fp16/fp32 conversions. One wave per row with 64-lane reductions; coalesced HBM access.
#include "common.hpp"
#include "kernels.hpp"

namespace ge {

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
    case 1: launch_kernel(embed_norm_kernel<1>, blocks, 256, 0, s, table.q, table.s, tokens, T, d, scale, norm_w, eps, x, h); break;
    case 2: launch_kernel(embed_norm_kernel<2>, blocks, 256, 0, s, table.q, table.s, tokens, T, d, scale, norm_w, eps, x, h); break;
    case 3: launch_kernel(embed_norm_kernel<3>, blocks, 256, 0, s, table.q, table.s, tokens, T, d, scale, norm_w, eps, x, h); break;
    default: launch_kernel(embed_norm_kernel<4>, blocks, 256, 0, s, table.q, table.s, tokens, T, d, scale, norm_w, eps, x, h); break;
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
    case 1: launch_kernel(residual_norm_kernel<1>, blocks, 256, 0, s, x, t, w, out_scale, next_w, eps, T, d, h); break;
    case 2: launch_kernel(residual_norm_kernel<2>, blocks, 256, 0, s, x, t, w, out_scale, next_w, eps, T, d, h); break;
    case 3: launch_kernel(residual_norm_kernel<3>, blocks, 256, 0, s, x, t, w, out_scale, next_w, eps, T, d, h); break;
    default: launch_kernel(residual_norm_kernel<4>, blocks, 256, 0, s, x, t, w, out_scale, next_w, eps, T, d, h); break;
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
    case 128: launch_kernel(qk_norm_rope_kernel<128>, blocks, 256, 0, s, qkv, T, H, KV, q_norm, k_norm, eps, positions, rope_table, q, k, v); break;
    case 256: launch_kernel(qk_norm_rope_kernel<256>, blocks, 256, 0, s, qkv, T, H, KV, q_norm, k_norm, eps, positions, rope_table, q, k, v); break;
    case 512: launch_kernel(qk_norm_rope_kernel<512>, blocks, 256, 0, s, qkv, T, H, KV, q_norm, k_norm, eps, positions, rope_table, q, k, v); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ============================================================================ mean pool
//
// pooled[s] = mean over the sequence's rows (reference Shaders/Elementwise.metal:243-256;
// Model/CPUReference.swift:277-282). Workgroup (64-column chunk, sequence): 4 row slices of 64
// threads each sum every fourth row, four loads in flight per thread, then the four partial sums
// combine in a fixed order, so the result does not depend on scheduling.
__global__ __launch_bounds__(256) void mean_pool_kernel(const float* __restrict__ x, const SeqRange* __restrict__ seqs,
                                                        int width, float* __restrict__ pooled) {
    __shared__ float part[4][64];
    const SeqRange sq = seqs[blockIdx.y];
    const int c = blockIdx.x * 64 + (threadIdx.x & 63), slice = threadIdx.x >> 6;
    float acc = 0.0f;
    if (c < width) {
        const float* p = x + (size_t)sq.start * width + c;
        const int n = int(sq.length);
        int r = slice;
        for (; r + 12 < n; r += 16) {
            const float a = p[(size_t)r * width], b = p[(size_t)(r + 4) * width];
            const float e = p[(size_t)(r + 8) * width], f = p[(size_t)(r + 12) * width];
            acc += a;
            acc += b;
            acc += e;
            acc += f;
        }
        for (; r < n; r += 4) acc += p[(size_t)r * width];
    }
    part[slice][threadIdx.x & 63] = acc;
    __syncthreads();
    if (slice == 0 && c < width) {
        const int i = threadIdx.x;
        const float sum = (part[0][i] + part[1][i]) + (part[2][i] + part[3][i]);
        pooled[(size_t)blockIdx.y * width + c] = sq.length ? sum / float(sq.length) : 0.0f;
    }
}

hipError_t launch_mean_pool(hipStream_t s, const float* x, const SeqRange* seqs, int n_seqs, int width, float* pooled) {
    if (n_seqs < 0 || width <= 0) return hipErrorInvalidValue;
    if (n_seqs == 0) return hipSuccess;
    launch_kernel(mean_pool_kernel, dim3((width + 63) / 64, n_seqs), 256, 0, s, x, seqs, width, pooled);
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
    launch_kernel(f32_to_f16_kernel, dim3(unsigned(blocks < 65536 ? blocks : 65536)), 256, 0, s, src, dst, n);
    return hipGetLastError();
}
hipError_t launch_f16_to_f32(hipStream_t s, const uint16_t* src, float* dst, size_t n) {
    if (n == 0) return hipSuccess;
    const size_t blocks = (n + 255) / 256;
    launch_kernel(f16_to_f32_kernel, dim3(unsigned(blocks < 65536 ? blocks : 65536)), 256, 0, s, src, dst, n);
    return hipGetLastError();
}


}  // namespace ge
