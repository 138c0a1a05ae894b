// Row-wise kernels: embedding gather + norm, fused residual norms, QK norm + RoPE, mean pool,
// fp16/fp32 conversions. One wave per row with 64-lane reductions; coalesced HBM access.
#include "common.hpp"
#include "kernels.hpp"

namespace ge {

// ============================================================================ embedding + norm
//
// One wave per token row; each lane owns 4 consecutive elements of every 256-wide chunk.
// x = dequant(table[id]) * scale, then h = rmsnorm(x) * w (reference Shaders/Elementwise.metal:8-35
// and :38-75; Model/CPUReference.swift:190-204, :217). An id -(r + 1) is row r of `vectors`
// ([rows][d] fp32), entered unscaled (Elementwise.metal:25-29); the host has checked r.
template <int CH>
__global__ __launch_bounds__(256) void embed_norm_kernel(const int8_t* __restrict__ tq, const uint16_t* __restrict__ ts,
                                                         const int32_t* __restrict__ tokens, int T, int d, float scale,
                                                         const float* __restrict__ vectors, const float* __restrict__ w,
                                                         float eps, float* __restrict__ x, uint16_t* __restrict__ h) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= T) return;
    const int id = tokens[row];
    float v[CH][4];
    float ss = 0.0f;
    // Every chunk's loads are issued before any is used (a lane past d reads chunk d - 4 and
    // discards it), so the row's loads are in flight together instead of one after another.
    if (id < 0) {
        const float* src = vectors + (size_t)(-(id + 1)) * d;
        float4 f[CH];
#pragma unroll
        for (int c = 0; c < CH; c++) f[c] = *reinterpret_cast<const float4*>(src + min(c * 256 + lane * 4, d - 4));
#pragma unroll
        for (int c = 0; c < CH; c++) {
            const int e = c * 256 + lane * 4;
            if (e < d) {
                v[c][0] = f[c].x, v[c][1] = f[c].y, v[c][2] = f[c].z, v[c][3] = f[c].w;
#pragma unroll
                for (int j = 0; j < 4; j++) ss += v[c][j] * v[c][j];
                *reinterpret_cast<float4*>(x + (size_t)row * d + e) = f[c];
            }
        }
    } else {
        const int8_t* q = tq + (size_t)id * d;
        const uint16_t* sc = ts + (size_t)id * (d / 32);
        uint32_t packed[CH];
        uint16_t sbits[CH];
#pragma unroll
        for (int c = 0; c < CH; c++) {
            const int ec = min(c * 256 + lane * 4, d - 4);
            packed[c] = *reinterpret_cast<const uint32_t*>(q + ec);
            sbits[c] = sc[ec / 32];
        }
#pragma unroll
        for (int c = 0; c < CH; c++) {
            const int e = c * 256 + lane * 4;
            if (e < d) {
                const float ds = h2f(sbits[c]);
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    v[c][j] = ds * float(int8_t((packed[c] >> (8 * j)) & 0xff)) * scale;
                    ss += v[c][j] * v[c][j];
                }
                *reinterpret_cast<float4*>(x + (size_t)row * d + e) = make_float4(v[c][0], v[c][1], v[c][2], v[c][3]);
            }
        }
    }
    float4 wa[CH];
#pragma unroll
    for (int c = 0; c < CH; c++) wa[c] = *reinterpret_cast<const float4*>(w + min(c * 256 + lane * 4, d - 4));
    ss = wave_sum(ss);
    const float inv = 1.0f / sqrtf(ss / float(d) + eps);
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int e = c * 256 + lane * 4;
        if (e < d) {
            const float wv[4] = {wa[c].x, wa[c].y, wa[c].z, wa[c].w};
            half4_t o;
#pragma unroll
            for (int j = 0; j < 4; j++) o[j] = _Float16(v[c][j] * inv * wv[j]);
            *reinterpret_cast<half4_t*>(h + (size_t)row * d + e) = o;
        }
    }
}

hipError_t launch_embed_norm(hipStream_t s, const Q8Dev& table, const int32_t* tokens, int T, float scale,
                             const float* vectors, const float* norm_w, float eps, float* x, uint16_t* h) {
    const int d = table.cols;
    if (T < 0 || d <= 0 || d % 32 != 0 || d > 1024) return hipErrorInvalidValue;
    if (T == 0) return hipSuccess;
    const int blocks = (T + 3) / 4, CH = (d + 255) / 256;
    switch (CH) {
    case 1: launch_kernel(embed_norm_kernel<1>, blocks, 256, 0, s, table.q, table.s, tokens, T, d, scale, vectors, norm_w, eps, x, h); break;
    case 2: launch_kernel(embed_norm_kernel<2>, blocks, 256, 0, s, table.q, table.s, tokens, T, d, scale, vectors, norm_w, eps, x, h); break;
    case 3: launch_kernel(embed_norm_kernel<3>, blocks, 256, 0, s, table.q, table.s, tokens, T, d, scale, vectors, norm_w, eps, x, h); break;
    default: launch_kernel(embed_norm_kernel<4>, blocks, 256, 0, s, table.q, table.s, tokens, T, d, scale, vectors, norm_w, eps, x, h); break;
    }
    return hipGetLastError();
}

// ============================================================================ residual + norms
//
// x = (x + rmsnorm(t) * w) * out_scale, then optionally h = rmsnorm(x) * next_w in fp16: the
// post-attention / post-FFN norm, the residual add and the next block's pre-norm in one pass
// (reference Shaders/Elementwise.metal:260-354; Model/CPUReference.swift:240-245, :254-257, :269).
//
// Modes (the layer's two residual steps without storing x in between):
//   kResStore  x = (x + rmsnorm(t) w) s stored; h = rmsnorm(x) next_w when next_w is given.
//   kResNoX    the same h; x is left as it was. The caller later runs kResTwo on the same x and t.
//   kResTwo    x1 = (x + rmsnorm(t) w) s as above, then x = (x1 + rmsnorm(t2) w2) s2 stored and
//              h = rmsnorm(x) next_w: the attention residual (t the o projection) recomputed
//              beside the FFN residual (t2 the down projection). x1 is formed by residual_add in
//              every mode, so it is the same number whether it was stored or recomputed.
// The sums of squares are fused multiply-adds in lane order, then a wave butterfly.
enum ResMode { kResStore = 0, kResNoX = 1, kResTwo = 2 };

__device__ __forceinline__ float residual_add(float x, float t, float inv, float w, float s) {
    return __builtin_fmaf(t * inv, w, x) * s;
}

template <int CH, bool F32OUT, int MODE>
__global__ __launch_bounds__(256) void residual_norm_kernel(float* __restrict__ x, const uint16_t* __restrict__ t16,
                                                            float t_eps, const float* __restrict__ w, float out_scale,
                                                            const uint16_t* __restrict__ t2_16, float t2_eps,
                                                            const float* __restrict__ w2, float out_scale2,
                                                            const float* __restrict__ next_w, float eps, int T, int d,
                                                            uint16_t* __restrict__ h, float* __restrict__ h32) {
#pragma clang fp contract(off)
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= T) return;
    // t (and t2) arrive as fp16 t * c (c a power of two) with t_eps = eps * c^2: the RMSNorm of
    // the stored values with t_eps is the RMSNorm of t.
    float tv[CH][4], t2v[CH][4], xv[CH][4];
    float ss = 0.0f, ss_t2 = 0.0f;
    // Every input's chunks are loaded before any is used (a lane past d reads chunk d - 4 and
    // discards it): the row's loads are in flight together.
    half4_t ta[CH], t2a[CH];
    float4 xa4[CH], wa[CH], w2a[CH], nwa[CH];
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int ec = min(c * 256 + lane * 4, d - 4);
        ta[c] = *reinterpret_cast<const half4_t*>(t16 + (size_t)row * d + ec);
        xa4[c] = *reinterpret_cast<const float4*>(x + (size_t)row * d + ec);
        wa[c] = *reinterpret_cast<const float4*>(w + ec);
        if constexpr (MODE == kResTwo) {
            t2a[c] = *reinterpret_cast<const half4_t*>(t2_16 + (size_t)row * d + ec);
            w2a[c] = *reinterpret_cast<const float4*>(w2 + ec);
        }
        if (next_w) nwa[c] = *reinterpret_cast<const float4*>(next_w + ec);
    }
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int e = c * 256 + lane * 4;
        if (e < d) {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                tv[c][j] = float(ta[c][j]);
                ss = __builtin_fmaf(tv[c][j], tv[c][j], ss);
                if constexpr (MODE == kResTwo) {
                    t2v[c][j] = float(t2a[c][j]);
                    ss_t2 = __builtin_fmaf(t2v[c][j], t2v[c][j], ss_t2);
                }
            }
        }
    }
    ss = wave_sum(ss);
    if constexpr (MODE == kResTwo) ss_t2 = wave_sum(ss_t2);
    const float inv = 1.0f / sqrtf(ss / float(d) + t_eps);
    const float inv_t2 = MODE == kResTwo ? 1.0f / sqrtf(ss_t2 / float(d) + t2_eps) : 0.0f;
    float ss2 = 0.0f;
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int e = c * 256 + lane * 4;
        if (e < d) {
            const float xa[4] = {xa4[c].x, xa4[c].y, xa4[c].z, xa4[c].w};
            const float wv[4] = {wa[c].x, wa[c].y, wa[c].z, wa[c].w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                xv[c][j] = residual_add(xa[j], tv[c][j], inv, wv[j], out_scale);
                if constexpr (MODE == kResTwo) {
                    const float w2v[4] = {w2a[c].x, w2a[c].y, w2a[c].z, w2a[c].w};
                    xv[c][j] = residual_add(xv[c][j], t2v[c][j], inv_t2, w2v[j], out_scale2);
                }
                ss2 = __builtin_fmaf(xv[c][j], xv[c][j], ss2);
            }
            if constexpr (MODE != kResNoX)
                *reinterpret_cast<float4*>(x + (size_t)row * d + e) = make_float4(xv[c][0], xv[c][1], xv[c][2], xv[c][3]);
        }
    }
    if (!next_w) return;
    ss2 = wave_sum(ss2);
    const float inv2 = 1.0f / sqrtf(ss2 / float(d) + eps);
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int e = c * 256 + lane * 4;
        if (e < d) {
            const float nw[4] = {nwa[c].x, nwa[c].y, nwa[c].z, nwa[c].w};
            if constexpr (F32OUT) {
                *reinterpret_cast<float4*>(h32 + (size_t)row * d + e) =
                    make_float4(xv[c][0] * inv2 * nw[0], xv[c][1] * inv2 * nw[1], xv[c][2] * inv2 * nw[2], xv[c][3] * inv2 * nw[3]);
            } else {
                half4_t o;
#pragma unroll
                for (int j = 0; j < 4; j++) o[j] = _Float16(xv[c][j] * inv2 * nw[j]);
                *reinterpret_cast<half4_t*>(h + (size_t)row * d + e) = o;
            }
        }
    }
}

namespace {
template <int MODE>
hipError_t residual_norm_dispatch(hipStream_t s, float* x, const uint16_t* t16, float t_eps, const float* w,
                                  float out_scale, const uint16_t* t2_16, float t2_eps, const float* w2, float out_scale2,
                                  const float* next_w, float eps, int T, int d, uint16_t* h, float* h32) {
    if (T < 0 || d <= 0 || d % 4 != 0 || d > 1024 || (next_w && !h && !h32) || !t16 || !x || !w) return hipErrorInvalidValue;
    if (T == 0) return hipSuccess;
    const int blocks = (T + 3) / 4, CH = (d + 255) / 256;
    // the fp32 output is a separate instantiation, so the fp16 one compiles as on its own
#define RN_LAUNCH(C)                                                                                              \
    (h32 ? launch_kernel(residual_norm_kernel<C, true, MODE>, blocks, 256, 0, s, x, t16, t_eps, w, out_scale, t2_16, \
                         t2_eps, w2, out_scale2, next_w, eps, T, d, h, h32)                                       \
         : launch_kernel(residual_norm_kernel<C, false, MODE>, blocks, 256, 0, s, x, t16, t_eps, w, out_scale, t2_16, \
                         t2_eps, w2, out_scale2, next_w, eps, T, d, h, h32))
    switch (CH) {
    case 1: RN_LAUNCH(1); break;
    case 2: RN_LAUNCH(2); break;
    case 3: RN_LAUNCH(3); break;
    default: RN_LAUNCH(4); break;
    }
#undef RN_LAUNCH
    return hipGetLastError();
}
}  // namespace

hipError_t launch_residual_norm(hipStream_t s, float* x, const uint16_t* t16, float t_eps, const float* w,
                                float out_scale, const float* next_w, float eps, int T, int d, uint16_t* h, float* h32) {
    return residual_norm_dispatch<kResStore>(s, x, t16, t_eps, w, out_scale, nullptr, 0.0f, nullptr, 0.0f, next_w, eps,
                                             T, d, h, h32);
}

hipError_t launch_residual_norm_h(hipStream_t s, const float* x, const uint16_t* t16, float t_eps, const float* w,
                                  float out_scale, const float* next_w, float eps, int T, int d, uint16_t* h) {
    if (!next_w || !h) return hipErrorInvalidValue;
    return residual_norm_dispatch<kResNoX>(s, const_cast<float*>(x), t16, t_eps, w, out_scale, nullptr, 0.0f, nullptr,
                                           0.0f, next_w, eps, T, d, h, nullptr);
}

hipError_t launch_residual_norm_two(hipStream_t s, float* x, const uint16_t* t16, float t_eps, const float* w,
                                    float out_scale, const uint16_t* t2_16, float t2_eps, const float* w2,
                                    float out_scale2, const float* next_w, float eps, int T, int d, uint16_t* h,
                                    float* h32) {
    if (!t2_16 || !w2) return hipErrorInvalidValue;
    return residual_norm_dispatch<kResTwo>(s, x, t16, t_eps, w, out_scale, t2_16, t2_eps, w2, out_scale2, next_w, eps, T,
                                           d, h, h32);
}

// ============================================================================ split-precision norm
//
// h3 = [hi | lo | hi] per row, with y = rmsnorm(x) * w in fp32 (the value the other norm kernels
// round to fp16, with the same lane order of the sum of squares), hi = fp16(y) and
// lo = fp16(y - hi). Against a weight stored as [W_hi | W_hi | W_lo] over 3 d columns the GEMM
// sums hi W_hi + lo W_hi + hi W_lo, which is y W to about 2^-20 relative instead of the 2^-11 of
// fp16 operands (the dropped lo W_lo term is below 2^-22).
template <int CH>
__global__ __launch_bounds__(256) void norm_split_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                         float eps, int T, int d, uint16_t* __restrict__ h3) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= T) return;
    float xv[CH][4];
    float ss = 0.0f;
    float4 xa4[CH], wa[CH];  // all chunks in flight together (a lane past d reads chunk d - 4, unused)
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int ec = min(c * 256 + lane * 4, d - 4);
        xa4[c] = *reinterpret_cast<const float4*>(x + (size_t)row * d + ec);
        wa[c] = *reinterpret_cast<const float4*>(w + ec);
    }
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int e = c * 256 + lane * 4;
        if (e < d) {
            xv[c][0] = xa4[c].x, xv[c][1] = xa4[c].y, xv[c][2] = xa4[c].z, xv[c][3] = xa4[c].w;
#pragma unroll
            for (int j = 0; j < 4; j++) ss += xv[c][j] * xv[c][j];
        }
    }
    ss = wave_sum(ss);
    const float inv = 1.0f / sqrtf(ss / float(d) + eps);
    uint16_t* out = h3 + (size_t)row * 3 * d;
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int e = c * 256 + lane * 4;
        if (e < d) {
            half4_t hi, lo;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float y = xv[c][j] * inv * wa[c][j];
                hi[j] = _Float16(y);
                lo[j] = _Float16(y - float(hi[j]));
            }
            *reinterpret_cast<half4_t*>(out + e) = hi;
            *reinterpret_cast<half4_t*>(out + d + e) = lo;
            *reinterpret_cast<half4_t*>(out + 2 * d + e) = hi;
        }
    }
}

hipError_t launch_norm_split(hipStream_t s, const float* x, const float* w, float eps, int T, int d, uint16_t* h3) {
    if (T < 0 || d <= 0 || d % 4 != 0 || d > 1024 || !x || !w || !h3) return hipErrorInvalidValue;
    if (T == 0) return hipSuccess;
    const int blocks = (T + 3) / 4, CH = (d + 255) / 256;
    switch (CH) {
    case 1: launch_kernel(norm_split_kernel<1>, blocks, 256, 0, s, x, w, eps, T, d, h3); break;
    case 2: launch_kernel(norm_split_kernel<2>, blocks, 256, 0, s, x, w, eps, T, d, h3); break;
    case 3: launch_kernel(norm_split_kernel<3>, blocks, 256, 0, s, x, w, eps, T, d, h3); break;
    default: launch_kernel(norm_split_kernel<4>, blocks, 256, 0, s, x, w, eps, T, d, h3); break;
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
                                                           uint16_t* __restrict__ k, uint16_t* __restrict__ v,
                                                           uint16_t* __restrict__ q_lo, uint16_t* __restrict__ k_lo) {
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
    uint16_t* dlo = nullptr;  // the split pair's low halves (q_lo / k_lo set)
    const float* w = nullptr;
    bool rope = true;
    if (slot < H) {
        dst = q + ((size_t)t * H + slot) * HD;
        if (q_lo) dlo = q_lo + ((size_t)t * H + slot) * HD;
        w = q_norm;
    } else if (slot < H + KV) {
        dst = k + ((size_t)t * KV + (slot - H)) * HD;
        if (k_lo) dlo = k_lo + ((size_t)t * KV + (slot - H)) * HD;
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
        if (dlo) {
            dlo[i] = f2h(a - h2f(dst[i]));
            dlo[HALF + i] = f2h(b - h2f(dst[HALF + i]));
        }
    }
}

hipError_t launch_qk_norm_rope(hipStream_t s, const float* qkv, int T, int H, int KV, int hd, const float* q_norm,
                               const float* k_norm, float eps, const int32_t* positions, const float* rope_table,
                               uint16_t* q, uint16_t* k, uint16_t* v, uint16_t* q_lo, uint16_t* k_lo) {
    if (T < 0 || H <= 0 || KV <= 0 || (q_lo == nullptr) != (k_lo == nullptr)) return hipErrorInvalidValue;
    if (T == 0) return hipSuccess;
    const long items = (long)T * (H + 2 * KV);
    const int blocks = int((items + 3) / 4);
    switch (hd) {
    case 128: launch_kernel(qk_norm_rope_kernel<128>, blocks, 256, 0, s, qkv, T, H, KV, q_norm, k_norm, eps, positions, rope_table, q, k, v, q_lo, k_lo); break;
    case 256: launch_kernel(qk_norm_rope_kernel<256>, blocks, 256, 0, s, qkv, T, H, KV, q_norm, k_norm, eps, positions, rope_table, q, k, v, q_lo, k_lo); break;
    case 512: launch_kernel(qk_norm_rope_kernel<512>, blocks, 256, 0, s, qkv, T, H, KV, q_norm, k_norm, eps, positions, rope_table, q, k, v, q_lo, k_lo); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ============================================================================ QK norm + RoPE, V transposed
//
// The arithmetic of qk_norm_rope_kernel on the QKV projection stored as scaled fp16 (see
// launch_qkv_norm_rope_vt), fused with the V transpose the LDS-copy attention reads. A workgroup
// of 16 waves takes 64 consecutive tokens, 4 per wave; per token a wave loads all S = H + 2 KV
// head slots before reducing any of them, and the S sums of squares go through the butterfly
// together. Each lane owns C = hd / 128 elements of the first half of every head and their NeoX
// partners. Normalised V
// rows are written row-major and also staged in LDS as [KV * hd][64 tokens], then written to
// V^T one d row (64 tokens, 128 contiguous bytes within a sequence) per wave instruction.
template <int HD, int S>
__global__ __launch_bounds__(1024) void qkv_norm_rope_vt_kernel(const uint16_t* __restrict__ qkv16, int T, int H, int KV,
                                                               const float* __restrict__ q_norm,
                                                               const float* __restrict__ k_norm, float eps,
                                                               const int32_t* __restrict__ positions,
                                                               const float* __restrict__ table,
                                                               uint16_t* __restrict__ q, uint16_t* __restrict__ k,
                                                               uint16_t* __restrict__ v, const int32_t* __restrict__ vcol,
                                                               int vt_cols, uint16_t* __restrict__ vt) {
    constexpr int C = HD / 128, HALF = HD / 2, TS = 66;  // tile row stride in halves
    extern __shared__ __attribute__((aligned(16))) uint16_t vtile[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int t0 = blockIdx.x * 64;
    float wq[2 * C], wk[2 * C];
#pragma unroll
    for (int j = 0; j < C; j++) {
        wq[j] = q_norm[lane * C + j];
        wq[C + j] = q_norm[HALF + lane * C + j];
        wk[j] = k_norm[lane * C + j];
        wk[C + j] = k_norm[HALF + lane * C + j];
    }
    for (int i = 0; i < 4; i++) {
        const int tok = wave * 4 + i, t = t0 + tok;
        if (t >= T) break;
        // The projection arrives as fp16 qkv * c (c a power of two, eps already scaled by c^2).
        const uint16_t* row = qkv16 + (size_t)t * S * HD + lane * C;
        float lo[S][C], hi[S][C], ss[S];
#pragma unroll
        for (int sl = 0; sl < S; sl++)
#pragma unroll
            for (int j = 0; j < C; j++) {
                lo[sl][j] = h2f(row[sl * HD + j]);
                hi[sl][j] = h2f(row[sl * HD + HALF + j]);
            }
        const float* cs = table + (size_t)positions[t] * HALF * 2 + lane * C * 2;
        float cr[2 * C];
#pragma unroll
        for (int j = 0; j < 2 * C; j++) cr[j] = cs[j];
#pragma unroll
        for (int sl = 0; sl < S; sl++) {
            ss[sl] = 0.0f;
#pragma unroll
            for (int j = 0; j < C; j++) ss[sl] += lo[sl][j] * lo[sl][j] + hi[sl][j] * hi[sl][j];
        }
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1)
#pragma unroll
            for (int sl = 0; sl < S; sl++) ss[sl] += __shfl_xor(ss[sl], m, 64);
#pragma unroll
        for (int sl = 0; sl < S; sl++) {
            const float inv = 1.0f / sqrtf(ss[sl] / float(HD) + eps);
            const bool isq = sl < H, isk = !isq && sl < H + KV;
            uint16_t* dst = isq ? q + ((size_t)t * H + sl) * HD
                                : (isk ? k + ((size_t)t * KV + (sl - H)) * HD : v + ((size_t)t * KV + (sl - H - KV)) * HD);
            uint16_t olo[C], ohi[C];
#pragma unroll
            for (int j = 0; j < C; j++) {
                float a = lo[sl][j] * inv, b = hi[sl][j] * inv;
                if (isq || isk) {
                    // a blend rather than a select between the two register arrays, which the
                    // compiler would turn into a select of their addresses (scratch memory)
                    const float fq = isq ? 1.0f : 0.0f, fk = 1.0f - fq;
                    a *= wq[j] * fq + wk[j] * fk;
                    b *= wq[C + j] * fq + wk[C + j] * fk;
                    const float c = cr[2 * j], sn = cr[2 * j + 1];
                    const float ra = a * c - b * sn, rb = a * sn + b * c;
                    a = ra;
                    b = rb;
                }
                olo[j] = f2h(a);
                ohi[j] = f2h(b);
            }
#pragma unroll
            for (int j = 0; j < C; j++) {
                dst[lane * C + j] = olo[j];
                dst[HALF + lane * C + j] = ohi[j];
            }
            if (!isq && !isk && vt) {
                const int r0 = (sl - H - KV) * HD;
#pragma unroll
                for (int j = 0; j < C; j++) {
                    vtile[(r0 + lane * C + j) * TS + tok] = olo[j];
                    vtile[(r0 + HALF + lane * C + j) * TS + tok] = ohi[j];
                }
            }
        }
    }
    if (!vt) return;
    __syncthreads();
    if (t0 + lane >= T) return;
    const int col = vcol[t0 + lane];
    for (int r = wave; r < KV * HD; r += 16) vt[(size_t)r * vt_cols + col] = vtile[r * TS + lane];
}

template <int HD, int S>
static hipError_t qkv_norm_rope_vt_launch(hipStream_t s, const uint16_t* qkv, int T, int H, int KV, const float* q_norm,
                                          const float* k_norm, float eps, const int32_t* positions, const float* rope_table,
                                          uint16_t* q, uint16_t* k, uint16_t* v, const int32_t* vcol, int vt_cols,
                                          uint16_t* vt) {
    const uint32_t lds = vt ? uint32_t(KV * HD * 66 * 2) : 0u;
    launch_kernel(qkv_norm_rope_vt_kernel<HD, S>, dim3((T + 63) / 64), dim3(1024), lds, s, qkv, T, H, KV, q_norm, k_norm, eps,
                  positions, rope_table, q, k, v, vcol, vt_cols, vt);
    return hipGetLastError();
}

template <int HD>
static hipError_t qkv_norm_rope_vt_dispatch(hipStream_t s, const uint16_t* qkv, int T, int H, int KV, const float* q_norm,
                                            const float* k_norm, float eps, const int32_t* positions,
                                            const float* rope_table, uint16_t* q, uint16_t* k, uint16_t* v,
                                            const int32_t* vcol, int vt_cols, uint16_t* vt) {
#define QNR_CASE(SL) \
    case SL: return qkv_norm_rope_vt_launch<HD, SL>(s, qkv, T, H, KV, q_norm, k_norm, eps, positions, rope_table, q, k, v, vcol, vt_cols, vt);
    switch (H + 2 * KV) {
        QNR_CASE(3) QNR_CASE(4) QNR_CASE(5) QNR_CASE(6) QNR_CASE(8) QNR_CASE(10)
    default: return hipErrorInvalidValue;
    }
#undef QNR_CASE
}

bool qkv_norm_rope_vt_supported(int hd, int H, int KV) {
    const int sl = H + 2 * KV;
    return (hd == 128 || hd == 256) && (sl == 3 || sl == 4 || sl == 5 || sl == 6 || sl == 8 || sl == 10) &&
           KV * hd * 66 * 2 <= 64 * 1024;
}

hipError_t launch_qkv_norm_rope_vt(hipStream_t s, const uint16_t* qkv, int T, int H, int KV, int hd,
                                   const float* q_norm, const float* k_norm, float eps, const int32_t* positions,
                                   const float* rope_table, uint16_t* q, uint16_t* k, uint16_t* v, const int32_t* vcol,
                                   int vt_cols, uint16_t* vt) {
    if (T < 0 || H <= 0 || KV <= 0 || !qkv_norm_rope_vt_supported(hd, H, KV) || (vt && (!vcol || vt_cols <= 0)))
        return hipErrorInvalidValue;
    if (T == 0) return hipSuccess;
    if (hd == 128)
        return qkv_norm_rope_vt_dispatch<128>(s, qkv, T, H, KV, q_norm, k_norm, eps, positions, rope_table, q, k, v, vcol, vt_cols, vt);
    return qkv_norm_rope_vt_dispatch<256>(s, qkv, T, H, KV, q_norm, k_norm, eps, positions, rope_table, q, k, v, vcol, vt_cols, vt);
}

// ============================================================================ mean pool
//
// pooled[s] = mean over the sequence's rows (reference Shaders/Elementwise.metal:243-256;
// Model/CPUReference.swift:277-282). Workgroup (64-column chunk, sequence) of 4 waves: 16 lanes
// hold a row's 64 columns (4 each, 16-byte loads), 16 row slots; slot j sums rows j, j + 16, ...
// in order, eight rows in flight; the 16 partial sums then combine in a fixed tree order, so the
// result does not depend on scheduling or on the sequence's place in the pack. 64-column chunks
// give a sequence's pool width / 64 workgroups, spread over that many CUs: with 256-column
// chunks of 16 waves, four 8192-token sequences ran on 12 CUs at 1 TB/s.
__global__ __launch_bounds__(256) void mean_pool_kernel(const float* __restrict__ x, const SeqRange* __restrict__ seqs,
                                                        int width, float* __restrict__ pooled) {
    __shared__ float4 part[16][16];
    const SeqRange sq = seqs[blockIdx.y];
    const int l16 = threadIdx.x & 15, slot = threadIdx.x >> 4;
    const int c = blockIdx.x * 64 + l16 * 4;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (c < width) {
        const float* p = x + (size_t)sq.start * width + c;
        const int n = int(sq.length);
        int r = slot;
        for (; r + 112 < n; r += 128) {
            float4 v[8];
#pragma unroll
            for (int u = 0; u < 8; u++) v[u] = *reinterpret_cast<const float4*>(p + (size_t)(r + 16 * u) * width);
#pragma unroll
            for (int u = 0; u < 8; u++) acc.x += v[u].x, acc.y += v[u].y, acc.z += v[u].z, acc.w += v[u].w;
        }
        for (; r < n; r += 16) {
            const float4 a = *reinterpret_cast<const float4*>(p + (size_t)r * width);
            acc.x += a.x, acc.y += a.y, acc.z += a.z, acc.w += a.w;
        }
    }
    part[slot][l16] = acc;
    __syncthreads();
    if (slot == 0 && c < width) {
        float4 t[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float4 u = part[2 * i][l16], v = part[2 * i + 1][l16];
            t[i] = make_float4(u.x + v.x, u.y + v.y, u.z + v.z, u.w + v.w);
        }
#pragma unroll
        for (int i = 0; i < 4; i++) t[i] = make_float4(t[2 * i].x + t[2 * i + 1].x, t[2 * i].y + t[2 * i + 1].y,
                                                     t[2 * i].z + t[2 * i + 1].z, t[2 * i].w + t[2 * i + 1].w);
#pragma unroll
        for (int i = 0; i < 2; i++) t[i] = make_float4(t[2 * i].x + t[2 * i + 1].x, t[2 * i].y + t[2 * i + 1].y,
                                                     t[2 * i].z + t[2 * i + 1].z, t[2 * i].w + t[2 * i + 1].w);
        const float4 sum = make_float4(t[0].x + t[1].x, t[0].y + t[1].y, t[0].z + t[1].z, t[0].w + t[1].w);
        const float4 m = sq.length ? make_float4(sum.x / float(sq.length), sum.y / float(sq.length), sum.z / float(sq.length),
                                                 sum.w / float(sq.length))
                                   : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        *reinterpret_cast<float4*>(pooled + (size_t)blockIdx.y * width + c) = m;
    }
}

hipError_t launch_mean_pool(hipStream_t s, const float* x, const SeqRange* seqs, int n_seqs, int width, float* pooled) {
    if (n_seqs < 0 || width <= 0 || width % 4) return hipErrorInvalidValue;
    if (n_seqs == 0) return hipSuccess;
    launch_kernel(mean_pool_kernel, dim3((width + 63) / 64, n_seqs), 256, 0, s, x, seqs, width, pooled);
    return hipGetLastError();
}

// ============================================================================ output projection
//
// The output projection applied to pooled rows: pooling is a mean and the projection is linear,
// so projecting the sequence's mean normed row equals the reference's mean of projected tokens
// (Model/CPUReference.swift:274-282) up to fp32 rounding, on one row per sequence instead of one
// per token, and in fp32 throughout: the Q8_0 weights as d * q (exact in fp32) and the normed rows
// as the final norm computed them, where the token-wise GEMM rounds both to fp16.
// One wave per output column n: lane l holds columns c * 256 + 4 l .. + 3 of the weight row
// (dequantised once), then walks the workgroup's rows; each row's dot product is summed per lane
// over its chunks in order, then over the lanes by a fixed butterfly, so a row's output depends
// on that row alone.
constexpr int kProjRows = 64;   // rows (sequences) per workgroup row of the grid
constexpr int kProjUnroll = 8;  // rows whose loads are in flight together

template <int CH>
__global__ __launch_bounds__(256) void pooled_projection_kernel(const float* __restrict__ in, int n_rows, int width,
                                                                const int8_t* __restrict__ q,
                                                                const uint16_t* __restrict__ sc, int n_out,
                                                                float* __restrict__ out) {
    const int n = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (n >= n_out) return;
    const int r0 = blockIdx.y * kProjRows, r1 = min(r0 + kProjRows, n_rows);
    float wv[CH][4];
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int ec = min(c * 256 + lane * 4, width - 4);
        const char4 q4 = *reinterpret_cast<const char4*>(q + (size_t)n * width + ec);
        const float dsc = h2f(sc[(size_t)n * (width / 32) + ec / 32]);
        wv[c][0] = dsc * float(q4.x), wv[c][1] = dsc * float(q4.y), wv[c][2] = dsc * float(q4.z), wv[c][3] = dsc * float(q4.w);
    }
    // kProjUnroll rows at a time, all their loads issued before any product (rows past r1 re-read
    // row r1 - 1, unused), so the loop waits for one batch of loads rather than for each row's
    for (int r = r0; r < r1; r += kProjUnroll) {
        float4 xa[kProjUnroll][CH];
#pragma unroll
        for (int u = 0; u < kProjUnroll; u++)
#pragma unroll
            for (int c = 0; c < CH; c++)
                xa[u][c] = *reinterpret_cast<const float4*>(in + (size_t)min(r + u, r1 - 1) * width +
                                                            min(c * 256 + lane * 4, width - 4));
#pragma unroll
        for (int u = 0; u < kProjUnroll; u++) {
            float acc = 0.0f;
#pragma unroll
            for (int c = 0; c < CH; c++)
                if (c * 256 + lane * 4 < width) {
                    acc = __builtin_fmaf(xa[u][c].x, wv[c][0], acc);
                    acc = __builtin_fmaf(xa[u][c].y, wv[c][1], acc);
                    acc = __builtin_fmaf(xa[u][c].z, wv[c][2], acc);
                    acc = __builtin_fmaf(xa[u][c].w, wv[c][3], acc);
                }
            acc = wave_sum(acc);
            if (lane == 0 && r + u < r1) out[(size_t)(r + u) * n_out + n] = acc;
        }
    }
}

hipError_t launch_pooled_projection(hipStream_t s, const float* in, int n_rows, int width, const Q8Dev& w, float* out) {
    if (n_rows < 0 || width <= 0 || width % 32 || width > 1024 || w.cols != width || w.rows <= 0 || !w.q || !w.s ||
        !in || !out)
        return hipErrorInvalidValue;
    if (n_rows == 0) return hipSuccess;
    const dim3 grid((w.rows + 3) / 4, (n_rows + kProjRows - 1) / kProjRows);
    switch ((width + 255) / 256) {
    case 1: launch_kernel(pooled_projection_kernel<1>, grid, 256, 0, s, in, n_rows, width, w.q, w.s, w.rows, out); break;
    case 2: launch_kernel(pooled_projection_kernel<2>, grid, 256, 0, s, in, n_rows, width, w.q, w.s, w.rows, out); break;
    case 3: launch_kernel(pooled_projection_kernel<3>, grid, 256, 0, s, in, n_rows, width, w.q, w.s, w.rows, out); break;
    default: launch_kernel(pooled_projection_kernel<4>, grid, 256, 0, s, in, n_rows, width, w.q, w.s, w.rows, out); break;
    }
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
