// Row kernels of the image tower (a pre-LayerNorm ViT over 16x16 patches,
// 3x3 pooling and a projection into the text space). One wave per row; lane l owns elements
// c * 256 + 4 l .. + 3 of every 256-wide chunk c. The GEMMs (patch embedding, QKV, output, MLP,
// projection) and the attention are the text path's kernels. Counterparts in the reference's
// gemma4v tower: position rows (Shaders/Elementwise.metal:207-222, Metal/VisionTower.swift:153-154),
// fused residual norms (Shaders/Elementwise.metal:300-350) and the pooling (:223-242,
// Model/CPUVisionReference.swift:67-83).
#include "common.hpp"
#include "kernels.hpp"

namespace ge {

__device__ __forceinline__ bool vit_valid(int c, int lane, int d) {
    return c * 256 + lane * 4 < d;
}

// LayerNorm statistics of a row held by a wave: mean, then the mean of squared deviations
// (two passes over the registers), rstd = 1 / sqrt(var + eps).
template <int CH>
__device__ __forceinline__ void vit_ln_stats(const float (&v)[CH][4], int d, int lane, float eps, float& mean,
                                             float& rstd) {
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < CH; c++)
        if (vit_valid(c, lane, d))
#pragma unroll
            for (int j = 0; j < 4; j++) s += v[c][j];
    mean = wave_sum(s) / float(d);
    float ss = 0.0f;
#pragma unroll
    for (int c = 0; c < CH; c++)
        if (vit_valid(c, lane, d))
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float t = v[c][j] - mean;
                ss += t * t;
            }
    rstd = 1.0f / sqrtf(wave_sum(ss) / float(d) + eps);
}

// The lane's chunks of a row vector (a lane past d reads the last chunk, unused): loaded before
// anything needs them, so a row's loads are in flight together rather than one after another.
template <int CH>
__device__ __forceinline__ void vit_load_chunks(const float* __restrict__ p, int d, int lane, float4 (&out)[CH]) {
#pragma unroll
    for (int c = 0; c < CH; c++) out[c] = *reinterpret_cast<const float4*>(p + min(c * 256 + lane * 4, d - 4));
}

// h = fp16((v - mean) * rstd * w + b) for the row's elements (w and b: the lane's chunks).
template <int CH>
__device__ __forceinline__ void vit_ln_store(const float (&v)[CH][4], int d, int lane, float mean, float rstd,
                                             const float4 (&w)[CH], const float4 (&b)[CH],
                                             uint16_t* __restrict__ hrow) {
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int e = c * 256 + lane * 4;
        if (e < d) {
            const float4 wv = w[c], bv = b[c];
            const float wa[4] = {wv.x, wv.y, wv.z, wv.w}, ba[4] = {bv.x, bv.y, bv.z, bv.w};
            half4_t o;
#pragma unroll
            for (int j = 0; j < 4; j++) o[j] = _Float16((v[c][j] - mean) * rstd * wa[j] + ba[j]);
            *reinterpret_cast<half4_t*>(hrow + e) = o;
        }
    }
}

// x = ((t + bias) + pos_x[px]) + pos_y[py], then h = LayerNorm(x) * w + b (fp16): the patch
// embedding's bias, the learned column and row position rows (table rows [0, npos) and
// [npos, 2 npos)), and the first layer's pre-norm.
template <int CH>
__global__ __launch_bounds__(256) void vit_embed_kernel(const float* __restrict__ t, const float* __restrict__ bias,
                                                        const float* __restrict__ pos, int npos,
                                                        const int32_t* __restrict__ px, const int32_t* __restrict__ py,
                                                        int T, int d, const float* __restrict__ w,
                                                        const float* __restrict__ b, float eps, float* __restrict__ x,
                                                        uint16_t* __restrict__ h) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= T) return;
    const float* pxr = pos + (size_t)px[row] * d;
    const float* pyr = pos + (size_t)(npos + py[row]) * d;
    float v[CH][4];
    float4 ta[CH], ba[CH], xa[CH], ya[CH], wa[CH], lb[CH];
    vit_load_chunks<CH>(t + (size_t)row * d, d, lane, ta);
    vit_load_chunks<CH>(bias, d, lane, ba);
    vit_load_chunks<CH>(pxr, d, lane, xa);
    vit_load_chunks<CH>(pyr, d, lane, ya);
    vit_load_chunks<CH>(w, d, lane, wa);
    vit_load_chunks<CH>(b, d, lane, lb);
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int e = c * 256 + lane * 4;
        if (e < d) {
            const float4 tv = ta[c], bv = ba[c], xv = xa[c], yv = ya[c];
            v[c][0] = ((tv.x + bv.x) + xv.x) + yv.x;
            v[c][1] = ((tv.y + bv.y) + xv.y) + yv.y;
            v[c][2] = ((tv.z + bv.z) + xv.z) + yv.z;
            v[c][3] = ((tv.w + bv.w) + xv.w) + yv.w;
            *reinterpret_cast<float4*>(x + (size_t)row * d + e) = make_float4(v[c][0], v[c][1], v[c][2], v[c][3]);
        }
    }
    float mean, rstd;
    vit_ln_stats<CH>(v, d, lane, eps, mean, rstd);
    vit_ln_store<CH>(v, d, lane, mean, rstd, wa, lb, h + (size_t)row * d);
}

// The layer's two residual steps with x stored once (the attention output o and the down
// projection t in fp16, times powers of two, so o_inv and t_inv scale them back exactly):
//   kVitResH      v = x + (o o_inv + bo); h = LayerNorm(v) * w + b; x is left as it was.
//   kVitResStore  the same v and h, and x = v stored (a trace of the sum after attention).
//   kVitResTwo    v = x + (o o_inv + bo) as above, then x = v + (t t_inv + bt) stored and, with w,
//                 h = LayerNorm(x) * w + b: the MLP residual beside the attention residual it
//                 recomputes, so the sum after attention is never stored.
enum VitResMode { kVitResH = 0, kVitResStore = 1, kVitResTwo = 2 };

template <int CH, int MODE>
__global__ __launch_bounds__(256) void vit_residual2_ln_kernel(float* __restrict__ x, const uint16_t* __restrict__ o16,
                                                               float o_inv, const float* __restrict__ bo,
                                                               const uint16_t* __restrict__ t16, float t_inv,
                                                               const float* __restrict__ bt,
                                                               const float* __restrict__ w, const float* __restrict__ b,
                                                               float eps, int T, int d, uint16_t* __restrict__ h) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= T) return;
    float v[CH][4];
    float4 xa[CH], ba[CH], bta[CH], wa[CH], lb[CH];
    half4_t oa[CH], ta[CH];
    vit_load_chunks<CH>(x + (size_t)row * d, d, lane, xa);
#pragma unroll
    for (int c = 0; c < CH; c++) oa[c] = *reinterpret_cast<const half4_t*>(o16 + (size_t)row * d + min(c * 256 + lane * 4, d - 4));
    vit_load_chunks<CH>(bo, d, lane, ba);
    if constexpr (MODE == kVitResTwo) {
#pragma unroll
        for (int c = 0; c < CH; c++) ta[c] = *reinterpret_cast<const half4_t*>(t16 + (size_t)row * d + min(c * 256 + lane * 4, d - 4));
        vit_load_chunks<CH>(bt, d, lane, bta);
    }
    if (w) {
        vit_load_chunks<CH>(w, d, lane, wa);
        vit_load_chunks<CH>(b, d, lane, lb);
    }
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int e = c * 256 + lane * 4;
        if (e < d) {
            const float xv[4] = {xa[c].x, xa[c].y, xa[c].z, xa[c].w}, bv[4] = {ba[c].x, ba[c].y, ba[c].z, ba[c].w};
#pragma unroll
            for (int j = 0; j < 4; j++) v[c][j] = xv[j] + (float(oa[c][j]) * o_inv + bv[j]);
            if constexpr (MODE == kVitResTwo) {
                const float btv[4] = {bta[c].x, bta[c].y, bta[c].z, bta[c].w};
#pragma unroll
                for (int j = 0; j < 4; j++) v[c][j] = v[c][j] + (float(ta[c][j]) * t_inv + btv[j]);
            }
            if constexpr (MODE != kVitResH)
                *reinterpret_cast<float4*>(x + (size_t)row * d + e) = make_float4(v[c][0], v[c][1], v[c][2], v[c][3]);
        }
    }
    if (!w) return;
    float mean, rstd;
    vit_ln_stats<CH>(v, d, lane, eps, mean, rstd);
    vit_ln_store<CH>(v, d, lane, mean, rstd, wa, lb, h + (size_t)row * d);
}

template <int CH>
constexpr auto vit_residual2_ln_kernel_h = vit_residual2_ln_kernel<CH, kVitResH>;
template <int CH>
constexpr auto vit_residual2_ln_kernel_store = vit_residual2_ln_kernel<CH, kVitResStore>;
template <int CH>
constexpr auto vit_residual2_ln_kernel_two = vit_residual2_ln_kernel<CH, kVitResTwo>;

// One wave per output token: the merge x merge patches of its window (row0 + dy * gx + dx), each
// through the final LayerNorm (pw, pb), summed in (dy, dx) order and scaled by 1 / merge^2;
// pooled (fp32) gets that mean, out (fp16) its RMSNorm times nw.
template <int CH>
__global__ __launch_bounds__(256) void vit_pool_kernel(const float* __restrict__ x, const int32_t* __restrict__ row0,
                                                       const int32_t* __restrict__ gx, int n_tokens, int merge, int d,
                                                       const float* __restrict__ pw, const float* __restrict__ pb,
                                                       float eps, const float* __restrict__ nw, float* __restrict__ pooled,
                                                       uint16_t* __restrict__ out) {
    const int tok = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (tok >= n_tokens) return;
    const int r0 = row0[tok], stride = gx[tok];
    float acc[CH][4];
#pragma unroll
    for (int c = 0; c < CH; c++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[c][j] = 0.0f;
    float4 pwa[CH], pba[CH], nwa[CH];
    vit_load_chunks<CH>(pw, d, lane, pwa);
    vit_load_chunks<CH>(pb, d, lane, pba);
    vit_load_chunks<CH>(nw, d, lane, nwa);
    for (int dy = 0; dy < merge; dy++)
        for (int dx = 0; dx < merge; dx++) {
            const float* xr = x + (size_t)(r0 + dy * stride + dx) * d;
            float v[CH][4];
            float4 xa[CH];
            vit_load_chunks<CH>(xr, d, lane, xa);
#pragma unroll
            for (int c = 0; c < CH; c++) {
                const int e = c * 256 + lane * 4;
                if (e < d) {
                    const float4 xv = xa[c];
                    v[c][0] = xv.x;
                    v[c][1] = xv.y;
                    v[c][2] = xv.z;
                    v[c][3] = xv.w;
                }
            }
            float mean, rstd;
            vit_ln_stats<CH>(v, d, lane, eps, mean, rstd);
#pragma unroll
            for (int c = 0; c < CH; c++) {
                const int e = c * 256 + lane * 4;
                if (e < d) {
                    const float4 wv = pwa[c], bv = pba[c];
                    const float wa[4] = {wv.x, wv.y, wv.z, wv.w}, ba[4] = {bv.x, bv.y, bv.z, bv.w};
#pragma unroll
                    for (int j = 0; j < 4; j++) acc[c][j] += (v[c][j] - mean) * rstd * wa[j] + ba[j];
                }
            }
        }
    const float inv_area = 1.0f / float(merge * merge);
    float ss = 0.0f;
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int e = c * 256 + lane * 4;
        if (e < d) {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                acc[c][j] *= inv_area;
                ss += acc[c][j] * acc[c][j];
            }
            *reinterpret_cast<float4*>(pooled + (size_t)tok * d + e) = make_float4(acc[c][0], acc[c][1], acc[c][2], acc[c][3]);
        }
    }
    const float inv = 1.0f / sqrtf(wave_sum(ss) / float(d) + eps);
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int e = c * 256 + lane * 4;
        if (e < d) {
            const float4 wv = nwa[c];
            const float wa[4] = {wv.x, wv.y, wv.z, wv.w};
            half4_t o;
#pragma unroll
            for (int j = 0; j < 4; j++) o[j] = _Float16(acc[c][j] * inv * wa[j]);
            *reinterpret_cast<half4_t*>(out + (size_t)tok * d + e) = o;
        }
    }
}

#define VIT_DISPATCH(KERNEL, CHV, ...)                                                                   \
    switch (CHV) {                                                                                      \
    case 1: launch_kernel(KERNEL<1>, __VA_ARGS__); break;                                               \
    case 2: launch_kernel(KERNEL<2>, __VA_ARGS__); break;                                               \
    case 3: launch_kernel(KERNEL<3>, __VA_ARGS__); break;                                               \
    case 4: launch_kernel(KERNEL<4>, __VA_ARGS__); break;                                               \
    case 5: launch_kernel(KERNEL<5>, __VA_ARGS__); break;                                               \
    case 6: launch_kernel(KERNEL<6>, __VA_ARGS__); break;                                               \
    case 7: launch_kernel(KERNEL<7>, __VA_ARGS__); break;                                               \
    default: launch_kernel(KERNEL<8>, __VA_ARGS__); break;                                              \
    }

static bool vit_width_ok(int d) { return d > 0 && d % 4 == 0 && d <= kVitMaxWidth; }

hipError_t launch_vit_embed(hipStream_t s, const float* t, const float* bias, const float* pos, int npos,
                            const int32_t* px, const int32_t* py, int T, int d, const float* w, const float* b, float eps,
                            float* x, uint16_t* h) {
    if (T < 0 || !vit_width_ok(d) || npos <= 0 || !t || !bias || !pos || !px || !py || !w || !b || !x || !h)
        return hipErrorInvalidValue;
    if (T == 0) return hipSuccess;
    const int CH = (d + 255) / 256;
    VIT_DISPATCH(vit_embed_kernel, CH, dim3((T + 3) / 4), dim3(256), 0, s, t, bias, pos, npos, px, py, T, d, w, b, eps, x, h)
    return hipGetLastError();
}

hipError_t launch_vit_residual2_ln(hipStream_t s, int mode, float* x, const uint16_t* o16, float o_inv, const float* bo,
                                   const uint16_t* t16, float t_inv, const float* bt, const float* w, const float* b,
                                   float eps, int T, int d, uint16_t* h) {
    if (T < 0 || !vit_width_ok(d) || !x || !o16 || !bo || (w && (!b || !h)) || mode < kVitResH || mode > kVitResTwo ||
        (mode == kVitResTwo && (!t16 || !bt)) || (mode != kVitResTwo && !w))
        return hipErrorInvalidValue;
    if (T == 0) return hipSuccess;
    const int CH = (d + 255) / 256;
    if (mode == kVitResH)
        VIT_DISPATCH(vit_residual2_ln_kernel_h, CH, dim3((T + 3) / 4), dim3(256), 0, s, x, o16, o_inv, bo, t16, t_inv, bt, w, b, eps, T, d, h)
    else if (mode == kVitResStore)
        VIT_DISPATCH(vit_residual2_ln_kernel_store, CH, dim3((T + 3) / 4), dim3(256), 0, s, x, o16, o_inv, bo, t16, t_inv, bt, w, b, eps, T, d, h)
    else
        VIT_DISPATCH(vit_residual2_ln_kernel_two, CH, dim3((T + 3) / 4), dim3(256), 0, s, x, o16, o_inv, bo, t16, t_inv, bt, w, b, eps, T, d, h)
    return hipGetLastError();
}

hipError_t launch_vit_pool(hipStream_t s, const float* x, const int32_t* row0, const int32_t* gx, int n_tokens, int merge,
                           int d, const float* pw, const float* pb, float eps, const float* nw, float* pooled,
                           uint16_t* out) {
    if (n_tokens < 0 || merge <= 0 || !vit_width_ok(d) || !x || !row0 || !gx || !pw || !pb || !nw || !pooled || !out)
        return hipErrorInvalidValue;
    if (n_tokens == 0) return hipSuccess;
    const int CH = (d + 255) / 256;
    VIT_DISPATCH(vit_pool_kernel, CH, dim3((n_tokens + 3) / 4), dim3(256), 0, s, x, row0, gx, n_tokens, merge, d, pw, pb,
                 eps, nw, pooled, out)
    return hipGetLastError();
}

#undef VIT_DISPATCH

}  // namespace ge
