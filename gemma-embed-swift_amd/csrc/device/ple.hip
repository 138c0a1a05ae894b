// Row kernels of the per-layer-input (PLE) branch of the reference's real architecture
// (Model/CPUReference.swift:206-210, :259-269; Model/Architecture.md:15-31):
//   ple = rmsnorm_pl(x0 @ Wplp^T / sqrt(d), per_layer_proj_norm)            once per forward
//   g = gelu_tanh(x @ Winp_gate^T) * ple[:, l, :]                           per layer
//   x = (x + rmsnorm(g @ Wproj^T, post_norm)) * layer_output_scale[l]
// The two projections whose inputs are not normalised (the residual x and the gated product g)
// run as fp16 GEMMs on per-row scaled copies: each row is divided by a power of two s that
// brings its 2-norm under 2^14, so every element fits fp16, and the consumer multiplies the
// row's products by s again. Both steps are exact, so the scaling changes no value beyond the
// fp16 rounding every GEMM input has. One wave per row, lane l owning elements
// c * 256 + 4 l .. + 3 of each 256-wide chunk c.
#include "common.hpp"
#include "kernels.hpp"

namespace ge {

namespace {

// The power of two s >= 1 with ||row||_2 / s < 2^14.
__device__ __forceinline__ float ple_row_scale(float sumsq) {
    const float n = sqrtf(sumsq);
    return n < 16384.0f ? 1.0f : exp2f(ceilf(log2f(n)) - 13.0f);
}

}  // namespace

// out[r] = rmsnorm(in[r] * mul * rscale[r / per_scale]) * w over rows of `width` (the per-layer
// input chunks: row t * L + l, scaled by token t's input scale).
template <int CH>
__global__ __launch_bounds__(256) void ple_rmsnorm_kernel(const float* __restrict__ in, int rows, int width, float mul,
                                                          const float* __restrict__ rscale, int per_scale,
                                                          const float* __restrict__ w, float eps, float* __restrict__ out) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float sc = mul * rscale[row / per_scale];
    float v[CH][4];
    float ss = 0.0f;
    // every chunk's loads before any use (a lane past the width reads the last chunk, unused)
    float4 ia[CH], wa[CH];
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int ec = min(c * 256 + lane * 4, width - 4);
        ia[c] = *reinterpret_cast<const float4*>(in + (size_t)row * width + ec);
        wa[c] = *reinterpret_cast<const float4*>(w + ec);
    }
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int e = c * 256 + lane * 4;
        if (e < width) {
            const float4 a = ia[c];
            v[c][0] = a.x * sc;
            v[c][1] = a.y * sc;
            v[c][2] = a.z * sc;
            v[c][3] = a.w * sc;
#pragma unroll
            for (int j = 0; j < 4; j++) ss += v[c][j] * v[c][j];
        }
    }
    const float inv = 1.0f / sqrtf(wave_sum(ss) / float(width) + eps);
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int e = c * 256 + lane * 4;
        if (e < width)
            *reinterpret_cast<float4*>(out + (size_t)row * width + e) =
                make_float4(v[c][0] * inv * wa[c].x, v[c][1] * inv * wa[c].y, v[c][2] * inv * wa[c].z, v[c][3] * inv * wa[c].w);
    }
}

// x16[r] = fp16(x[r] / s_r), rscale[r] = s_r.
template <int CH>
__global__ __launch_bounds__(256) void ple_input_kernel(const float* __restrict__ x, int T, int d,
                                                        uint16_t* __restrict__ x16, float* __restrict__ rscale) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= T) return;
    float v[CH][4];
    float ss = 0.0f;
    float4 xa[CH];  // every chunk in flight before any use (a lane past d reads the last chunk, unused)
#pragma unroll
    for (int c = 0; c < CH; c++) xa[c] = *reinterpret_cast<const float4*>(x + (size_t)row * d + min(c * 256 + lane * 4, d - 4));
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int e = c * 256 + lane * 4;
        if (e < d) {
            const float4 a = xa[c];
            v[c][0] = a.x;
            v[c][1] = a.y;
            v[c][2] = a.z;
            v[c][3] = a.w;
#pragma unroll
            for (int j = 0; j < 4; j++) ss += v[c][j] * v[c][j];
        }
    }
    const float s = ple_row_scale(wave_sum(ss)), is = 1.0f / s;
    if (lane == 0) rscale[row] = s;
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int e = c * 256 + lane * 4;
        if (e < d) {
            half4_t o;
#pragma unroll
            for (int j = 0; j < 4; j++) o[j] = _Float16(v[c][j] * is);
            *reinterpret_cast<half4_t*>(x16 + (size_t)row * d + e) = o;
        }
    }
}

// The FFN residual of a layer with the branch, fused with the branch's row-scaled input:
// x = x + rmsnorm(t) * w (t as fp16 t * c with t_eps = eps * c^2, as residual_norm_kernel takes
// it), then x16[r] = fp16(x[r] / s_r), rscale[r] = s_r.
template <int CH>
__global__ __launch_bounds__(256) void ple_residual_input_kernel(float* __restrict__ x, const uint16_t* __restrict__ t16,
                                                                 float t_eps, const float* __restrict__ w, int T, int d,
                                                                 uint16_t* __restrict__ x16, float* __restrict__ rscale) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= T) return;
    float tv[CH][4], xv[CH][4];
    float ss = 0.0f;
    // every chunk's loads before any use (a lane past d reads the last chunk, unused)
    half4_t ta[CH];
    float4 xa4[CH], wa[CH];
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int ec = min(c * 256 + lane * 4, d - 4);
        ta[c] = *reinterpret_cast<const half4_t*>(t16 + (size_t)row * d + ec);
        xa4[c] = *reinterpret_cast<const float4*>(x + (size_t)row * d + ec);
        wa[c] = *reinterpret_cast<const float4*>(w + ec);
    }
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int e = c * 256 + lane * 4;
        if (e < d) {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                tv[c][j] = float(ta[c][j]);
                ss += tv[c][j] * tv[c][j];
            }
        }
    }
    const float inv = 1.0f / sqrtf(wave_sum(ss) / float(d) + t_eps);
    float ss2 = 0.0f;
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int e = c * 256 + lane * 4;
        if (e < d) {
            const float xa[4] = {xa4[c].x, xa4[c].y, xa4[c].z, xa4[c].w};
            const float wv[4] = {wa[c].x, wa[c].y, wa[c].z, wa[c].w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                xv[c][j] = xa[j] + tv[c][j] * inv * wv[j];
                ss2 += xv[c][j] * xv[c][j];
            }
            *reinterpret_cast<float4*>(x + (size_t)row * d + e) = make_float4(xv[c][0], xv[c][1], xv[c][2], xv[c][3]);
        }
    }
    const float sc = ple_row_scale(wave_sum(ss2)), is = 1.0f / sc;
    if (lane == 0) rscale[row] = sc;
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int e = c * 256 + lane * 4;
        if (e < d) {
            half4_t o;
#pragma unroll
            for (int j = 0; j < 4; j++) o[j] = _Float16(xv[c][j] * is);
            *reinterpret_cast<half4_t*>(x16 + (size_t)row * d + e) = o;
        }
    }
}

// g = gelu_tanh(graw[r] * rscale[r]) * ple[r][layer]; g16[r] = fp16(g / s2_r), rscale2[r] = s2_r.
template <int CH>
__global__ __launch_bounds__(256) void ple_gate_kernel(const float* __restrict__ graw, const float* __restrict__ rscale,
                                                       const float* __restrict__ ple, int layer, int layers, int T, int pl,
                                                       uint16_t* __restrict__ g16, float* __restrict__ rscale2) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= T) return;
    const float s = rscale[row];
    const float* pr = ple + ((size_t)row * layers + layer) * pl;
    float v[CH][4];
    float ss = 0.0f;
    float4 ga[CH], pa[CH];  // every chunk in flight before any use (a lane past pl reads the last chunk, unused)
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int ec = min(c * 256 + lane * 4, pl - 4);
        ga[c] = *reinterpret_cast<const float4*>(graw + (size_t)row * pl + ec);
        pa[c] = *reinterpret_cast<const float4*>(pr + ec);
    }
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int e = c * 256 + lane * 4;
        if (e < pl) {
            const float4 a = ga[c];
            const float4 p = pa[c];
            v[c][0] = gelu_tanh(a.x * s) * p.x;
            v[c][1] = gelu_tanh(a.y * s) * p.y;
            v[c][2] = gelu_tanh(a.z * s) * p.z;
            v[c][3] = gelu_tanh(a.w * s) * p.w;
#pragma unroll
            for (int j = 0; j < 4; j++) ss += v[c][j] * v[c][j];
        }
    }
    const float s2 = ple_row_scale(wave_sum(ss)), is2 = 1.0f / s2;
    if (lane == 0) rscale2[row] = s2;
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int e = c * 256 + lane * 4;
        if (e < pl) {
            half4_t o;
#pragma unroll
            for (int j = 0; j < 4; j++) o[j] = _Float16(v[c][j] * is2);
            *reinterpret_cast<half4_t*>(g16 + (size_t)row * pl + e) = o;
        }
    }
}

// p = praw[r] * rscale2[r]; x = (x + rmsnorm(p) * w) * out_scale; with next_w also
// h = rmsnorm(x) * next_w (fp16), the next layer's pre-norm.
template <int CH, bool F32OUT>
__global__ __launch_bounds__(256) void ple_residual_norm_kernel(float* __restrict__ x, const float* __restrict__ praw,
                                                                const float* __restrict__ rscale2,
                                                                const float* __restrict__ w, float out_scale,
                                                                const float* __restrict__ next_w, float eps, int T, int d,
                                                                uint16_t* __restrict__ h, float* __restrict__ h32) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= T) return;
    const float s2 = rscale2[row];
    float p[CH][4], xv[CH][4];
    float ss = 0.0f;
    // every chunk's loads before any use (a lane past d reads the last chunk, unused)
    float4 pa[CH], xa4[CH], wa[CH], nwa[CH];
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int ec = min(c * 256 + lane * 4, d - 4);
        pa[c] = *reinterpret_cast<const float4*>(praw + (size_t)row * d + ec);
        xa4[c] = *reinterpret_cast<const float4*>(x + (size_t)row * d + ec);
        wa[c] = *reinterpret_cast<const float4*>(w + ec);
        if (next_w) nwa[c] = *reinterpret_cast<const float4*>(next_w + ec);
    }
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int e = c * 256 + lane * 4;
        if (e < d) {
            const float4 a = pa[c];
            p[c][0] = a.x * s2;
            p[c][1] = a.y * s2;
            p[c][2] = a.z * s2;
            p[c][3] = a.w * s2;
#pragma unroll
            for (int j = 0; j < 4; j++) ss += p[c][j] * p[c][j];
        }
    }
    const float inv = 1.0f / sqrtf(wave_sum(ss) / float(d) + eps);
    float ss2 = 0.0f;
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int e = c * 256 + lane * 4;
        if (e < d) {
            const float xa[4] = {xa4[c].x, xa4[c].y, xa4[c].z, xa4[c].w};
            const float wv[4] = {wa[c].x, wa[c].y, wa[c].z, wa[c].w};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                xv[c][j] = (xa[j] + p[c][j] * inv * wv[j]) * out_scale;
                ss2 += xv[c][j] * xv[c][j];
            }
            *reinterpret_cast<float4*>(x + (size_t)row * d + e) = make_float4(xv[c][0], xv[c][1], xv[c][2], xv[c][3]);
        }
    }
    if (!next_w) return;
    const float inv2 = 1.0f / sqrtf(wave_sum(ss2) / float(d) + eps);
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int e = c * 256 + lane * 4;
        if (e < d) {
            if constexpr (F32OUT) {
                *reinterpret_cast<float4*>(h32 + (size_t)row * d + e) =
                    make_float4(xv[c][0] * inv2 * nwa[c][0], xv[c][1] * inv2 * nwa[c][1], xv[c][2] * inv2 * nwa[c][2],
                                xv[c][3] * inv2 * nwa[c][3]);
            } else {
                half4_t o;
#pragma unroll
                for (int j = 0; j < 4; j++) o[j] = _Float16(xv[c][j] * inv2 * nwa[c][j]);
                *reinterpret_cast<half4_t*>(h + (size_t)row * d + e) = o;
            }
        }
    }
}

template <int CH>
constexpr auto ple_residual_norm_f16 = ple_residual_norm_kernel<CH, false>;
template <int CH>
constexpr auto ple_residual_norm_f32 = ple_residual_norm_kernel<CH, true>;

#define PLE_DISPATCH(KERNEL, WIDTH, ROWS, ...)                                                          \
    do {                                                                                                \
        const dim3 grid_((ROWS + 3) / 4);                                                               \
        switch ((WIDTH + 255) / 256) {                                                                  \
        case 1: launch_kernel(KERNEL<1>, grid_, dim3(256), 0, __VA_ARGS__); break;                      \
        case 2: launch_kernel(KERNEL<2>, grid_, dim3(256), 0, __VA_ARGS__); break;                      \
        case 3: launch_kernel(KERNEL<3>, grid_, dim3(256), 0, __VA_ARGS__); break;                      \
        default: launch_kernel(KERNEL<4>, grid_, dim3(256), 0, __VA_ARGS__); break;                     \
        }                                                                                               \
    } while (0)

static bool ple_width_ok(int w) { return w > 0 && w % 4 == 0 && w <= 1024; }

hipError_t launch_ple_rmsnorm(hipStream_t s, const float* in, int rows, int width, float mul, const float* rscale,
                              int per_scale, const float* w, float eps, float* out) {
    if (rows < 0 || !ple_width_ok(width) || per_scale <= 0 || !in || !rscale || !w || !out) return hipErrorInvalidValue;
    if (rows == 0) return hipSuccess;
    PLE_DISPATCH(ple_rmsnorm_kernel, width, rows, s, in, rows, width, mul, rscale, per_scale, w, eps, out);
    return hipGetLastError();
}

hipError_t launch_ple_input(hipStream_t s, const float* x, int T, int d, uint16_t* x16, float* rscale) {
    if (T < 0 || !ple_width_ok(d) || !x || !x16 || !rscale) return hipErrorInvalidValue;
    if (T == 0) return hipSuccess;
    PLE_DISPATCH(ple_input_kernel, d, T, s, x, T, d, x16, rscale);
    return hipGetLastError();
}

hipError_t launch_ple_residual_input(hipStream_t s, float* x, const uint16_t* t16, float t_eps, const float* w, int T,
                                     int d, uint16_t* x16, float* rscale) {
    if (T < 0 || !ple_width_ok(d) || !x || !t16 || !w || !x16 || !rscale) return hipErrorInvalidValue;
    if (T == 0) return hipSuccess;
    PLE_DISPATCH(ple_residual_input_kernel, d, T, s, x, t16, t_eps, w, T, d, x16, rscale);
    return hipGetLastError();
}

hipError_t launch_ple_gate(hipStream_t s, const float* graw, const float* rscale, const float* ple, int layer, int layers,
                           int T, int pl, uint16_t* g16, float* rscale2) {
    if (T < 0 || !ple_width_ok(pl) || layer < 0 || layer >= layers || !graw || !rscale || !ple || !g16 || !rscale2)
        return hipErrorInvalidValue;
    if (T == 0) return hipSuccess;
    PLE_DISPATCH(ple_gate_kernel, pl, T, s, graw, rscale, ple, layer, layers, T, pl, g16, rscale2);
    return hipGetLastError();
}

hipError_t launch_ple_residual_norm(hipStream_t s, float* x, const float* praw, const float* rscale2, const float* w,
                                    float out_scale, const float* next_w, float eps, int T, int d, uint16_t* h, float* h32) {
    if (T < 0 || !ple_width_ok(d) || !x || !praw || !rscale2 || !w || (next_w && !h && !h32)) return hipErrorInvalidValue;
    if (T == 0) return hipSuccess;
    // the fp32 output is a separate instantiation, so the fp16 one compiles as on its own
    if (h32)
        PLE_DISPATCH(ple_residual_norm_f32, d, T, s, x, praw, rscale2, w, out_scale, next_w, eps, T, d, h, h32);
    else
        PLE_DISPATCH(ple_residual_norm_f16, d, T, s, x, praw, rscale2, w, out_scale, next_w, eps, T, d, h, h32);
    return hipGetLastError();
}

#undef PLE_DISPATCH

}  // namespace ge
