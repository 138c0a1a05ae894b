// Device helpers shared by the gfx950 kernels.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

namespace ge {

// Events the next launch records from its own dispatch timestamps (set by the runtime while
// profiling; null otherwise). hipExtLaunchKernelGGL stamps the kernel's start and end the way
// the profiler does, without separate marker packets between kernels.
struct LaunchEvents {
    hipEvent_t start = nullptr, stop = nullptr;
};
LaunchEvents& launch_events();

template <typename... KArgs, typename... Args>
inline void launch_kernel(void (*kernel)(KArgs...), dim3 grid, dim3 block, uint32_t lds, hipStream_t s, Args... args) {
    const LaunchEvents& ev = launch_events();
    if (ev.start)
        hipExtLaunchKernelGGL(kernel, grid, block, lds, s, ev.start, ev.stop, 0u, static_cast<KArgs>(args)...);
    else
        hipLaunchKernelGGL(kernel, grid, block, lds, s, static_cast<KArgs>(args)...);
}


typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));
// Native 4 x 32-bit vector for 16-byte moves: unlike HIP's uint4 struct, arrays of it stay in
// registers.
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

__device__ __forceinline__ float gelu_tanh(float x) {
    // 0.5 x (1 + tanh(u)), u = sqrt(2 / pi) (x + 0.044715 x^3) (ggml's gelu_tanh, reference
    // Shaders/Common.metal:18-21, Model/Architecture.md:45), evaluated through the identity
    // 0.5 (1 + tanh(u)) = 1 / (1 + e^(-2u)): one v_exp_f32 and one v_rcp_f32 instead of tanhf.
    // e^(-2u) = 2^(-2u log2 e); it overflows to +inf for very negative x, giving x * 0.
    const float c = 0.79788456080286535587989211986876f;
    const float u = c * x * (1.0f + 0.044715f * x * x);
    const float e = __builtin_amdgcn_exp2f(-2.0f * 1.4426950408889634f * u);
    return x * __builtin_amdgcn_rcpf(1.0f + e);
}

__device__ __forceinline__ float h2f(uint16_t b) { return float(__builtin_bit_cast(_Float16, b)); }
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, _Float16(f)); }

// ---------------------------------------------------------------- wait counters, LDS copies

// s_waitcnt lgkmcnt(0) alone (vmcnt and expcnt at their maxima; gfx9 encoding: vmcnt in bits
// 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
__device__ __forceinline__ void wait_lgkmcnt0() { __builtin_amdgcn_s_waitcnt(0xc07f); }

// s_waitcnt with only the vector-memory counter constrained.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Buffer resource over [p, p + bytes): raw (untyped) dword access, no swizzle; reads past the
// end return zero. p and bytes must be wave-uniform.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, bytes, 0x00020000);
}

// buffer_load_dwordx4 ... lds: lane l's 16 bytes at byte offset voff + soff of r land at
// lds_base + 16 l (lds_base and soff wave-uniform). The copy counts against vmcnt like a load.
// (The global_load_lds form of the same copy is a FLAT instruction, after which the compiler
// treats every LDS wait as a full lgkmcnt(0), serialising fragment reads with the MFMAs.)
__device__ __forceinline__ void lds_copy16(__amdgpu_buffer_rsrc_t r, void* lds_base, uint32_t voff, uint32_t soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds_base, 16, voff, soff, 0, 0);
}

// A workgroup barrier without the release fence of __syncthreads(): that fence would wait for
// every outstanding global->LDS copy, including the ones meant to stay in flight. The asm
// memory clobbers keep the compiler from moving LDS accesses across it; the copies a barrier
// must cover are waited for explicitly (wait_vmcnt) before it, and the LDS reads that must be
// complete (wait_lgkmcnt0).
__device__ __forceinline__ void workgroup_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

}  // namespace ge
