// Scalar math shared by the gfx950 kernels, in the reference CPU backend's
// operation order (each file is built with -ffp-contract=off).
#pragma once
#include <hip/hip_runtime.h>
#include <math.h>

// sqrt(2 / pi) rounded to f32, as (2.0f32 / PI).sqrt() in rust/src/backend_cpu.rs:56
constexpr float G4A_GELU_C = 0x1.988452p-1f;

// gelu_tanh_scalar (rust/src/backend_cpu.rs:55-58):
// 0.5 * v * (1 + tanh(c * (v + 0.044715 * v * v * v)))
__device__ __forceinline__ float g4a_gelu_tanh(float v) {
    return 0.5f * v * (1.0f + tanhf(G4A_GELU_C * (v + 0.044715f * v * v * v)));
}

constexpr float G4A_NEG_INF = -__builtin_huge_valf();

// Butterfly max / sum over the 64 lanes of a wave (every lane gets the result).
__device__ __forceinline__ float g4a_wave_max(float x) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o, 64));
    return x;
}

__device__ __forceinline__ float g4a_wave_sum(float x) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o, 64);
    return x;
}

// A float4 store of data the next kernel reads once (split partials, output
// rows): non-temporal, so it does not sit in this kernel's L2 as a dirty line
// that the end-of-kernel write-back has to flush.
__device__ __forceinline__ void g4a_store_nt(float* p, const float4& v) {
    __builtin_nontemporal_store(v.x, p);
    __builtin_nontemporal_store(v.y, p + 1);
    __builtin_nontemporal_store(v.z, p + 2);
    __builtin_nontemporal_store(v.w, p + 3);
}
