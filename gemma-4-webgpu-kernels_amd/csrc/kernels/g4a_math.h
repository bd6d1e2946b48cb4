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


// x of another lane of the same 16-lane row, by a DPP pattern (no LDS round trip).
constexpr int G4A_DPP_XOR1 = 0xB1;         // quad_perm [1,0,3,2]
constexpr int G4A_DPP_XOR2 = 0x4E;         // quad_perm [2,3,0,1]
constexpr int G4A_DPP_HALF_MIRROR = 0x141;  // lane i of each 8-lane half reads lane 7 - i
constexpr int G4A_DPP_ROW_MIRROR = 0x140;   // lane i of each 16-lane row reads lane 15 - i
template <int CTRL>
__device__ __forceinline__ float g4a_dpp(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}

// Sum / max over each 16-lane row: pairs, quads, half rows, rows. Every lane of
// a row computes the same additions with the operands swapped, so all 16 hold
// the same bits.
__device__ __forceinline__ float g4a_row_sum16(float x) {
    x += g4a_dpp<G4A_DPP_XOR1>(x);
    x += g4a_dpp<G4A_DPP_XOR2>(x);
    x += g4a_dpp<G4A_DPP_HALF_MIRROR>(x);
    x += g4a_dpp<G4A_DPP_ROW_MIRROR>(x);
    return x;
}

__device__ __forceinline__ float g4a_row_max16(float x) {
    x = fmaxf(x, g4a_dpp<G4A_DPP_XOR1>(x));
    x = fmaxf(x, g4a_dpp<G4A_DPP_XOR2>(x));
    x = fmaxf(x, g4a_dpp<G4A_DPP_HALF_MIRROR>(x));
    x = fmaxf(x, g4a_dpp<G4A_DPP_ROW_MIRROR>(x));
    return x;
}

// Max / sum over the 64 lanes of a wave (every lane gets the same bits): the
// 16-lane rows by DPP, then the four row results through readlane, with no LDS
// round trip. The whole wave must be active (readlane reads lanes 0, 16, 32
// and 48 whatever EXEC holds).
__device__ __forceinline__ float g4a_lane(float x, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), l));
}

__device__ __forceinline__ float g4a_wave_max(float x) {
    x = g4a_row_max16(x);
    return fmaxf(fmaxf(g4a_lane(x, 0), g4a_lane(x, 16)), fmaxf(g4a_lane(x, 32), g4a_lane(x, 48)));
}

__device__ __forceinline__ float g4a_wave_sum(float x) {
    x = g4a_row_sum16(x);
    return (g4a_lane(x, 0) + g4a_lane(x, 16)) + (g4a_lane(x, 32) + g4a_lane(x, 48));
}

// Lane l's x and lane (l ^ 16)'s (or (l ^ 32)'s) by a gfx950 permlane swap with
// both operands x: .x holds the lower row's value, .y the upper row's, in both
// lanes of the pair, so a sum of the two has the same bits in both.
__device__ __forceinline__ float2 g4a_pair16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return make_float2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float2 g4a_pair32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return make_float2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Max / sum over lanes l, l ^ 16, l ^ 32, l ^ 48 (the four rows' lanes of one
// column), in every one of them: the order and bits of an xor 16, 32 butterfly.
__device__ __forceinline__ float g4a_col_max4(float x) {
    float2 t = g4a_pair16(x);
    x = fmaxf(t.x, t.y);
    t = g4a_pair32(x);
    return fmaxf(t.x, t.y);
}

__device__ __forceinline__ float g4a_col_sum4(float x) {
    float2 t = g4a_pair16(x);
    x = t.x + t.y;
    t = g4a_pair32(x);
    return t.x + t.y;
}

// Max over each 8-lane group (lanes 8g .. 8g+7), in every lane of the group.
__device__ __forceinline__ float g4a_max8(float x) {
    x = fmaxf(x, g4a_dpp<G4A_DPP_XOR1>(x));
    x = fmaxf(x, g4a_dpp<G4A_DPP_XOR2>(x));
    x = fmaxf(x, g4a_dpp<G4A_DPP_HALF_MIRROR>(x));
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
