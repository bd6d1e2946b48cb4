// The rest of the backend trait's op surface for gfx950: elementwise ops, the
// column slice, the fused residual + RMSNorm (+ layer scalar) of every Gemma-4
// post-norm, RMSNorm over rows of any width, and the f32 embedding gather.
//
// Replaces, behind the backend trait, the WGSL ELEMENTWISE, SLICE_COLS, RMSNORM
// and EMBED kernels (rust/src/kernels/elementwise.wgsl, slice_cols.wgsl,
// rmsnorm.wgsl, embed.wgsl; dispatched by rust/src/backend_wgpu.rs:560-622,
// :734-760, :834-876). Semantics are the CPU backend's
// (rust/src/backend_cpu.rs:127-145 embed_rows, :149-172 rms_norm, :224-244 the
// elementwise ops, :343-350 slice_cols) and the trait's add_rms_norm
// composition (rust/src/backend.rs:136-145), each f32 operation separately
// rounded in the same order. These ops move a few bytes per element: the
// kernels are HBM- or launch-bound and are written for coalesced access.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "g4a_math.h"
#include "g4a_params.h"

namespace {

// y[i] = op(a[i], b[i]) over n elements, grid-stride.
__device__ __forceinline__ void ew(const G4aEwParams& p) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    const float s = p.op == G4A_EW_SCALE_BY ? p.sp[0] : p.s;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < p.n; i += stride) {
        const float v = p.op == G4A_EW_FILL ? 0.0f : p.a[i];
        float o;
        switch (p.op) {
            case G4A_EW_ADD: o = v + p.b[i]; break;
            case G4A_EW_MUL: o = v * p.b[i]; break;
            case G4A_EW_SCALE:
            case G4A_EW_SCALE_BY: o = v * s; break;
            case G4A_EW_GELU: o = g4a_gelu_tanh(v); break;
            case G4A_EW_GEGLU: o = g4a_gelu_tanh(v) * p.b[i]; break;
            case G4A_EW_FILL: o = s; break;
            default: o = s * tanhf(v / s); break;  // softcap: cap * tanh(v / cap)
        }
        p.y[i] = o;
    }
}

// y[r, c] = x[r * stride + offset + c]
__device__ __forceinline__ void slice_cols(const G4aSliceColsParams& p) {
    const size_t n = (size_t)p.rows * p.width;
    for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < n; e += (size_t)gridDim.x * blockDim.x) {
        const size_t r = e / p.width, c = e - r * p.width;
        p.y[e] = p.x[r * p.stride + p.offset + c];
    }
}

// One workgroup per row of any width: ss = sum of x^2 (256 strided partial sums,
// then a tree through LDS: another order than the reference's sequential sum),
// inv = 1 / sqrt(ss / D + eps), y = (res + x * inv * w) * s[0], with the
// residual, weight and scalar each optional.
__device__ __forceinline__ void rms_rows(const G4aRmsRowsParams& p) {
    __shared__ float part[256];
    const uint32_t row = blockIdx.x, tid = threadIdx.x;
    const float* __restrict__ xr = p.x + (size_t)row * p.D;
    // RU chunks of 256 at a time: their loads go out together (indices clamped into
    // the row), then the chunk's terms are added in the same order as one by one
    constexpr uint32_t RU = 8;
    float ss = 0.0f;
    for (uint32_t d0 = tid; d0 < p.D; d0 += RU * 256) {
        float xv[RU];
#pragma unroll
        for (uint32_t u = 0; u < RU; ++u) xv[u] = xr[min(d0 + 256 * u, p.D - 1)];
#pragma unroll
        for (uint32_t u = 0; u < RU; ++u) {
            const float t = ss + xv[u] * xv[u];
            ss = d0 + 256 * u < p.D ? t : ss;
        }
    }
    part[tid] = ss;
    __syncthreads();
    for (uint32_t st = 128; st > 0; st >>= 1) {
        if (tid < st) part[tid] += part[tid + st];
        __syncthreads();
    }
    const float inv = 1.0f / sqrtf(part[0] / (float)p.D + p.eps);
    const float sc = p.scale_by ? p.scale_by[0] : 1.0f;
    float* __restrict__ yr = p.y + (size_t)row * p.D;
    const float* __restrict__ rr = p.res ? p.res + (size_t)row * p.D : nullptr;
    const float* __restrict__ wr = p.w;
    // the chunk's loads all go out before its stores: a load after a store to y
    // (which may alias x, w or the residual as far as the compiler knows) waited
    for (uint32_t d0 = tid; d0 < p.D; d0 += RU * 256) {
        float xv[RU], wv[RU], rv[RU];
#pragma unroll
        for (uint32_t u = 0; u < RU; ++u) {
            const uint32_t d = min(d0 + 256 * u, p.D - 1);
            xv[u] = xr[d];
            if (wr) wv[u] = wr[d];
            if (rr) rv[u] = rr[d];
        }
#pragma unroll
        for (uint32_t u = 0; u < RU; ++u) {
            const uint32_t d = d0 + 256 * u;
            if (d >= p.D) break;
            float n = xv[u] * inv;
            if (wr) n = n * wv[u];
            if (rr) n = rv[u] + n;
            if (p.scale_by) n = n * sc;
            yr[d] = n;
        }
    }
}

// embed_rows on an f32 table (rust/src/backend_cpu.rs:138-144): out[i, d] = table[ids[i], d] * scale
__device__ __forceinline__ void embed_rows_f32(const G4aEmbedF32Params& p) {
    const size_t n = (size_t)p.T * p.D;
    for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < n; e += (size_t)gridDim.x * blockDim.x) {
        const size_t i = e / p.D, d = e - i * p.D;
        p.out[e] = p.table[(size_t)p.ids[i] * p.D + d] * p.scale;
    }
}

// counters[i] += inc (u32, wrapping): one thread per counter, vector loads and stores
__device__ __forceinline__ void u32_add(const G4aCounterParams& p) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < p.n) p.c[i] = p.c[i] + p.inc;
}

}  // namespace

extern "C" __global__ __launch_bounds__(256) void g4a_ew(G4aEwParams p) { ew(p); }
extern "C" __global__ __launch_bounds__(256) void g4a_u32_add(G4aCounterParams p) { u32_add(p); }
extern "C" __global__ __launch_bounds__(256) void g4a_slice_cols(G4aSliceColsParams p) { slice_cols(p); }
extern "C" __global__ __launch_bounds__(256) void g4a_rms_rows(G4aRmsRowsParams p) { rms_rows(p); }
extern "C" __global__ __launch_bounds__(256) void g4a_embed_rows_f32(G4aEmbedF32Params p) { embed_rows_f32(p); }
