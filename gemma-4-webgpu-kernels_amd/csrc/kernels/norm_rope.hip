// The attention producer for gfx950: per-head RMSNorm and half-split partial
// RoPE of the q/k projections, the unweighted per-head RMSNorm of v, and the
// write of the new K/V rows into the layer's cache (linear or ring), in one
// launch.
//
// Replaces, behind the backend trait, the WGSL RMSNORM_ROPE kernel
// (rust/src/kernels/rmsnorm_rope.wgsl, dispatched by
// rust/src/backend_wgpu.rs:877-893) and the COPY of the KV append
// (rust/src/backend_wgpu.rs:1014-1055); the semantics are the CPU
// composition the trait defines (rust/src/backend.rs:146-154):
//   rms_norm (rust/src/backend_cpu.rs:149-172): inv = 1/sqrt(ss/Dh + eps),
//            y = x*inv*w (w optional),
//   rope     (rust/src/backend_cpu.rs:248-268): for j < rot/2,
//            freq = theta^(-2j/rot), ang = pos*freq,
//            out[j] = a*cos - b*sin, out[j + rot/2] = b*cos + a*sin
//            (a = y[j], b = y[j + rot/2]); dims >= rot pass through,
// as the model applies them to one attention block (rust/src/model.rs:256-281).
//
// One wave per row (token, head) of Dh values; lane l owns dims 4l..4l+3
// (+256, +512, +768). Every operation is the reference's, separately rounded
// (this file is built with -ffp-contract=off), so the rows come out
// bit-identical to the CPU backend's:
//   - the sum of squares runs d = 0..Dh-1 in order, as the reference's
//     iterator sum does: the rows' squares go to LDS and lane r of wave 0 adds
//     row r's in sequence (one dependent chain of Dh adds per row, the rows of
//     a workgroup side by side). A tree reduction over the wave moves inv by
//     an ulp now and then, which scores of ~90 turn into ~5e-5 of attention
//     output;
//   - sin and cos of the angle come from a table the host fills with libm's
//     sinf / cosf of pos * freq (Rust's f32::sin_cos on the same platform)
//     for positions below the table's size; the device's sincosf differs from
//     libm by an ulp in places. Past the table (positions the host did not
//     tabulate) the kernel falls back to sincosf of pos * freq;
//   - the frequencies come from the host too (libm powf, as Rust's f32::powf):
//     a one-ulp difference in freq would move the angle by pos * ulp, i.e. by
//     ~2e-3 rad at position 32768.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "g4a_params.h"

namespace {

constexpr int NR_WAVES = 4;    // rows per workgroup
constexpr int NR_MAXE = 4;     // float4 groups per lane: Dh <= 1024

// Row stride of the LDS stage: 4 floats of padding put the rows of the
// sequential sums (lane r reads row r) on different banks.
constexpr int NR_STRIDE = NR_MAXE * 256 + 4;

// HOIST (the short form, for launches of at most one workgroup per CU: decode
// steps) issues the norm weights and the rotation's sin/cos together right after
// the norm's barriers, at indices clamped into range; the long form (prefill)
// loads each where it is used, which keeps registers free for occupancy (the
// short form's loads made a 2048-token prefill 14 % slower). The operations and
// their order are the same in both, so the rows are bit-identical.
template <bool HOIST>
__device__ __forceinline__ void norm_rope_rows(const G4aNormRopeParams& p) {
    __shared__ __attribute__((aligned(16))) float stage[NR_WAVES][NR_STRIDE];
    __shared__ float row_ss[NR_WAVES];
    const int lane = threadIdx.x & 63;
    // wave-uniform (readfirstlane): the row, its segment and the segment's fields then
    // stay in scalar registers, read from the kernel arguments by scalar loads; a
    // per-lane row index made every field a vector load with a wait at each use
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t row = blockIdx.x * NR_WAVES + w;
    // a device position (T = 1) is read at run time; past max_pos the launch writes nothing
    // (every thread of the grid leaves here, before any barrier)
    uint32_t pos0 = p.pos0, cache_row = p.cache_row;
    if (p.dpos) {
        pos0 = __builtin_amdgcn_readfirstlane(*p.dpos);
        if (pos0 > p.max_pos) return;
        cache_row = pos0;
    }
    // no early return: every wave reaches the workgroup barriers of the norm
    bool live = row < p.total_rows;
    // segment of this row (rows are segment-major: seg s covers T * heads_s rows)
    int si = 0;
    uint32_t r = live ? row : 0u;
    while (si + 1 < (int)p.nseg && r >= p.T * p.seg[si].heads) {
        r -= p.T * p.seg[si].heads;
        ++si;
    }
    const G4aNormRopeSeg S = p.seg[si];
    const uint32_t t = r / S.heads, h = r % S.heads;
    live = live && t >= S.first_t;  // else its ring slot is taken by a later token of this call
    const uint32_t Dh = p.Dh;
    const float* __restrict__ xr = S.x + ((size_t)t * S.heads + h) * Dh;
    float4 v[NR_MAXE];
#pragma unroll
    for (int e = 0; e < NR_MAXE; ++e) {
        const uint32_t d = 4 * lane + 256 * e;
        v[e] = live && d < Dh ? *reinterpret_cast<const float4*>(xr + d) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    const bool norm_row = live && S.norm;
    if (p.any_norm) {
        // squares (each rounded, as v * v) into the stage, then lane r of wave 0 sums row r
        // in order: ss = ((x0^2 + x1^2) + x2^2) + ...
        if (norm_row) {
#pragma unroll
            for (int e = 0; e < NR_MAXE; ++e) {
                const uint32_t d = 4 * lane + 256 * e;
                if (d < Dh) {
                    const float4 sq = make_float4(v[e].x * v[e].x, v[e].y * v[e].y, v[e].z * v[e].z, v[e].w * v[e].w);
                    *reinterpret_cast<float4*>(&stage[w][d]) = sq;
                }
            }
        }
        __syncthreads();
        if (w == 0 && lane < NR_WAVES) {
            const float* const sr = stage[lane];
            float ss = 0.0f;
            uint32_t d = 0;
            for (; d + 16 <= Dh; d += 16) {
                const float4 a = *reinterpret_cast<const float4*>(sr + d);
                const float4 b = *reinterpret_cast<const float4*>(sr + d + 4);
                const float4 c = *reinterpret_cast<const float4*>(sr + d + 8);
                const float4 e = *reinterpret_cast<const float4*>(sr + d + 12);
                ss = ss + a.x; ss = ss + a.y; ss = ss + a.z; ss = ss + a.w;
                ss = ss + b.x; ss = ss + b.y; ss = ss + b.z; ss = ss + b.w;
                ss = ss + c.x; ss = ss + c.y; ss = ss + c.z; ss = ss + c.w;
                ss = ss + e.x; ss = ss + e.y; ss = ss + e.z; ss = ss + e.w;
            }
            for (; d < Dh; d += 4) {  // head_dim % 16 != 0
                const float4 a = *reinterpret_cast<const float4*>(sr + d);
                ss = ss + a.x; ss = ss + a.y; ss = ss + a.z; ss = ss + a.w;
            }
            row_ss[lane] = ss;
        }
        __syncthreads();
    }
    if (!live) return;
    // short form: every load the rest of the row needs goes out here, before the first
    // use, at indices clamped into range and under wave-uniform tests only (loads under
    // the per-dim bounds tests below wait one at a time: the norm weights per 256 dims,
    // the sin/cos per dim)
    const uint32_t rot = p.rotary_dim, half = rot / 2;
    const bool rope = S.rope && rot;
    float4 wv[NR_MAXE];
    if (HOIST && S.norm && S.w) {
#pragma unroll
        for (int e = 0; e < NR_MAXE; ++e)
            if (256u * e < Dh) wv[e] = *reinterpret_cast<const float4*>(S.w + min(4u * lane + 256u * e, Dh - 4));
    }
    uint32_t ipos = 0;
    bool tab = false;
    float2 scv[NR_MAXE][4];
    if (rope) {
        ipos = p.pos ? p.pos[t] : pos0 + t;
        tab = ipos < p.sc_rows;
        if (HOIST && tab) {
            const float2* const sc_row = p.sc + (size_t)ipos * half;
#pragma unroll
            for (int e = 0; e < NR_MAXE; ++e)
                if (256u * e < rot) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const uint32_t d = min(4u * lane + 256u * e + i, rot - 1);
                        scv[e][i] = sc_row[d < half ? d : d - half];
                    }
                }
        }
    }
    if (S.norm) {
        const float ss = row_ss[w];
        const float inv = 1.0f / sqrtf(ss / (float)Dh + p.eps);
#pragma unroll
        for (int e = 0; e < NR_MAXE; ++e) {
            const uint32_t d = 4 * lane + 256 * e;
            if (d >= Dh) continue;
            v[e].x = v[e].x * inv;
            v[e].y = v[e].y * inv;
            v[e].z = v[e].z * inv;
            v[e].w = v[e].w * inv;
            if (S.w) {
                const float4 ww = HOIST ? wv[e] : *reinterpret_cast<const float4*>(S.w + d);
                v[e].x = v[e].x * ww.x;
                v[e].y = v[e].y * ww.y;
                v[e].z = v[e].z * ww.z;
                v[e].w = v[e].w * ww.w;
            }
        }
    }
    if (rope) {
        float* const ys = stage[w];
#pragma unroll
        for (int e = 0; e < NR_MAXE; ++e) {
            const uint32_t d = 4 * lane + 256 * e;
            if (d < Dh) *reinterpret_cast<float4*>(ys + d) = v[e];
        }
        __builtin_amdgcn_wave_barrier();
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        const float pos = (float)ipos;
        const float2* const sc_row = p.sc + (size_t)(tab ? ipos : 0u) * half;
#pragma unroll
        for (int e = 0; e < NR_MAXE; ++e) {
            const uint32_t d0 = 4 * lane + 256 * e;
            if (d0 >= rot) continue;
            float o[4] = {v[e].x, v[e].y, v[e].z, v[e].w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t d = d0 + i;
                if (d >= rot) continue;  // pass-through tail
                const uint32_t j = d < half ? d : d - half;
                const float a = ys[j], b = ys[j + half];
                float sn, cs;
                if (tab) {
                    const float2 v2 = HOIST ? scv[e][i] : sc_row[j];
                    sn = v2.x;
                    cs = v2.y;
                } else {
                    sincosf(pos * p.freq[j], &sn, &cs);
                }
                o[i] = d < half ? a * cs - b * sn : b * cs + a * sn;
            }
            v[e] = make_float4(o[0], o[1], o[2], o[3]);
        }
    }
    size_t orow = (size_t)t;
    if (S.cache) {
        const uint64_t lr = (uint64_t)cache_row + t;
        orow = p.ring_cap ? (size_t)(lr % p.ring_cap) : (size_t)lr;
    }
    float* const yr = S.y + (orow * S.heads + h) * Dh;
#pragma unroll
    for (int e = 0; e < NR_MAXE; ++e) {
        const uint32_t d = 4 * lane + 256 * e;
        if (d < Dh) *reinterpret_cast<float4*>(yr + d) = v[e];
    }
}

}  // namespace

extern "C" __global__ __launch_bounds__(256) void g4a_norm_rope(G4aNormRopeParams p) { norm_rope_rows<false>(p); }
extern "C" __global__ __launch_bounds__(256) void g4a_norm_rope_short(G4aNormRopeParams p) {
    norm_rope_rows<true>(p);
}
