// Split-K flash-decode attention for gfx950 (CDNA4), MQA/GQA groups of 4 or 8
// query heads per kv head, head_dim 256 or 512, f32 everywhere.
//
// Replaces the reference's ATTN_SPLIT / ATTN_COMBINE WGSL kernels
// (rust/src/kernels/attention_split.wgsl, attention_combine.wgsl) behind
// Backend::attention (rust/src/backend.rs:119-120). Results follow the CPU
// reference rust/src/backend_cpu.rs:270-336.
//
// Exactness. The attention scores are computed exactly as the CPU reference
// does: dot = ((0 + q0*k0) + q1*k1) + ... over d = 0..Dh-1 with every multiply
// and add rounded separately (this file is built with -ffp-contract=off; the
// only fused multiply-adds are the explicit __builtin_fmaf in the P.V fold),
// then *scale, then the optional soft-cap. With unit-RMS q/k and scale 1 the
// scores reach ~90, so any other summation order moves them by ~1e-5 and the
// output by up to ~5e-5; bit-equal scores keep the output within ~1e-7.
//
// Work decomposition. A workgroup is 4 waves and owns one key split of one
// (query, kv head). Each wave owns 4 query heads ("head group") and walks
// 64-key tiles of its split: in the score phase lane = key, each lane runs 4
// sequential dots (q is wave-uniform, so it streams through the scalar cache),
// then an online softmax per head; in the P.V phase lane = output dims and the
// wave's probabilities are broadcast from LDS. The 4 waves of a workgroup are
// (key-tile slot, head group) pairs; at the end the key-tile slots of a head
// group merge through LDS and the split's (m, l, acc) partial is written,
// or the normalised output when there is a single split.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "g4a_params.h"

namespace {

constexpr float NEG_INF = -__builtin_huge_valf();

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o, 64));
    return x;
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o, 64);
    return x;
}

__device__ __forceinline__ float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }

// Read-only, wave-uniform data (the query rows) is addressed through the
// constant address space so the compiler can fetch it with scalar loads into
// SGPRs instead of per-lane vector loads.
typedef __attribute__((address_space(4))) const float cfloat;
__device__ __forceinline__ cfloat* as_const(const float* p) { return (cfloat*)(p); }

__device__ __forceinline__ float f4get(const float4& v, int e) {
    return e == 0 ? v.x : e == 1 ? v.y : e == 2 ? v.z : v.w;
}

// Physical row of logical key j: a ring of ring_cap slots, or the identity.
__device__ __forceinline__ uint32_t phys_row(uint32_t j, uint32_t ring_cap) {
    return ring_cap ? j % ring_cap : j;
}

__device__ __forceinline__ float score_epilogue(float dot, float scale, float softcap) {
    dot *= scale;
    if (softcap > 0.0f) dot = softcap * tanhf(dot / softcap);
    return dot;
}

typedef float f4v __attribute__((ext_vector_type(4)));  // MFMA accumulator (4 VGPRs)

// One float4 chunk (dims d..d+3) of the 4 per-lane dots of a head group:
// for each head, dot = (((dot + q[d]k[d]) + q[d+1]k[d+1]) + ...) with separately
// rounded multiplies and adds, exactly the CPU reference's order.
template <int DH>
__device__ __forceinline__ void qk_chunk(float (&s)[4], cfloat* __restrict__ qh, int d, const float4& kk, int c) {
    // bound how far the scheduler hoists the scalar q loads (SGPR budget)
    if ((c & 1) == 0) __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int h = 0; h < 4; ++h) {
        cfloat* qd = qh + h * DH + d;
        float a = s[h];
        a = a + qd[0] * kk.x;
        a = a + qd[1] * kk.y;
        a = a + qd[2] * kk.z;
        a = a + qd[3] * kk.w;
        s[h] = a;
    }
}

template <int DH, int GROUP>
struct DecodeCfg {
    static constexpr int HG = GROUP / 4;                 // head-group waves per key-tile slot
    static constexpr int KT = 4 / HG;                    // key-tile slots per workgroup
    static constexpr int DC = KT == 2 ? 64 : 32;         // dims per K stage
    static constexpr int NST = DH / DC;                  // K stages per tile
    static constexpr int C4 = DC / 4;                    // float4 per row per stage
    static constexpr int RS = DC + 4;                    // LDS row stride in floats (padded: no bank conflicts)
    static constexpr int SLOT_THREADS = 64 * HG;
    static constexpr int LPT = 64 * C4 / SLOT_THREADS;   // float4 loads per thread per stage
    static constexpr int NV4 = DH / 256;                 // V float4 per lane per row
    static constexpr int PVK = 64 / HG;                  // keys per wave in the P.V phase
    static constexpr int VB = 8;                         // V prefetch depth (keys)
    static constexpr int NHQ = GROUP / 4;                // MFMA head quarters
    // shared memory (floats)
    static constexpr int KST = KT * 2 * 64 * RS;         // double-buffered K stages
    static constexpr int MERGE = 4 * GROUP * DH;         // end-of-kernel merge (overlays KST)
    static constexpr int BIG = KST > MERGE ? KST : MERGE;
    static constexpr int PBUF = KT * 64 * 4 * HG;        // probabilities [slot][key][i][hh]
    static constexpr int CORR = KT * GROUP;
    static constexpr int ML = KT * 2 * GROUP;
    static constexpr int SMEM = BIG + PBUF + CORR + ML;
    static_assert(LPT * SLOT_THREADS == 64 * C4, "stage must split evenly over the slot's threads");
    static_assert(PVK % VB == 0, "P.V key range must be a multiple of the prefetch depth");
};

// Split-K flash decode: see the file header for the decomposition.
template <int DH, int GROUP>
__device__ __forceinline__ void decode_split(const G4aDecodeParams& p) {
    static_assert(DH == 256 || DH == 512, "fast decode handles head_dim 256 / 512");
    static_assert(GROUP == 4 || GROUP == 8, "fast decode handles groups of 4 / 8 heads");
    using C = DecodeCfg<DH, GROUP>;
    constexpr int HG = C::HG, KT = C::KT, DC = C::DC, NST = C::NST, C4 = C::C4, RS = C::RS, LPT = C::LPT,
                  NV4 = C::NV4, PVK = C::PVK, VB = C::VB, NHQ = C::NHQ, SLOT_THREADS = C::SLOT_THREADS;

    __shared__ __attribute__((aligned(16))) float smem[C::SMEM];
    float* const kst = smem;                          // [KT][2][64*RS]
    float* const mrg = smem;                          // [4][GROUP][DH] after the tile loop
    float* const pbuf = smem + C::BIG;                // [KT][64][4][HG]
    float* const corrbuf = pbuf + C::PBUF;            // [KT][GROUP]
    float* const mlbuf = corrbuf + C::CORR;           // [KT][2][GROUP]

    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int hg = w % HG;
    const int kt = w / HG;
    const int stid = hg * 64 + lane;
    const uint32_t split = blockIdx.x, qi = blockIdx.y, kvh = blockIdx.z;
    const uint32_t qpos = p.q_pos ? p.q_pos[qi] : p.q_pos0 + qi;
    const uint32_t ks = p.k_start + split * p.keys_per_split;
    const uint32_t ke = min(ks + p.keys_per_split, p.k_end);
    const uint32_t h0 = kvh * GROUP;
    cfloat* __restrict__ qh = as_const(p.q + ((size_t)qi * p.Hq + h0 + hg * 4) * DH);
    const size_t row_stride = (size_t)p.Hkv * DH;
    const float* __restrict__ kbase = p.k + (size_t)kvh * DH;
    const float* __restrict__ vbase = p.v + (size_t)kvh * DH + 4 * lane;
    float* const my_kst = kst + kt * 2 * 64 * RS;
    float* const my_pbuf = pbuf + kt * 64 * 4 * HG;

    float m[4], lpart[4];
#pragma unroll
    for (int h = 0; h < 4; ++h) {
        m[h] = NEG_INF;
        lpart[h] = 0.0f;
    }
    f4v acc[NHQ][NV4][4];
#pragma unroll
    for (int a = 0; a < NHQ; ++a)
#pragma unroll
        for (int b = 0; b < NV4; ++b)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[a][b][e] = f4v{0.0f, 0.0f, 0.0f, 0.0f};

    const uint32_t ntiles = ke > ks ? (ke - ks + 63) / 64 : 0;
    const uint32_t niter = (ntiles + KT - 1) / KT;
    for (uint32_t it = 0; it < niter; ++it) {
        const uint32_t t = it * KT + kt;
        const uint32_t t0 = ks + t * 64;
        bool active = t < ntiles;
        if (active) {
            const uint32_t kpos_first = p.k_pos ? p.k_pos[t0] : p.k_pos0 + t0;
            active = kpos_first <= qpos;  // ascending positions: a future first key means a future tile
        }
        const uint32_t nk = active ? min(64u, ke - t0) : 1u;
        const uint32_t row0 = active ? phys_row(t0, p.ring_cap) : 0u;
        auto prow = [&](uint32_t r) -> uint32_t {  // physical row of tile key r (clamped to the tile)
            uint32_t x = row0 + min(r, nk - 1);
            if (p.ring_cap && x >= p.ring_cap) x -= p.ring_cap;
            return x;
        };

        // ---- scores: K streams through LDS in stages of DC dims, lane = key ----
        float4 kreg[2][LPT];
        auto load_stage = [&](int st, float4 (&r)[LPT]) {
#pragma unroll
            for (int i = 0; i < LPT; ++i) {
                const int f = stid + SLOT_THREADS * i;
                r[i] = ld4(kbase + (size_t)prow(f / C4) * row_stride + st * DC + 4 * (f % C4));
            }
        };
        auto store_stage = [&](int buf, const float4 (&r)[LPT]) {
#pragma unroll
            for (int i = 0; i < LPT; ++i) {
                const int f = stid + SLOT_THREADS * i;
                *reinterpret_cast<float4*>(my_kst + buf * 64 * RS + (f / C4) * RS + 4 * (f % C4)) = r[i];
            }
        };
        float4 vb[VB][NV4];
        const uint32_t kv0 = hg * PVK;  // first key of this wave's P.V range
        auto load_v = [&](uint32_t kk, float4 (&r)[NV4]) {
            const float* vr = vbase + (size_t)prow(kk) * row_stride;
#pragma unroll
            for (int q4 = 0; q4 < NV4; ++q4) r[q4] = ld4(vr + 256 * q4);
        };

        float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (active) {
            load_stage(0, kreg[0]);
            if (NST > 1) load_stage(1, kreg[1]);
        }
#pragma unroll
        for (int st = 0; st < NST; ++st) {
            if (active) store_stage(st & 1, kreg[st & 1]);
            __syncthreads();
            if (active) {
                if (st + 2 < NST) load_stage(st + 2, kreg[st & 1]);
                if (st == NST - 1) {
#pragma unroll
                    for (int b = 0; b < VB; ++b) load_v(kv0 + b, vb[b]);  // overlap V latency with the last stage
                }
                const float* kr = my_kst + (st & 1) * 64 * RS + lane * RS;
#pragma unroll
                for (int c = 0; c < C4; ++c) {
                    const float4 kk = *reinterpret_cast<const float4*>(kr + 4 * c);
                    qk_chunk<DH>(s, qh, st * DC + 4 * c, kk, c);
                }
            }
        }

        // ---- online softmax for this wave's 4 heads (lane = key) ----
        if (active) {
            const uint32_t j = t0 + min((uint32_t)lane, nk - 1);
            const uint32_t kp = p.k_pos ? p.k_pos[j] : p.k_pos0 + j;
            const bool vis = (uint32_t)lane < nk && kp <= qpos && (p.window == 0 || qpos - kp < p.window);
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                const float sc = vis ? score_epilogue(s[h], p.scale, p.softcap) : NEG_INF;
                const float mn = fmaxf(m[h], wave_max(sc));
                const float corr = (m[h] == NEG_INF) ? 0.0f : expf(m[h] - mn);
                const float pr = (sc == NEG_INF) ? 0.0f : expf(sc - mn);
                lpart[h] = lpart[h] * corr + pr;
                m[h] = mn;
                my_pbuf[lane * 4 * HG + h * HG + hg] = pr;
                if (lane == 0) corrbuf[kt * GROUP + hg * 4 + h] = corr;
            }
        }
        __syncthreads();

        // ---- P.V on the matrix cores: this wave's PVK keys, all GROUP heads ----
        // v_mfma_f32_4x4x1_16b_f32: 16 blocks of D[4 heads][4 dims] += P[head] * V[dim];
        // lane l gives A = P[hq*4 + l%4] and B = V[key][256*q4 + 4*l + e]; its
        // result register r holds out[hq*4 + r][256*q4 + 4*l + e].
        if (active) {
#pragma unroll
            for (int hq = 0; hq < NHQ; ++hq) {
                const float* cb = corrbuf + kt * GROUP + hq * 4;
                const f4v cr = f4v{cb[0], cb[1], cb[2], cb[3]};
#pragma unroll
                for (int q4 = 0; q4 < NV4; ++q4)
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[hq][q4][e] *= cr;
            }
            const float* pb = my_pbuf + (lane & 3) * HG;
            for (int kb = 0; kb < PVK; kb += VB) {
#pragma unroll
                for (int b = 0; b < VB; ++b) {
                    const uint32_t kk = kv0 + kb + b;
                    float a[NHQ];
#pragma unroll
                    for (int hq = 0; hq < NHQ; ++hq) a[hq] = pb[kk * 4 * HG + hq];
#pragma unroll
                    for (int hq = 0; hq < NHQ; ++hq)
#pragma unroll
                        for (int q4 = 0; q4 < NV4; ++q4) {
                            acc[hq][q4][0] = __builtin_amdgcn_mfma_f32_4x4x1f32(a[hq], vb[b][q4].x, acc[hq][q4][0], 0, 0, 0);
                            acc[hq][q4][1] = __builtin_amdgcn_mfma_f32_4x4x1f32(a[hq], vb[b][q4].y, acc[hq][q4][1], 0, 0, 0);
                            acc[hq][q4][2] = __builtin_amdgcn_mfma_f32_4x4x1f32(a[hq], vb[b][q4].z, acc[hq][q4][2], 0, 0, 0);
                            acc[hq][q4][3] = __builtin_amdgcn_mfma_f32_4x4x1f32(a[hq], vb[b][q4].w, acc[hq][q4][3], 0, 0, 0);
                        }
                    if (kb + VB < PVK) load_v(kk + VB, vb[b]);
                }
            }
        }
    }

    // ---- per-slot (m, l), then merge the 4 waves' accumulators through LDS ----
#pragma unroll
    for (int h = 0; h < 4; ++h) lpart[h] = wave_sum(lpart[h]);
    if (lane == 0) {
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            mlbuf[kt * 2 * GROUP + hg * 4 + h] = m[h];
            mlbuf[kt * 2 * GROUP + GROUP + hg * 4 + h] = lpart[h];
        }
    }
    __syncthreads();  // every wave is done with the K stages: the merge buffer may overlay them
#pragma unroll
    for (int hq = 0; hq < NHQ; ++hq)
#pragma unroll
        for (int q4 = 0; q4 < NV4; ++q4)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                *reinterpret_cast<float4*>(mrg + ((size_t)w * GROUP + hq * 4 + r) * DH + 256 * q4 + 4 * lane) =
                    make_float4(acc[hq][q4][0][r], acc[hq][q4][1][r], acc[hq][q4][2][r], acc[hq][q4][3][r]);
    __syncthreads();
    // wave w finalises heads [w*GROUP/4, (w+1)*GROUP/4)
#pragma unroll
    for (int hh = 0; hh < GROUP / 4; ++hh) {
        const int h = w * (GROUP / 4) + hh;
        float M = NEG_INF;
#pragma unroll
        for (int sl = 0; sl < KT; ++sl) M = fmaxf(M, mlbuf[sl * 2 * GROUP + h]);
        float L = 0.0f, es[KT];
#pragma unroll
        for (int sl = 0; sl < KT; ++sl) {
            const float ms = mlbuf[sl * 2 * GROUP + h];
            es[sl] = (ms == NEG_INF) ? 0.0f : expf(ms - M);
            L += mlbuf[sl * 2 * GROUP + GROUP + h] * es[sl];
        }
        const size_t ih = (size_t)qi * p.Hq + h0 + h;
#pragma unroll
        for (int q4 = 0; q4 < NV4; ++q4) {
            float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
            for (int sl = 0; sl < KT; ++sl) {
                float4 a = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
                for (int g = 0; g < HG; ++g) {
                    const float4 x = *reinterpret_cast<const float4*>(mrg + ((size_t)(sl * HG + g) * GROUP + h) * DH + 256 * q4 + 4 * lane);
                    a.x += x.x; a.y += x.y; a.z += x.z; a.w += x.w;
                }
                o.x += a.x * es[sl]; o.y += a.y * es[sl]; o.z += a.z * es[sl]; o.w += a.w * es[sl];
            }
            if (p.nsplit == 1) {
                const float inv = L > 0.0f ? 1.0f / L : 0.0f;
                *reinterpret_cast<float4*>(p.out + ih * DH + 256 * q4 + 4 * lane) =
                    make_float4(o.x * inv, o.y * inv, o.z * inv, o.w * inv);
            } else {
                *reinterpret_cast<float4*>(p.part + (ih * p.nsplit + split) * DH + 256 * q4 + 4 * lane) = o;
            }
        }
        if (p.nsplit > 1 && lane == 0) {
            float* ml = p.part + (size_t)p.T * p.Hq * p.nsplit * DH + (ih * p.nsplit + split) * 2;
            ml[0] = M;
            ml[1] = L;
        }
    }
}

// out = sum_s acc_s * e^(m_s - M) / sum_s l_s * e^(m_s - M), M = max_s m_s; 0 when the
// denominator is 0 (the semantics of rust/src/kernels/attention_combine.wgsl:1-28).
// One block per (64 output dims, head, query). The split weights e^(m_s - M) are
// computed once per block into LDS; the 4 waves then stream disjoint quarters of
// the splits with several loads in flight per lane and reduce through LDS.
constexpr int COMBINE_MAX_SPLITS = 1024;

template <int DH>
__device__ __forceinline__ void combine(const G4aCombineParams& p) {
    __shared__ float wgt[COMBINE_MAX_SPLITS];
    __shared__ float red[4][64];
    __shared__ float redm[4], redl[4];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = tid >> 6;
    const uint32_t d = blockIdx.x * 64 + lane;
    const size_t ih = (size_t)blockIdx.z * p.Hq + blockIdx.y;
    const float* __restrict__ ml = p.part + (size_t)p.T * p.Hq * p.nsplit * DH + ih * p.nsplit * 2;
    const float* __restrict__ acc = p.part + ih * p.nsplit * DH + d;
    const uint32_t ns = p.nsplit;
    float M = NEG_INF;
    for (uint32_t s = tid; s < ns; s += 256) M = fmaxf(M, ml[2 * s]);
    M = wave_max(M);
    if (lane == 0) redm[w] = M;
    __syncthreads();
    M = fmaxf(fmaxf(redm[0], redm[1]), fmaxf(redm[2], redm[3]));
    float L = 0.0f;
    for (uint32_t s = tid; s < ns; s += 256) {
        const float ms = ml[2 * s];
        const float e = (ms == NEG_INF) ? 0.0f : expf(ms - M);
        wgt[s] = e;
        L += ml[2 * s + 1] * e;
    }
    L = wave_sum(L);
    if (lane == 0) redl[w] = L;
    __syncthreads();
    L = redl[0] + redl[1] + redl[2] + redl[3];
    constexpr int U = 8;
    float A = 0.0f;
    uint32_t s = w;
    for (; s + 4 * (U - 1) < ns; s += 4 * U) {
        float x[U];
#pragma unroll
        for (int u = 0; u < U; ++u) x[u] = acc[(size_t)(s + 4 * u) * DH];
#pragma unroll
        for (int u = 0; u < U; ++u) A += x[u] * wgt[s + 4 * u];
    }
    for (; s < ns; s += 4) A += acc[(size_t)s * DH] * wgt[s];
    red[w][lane] = A;
    __syncthreads();
    if (w == 0) {
        A = red[0][lane] + red[1][lane] + red[2][lane] + red[3][lane];
        p.out[ih * DH + d] = L > 0.0f ? A / L : 0.0f;
    }
}

// Generic masked online-softmax attention, one wave per (query, head), for any
// head dims (Dh <= 1024, Dv <= 1024) and group sizes. Same exact score
// arithmetic as the fast path; the semantics of rust/src/kernels/attention.wgsl
// plus the soft-cap of rust/src/backend_cpu.rs:303-305.
__device__ __forceinline__ void generic_attention(const G4aGenericParams& p) {
    constexpr int MAXV = 16;  // Dv <= 64 * MAXV
    __shared__ float qs[1024];
    __shared__ float pb[64];
    const int lane = threadIdx.x;
    const uint32_t h = blockIdx.x, qi = blockIdx.y;
    const uint32_t group = p.Hq / p.Hkv;
    const uint32_t kvh = h / group;
    const uint32_t qpos = p.q_pos[qi];
    const float* __restrict__ qr = p.q + ((size_t)qi * p.Hq + h) * p.Dh;
    for (uint32_t d = lane; d < p.Dh; d += 64) qs[d] = qr[d];
    __syncthreads();
    float m = NEG_INF, l = 0.0f;
    float acc[MAXV];
#pragma unroll
    for (int e = 0; e < MAXV; ++e) acc[e] = 0.0f;
    for (uint32_t t0 = p.k_start; t0 < p.k_end; t0 += 64) {
        const uint32_t nk = min(64u, p.k_end - t0);
        const bool inr = (uint32_t)lane < nk;
        const uint32_t j = inr ? t0 + lane : t0;
        const float* __restrict__ kr = p.k + ((size_t)phys_row(j, p.ring_cap) * p.Hkv + kvh) * p.Dh;
        float dot = 0.0f;
        for (uint32_t d = 0; d < p.Dh; ++d) dot = dot + qs[d] * kr[d];
        const uint32_t kp = p.k_pos[j];
        const bool vis = inr && kp <= qpos && (p.window == 0 || qpos - kp < p.window);
        const float sc = vis ? score_epilogue(dot, p.scale, p.softcap) : NEG_INF;
        const float mn = fmaxf(m, wave_max(sc));
        const float corr = (m == NEG_INF) ? 0.0f : expf(m - mn);
        const float pr = (sc == NEG_INF) ? 0.0f : expf(sc - mn);
        l = l * corr + pr;
        m = mn;
#pragma unroll
        for (int e = 0; e < MAXV; ++e) acc[e] *= corr;
        pb[lane] = pr;
        __syncthreads();
        for (uint32_t jj = 0; jj < nk; ++jj) {
            const float pj = pb[jj];
            const float* __restrict__ vr = p.v + ((size_t)phys_row(t0 + jj, p.ring_cap) * p.Hkv + kvh) * p.Dv;
#pragma unroll
            for (int e = 0; e < MAXV; ++e) {
                const uint32_t d = lane + 64 * e;
                if (d < p.Dv) acc[e] = __builtin_fmaf(pj, vr[d], acc[e]);
            }
        }
        __syncthreads();
    }
    l = wave_sum(l);
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    float* o = p.out + ((size_t)qi * p.Hq + h) * p.Dv;
#pragma unroll
    for (int e = 0; e < MAXV; ++e) {
        const uint32_t d = lane + 64 * e;
        if (d < p.Dv) o[d] = acc[e] * inv;
    }
}

}  // namespace

extern "C" {
__global__ __launch_bounds__(256) void g4a_decode_d256_g8(G4aDecodeParams p) { decode_split<256, 8>(p); }
__global__ __launch_bounds__(256) void g4a_decode_d512_g8(G4aDecodeParams p) { decode_split<512, 8>(p); }
__global__ __launch_bounds__(256) void g4a_decode_d256_g4(G4aDecodeParams p) { decode_split<256, 4>(p); }
__global__ __launch_bounds__(256) void g4a_decode_d512_g4(G4aDecodeParams p) { decode_split<512, 4>(p); }
__global__ __launch_bounds__(256) void g4a_combine_d256(G4aCombineParams p) { combine<256>(p); }
__global__ __launch_bounds__(256) void g4a_combine_d512(G4aCombineParams p) { combine<512>(p); }
__global__ __launch_bounds__(64) void g4a_generic_attention(G4aGenericParams p) { generic_attention(p); }
}
