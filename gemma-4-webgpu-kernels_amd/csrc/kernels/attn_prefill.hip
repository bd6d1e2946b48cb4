// Query-tiled prefill attention on the fp32 matrix cores (gfx950), with exact
// scores where they matter. Replaces the reference's per-query ATTN_SPLIT
// dispatch for T > 1 (rust/src/backend_wgpu.rs:944-957, grid (T, Hkv, splits))
// behind Backend::attention; results follow rust/src/backend_cpu.rs:270-336.
//
// Tiling. A workgroup (4 waves) owns 8 consecutive queries of one kv head; a
// wave owns 16 rows = 2 queries x the 8 query heads of the kv group, all of
// which read the same K/V (MQA). K/V stream through LDS in double-buffered
// 16-key tiles (register-staged, one tile ahead). Per tile a wave computes
// S^T = K Q^T with v_mfma_f32_16x16x4_f32 (A = K from LDS, B = Q held in
// registers), so the scores land as lane = row, 4 keys per lane: exactly the
// A-operand layout of the following P.V product (another 16x16x4 chain, B = V
// from LDS), with no transpose.
//
// Exactness. The matrix cores sum the 256/512-term dots in their own order, a
// few 1e-5 away from the CPU reference's sequential f32 sum - enough to move
// outputs by up to ~1e-4 when two keys nearly tie. So every key whose
// approximate score is within TAU of its row's running maximum is recorded
// (per-wave list in LDS); once the row block is done, the survivors
// (still within TAU of the final maximum) get their score recomputed in the
// reference's exact order and their contribution corrected:
//   O[row] += (e^{s_exact - m} - e^{s_approx - m}) * v[key],  l[row] += same.
// Keys farther than TAU below the maximum carry weight < e^-10 relative to it,
// so their ~1e-5 score error changes the output by < 1e-9. If the list fills
// up (many near-ties), it is compacted against the current maxima and, if
// still full, corrected on the spot.
#include "g4a_params.h"

namespace {

constexpr float PF_TAU = 10.0f;

template <int DH>
struct PrefillCfg {
    static constexpr int BK = 16;                        // keys per tile (one MFMA K-block)
    static constexpr int KRS = DH + 4;                   // padded K row stride in LDS
    static constexpr int TILE = BK * KRS + BK * DH;      // floats per tile buffer: K then V
    static constexpr int LPT = (2 * BK * DH / 4) / 256;  // float4 loads per thread per tile
    static constexpr int NC = DH / 64;                   // O column groups (x4 MFMA blocks)
    static constexpr int QT = DH / 16;                   // Q float4 per lane
    static constexpr int CAP = DH == 256 ? 2048 : 640;   // candidate entries per wave
    static constexpr int SMEM = 2 * TILE + 4 * 2 * CAP + 4 * 16;
};

__device__ __forceinline__ uint64_t ballot(bool b) { return __ballot(b); }
__device__ __forceinline__ int lanes_below(uint64_t m) {
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0));
}
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int DH>
__device__ __forceinline__ void prefill(const G4aPrefillParams& p) {
    using C = PrefillCfg<DH>;
    constexpr int BK = C::BK, KRS = C::KRS, LPT = C::LPT, NC = C::NC, QT = C::QT, CAP = C::CAP;
    __shared__ __attribute__((aligned(16))) float smem[C::SMEM];

    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, rl = lane & 15;
    const uint32_t kvh = blockIdx.y;
    const uint32_t qb = blockIdx.x * 8;
    const uint32_t qw = qb + 2 * w;
    const uint32_t h0 = kvh * 8;
    const size_t row_stride = (size_t)p.Hkv * DH;
    const float* __restrict__ kbase = p.k + (size_t)kvh * DH;
    const float* __restrict__ vbase = p.v + (size_t)kvh * DH;
    uint32_t* const my_keys = reinterpret_cast<uint32_t*>(smem + 2 * C::TILE + w * 2 * CAP);
    float* const my_s = smem + 2 * C::TILE + w * 2 * CAP + CAP;
    float* const my_m = smem + 2 * C::TILE + 4 * 2 * CAP + w * 16;

    // visible key-index range [lo, hi) of query i
    auto key_hi = [&](int64_t i) -> int64_t {
        const int64_t lim = (int64_t)p.q_pos0 + i - (int64_t)p.k_pos0 + 1;
        return lim <= 0 ? 0 : (lim < (int64_t)p.S ? lim : (int64_t)p.S);
    };
    auto key_lo = [&](int64_t i) -> int64_t {
        if (p.window == 0) return 0;
        const int64_t lo = (int64_t)p.q_pos0 + i - (int64_t)p.k_pos0 - (int64_t)p.window + 1;
        return lo > 0 ? lo : 0;
    };
    auto prow = [&](uint32_t j) -> size_t { return p.ring_cap ? j % p.ring_cap : j; };

    const uint32_t qlast = min(qb + 7, p.T - 1);
    const int64_t wg_lo = key_lo(qb), wg_hi = key_hi(qlast);
    const uint32_t nt = wg_hi > wg_lo ? (uint32_t)((wg_hi - wg_lo + BK - 1) / BK) : 0;
    const bool wave_valid = qw < p.T;
    const int64_t w_lo = wave_valid ? key_lo(qw) : 0;
    const int64_t w_hi = wave_valid ? key_hi(min(qw + 1, p.T - 1)) : 0;

    // this lane's softmax row: query qw + rl/8, head h0 + rl%8
    const uint32_t myq = qw + (rl >> 3);
    const bool qvalid = myq < p.T;
    const int64_t my_lo = key_lo(myq), my_hi = qvalid ? key_hi(myq) : 0;
    float4 qr[QT];
    {
        const float* qrow = p.q + ((size_t)min(myq, p.T - 1) * p.Hq + h0 + (rl & 7)) * DH + 4 * g;
#pragma unroll
        for (int t = 0; t < QT; ++t) qr[t] = ld4(qrow + 16 * t);
    }

    auto load_tile = [&](uint32_t t, float4 (&r)[LPT]) {
        const int64_t t0 = wg_lo + (int64_t)t * BK;
#pragma unroll
        for (int i = 0; i < LPT; ++i) {
            const int f = (tid + 256 * i) % (BK * DH / 4);
            int64_t key = t0 + f / (DH / 4);
            if (key > wg_hi - 1) key = wg_hi - 1;
            const float* base = i < LPT / 2 ? kbase : vbase;
            r[i] = ld4(base + prow((uint32_t)key) * row_stride + 4 * (f % (DH / 4)));
        }
    };
    auto store_tile = [&](float* buf, const float4 (&r)[LPT]) {
#pragma unroll
        for (int i = 0; i < LPT; ++i) {
            const int f = (tid + 256 * i) % (BK * DH / 4);
            float* dst = i < LPT / 2 ? buf + (f / (DH / 4)) * KRS + 4 * (f % (DH / 4))
                                     : buf + BK * KRS + (f / (DH / 4)) * DH + 4 * (f % (DH / 4));
            *reinterpret_cast<float4*>(dst) = r[i];
        }
    };

    float m_run = NEG_INF, l_part = 0.0f;
    f4v O[NC][4];
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int e = 0; e < 4; ++e) O[c][e] = f4v{0.0f, 0.0f, 0.0f, 0.0f};
    int cnt = 0;  // wave-uniform number of recorded candidates

    // Publish every row's reference maximum to the wave's m table.
    auto publish_m = [&](float mref) {
        if (g == 0) my_m[rl] = mref;
        wave_sync();
    };
    // Drop recorded candidates more than TAU below their row's published maximum.
    auto compact = [&]() {
        int nc = 0;
        for (int base = 0; base < cnt; base += 64) {
            const int e = base + lane;
            const bool has = e < cnt;
            const uint32_t pk = has ? my_keys[e] : 0u;
            const float sa = has ? my_s[e] : 0.0f;
            const bool keep = has && sa > my_m[pk >> 28] - PF_TAU;
            wave_sync();
            const uint64_t b = ballot(keep);
            if (keep) {
                const int pos = nc + lanes_below(b);
                my_keys[pos] = pk;
                my_s[pos] = sa;
            }
            nc += __builtin_popcountll(b);
            wave_sync();
        }
        cnt = nc;
    };
    // Exact rescoring of every recorded candidate and correction of O and l,
    // against the published maxima (the scale O and l are currently held at).
    auto flush = [&]() {
        for (int base = 0; base < cnt; base += 64) {
            const int e = base + lane;
            const bool has = e < cnt;
            const uint32_t pk = has ? my_keys[e] : 0u;
            const uint32_t rho = pk >> 28, kap = pk & 0x0fffffffu;
            float delta = 0.0f;
            if (has) {
                const float* qrow = p.q + ((size_t)(qw + (rho >> 3)) * p.Hq + h0 + (rho & 7)) * DH;
                const float* krow = kbase + prow(kap) * row_stride;
                float dot = 0.0f;
#pragma unroll 4
                for (int d = 0; d < DH; d += 16) {
                    float4 qa[4], ka[4];
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        qa[u] = ld4(qrow + d + 4 * u);
                        ka[u] = ld4(krow + d + 4 * u);
                    }
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        dot = dot + qa[u].x * ka[u].x;
                        dot = dot + qa[u].y * ka[u].y;
                        dot = dot + qa[u].z * ka[u].z;
                        dot = dot + qa[u].w * ka[u].w;
                    }
                }
                const float sx = dot * p.scale;
                const float m = my_m[rho];
                delta = expf(sx - m) - expf(my_s[e] - m);
            }
            const int nb = min(64, cnt - base);
            for (int i = 0; i < nb; ++i) {
                const float di = __builtin_amdgcn_readlane(__float_as_int(delta), i) == 0
                                     ? 0.0f
                                     : __int_as_float(__builtin_amdgcn_readlane(__float_as_int(delta), i));
                if (di == 0.0f) continue;
                const uint32_t ri = __builtin_amdgcn_readlane(rho, i);
                const uint32_t ki = __builtin_amdgcn_readlane(kap, i);
                if (lane == (int)ri) l_part += di;
                if (g == (int)(ri >> 2)) {
                    const float* vrow = vbase + prow(ki) * row_stride + 4 * rl;
#pragma unroll
                    for (int c = 0; c < NC; ++c) {
                        const float4 v4 = ld4(vrow + 64 * c);
                        const float vv[4] = {v4.x, v4.y, v4.z, v4.w};
#pragma unroll
                        for (int ee = 0; ee < 4; ++ee) {
                            switch (ri & 3) {
                                case 0: O[c][ee][0] = __builtin_fmaf(di, vv[ee], O[c][ee][0]); break;
                                case 1: O[c][ee][1] = __builtin_fmaf(di, vv[ee], O[c][ee][1]); break;
                                case 2: O[c][ee][2] = __builtin_fmaf(di, vv[ee], O[c][ee][2]); break;
                                default: O[c][ee][3] = __builtin_fmaf(di, vv[ee], O[c][ee][3]); break;
                            }
                        }
                    }
                }
            }
        }
        cnt = 0;
    };

    float4 pre[LPT];
    if (nt > 0) load_tile(0, pre);  // no visible key at all: nothing to load (the clamp needs wg_hi >= 1)
    for (uint32_t t = 0; t < nt; ++t) {
        float* const buf = smem + (t & 1) * C::TILE;
        store_tile(buf, pre);
        __syncthreads();
        load_tile(min(t + 1, nt - 1), pre);  // always issued: exact load counting; the last one re-reads
        const int64_t t0 = wg_lo + (int64_t)t * BK;
        if (!wave_valid || t0 >= w_hi || t0 + BK <= w_lo) continue;
        const float* Kt = buf;
        const float* Vt = buf + BK * KRS;

        // ---- approximate scores S^T = K Q^T: lane holds keys 4g + r of row rl ----
        f4v S = f4v{0.0f, 0.0f, 0.0f, 0.0f};
        const float* kr = Kt + rl * KRS + 4 * g;
#pragma unroll
        for (int tt = 0; tt < QT; ++tt) {
            const float4 kk = *reinterpret_cast<const float4*>(kr + 16 * tt);
            S = __builtin_amdgcn_mfma_f32_16x16x4f32(kk.x, qr[tt].x, S, 0, 0, 0);
            S = __builtin_amdgcn_mfma_f32_16x16x4f32(kk.y, qr[tt].y, S, 0, 0, 0);
            S = __builtin_amdgcn_mfma_f32_16x16x4f32(kk.z, qr[tt].z, S, 0, 0, 0);
            S = __builtin_amdgcn_mfma_f32_16x16x4f32(kk.w, qr[tt].w, S, 0, 0, 0);
        }
        float s[4];
        bool vis[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t j = t0 + 4 * g + r;
            vis[r] = j >= my_lo && j < my_hi;
            s[r] = vis[r] ? S[r] * p.scale : NEG_INF;
        }
        float tm = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
        tm = fmaxf(tm, __shfl_xor(tm, 16, 64));
        tm = fmaxf(tm, __shfl_xor(tm, 32, 64));
        const float mn = fmaxf(m_run, tm);

        // ---- record the keys within TAU of the running maximum ----
        if (cnt + 4 * 64 > CAP) {
            publish_m(mn);
            compact();
            if (cnt + 4 * 64 > CAP) {
                publish_m(m_run);  // O and l are still held at m_run
                flush();
            }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const bool cand = vis[r] && s[r] > mn - PF_TAU;
            const uint64_t b = ballot(cand);
            if (cand) {
                const int pos = cnt + lanes_below(b);
                my_keys[pos] = ((uint32_t)rl << 28) | (uint32_t)(t0 + 4 * g + r);
                my_s[pos] = s[r];
            }
            cnt += __builtin_popcountll(b);
        }

        // ---- online softmax (row rl) and P.V on the matrix cores ----
        float pr[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) pr[r] = vis[r] ? expf(s[r] - mn) : 0.0f;
        const float corr = (m_run == NEG_INF) ? 0.0f : expf(m_run - mn);
        l_part = l_part * corr + ((pr[0] + pr[1]) + (pr[2] + pr[3]));
        m_run = mn;
        // O rows are 4g + r'; their correction factors live in lanes 4g + r'
        const f4v cr = f4v{__shfl(corr, 4 * g + 0, 64), __shfl(corr, 4 * g + 1, 64), __shfl(corr, 4 * g + 2, 64),
                           __shfl(corr, 4 * g + 3, 64)};
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int e = 0; e < 4; ++e) O[c][e] *= cr;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float* vr = Vt + (4 * g + r) * DH + 4 * rl;
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const float4 vv = *reinterpret_cast<const float4*>(vr + 64 * c);
                O[c][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(pr[r], vv.x, O[c][0], 0, 0, 0);
                O[c][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(pr[r], vv.y, O[c][1], 0, 0, 0);
                O[c][2] = __builtin_amdgcn_mfma_f32_16x16x4f32(pr[r], vv.z, O[c][2], 0, 0, 0);
                O[c][3] = __builtin_amdgcn_mfma_f32_16x16x4f32(pr[r], vv.w, O[c][3], 0, 0, 0);
            }
        }
    }
    if (!wave_valid) return;  // no barrier follows

    // ---- exact corrections for the keys still within TAU of the final maxima ----
    publish_m(m_run);
    compact();
    flush();

    // ---- normalise and write: O row 4g + r' is query qw + row/8, head h0 + row%8 ----
    float l = l_part;
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int row = 4 * g + r;
        const float lr = __shfl(l, row, 64);
        const float inv = lr > 0.0f ? 1.0f / lr : 0.0f;
        const uint32_t qi = qw + (row >> 3);
        if (qi >= p.T) continue;
        float* orow = p.out + ((size_t)qi * p.Hq + h0 + (row & 7)) * DH + 4 * rl;
#pragma unroll
        for (int c = 0; c < NC; ++c)
            *reinterpret_cast<float4*>(orow + 64 * c) =
                make_float4(O[c][0][r] * inv, O[c][1][r] * inv, O[c][2][r] * inv, O[c][3][r] * inv);
    }
}

}  // namespace

extern "C" {
__global__ __launch_bounds__(256) void g4a_prefill_d256(G4aPrefillParams p) { prefill<256>(p); }
__global__ __launch_bounds__(256) void g4a_prefill_d512(G4aPrefillParams p) { prefill<512>(p); }
}
