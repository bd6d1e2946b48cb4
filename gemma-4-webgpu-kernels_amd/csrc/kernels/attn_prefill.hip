// Query-tiled prefill attention on the matrix cores (gfx950), with exact
// scores where they matter. Replaces the reference's per-query ATTN_SPLIT
// dispatch for T > 1 (rust/src/backend_wgpu.rs:944-957, grid (T, Hkv, splits))
// behind Backend::attention; results follow rust/src/backend_cpu.rs:270-336.
//
// Tiling. A wave owns 16 rows = 2 queries x the 8 query heads of the kv group,
// all of which read the same K/V (MQA). K/V stream through LDS in 16-key tiles.
// Per tile a wave computes S^T = K Q^T on the matrix cores (A = K from LDS,
// B = Q held in registers), so the scores land as lane = row, 4 keys per lane:
// exactly the A-operand layout of the following P.V product (B = V from LDS),
// with no transpose. Two 8-wave kernels, both on K and V pre-split by
// split_kv, scores from fp16 hi/lo splits of K and q each scaled by a power of
// two (K per 16-key tile, q per wave) into fp16's top binade, P.V from fp16
// hi/lo splits:
//   prefill_pair<256>   two waves per row block take the even / odd key tiles;
//   prefill_dsplit<512> two waves per row block split the head dim.
//
// Exactness. The matrix cores sum the 256/512-term dots in their own order
// (and the split forms round their inputs to ~22 bits), a few 1e-5 away from
// the CPU reference's sequential f32 sum on scores of ~90 - enough to move
// outputs by more than the 1e-5 bar when keys nearly tie. So every key whose
// approximate score is within TAU of its row's running maximum is recorded
// (per-wave list in LDS); once the row block is done, the survivors (still
// within TAU of the final maximum) get their score recomputed in the
// reference's exact order and their contribution corrected:
//   O[row] += (e^{s_exact - m} - e^{s_approx - m}) * v[key],  l[row] += same.
// Keys farther than TAU below the maximum keep their estimate, each with weight
// < e^-TAU relative to the maximum's. Their errors delta move the output by at
// most max|delta| * (W_out / l) * max|v - out|, W_out / l the weight share of
// those keys, <= N e^-TAU / (1 + N e^-TAU) for N keys in a row. So TAU
// (G4aPrefillParams::tau) grows with the key range: the host passes
// max(7, ln N + 2), which keeps that share below e^-2 even when every key sits
// just outside the band and every error pushes the same way (worst case with
// the scaled fp16 estimate ~5e-7 on the outputs).
// If the list fills up (many near-ties), it is compacted against the current
// maxima and, if still full, corrected on the spot.
#include "g4a_params.h"

namespace {

// Probabilities are held as P = PSCALE * e^(s - m_ref), m_ref a lagging row
// maximum that is raised (with O and l rescaled) once the running maximum
// passes it by RESCALE. With fp16 P.V splits P <= PSCALE * e^RESCALE = 55.9e3
// stays below the fp16 maximum, and the 2^10 scale keeps the P of keys down to
// e^-16 below m_ref in fp16's normal range (relative error 2^-22 after the
// hi/lo split) instead of its subnormals, whose absolute steps would add up
// over many small weights. O and l carry the same scale, so O / l is unchanged.
constexpr float PF_RESCALE = 4.0f;
// Bound of the wait for a pair partner's half of the end-of-kernel dots (each
// try sleeps ~64 cycles: ~1.7 ms in all, against a few microseconds expected).
// Built with G4A_PF_PAIR_SPIN=0, every wave computes every dot itself (the path
// a wave takes once a wait has run out), for testing that path.
#ifndef G4A_PF_PAIR_SPIN
#define G4A_PF_PAIR_SPIN (1 << 16)
#endif
constexpr int PF_PAIR_SPIN = G4A_PF_PAIR_SPIN;
constexpr float PF_PSCALE = 1024.0f;

// e^x for the in-loop probabilities: the hardware 2^x of x log2(e). The rounded
// product moves a weight by ~|x| 1e-7 relatively, ~4e-8 at most once weighted
// by e^x itself; the exact rescoring cancels this same form, so only the
// estimate's contribution changes.
constexpr float PF_LOG2E = 1.44269504088896341f;
__device__ __forceinline__ float pf_exp(float x) { return __builtin_amdgcn_exp2f(x * PF_LOG2E); }

__device__ __forceinline__ uint64_t ballot(bool b) { return __ballot(b); }
__device__ __forceinline__ int lanes_below(uint64_t m) {
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0));
}
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// ---------------------------------------------------------------------------
// Head-dim 256 prefill with two waves per SIMD. A workgroup is 8 waves over the
// same 8 queries as above: wave w owns rows 16*(w%4) .. +15 (2 queries x 8
// heads) and the tiles of parity w/4 (even or odd 16-key tiles), so the two
// waves sharing a SIMD (w and w+4) never wait on each other and the hardware
// overlaps one wave's LDS and memory waits with the other's work. Per step both
// tiles sit in LDS (global->LDS copies of the next pair in flight meanwhile). At
// the end each wave compacts its candidates against the maximum over both
// parities, corrects them exactly, and the parities merge through LDS.
typedef _Float16 h4v __attribute__((ext_vector_type(4)));
typedef _Float16 h8v __attribute__((ext_vector_type(8)));

// The exponent a that puts values whose largest magnitude is mx into
// [2^14, 2^15) once divided by 2^a (mx = 0 gives any a; the values stay 0).
__device__ __forceinline__ int fp16_scale_exp(float mx) { return __builtin_amdgcn_frexp_expf(mx) - 15; }

// x * 2^-a = hi + lo + O(2^-22 |x * 2^-a|): hi = fp16(x 2^-a), lo = fp16(x 2^-a - hi), both
// rounded to nearest even; the scaling by a power of two is exact.
__device__ __forceinline__ void split8h(const float4& x0, const float4& x1, int a, h8v& hi, h8v& lo) {
    const float x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float y = ldexpf(x[i], -a);
        hi[i] = (_Float16)y;
        lo[i] = (_Float16)(y - (float)hi[i]);
    }
}

// The largest of the wave's 64 non-negative values, as a scalar: read lane by
// lane (once per kernel; a butterfly of shuffles here would share its lane-index
// registers with the tile loop's shuffles and keep them live across it).
__device__ __forceinline__ float wave_max_scalar(float x) {
    uint32_t m = 0;
    const int bits = __float_as_int(x);
#pragma unroll
    for (int l = 0; l < 64; ++l) m = max(m, (uint32_t)__builtin_amdgcn_readlane(bits, l));
    return __int_as_float((int)m);
}

__device__ __forceinline__ float absmax8(const float4& x0, const float4& x1) {
    return fmaxf(fmaxf(fmaxf(fabsf(x0.x), fabsf(x0.y)), fmaxf(fabsf(x0.z), fabsf(x0.w))),
                 fmaxf(fmaxf(fabsf(x1.x), fabsf(x1.y)), fmaxf(fabsf(x1.z), fabsf(x1.w))));
}

// The factor 2^a the split K rows of the 16-key tile starting at key t0 were
// divided by (a scalar load: the address is uniform).
__device__ __forceinline__ float tile_kscale(const G4aPrefillParams& p, uint32_t kvh, int32_t t0) {
    typedef const __attribute__((address_space(4))) float cfloat;
    const uint32_t idx = kvh * (p.split_n / 16) + ((uint32_t)t0 - p.split0) / 16;
    return ((cfloat*)p.kscale)[__builtin_amdgcn_readfirstlane(idx)];
}

// x = hi + lo + O(2^-22 |x|) (for |x| >= 2^-3; below, an absolute 2^-25):
// hi = fp16(x), lo = fp16(x - hi), both rounded to nearest even.
__device__ __forceinline__ void split16(float x, h4v& hi, h4v& lo, int i) {
    const _Float16 h = (_Float16)x;
    hi[i] = h;
    lo[i] = (_Float16)(x - (float)h);
}

// The G4aSplitParams pre-pass. Blocks [0, nkeys/16 * Hkv) split K: one
// 256-thread block per (16-key tile, kv head) finds the tile's largest |k|,
// scales the tile by the power of two that puts it in [2^14, 2^15) and writes
// fp16 hi/lo pairs (items = 8-dim blocks of the tile's rows, strided over the
// threads). The blocks after them split V key quads into fp16 hi/lo pairs (one
// thread per 4 dims 64c + 4n .. +3 of a quad), flagging V values outside the
// fp16 range.
__device__ __forceinline__ void split_kv(const G4aSplitParams& p) {
    const uint32_t nbk = p.Dh / 8, nc = p.Dh / 64;
    const uint32_t kblocks = (p.nkeys / 16) * p.Hkv;
    const size_t nv_items = (size_t)(p.nkeys / 4) * p.Hkv * nc * 16;
    auto row_of = [&](size_t jj) -> size_t {  // physical row of key k0 + jj
        uint32_t j = p.k0 + (uint32_t)jj;
        if (!p.ring_cap && j >= p.S) j = p.S - 1;
        return p.ring_cap ? j % p.ring_cap : j;
    };
    auto seen = [&](size_t jj) -> bool {  // key k0 + jj lies in the call's key range
        const uint32_t j = p.k0 + (uint32_t)jj;
        return j >= p.vis_lo && j < p.vis_hi;
    };
    const float4 zero4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (blockIdx.x < kblocks) {
        constexpr int MAXI = 4;  // items per thread: 16 rows x Dh/8 blocks over 256 threads (Dh <= 512)
        __shared__ float redmax[4];
        const uint32_t tile = blockIdx.x / p.Hkv, h = blockIdx.x % p.Hkv;
        const uint32_t nitems = 16 * nbk;
        // every row is loaded whatever `seen` says (row_of keeps each inside the cache)
        // and an unseen one is replaced by zeros where it is used: a load under the test,
        // or zeros written over its registers, waited for the load on the spot
        float4 x0[MAXI], x1[MAXI];
        bool ok[MAXI];
#pragma unroll
        for (int u = 0; u < MAXI; ++u) {
            const uint32_t it = threadIdx.x + 256 * u;
            const size_t jj = (size_t)tile * 16 + it / nbk;
            const float* src = p.k + (row_of(jj) * p.Hkv + h) * p.Dh + 8 * (it % nbk);
            x0[u] = ld4(src);
            x1[u] = ld4(src + 4);
            ok[u] = it < nitems && seen(jj);
        }
        float mx = 0.0f;  // unseen rows count as zeros, which cannot raise it
#pragma unroll
        for (int u = 0; u < MAXI; ++u) {
            const float m8 = absmax8(x0[u], x1[u]);
            mx = ok[u] ? fmaxf(mx, m8) : mx;
        }
        mx = g4a_wave_max(mx);
        if ((threadIdx.x & 63) == 0) redmax[threadIdx.x >> 6] = mx;
        __syncthreads();
        mx = fmaxf(fmaxf(redmax[0], redmax[1]), fmaxf(redmax[2], redmax[3]));
        const int a = fp16_scale_exp(mx);
#pragma unroll
        for (int u = 0; u < MAXI; ++u) {
            const uint32_t it = threadIdx.x + 256 * u;
            if (it < nitems) {
                const size_t jj = (size_t)tile * 16 + it / nbk;
                h8v hi, lo;
                split8h(ok[u] ? x0[u] : zero4, ok[u] ? x1[u] : zero4, a, hi, lo);
                float* dst = p.kout + (jj * p.Hkv + h) * p.Dh + 8 * (it % nbk);
                *reinterpret_cast<h8v*>(dst) = hi;
                *reinterpret_cast<h8v*>(dst + 4) = lo;
            }
        }
        if (threadIdx.x == 0) p.kscale[h * (p.nkeys / 16) + tile] = ldexpf(1.0f, a);
        return;
    }
    size_t i = (size_t)(blockIdx.x - kblocks) * blockDim.x + threadIdx.x;
    if (i >= nv_items) return;
    const uint32_t n = (uint32_t)(i % 16);
    size_t t = i / 16;
    const uint32_t c = (uint32_t)(t % nc);
    t /= nc;
    const uint32_t h = (uint32_t)(t % p.Hkv);
    const size_t qd = t / p.Hkv;
    float4 x[4];
    bool ok[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {  // all four rows in flight at once; an unseen one is zeros where used
        x[kk] = ld4(p.v + (row_of(4 * qd + kk) * p.Hkv + h) * p.Dh + 64 * c + 4 * n);
        ok[kk] = seen(4 * qd + kk);
    }
    float* const blk = p.vout + (qd * p.Hkv + h) * 4 * p.Dh;
    bool bad = false;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        h4v hi, lo;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            const float xl = e == 0 ? x[kk].x : (e == 1 ? x[kk].y : (e == 2 ? x[kk].z : x[kk].w));
            const float xv = ok[kk] ? xl : 0.0f;
            bad |= !(fabsf(xv) <= 32768.0f);
            split16(xv, hi, lo, kk);
        }
        float* const dst = blk + 4 * ((4 * c + e) * 16 + n);
        *reinterpret_cast<h4v*>(dst) = hi;
        *reinterpret_cast<h4v*>(dst + 2) = lo;
    }
    if (bad) *p.vflag = p.epoch;
}

template <int DH>
struct PairCfg {
    static constexpr int BK = 16;
    static constexpr int KRS = DH + 4;
    static constexpr int TILE = BK * KRS + BK * DH;
    static constexpr int RPW = 2 * 2 * BK * (DH / 256) / 8;  // 1 KiB row copies per wave per tile pair
    static constexpr int NC = DH / 64;
    static constexpr int QT = DH / 16;
    static constexpr int CAP = 256;                          // candidate entries per wave
    static constexpr int SR = 20;                            // staged row stride (floats): 16 dims + pad
    static constexpr int STAGE = (64 + 16) * SR;             // per-wave staging floats (in-loop overflow path)
    static constexpr int QRS = DH + 4;                       // q row stride in the end-of-kernel LDS copy
    static constexpr int FLUSH = 4 * 16 * QRS;               // q rows of the 4 row blocks
    static constexpr int MERGE = 4 * (NC * 16 * 64 + 2 * 64);  // odd-parity O, l, m of the 4 row blocks
    static constexpr int BIG00 = 4 * TILE > 8 * STAGE ? 4 * TILE : 8 * STAGE;  // two tile pairs in flight
    static constexpr int BIG0 = BIG00 > FLUSH ? BIG00 : FLUSH;
    static constexpr int BIG = BIG0 > MERGE ? BIG0 : MERGE;
    static constexpr int SMEM = BIG + 8 * 2 * CAP + 8 * 16;
    static_assert(RPW * 8 * 256 == 2 * 2 * BK * DH, "tile pair split into 1 KiB row copies");
    static_assert(DH % 256 == 0, "rows are copied in 1 KiB pieces");
};

template <int DH>
__device__ __forceinline__ void prefill_pair(const G4aPrefillParams& p) {
    using C = PairCfg<DH>;
    constexpr int BK = C::BK, KRS = C::KRS, RPW = C::RPW, NC = C::NC, QT = C::QT, CAP = C::CAP, SR = C::SR;
    __shared__ __attribute__((aligned(16))) float smem[C::SMEM];

    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rb = w & 3, par = w >> 2;
    const int g = lane >> 4, rl = lane & 15;
    const uint32_t kvh = blockIdx.y;
    const uint32_t qb = blockIdx.x * 8;
    const uint32_t qw = qb + 2 * rb;
    const uint32_t h0 = kvh * 8;
    const size_t row_stride = (size_t)p.Hkv * DH;
    const float* __restrict__ kbase = p.k + (size_t)kvh * DH;
    const float* __restrict__ vbase = p.v + (size_t)kvh * DH;
    uint32_t* const my_keys = reinterpret_cast<uint32_t*>(smem + C::BIG + w * 2 * CAP);
    float* const my_s = smem + C::BIG + w * 2 * CAP + CAP;
    float* const mtab = smem + C::BIG + 8 * 2 * CAP;  // [8 waves][16 rows]
    float* const my_m = mtab + w * 16;

    auto key_hi = [&](int64_t i) -> int32_t {
        const int64_t lim = (int64_t)p.q_pos0 + i - (int64_t)p.k_pos0 + 1;
        return (int32_t)(lim <= 0 ? 0 : (lim < (int64_t)p.S ? lim : (int64_t)p.S));
    };
    auto key_lo = [&](int64_t i) -> int32_t {
        if (p.window == 0) return 0;
        const int64_t lo = (int64_t)p.q_pos0 + i - (int64_t)p.k_pos0 - (int64_t)p.window + 1;
        return (int32_t)(lo <= 0 ? 0 : (lo < (int64_t)p.S ? lo : (int64_t)p.S));
    };
    auto prow = [&](uint32_t j) -> size_t { return p.ring_cap ? j % p.ring_cap : j; };

    const uint32_t qlast = min(qb + 7, p.T - 1);
    const int32_t wg_lo = key_lo(qb), wg_hi = key_hi(qlast);
    // tiles start on multiples of BK (the pre-split V quads are aligned to them);
    // keys of the first tile before wg_lo are masked like any invisible key
    const int32_t wg_base = wg_lo & ~(BK - 1);
    const uint32_t nt = wg_hi > wg_lo ? (uint32_t)((wg_hi - wg_base + BK - 1) / BK) : 0;
    const uint32_t nsteps = (nt + 1) / 2;
    // P.V from fp16 hi/lo splits of P and V unless some V value is outside their range
    const bool v16 = __builtin_amdgcn_readfirstlane(*p.vflag) != p.epoch;
    const float psc = v16 ? PF_PSCALE : 1.0f;  // scale of P, O and l (the f32 P.V path needs none)
    const bool wave_valid = qw < p.T;
    const int32_t w_lo = wave_valid ? key_lo(qw) : 0;
    const int32_t w_hi = wave_valid ? key_hi(min(qw + 1, p.T - 1)) : 0;
    const uint32_t myq = qw + (rl >> 3);
    const bool qvalid = myq < p.T;
    const int32_t my_lo = key_lo(myq), my_hi = qvalid ? key_hi(myq) : 0;
    // q rows in the B layout of v_mfma_f32_16x16x32_f16, split into fp16 hi/lo of
    // q * 2^-aq (aq per wave: its largest |q 2^-aq| in [2^14, 2^15)): lane (g, rl)
    // holds row rl's dims 32kb + 8g .. +7
    constexpr int QB = DH / 32;
    h8v qh[QB], ql[QB];
    float qsc;  // 2^aq
    {
        const float* qrow = p.q + ((size_t)min(myq, p.T - 1) * p.Hq + h0 + (rl & 7)) * DH + 8 * g;
        float4 qa[QB], qb4[QB];
        float mx = 0.0f;
#pragma unroll
        for (int kb = 0; kb < QB; ++kb) {
            qa[kb] = ld4(qrow + 32 * kb);
            qb4[kb] = ld4(qrow + 32 * kb + 4);
            mx = fmaxf(mx, absmax8(qa[kb], qb4[kb]));
        }
        const int aq = fp16_scale_exp(wave_max_scalar(mx));
        qsc = ldexpf(1.0f, aq);
#pragma unroll
        for (int kb = 0; kb < QB; ++kb) split8h(qa[kb], qb4[kb], aq, qh[kb], ql[kb]);
    }
    const float* __restrict__ ksbase = p.ksplit + (size_t)kvh * DH;
    static_assert(DH == 256, "the V quads of a tile are 16 1 KiB pieces");

    // Tile pair of step st (tiles 2st and 2st+1) goes to ring slot st&1, each
    // tile K (16 split rows of KRS 4-byte slots) then V (16 rows of DH floats,
    // or its 4 pre-split key quads), with global->LDS copies: 64 pieces of 1 KiB
    // per pair, RPW per wave. K rows past the last visible key re-read it.
    auto issue_pair = [&](uint32_t st) {
        float* const slot = smem + (st & 1) * 2 * C::TILE;
#pragma unroll
        for (int j = 0; j < RPW; ++j) {
            const int idx = w * RPW + j;                  // 1 KiB piece of the pair
            const int row = idx / (DH / 256), piece = idx % (DH / 256);
            const int tsel = row / (2 * BK), isv = (row / BK) & 1, kf = row % BK;
            const uint32_t tile0 = (uint32_t)wg_base + (2 * st + tsel) * BK;
            // keys outside the workgroup's visible range [wg_lo, wg_hi) read its nearest
            // visible row (their P is 0; an unwritten slot could hold NaN)
            const uint32_t key = min(max(tile0 + kf, (uint32_t)wg_lo), (uint32_t)wg_hi - 1u);
            // K rows come from the split copy (row key - split0); V from the split
            // quads (piece kf: quad kf/4, its 1 KiB piece kf%4) or the cache rows
            const uint32_t ks = min(key - min(key, p.split0), p.split_n - 1u);
            const uint32_t qd = min(tile0 - min(tile0, p.split0), p.split_n - (uint32_t)BK) / 4 + (kf >> 2);
            const float* src = !isv ? ksbase + (size_t)ks * row_stride + 256 * piece + 4 * lane
                               : v16 ? p.vsplit + ((size_t)qd * p.Hkv + kvh) * 4 * DH + 256 * (kf & 3) + 4 * lane
                                     : vbase + prow(key) * row_stride + 256 * piece + 4 * lane;
            float* dst = slot + tsel * C::TILE + (isv ? BK * KRS + kf * DH : kf * KRS) + 256 * piece;
            copy16_to_lds(src, dst);
        }
    };

    float m_run = NEG_INF, m_ref = NEG_INF, l_part = 0.0f;
    f4v O[NC][4];
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int e = 0; e < 4; ++e) O[c][e] = f4v{0.0f, 0.0f, 0.0f, 0.0f};
    int cnt = 0;

    auto publish_m = [&](float mref) {
        if (g == 0) my_m[rl] = mref;
        wave_sync();
    };
    auto compact = [&]() {
        int nc = 0;
        for (int base = 0; base < cnt; base += 64) {
            const int e = base + lane;
            const bool has = e < cnt;
            const uint32_t pk = has ? my_keys[e] : 0u;
            const float sa = has ? my_s[e] : 0.0f;
            const bool keep = has && sa > my_m[pk >> 28] - p.tau;
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
    // Exact correction of the recorded candidates against the published
    // maxima (the scale O and l are held at), 64 candidates per pass, lane =
    // candidate: its exact dot in the reference's order, then
    // delta = e^{s_exact - m} - e^{s_approx - m} added to its row's l, then
    // O += Delta V on the matrix cores. The in-loop form reads q and k rows
    // straight from memory 16 dims at a time (few registers; it only runs when
    // a list overflows).
    auto delta_and_l = [&](int base, bool has, uint32_t rho, float dot, int e) -> float {
        float delta = 0.0f;
        if (has) {
            const float m = my_m[rho];
            delta = psc * (expf(dot * p.scale - m) - pf_exp(my_s[e] - m));
        }
        const int nb = min(64, cnt - base);
        for (int i = 0; i < nb; ++i) {
            const float di = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(delta), i));
            const uint32_t ri = __builtin_amdgcn_readlane(rho, i);
            if (lane == (int)ri) l_part += di;
        }
        return delta;
    };
    // O += Delta V with Delta[row][cand] = delta if the candidate belongs to the
    // row, else 0: K-step s of the 16x16x4 chain takes candidates 4s .. 4s+3
    // (lane l: A = Delta[l%16][4s + l/16], B = V[key(4s + l/16)][64c + 4(l%16) + e]),
    // V rows DEPTH K-steps ahead (DEPTH 4 at the end of the kernel, 2 in the
    // loop where registers are short).
    auto load_v = [&](int s4, uint32_t kap, float4 (&vb)[NC]) {
        const uint32_t kk = (uint32_t)__shfl((int)kap, s4 + g, 64);
        const float* vrow = vbase + prow(kk) * row_stride + 4 * rl;
#pragma unroll
        for (int c = 0; c < NC; ++c) vb[c] = ld4(vrow + 64 * c);
    };
    // With lc, the same A (Delta of 4 candidates by row) times a block of ones also
    // accumulates each row's l correction: lc register r of lane (g, rl) is row 4g + r.
    auto apply_v = [&](int s4, float delta, uint32_t rho, const float4 (&vb)[NC], f4v* lc) {
        const float dl = __shfl(delta, s4 + g, 64);
        const uint32_t rr = (uint32_t)__shfl((int)rho, s4 + g, 64);
        const float a = rr == (uint32_t)rl ? dl : 0.0f;
        if (lc) *lc = __builtin_amdgcn_mfma_f32_16x16x4f32(a, 1.0f, *lc, 0, 0, 0);
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            O[c][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, vb[c].x, O[c][0], 0, 0, 0);
            O[c][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, vb[c].y, O[c][1], 0, 0, 0);
            O[c][2] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, vb[c].z, O[c][2], 0, 0, 0);
            O[c][3] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, vb[c].w, O[c][3], 0, 0, 0);
        }
    };
    auto correct_o2 = [&](int base, float delta, uint32_t rho, uint32_t kap) {
        __builtin_amdgcn_sched_barrier(0);
        const int nb = min(64, cnt - base);
        float4 vA[NC], vB[NC];
        auto step = [&](int s4, float4 (&vb)[NC]) {
            if (s4 < nb) {
                apply_v(s4, delta, rho, vb, nullptr);
                if (s4 + 8 < nb) load_v(s4 + 8, kap, vb);
            }
        };
        load_v(0, kap, vA);
        if (4 < nb) load_v(4, kap, vB);
        for (int s4 = 0; s4 < nb; s4 += 8) {
            step(s4, vA);
            step(s4 + 4, vB);
        }
    };
    auto correct_o4 = [&](int base, float delta, uint32_t rho, uint32_t kap, f4v* lc) {
        __builtin_amdgcn_sched_barrier(0);
        const int nb = min(64, cnt - base);
        float4 vA[NC], vB[NC], vC[NC], vD[NC];
        auto step = [&](int s4, float4 (&vb)[NC]) {
            if (s4 < nb) {
                apply_v(s4, delta, rho, vb, lc);
                if (s4 + 16 < nb) load_v(s4 + 16, kap, vb);
            }
        };
        load_v(0, kap, vA);
        if (4 < nb) load_v(4, kap, vB);
        if (8 < nb) load_v(8, kap, vC);
        if (12 < nb) load_v(12, kap, vD);
        for (int s4 = 0; s4 < nb; s4 += 16) {
            step(s4, vA);
            step(s4 + 4, vB);
            step(s4 + 8, vC);
            step(s4 + 12, vD);
        }
    };
    auto flush_light = [&]() {
        for (int base = 0; base < cnt; base += 64) {
            const int e = base + lane;
            const bool has = e < cnt;
            const uint32_t pk = has ? my_keys[e] : 0u;
            const uint32_t rho = pk >> 28, kap = has ? (pk & 0x0fffffffu) : (uint32_t)wg_lo;
            const float* qrow = p.q + ((size_t)min(qw + (rho >> 3), p.T - 1) * p.Hq + h0 + (rho & 7)) * DH;
            const float* krow = kbase + prow(kap) * row_stride;
            float dot = 0.0f;
#pragma unroll 1
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
            const float delta = delta_and_l(base, has, rho, dot, e);
            correct_o2(base, delta, rho, kap);
        }
        cnt = 0;
    };
    // End-of-kernel form, one candidate per lane (64 per batch). Lane e runs
    // candidate e's sequential dot: its q row from LDS (qlds, copied from the
    // registers), its k row straight from memory (the keys of this workgroup
    // were just streamed, so they sit in L2), 64 dims per register chunk with
    // the next chunk already loading. Delta V then goes through correct_o4.
    auto flush_rows = [&](const float* qlds) {
        constexpr int QRS = C::QRS, NCH = DH / 64;
        static_assert(NCH % 2 == 0, "chunks are processed in pairs");
        for (int base = 0; base < cnt; base += 64) {
            const int e = base + lane;
            const bool has = e < cnt;
            const uint32_t pk = has ? my_keys[e] : 0u;
            const uint32_t rho = pk >> 28, kap = has ? (pk & 0x0fffffffu) : (uint32_t)wg_lo;
            const float* const krow = kbase + prow(kap) * row_stride;
            const float* const qv = qlds + rho * QRS;
            float4 kA[16], kB[16];
            auto load_chunk = [&](int ch, float4 (&kc)[16]) {
#pragma unroll
                for (int u = 0; u < 16; ++u) kc[u] = ld4(krow + 64 * ch + 4 * u);
            };
            float dot = 0.0f;
            auto dot_chunk = [&](int ch, const float4 (&kc)[16]) {
#pragma unroll
                for (int u = 0; u < 16; ++u) {
                    const float4 q4 = *reinterpret_cast<const float4*>(qv + 64 * ch + 4 * u);
                    dot = dot + q4.x * kc[u].x;
                    dot = dot + q4.y * kc[u].y;
                    dot = dot + q4.z * kc[u].z;
                    dot = dot + q4.w * kc[u].w;
                }
            };
            load_chunk(0, kA);
            load_chunk(1, kB);
#pragma unroll
            for (int ch = 0; ch < NCH; ch += 2) {
                dot_chunk(ch, kA);
                if (ch + 2 < NCH) load_chunk(ch + 2, kA);
                dot_chunk(ch + 1, kB);
                if (ch + 3 < NCH) load_chunk(ch + 3, kB);
            }
            float delta = 0.0f;
            if (has) {
                const float m = my_m[rho];
                delta = psc * (expf(dot * p.scale - m) - pf_exp(my_s[e] - m));
            }
            f4v lc = f4v{0.0f, 0.0f, 0.0f, 0.0f};
            correct_o4(base, delta, rho, kap, &lc);
            // row rl's l correction sits in register rl%4 of lanes 16*(rl/4) ..; lanes g == 0 own l
            const int src = 16 * (rl >> 2);
            const float c0 = __shfl(lc[0], src, 64), c1 = __shfl(lc[1], src, 64);
            const float c2 = __shfl(lc[2], src, 64), c3 = __shfl(lc[3], src, 64);
            const int rr = rl & 3;
            const float cl = rr == 0 ? c0 : (rr == 1 ? c1 : (rr == 2 ? c2 : c3));
            if (g == 0) l_part += cl;
        }
        cnt = 0;
    };

    if (nsteps > 0) issue_pair(0);
    for (uint32_t st = 0; st < nsteps; ++st) {
        wait_vm<0>();   // this wave's copies of pair st have landed (nothing else is in flight)
        barrier_lds();  // every wave's have; every wave is done with slot (st+1)&1 (pair st-1)
        if (st + 1 < nsteps) issue_pair(st + 1);
        const uint32_t t = 2 * st + par;
        const int32_t t0 = wg_base + (int32_t)(t * BK);
        if (!wave_valid || t >= nt || t0 >= w_hi || t0 + BK <= w_lo) continue;
        const float* Kt = smem + (st & 1) * 2 * C::TILE + par * C::TILE;
        const float* Vt = Kt + BK * KRS;

        // score estimate S^T = K Q^T from the scaled fp16 splits: Khi Qhi + Klo Qhi + Khi Qlo
        // (error ~2^-21 relative per term), three independent accumulators, then the
        // wave's and the tile's powers of two. Lane (g, rl) reads key rl's 8-dim block
        // 4kb + g: hi then lo, 16 bytes each.
        f4v SA[3];
#pragma unroll
        for (int a = 0; a < 3; ++a) SA[a] = f4v{0.0f, 0.0f, 0.0f, 0.0f};
        const float* kr = Kt + rl * KRS + 8 * g;
#pragma unroll
        for (int kb = 0; kb < QB; ++kb) {
            const h8v khi = *reinterpret_cast<const h8v*>(kr + 32 * kb);
            const h8v klo = *reinterpret_cast<const h8v*>(kr + 32 * kb + 4);
            SA[0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(khi, qh[kb], SA[0], 0, 0, 0);
            SA[1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(klo, qh[kb], SA[1], 0, 0, 0);
            SA[2] = __builtin_amdgcn_mfma_f32_16x16x32_f16(khi, ql[kb], SA[2], 0, 0, 0);
        }
        const f4v S = (SA[0] + SA[1]) + SA[2];
        const float sc = qsc * tile_kscale(p, kvh, t0);  // a power of two: exact
        float s[4];
        bool vis[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int32_t j = t0 + 4 * g + r;
            vis[r] = j >= my_lo && j < my_hi;
            s[r] = vis[r] ? (S[r] * sc) * p.scale : NEG_INF;
        }
        float tm = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
        tm = g4a_col_max4(tm);
        const float mn = fmaxf(m_run, tm);

        // candidates: count first, make room if needed, then record
        bool cand[4];
        uint64_t bal[4];
        int nnew = 0;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            cand[r] = vis[r] && s[r] > mn - p.tau;
            bal[r] = ballot(cand[r]);
            nnew += __builtin_popcountll(bal[r]);
        }
        if (cnt + nnew > CAP) {
            publish_m(mn);
            compact();
            if (cnt + nnew > CAP) {
                publish_m(m_ref);
                flush_light();
            }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            if (cand[r]) {
                const int pos = cnt + lanes_below(bal[r]);
                my_keys[pos] = ((uint32_t)rl << 28) | (uint32_t)(t0 + 4 * g + r);
                my_s[pos] = s[r];
            }
            cnt += __builtin_popcountll(bal[r]);
        }
        m_run = mn;

        if (ballot(mn > m_ref + PF_RESCALE) != 0) {
            const float corr = (m_ref == NEG_INF) ? 0.0f : expf(m_ref - mn);
            l_part *= corr;
            m_ref = mn;
            const f4v cr = f4v{__shfl(corr, 4 * g + 0, 64), __shfl(corr, 4 * g + 1, 64), __shfl(corr, 4 * g + 2, 64),
                               __shfl(corr, 4 * g + 3, 64)};
#pragma unroll
            for (int c = 0; c < NC; ++c)
#pragma unroll
                for (int e = 0; e < 4; ++e) O[c][e] *= cr;
        }

        float pr[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) pr[r] = vis[r] ? psc * pf_exp(s[r] - m_ref) : 0.0f;
        l_part += (pr[0] + pr[1]) + (pr[2] + pr[3]);
        if (v16) {
            // O += P V on v_mfma_f32_16x16x16_f16: Phi Vhi + Phi Vlo + Plo Vhi (relative error
            // ~2^-21). Lane (g, rl) gives A = P[row rl][keys 4g .. 4g+3] (its pr) and
            // B = V[keys 4g .. 4g+3][dim 64c + 4rl + e]: quad g's 16 bytes (4 hi, 4 lo).
            h4v ah, al;
#pragma unroll
            for (int r = 0; r < 4; ++r) split16(pr[r], ah, al, r);
            const float* const vq = Vt + g * 4 * DH + 4 * rl;
#pragma unroll
            for (int c = 0; c < NC; ++c)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float4 raw = *reinterpret_cast<const float4*>(vq + 4 * 16 * (4 * c + e));
                    h4v bh, bl;
                    __builtin_memcpy(&bh, &raw.x, 8);
                    __builtin_memcpy(&bl, &raw.z, 8);
                    O[c][e] = __builtin_amdgcn_mfma_f32_16x16x16f16(ah, bh, O[c][e], 0, 0, 0);
                    O[c][e] = __builtin_amdgcn_mfma_f32_16x16x16f16(ah, bl, O[c][e], 0, 0, 0);
                    O[c][e] = __builtin_amdgcn_mfma_f32_16x16x16f16(al, bh, O[c][e], 0, 0, 0);
                }
            continue;
        }
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

    // ---- end: compact against the maximum over both parities, correct, merge ----
    wait_vm<0>();
    // the f32 q rows of this row block (row rl: query qw + rl/8, head rl%8) for the
    // exact rescoring load from memory while the lists are compacted
    float4 qf[QT];
    if (par == 0) {
        const float* qrow = p.q + ((size_t)min(myq, p.T - 1) * p.Hq + h0 + (rl & 7)) * DH + 4 * g;
#pragma unroll
        for (int t = 0; t < QT; ++t) qf[t] = ld4(qrow + 16 * t);
    }
    publish_m(m_run);
    __syncthreads();  // tile buffers free; both parities' maxima published
    {
        const float mo = mtab[(w ^ 4) * 16 + rl];  // the other parity's running maximum of row rl
        publish_m(fmaxf(m_run, mo));
    }
    float* const qlds = smem + rb * 16 * C::QRS;
    if (wave_valid) compact();
    if (par == 0) {
#pragma unroll
        for (int t = 0; t < QT; ++t) *reinterpret_cast<float4*>(qlds + rl * C::QRS + 16 * t + 4 * g) = qf[t];
    }
    publish_m(m_ref);
    __syncthreads();  // the q rows are visible
    if (wave_valid) flush_rows(qlds);
    float l = l_part;
    l = g4a_col_sum4(l);
    __syncthreads();  // staging done: the merge area overlays it
    float* const mo_ = smem + rb * (NC * 16 * 64 + 2 * 64);  // odd parity -> even parity, per row block
    if (par == 1) {
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int r = 0; r < 4; ++r) mo_[((c * 4 + e) * 4 + r) * 64 + lane] = O[c][e][r];
        mo_[NC * 16 * 64 + lane] = l;
        mo_[NC * 16 * 64 + 64 + lane] = m_ref;
    }
    __syncthreads();
    if (par == 1 || !wave_valid) return;
    {
        // rows: lane (g, rl) holds l and m of row rl; O register r of lane (g, rl) is row 4g + r
        const float l1 = mo_[NC * 16 * 64 + lane];
        const float m1 = mo_[NC * 16 * 64 + 64 + lane];
        const float M = fmaxf(m_ref, m1);
        const float e0 = (m_ref == NEG_INF) ? 0.0f : expf(m_ref - M);
        const float e1 = (m1 == NEG_INF) ? 0.0f : expf(m1 - M);
        const float lt = l * e0 + l1 * e1;
        const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
        float a0[4], a1[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float iv = __shfl(inv, 4 * g + r, 64);
            a0[r] = __shfl(e0, 4 * g + r, 64) * iv;
            a1[r] = __shfl(e1, 4 * g + r, 64) * iv;
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = 4 * g + r;
            const uint32_t qi = qw + (row >> 3);
            if (qi >= p.T) continue;
            float* orow = p.out + ((size_t)qi * p.Hq + h0 + (row & 7)) * DH + 4 * rl;
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                float4 o;
                o.x = O[c][0][r] * a0[r] + mo_[((c * 4 + 0) * 4 + r) * 64 + lane] * a1[r];
                o.y = O[c][1][r] * a0[r] + mo_[((c * 4 + 1) * 4 + r) * 64 + lane] * a1[r];
                o.z = O[c][2][r] * a0[r] + mo_[((c * 4 + 2) * 4 + r) * 64 + lane] * a1[r];
                o.w = O[c][3][r] * a0[r] + mo_[((c * 4 + 3) * 4 + r) * 64 + lane] * a1[r];
                *reinterpret_cast<float4*>(orow + 64 * c) = o;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Head-dim 512 prefill with two waves per SIMD. The split q rows and the O
// accumulator of a 16-row block take 128 registers each at head_dim 512, more
// than two waves per SIMD can hold, so a row block is shared by two waves that
// split the head dim: wave w owns rows 16*(w%4) .. +15 (2 queries x 8 heads)
// and dims 256*(w/4) .. +255. Per 16-key tile each wave computes its half of
// the score estimate (scaled fp16 hi/lo splits), the pair adds the halves through LDS
// in a fixed order (both waves then hold bit-identical scores, maxima,
// candidate lists and l), and each wave runs P.V (fp16 hi/lo splits) and the
// exact corrections for its own 256 output columns. Tiles stream into a 2-slot
// LDS ring with global->LDS copies, one tile ahead.
// Causal balance: a query block with more key tiles than the average runs as
// two workgroups over the two halves of its tiles (p.nbig, see G4aPrefillParams);
// each writes its partial (O, l, m) and prefill_merge combines them.
template <int DH>
struct DsplitCfg {
    static constexpr int BK = 16;
    static constexpr int HD = DH / 2;                 // dims per wave
    static constexpr int KRS = DH + 4;                // K split row stride in LDS (4-byte slots)
    static constexpr int TILE = BK * KRS + BK * DH;   // K rows then V (4 split key quads, or 16 rows)
    static constexpr int NPR = DH / 256;              // 1 KiB pieces per row
    static constexpr int NCH = HD / 64;               // O column groups per wave (x4 MFMA blocks)
    static constexpr int QBH = HD / 32;               // 32-dim K-blocks of a wave's partial score
    static constexpr int CAP = 256;                   // candidate entries per wave
    static constexpr int XS = 8 * 64 * 4;             // partial-score exchange [wave][lane][4]
    static constexpr int STAGE = (64 + 16) * 36;      // per-wave staging floats at the end (in the tile buffers)
    static constexpr int SMEM = 2 * TILE + XS + 8 * 2 * CAP + 8 * 16 + 8;  // ..., pair flags
    static constexpr int PART_WAVE = NCH * 16 * 64 + 2 * 16;  // a wave's partial: O, then l and m of its rows
    static_assert(8 * STAGE <= 2 * TILE, "the end-of-kernel staging areas fit in the tile buffers");
    static_assert(BK * NPR == 8 * 4, "a tile is 64 pieces of 1 KiB: 8 per wave");
    static_assert(SMEM * 4 <= 160 * 1024, "LDS budget of a CU");
};

template <int DH>
__device__ __forceinline__ void prefill_dsplit(const G4aPrefillParams& p) {
    using C = DsplitCfg<DH>;
    constexpr int BK = C::BK, HD = C::HD, KRS = C::KRS, NPR = C::NPR, NCH = C::NCH, QBH = C::QBH, CAP = C::CAP;
    __shared__ __attribute__((aligned(16))) float smem[C::SMEM];

    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rb = w & 3, dhf = w >> 2;
    const int g = lane >> 4, rl = lane & 15;
    const uint32_t kvh = blockIdx.y;
    // work item: the two halves of each of the last nbig query blocks, then the
    // other blocks, heaviest (latest queries) first
    const uint32_t NB = (p.T + 7) / 8;
    const uint32_t item = blockIdx.x;
    const bool split = item < 2 * p.nbig;
    const uint32_t half_id = split ? (item & 1u) : 0u;
    const uint32_t blk = split ? NB - 1 - item / 2 : NB - 1 - p.nbig - (item - 2 * p.nbig);
    const uint32_t qb = blk * 8;
    const uint32_t qw = qb + 2 * rb;
    const uint32_t h0 = kvh * 8;
    const size_t row_stride = (size_t)p.Hkv * DH;
    const float* __restrict__ kbase = p.k + (size_t)kvh * DH;
    const float* __restrict__ vbase = p.v + (size_t)kvh * DH;
    float4* const xs = reinterpret_cast<float4*>(smem + 2 * C::TILE);            // [8 waves][64 lanes]
    uint32_t* const my_keys = reinterpret_cast<uint32_t*>(smem + 2 * C::TILE + C::XS + w * 2 * CAP);
    float* const my_s = smem + 2 * C::TILE + C::XS + w * 2 * CAP + CAP;
    float* const my_m = smem + 2 * C::TILE + C::XS + 8 * 2 * CAP + w * 16;
    // end-of-kernel exchange of the pair's dots: flags (one per wave) in their own
    // slots, set to 0 before the first barrier; the dots over the partial-score
    // exchange area, which the tile loop no longer uses by then
    uint32_t* const pair_flags = reinterpret_cast<uint32_t*>(smem + 2 * C::TILE + C::XS + 8 * 2 * CAP + 8 * 16);
    if (lane == 0) pair_flags[w] = 0u;
    float* const pair_dots = smem + 2 * C::TILE + (w & 3) * 128;  // [2 batch parities][64]

    auto key_hi = [&](int64_t i) -> int32_t {
        const int64_t lim = (int64_t)p.q_pos0 + i - (int64_t)p.k_pos0 + 1;
        return (int32_t)(lim <= 0 ? 0 : (lim < (int64_t)p.S ? lim : (int64_t)p.S));
    };
    auto key_lo = [&](int64_t i) -> int32_t {
        if (p.window == 0) return 0;
        const int64_t lo = (int64_t)p.q_pos0 + i - (int64_t)p.k_pos0 - (int64_t)p.window + 1;
        return (int32_t)(lo <= 0 ? 0 : (lo < (int64_t)p.S ? lo : (int64_t)p.S));
    };
    auto prow = [&](uint32_t j) -> size_t { return p.ring_cap ? j % p.ring_cap : j; };

    const uint32_t qlast = min(qb + 7, p.T - 1);
    const int32_t wg_lo = key_lo(qb), wg_hi = key_hi(qlast);
    // tiles start on multiples of BK (the pre-split V quads are aligned to them);
    // keys of the first tile before wg_lo are masked like any invisible key
    const int32_t wg_base = wg_lo & ~(BK - 1);
    const uint32_t nt = wg_hi > wg_lo ? (uint32_t)((wg_hi - wg_base + BK - 1) / BK) : 0;
    // this workgroup's tiles [t_begin, t_end): all of them, or one half of a split block
    const uint32_t t_begin = split && half_id ? nt / 2 : 0u;
    const uint32_t t_end = split && !half_id ? nt / 2 : nt;
    const bool v16 = __builtin_amdgcn_readfirstlane(*p.vflag) != p.epoch;
    const float psc = v16 ? PF_PSCALE : 1.0f;  // scale of P, O and l (the f32 P.V path needs none)
    const bool wave_valid = qw < p.T;
    const int32_t w_lo = wave_valid ? key_lo(qw) : 0;
    const int32_t w_hi = wave_valid ? key_hi(min(qw + 1, p.T - 1)) : 0;
    const uint32_t myq = qw + (rl >> 3);
    const bool qvalid = myq < p.T;
    const int32_t my_lo = key_lo(myq), my_hi = qvalid ? key_hi(myq) : 0;
    // this wave's half of the q rows in the B layout of v_mfma_f32_16x16x32_f16, split
    // into fp16 hi/lo of q * 2^-aq (aq per wave: its largest |q 2^-aq| in
    // [2^14, 2^15)): lane (g, rl) holds row rl's dims HD*dhf + 32kb + 8g .. +7
    h8v qh[QBH], ql[QBH];
    float qsc;  // 2^aq
    {
        const float* qrow = p.q + ((size_t)min(myq, p.T - 1) * p.Hq + h0 + (rl & 7)) * DH + HD * dhf + 8 * g;
        float4 qa[QBH], qb4[QBH];
        float mx = 0.0f;
#pragma unroll
        for (int kb = 0; kb < QBH; ++kb) {
            qa[kb] = ld4(qrow + 32 * kb);
            qb4[kb] = ld4(qrow + 32 * kb + 4);
            mx = fmaxf(mx, absmax8(qa[kb], qb4[kb]));
        }
        const int aq = fp16_scale_exp(wave_max_scalar(mx));
        qsc = ldexpf(1.0f, aq);
#pragma unroll
        for (int kb = 0; kb < QBH; ++kb) split8h(qa[kb], qb4[kb], aq, qh[kb], ql[kb]);
    }
    const float* __restrict__ ksbase = p.ksplit + (size_t)kvh * DH;

    // Tile t (keys tile0 .. tile0+BK-1, tile0 = wg_base + t*BK) into buffer t&1:
    // waves 0-3 copy K split rows 4w .. 4w+3, waves 4-7 V (key quad w-4, or raw
    // rows 4(w-4) .. +3). K rows past the last visible key re-read it.
    auto issue_tile = [&](uint32_t t) {
        float* const buf = smem + (t & 1) * C::TILE;
        const uint32_t tile0 = (uint32_t)wg_base + t * BK;
        const uint32_t last = (uint32_t)wg_hi - 1u;
        if (w < 4) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int kf = 4 * w + i;
                const uint32_t key = min(tile0 + kf, last);
                const uint32_t ks = min(key - min(key, p.split0), p.split_n - 1u);
                const float* src = ksbase + (size_t)ks * row_stride + 4 * lane;
#pragma unroll
                for (int pc = 0; pc < NPR; ++pc) copy16_to_lds(src + 256 * pc, buf + kf * KRS + 256 * pc);
            }
        } else if (v16) {
            const uint32_t qd = min(tile0 - min(tile0, p.split0), p.split_n - (uint32_t)BK) / 4 + (w - 4);
            const float* src = p.vsplit + ((size_t)qd * p.Hkv + kvh) * 4 * DH + 4 * lane;
            float* const dst = buf + BK * KRS + (w - 4) * 4 * DH;
#pragma unroll
            for (int pc = 0; pc < 4 * NPR; ++pc) copy16_to_lds(src + 256 * pc, dst + 256 * pc);
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int kf = 4 * (w - 4) + i;
                // keys before the workgroup's first visible key read its row (P is 0 there)
                const float* src = vbase + prow(min(max(tile0 + kf, (uint32_t)wg_lo), last)) * row_stride + 4 * lane;
#pragma unroll
                for (int pc = 0; pc < NPR; ++pc) copy16_to_lds(src + 256 * pc, buf + BK * KRS + kf * DH + 256 * pc);
            }
        }
    };

    float m_run = NEG_INF, m_ref = NEG_INF, l_part = 0.0f;
    f4v O[NCH][4];
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
        for (int e = 0; e < 4; ++e) O[c][e] = f4v{0.0f, 0.0f, 0.0f, 0.0f};
    int cnt = 0;  // wave-uniform number of recorded candidates (the same in both waves of a pair)

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
            const bool keep = has && sa > my_m[pk >> 28] - p.tau;
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
    // delta = e^{s_exact - m} - e^{s_approx - m} of candidate e against its row's
    // published maximum, added to that row's l.
    auto delta_and_l = [&](int base, bool has, uint32_t rho, float dot, int e) -> float {
        float delta = 0.0f;
        if (has) {
            const float m = my_m[rho];
            delta = psc * (expf(dot * p.scale - m) - pf_exp(my_s[e] - m));
        }
        const int nb = min(64, cnt - base);
        for (int i = 0; i < nb; ++i) {
            const float di = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(delta), i));
            const uint32_t ri = __builtin_amdgcn_readlane(rho, i);
            if (lane == (int)ri) l_part += di;
        }
        return delta;
    };
    // O += Delta V for this wave's columns: K-step s of the 16x16x4 chain takes
    // candidates 4s .. 4s+3 (lane l: A = Delta[l%16][4s + l/16], B = V[key(4s + l/16)]
    // [HD*dhf + 64c + 4(l%16) + e]); V rows straight from memory, two K-steps ahead.
    auto correct_o = [&](int base, float delta, uint32_t rho, uint32_t kap) {
        const int nb = min(64, cnt - base);
        auto load_v = [&](int s4, float4 (&vb)[NCH]) {
            const uint32_t kk = (uint32_t)__shfl((int)kap, s4 + g, 64);
            const float* vrow = vbase + prow(kk) * row_stride + HD * dhf + 4 * rl;
#pragma unroll
            for (int c = 0; c < NCH; ++c) vb[c] = ld4(vrow + 64 * c);
        };
        auto apply_v = [&](int s4, const float4 (&vb)[NCH]) {
            const float dl = __shfl(delta, s4 + g, 64);
            const uint32_t rr = (uint32_t)__shfl((int)rho, s4 + g, 64);
            const float a = rr == (uint32_t)rl ? dl : 0.0f;
#pragma unroll
            for (int c = 0; c < NCH; ++c) {
                O[c][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, vb[c].x, O[c][0], 0, 0, 0);
                O[c][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, vb[c].y, O[c][1], 0, 0, 0);
                O[c][2] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, vb[c].z, O[c][2], 0, 0, 0);
                O[c][3] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, vb[c].w, O[c][3], 0, 0, 0);
            }
        };
        float4 vA[NCH], vB[NCH];
        load_v(0, vA);
        if (4 < nb) load_v(4, vB);
        for (int s4 = 0; s4 < nb; s4 += 8) {
            apply_v(s4, vA);
            if (s4 + 8 < nb) load_v(s4 + 8, vA);
            if (s4 + 4 < nb) {
                apply_v(s4 + 4, vB);
                if (s4 + 12 < nb) load_v(s4 + 12, vB);
            }
        }
    };
    // In-loop correction (a list overflowed): exact dots with q and k rows straight
    // from memory, 16 dims per step (the split q rows stay live in registers).
    auto flush_light = [&]() {
        for (int base = 0; base < cnt; base += 64) {
            const int e = base + lane;
            const bool has = e < cnt;
            const uint32_t pk = has ? my_keys[e] : 0u;
            const uint32_t rho = pk >> 28, kap = has ? (pk & 0x0fffffffu) : (uint32_t)wg_lo;
            const float* qrow = p.q + ((size_t)min(qw + (rho >> 3), p.T - 1) * p.Hq + h0 + (rho & 7)) * DH;
            const float* krow = kbase + prow(kap) * row_stride;
            float dot = 0.0f;
#pragma unroll 1
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
            const float delta = delta_and_l(base, has, rho, dot, e);
            correct_o(base, delta, rho, kap);
        }
        cnt = 0;
    };
    // End-of-kernel correction. The two waves of a pair hold the same candidate
    // list, so each computes the exact dots of one half of every batch of 64
    // (wave dhf: candidates base + 32 dhf + j, lane j) and the halves meet in LDS:
    // 32-dim segments of the wave's 16 q rows and of its 32 candidates' k rows are
    // staged in its LDS area with coalesced reads (two segments in flight), each
    // lane runs its candidate's sequential dot from LDS, and the dots go to the
    // pair's exchange slots (double-buffered by batch parity) with a flag. Every
    // dot is the same sequence of operations whichever wave computes it. The wait
    // for the partner's flag is bounded: past the bound the wave computes the
    // partner's half itself, so a wave never waits on a flag forever.
    auto flush_staged = [&](float* stage, float* xch, uint32_t* flags) {
        constexpr int SR = 36;
        constexpr int NSEG = DH / 32;
        constexpr int NC = 32;                 // candidates per wave and batch
        float* const kst = stage;              // [NC candidates][SR]
        float* const qst = stage + NC * SR;    // [16 rows][SR]
        const int seg = lane >> 3, part = lane & 7;
        const float* const q0 = p.q + ((size_t)min(qw, p.T - 1) * p.Hq + h0 + seg) * DH + 4 * part;
        const float* const q1 = p.q + ((size_t)min(qw + 1, p.T - 1) * p.Hq + h0 + seg) * DH + 4 * part;
        uint32_t* const my_flag = flags + w;
        const uint32_t* const other_flag = flags + (w ^ 4);
        uint32_t batch = 0;
        bool solo = false;
        for (int base = 0; base < cnt; base += 64, ++batch) {
            const int e = base + lane;
            const bool has = e < cnt;
            const uint32_t pk = has ? my_keys[e] : 0u;
            const uint32_t rho = pk >> 28, kap = has ? (pk & 0x0fffffffu) : (uint32_t)wg_lo;
            // exact dots of candidates base + NC * hs + (lane % NC), read back from the lanes that hold them
            auto dots_of_half = [&](int hs) -> float {
                const float* krow[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t ki = (uint32_t)__shfl((int)kap, NC * hs + 8 * i + seg, 64);
                    krow[i] = kbase + prow(ki) * row_stride + 4 * part;
                }
                const uint32_t rc = (uint32_t)__shfl((int)rho, NC * hs + (lane & (NC - 1)), 64);
                float4 kA[4], qA[2], kB[4], qB[2];
                auto load_seg = [&](int sg, float4 (&kk)[4], float4 (&qq)[2]) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) kk[i] = ld4(krow[i] + 32 * sg);
                    qq[0] = ld4(q0 + 32 * sg);
                    qq[1] = ld4(q1 + 32 * sg);
                };
                float dot = 0.0f;
                // prefetch (a constant at every call site) reloads kk, qq with segment sg + 2
                auto consume = [&](int sg, float4 (&kk)[4], float4 (&qq)[2], bool prefetch) {
                    wave_sync();  // the previous segment's reads are done
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        *reinterpret_cast<float4*>(kst + (8 * i + seg) * SR + 4 * part) = kk[i];
                    *reinterpret_cast<float4*>(qst + seg * SR + 4 * part) = qq[0];
                    *reinterpret_cast<float4*>(qst + (8 + seg) * SR + 4 * part) = qq[1];
                    if (prefetch) load_seg(sg + 2, kk, qq);
                    wave_sync();
                    const float* kr = kst + (lane & (NC - 1)) * SR;  // lanes NC.. repeat lanes 0 .. NC-1
                    const float* qv = qst + rc * SR;
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        const float4 k4 = *reinterpret_cast<const float4*>(kr + 4 * u);
                        const float4 q4 = *reinterpret_cast<const float4*>(qv + 4 * u);
                        dot = dot + q4.x * k4.x;
                        dot = dot + q4.y * k4.y;
                        dot = dot + q4.z * k4.z;
                        dot = dot + q4.w * k4.w;
                    }
                };
                static_assert(NSEG % 2 == 0 && NSEG >= 4, "segments are consumed in pairs");
                load_seg(0, kA, qA);
                load_seg(1, kB, qB);
                // the last pair is peeled off so the loop's loads are unconditional: the
                // waits before each store then count only the older segment's loads
#pragma unroll 1
                for (int sg = 0; sg < NSEG - 2; sg += 2) {
                    consume(sg, kA, qA, true);
                    consume(sg + 1, kB, qB, true);
                }
                consume(NSEG - 2, kA, qA, false);
                consume(NSEG - 1, kB, qB, false);
                return dot;
            };
            float* const slot = xch + (batch & 1u) * 64;
            const float mine = dots_of_half(dhf);
            bool seen = false;
            if (!solo) {
                if (lane < NC) slot[NC * dhf + lane] = mine;
                // publish this batch's half (the exchange writes above are ordered before the flag)
                __hip_atomic_store(my_flag, batch + 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
                for (int spin = 0; spin < PF_PAIR_SPIN; ++spin) {
                    if (__hip_atomic_load(other_flag, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) >= batch + 1u) {
                        seen = true;
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
                }
            }
            float dot;
            if (seen) {
                dot = slot[lane];
            } else {
                // no half from the partner in time: this wave computes both from here on and
                // leaves the exchange slots alone (the partner may still read its last half)
                solo = true;
                const float theirs = dots_of_half(dhf ^ 1);
                const float a = __shfl(mine, lane & (NC - 1), 64);
                const float b = __shfl(theirs, lane & (NC - 1), 64);
                dot = (lane >> 5) == dhf ? a : b;
            }
            const float delta = delta_and_l(base, has, rho, dot, e);
            correct_o(base, delta, rho, kap);
        }
        cnt = 0;
    };

    auto tile_active = [&](uint32_t t) -> bool {
        const int32_t t0 = wg_base + (int32_t)(t * BK);
        return wave_valid && t < nt && t0 < w_hi && t0 + BK > w_lo;
    };
    if (t_begin < t_end) issue_tile(t_begin);
    for (uint32_t t = t_begin; t < t_end; ++t) {
        wait_vm<0>();   // this wave's copies of tile t have landed (nothing else is in flight)
        barrier_lds();  // every wave's have; buffer (t+1)&1 and the exchange slots are free
        if (t + 1 < t_end) issue_tile(t + 1);
        // both waves of a pair share the row block, hence the activity of a tile
        const bool act = tile_active(t);
        const int32_t t0 = wg_base + (int32_t)(t * BK);
        const float* const Kt = smem + (t & 1) * C::TILE;
        const float* const Vt = Kt + BK * KRS;
        f4v Sp = f4v{0.0f, 0.0f, 0.0f, 0.0f};
        if (act) {
            // this wave's half of S^T = K Q^T from the scaled fp16 splits: Khi Qhi + Klo Qhi +
            // Khi Qlo, then the wave's and the tile's powers of two
            f4v SA[3];
#pragma unroll
            for (int a = 0; a < 3; ++a) SA[a] = f4v{0.0f, 0.0f, 0.0f, 0.0f};
            const float* kr = Kt + rl * KRS + HD * dhf + 8 * g;
#pragma unroll
            for (int kb = 0; kb < QBH; ++kb) {
                const h8v khi = *reinterpret_cast<const h8v*>(kr + 32 * kb);
                const h8v klo = *reinterpret_cast<const h8v*>(kr + 32 * kb + 4);
                SA[0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(khi, qh[kb], SA[0], 0, 0, 0);
                SA[1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(klo, qh[kb], SA[1], 0, 0, 0);
                SA[2] = __builtin_amdgcn_mfma_f32_16x16x32_f16(khi, ql[kb], SA[2], 0, 0, 0);
            }
            Sp = (SA[0] + SA[1]) + SA[2];
            const float sc = qsc * tile_kscale(p, kvh, t0);  // a power of two: exact
#pragma unroll
            for (int r = 0; r < 4; ++r) Sp[r] = Sp[r] * sc;
            xs[w * 64 + lane] = make_float4(Sp[0], Sp[1], Sp[2], Sp[3]);
        }
        barrier_lds();  // both halves of every active pair are in the exchange slots
        if (!act) continue;
        const float4 o4 = xs[(w ^ 4) * 64 + lane];
        const f4v So = f4v{o4.x, o4.y, o4.z, o4.w};
        const f4v S = dhf == 0 ? Sp + So : So + Sp;  // the low half first in both waves
        float s[4];
        bool vis[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int32_t j = t0 + 4 * g + r;
            vis[r] = j >= my_lo && j < my_hi;
            s[r] = vis[r] ? S[r] * p.scale : NEG_INF;
        }
        float tm = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
        tm = g4a_col_max4(tm);
        const float mn = fmaxf(m_run, tm);

        // ---- record the keys within TAU of the running maximum ----
        bool cand[4];
        uint64_t bal[4];
        int nnew = 0;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            cand[r] = vis[r] && s[r] > mn - p.tau;
            bal[r] = ballot(cand[r]);
            nnew += __builtin_popcountll(bal[r]);
        }
        if (cnt + nnew > CAP) {
            publish_m(mn);
            compact();
            if (cnt + nnew > CAP) {
                publish_m(m_ref);  // O and l are held at m_ref
                flush_light();
            }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            if (cand[r]) {
                const int pos = cnt + lanes_below(bal[r]);
                my_keys[pos] = ((uint32_t)rl << 28) | (uint32_t)(t0 + 4 * g + r);
                my_s[pos] = s[r];
            }
            cnt += __builtin_popcountll(bal[r]);
        }
        m_run = mn;

        // ---- rescale O and l when some row's maximum moved RESCALE above its reference ----
        if (ballot(mn > m_ref + PF_RESCALE) != 0) {
            const float corr = (m_ref == NEG_INF) ? 0.0f : expf(m_ref - mn);
            l_part *= corr;
            m_ref = mn;
            const f4v cr = f4v{__shfl(corr, 4 * g + 0, 64), __shfl(corr, 4 * g + 1, 64),
                               __shfl(corr, 4 * g + 2, 64), __shfl(corr, 4 * g + 3, 64)};
#pragma unroll
            for (int c = 0; c < NCH; ++c)
#pragma unroll
                for (int e = 0; e < 4; ++e) O[c][e] *= cr;
        }

        // ---- probabilities against m_ref and P.V for this wave's columns ----
        float pr[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) pr[r] = vis[r] ? psc * pf_exp(s[r] - m_ref) : 0.0f;
        l_part += (pr[0] + pr[1]) + (pr[2] + pr[3]);
        if (v16) {
            // O += P V on v_mfma_f32_16x16x16_f16: Phi Vhi + Phi Vlo + Plo Vhi. Lane (g, rl)
            // gives A = P[row rl][keys 4g .. 4g+3] and B = V[keys 4g .. 4g+3][dim
            // 64 cg + 4rl + e] (cg = NCH*dhf + c): quad g's 16 bytes (4 hi, 4 lo).
            h4v ah, al;
#pragma unroll
            for (int r = 0; r < 4; ++r) split16(pr[r], ah, al, r);
            const float* const vq = Vt + g * 4 * DH + 4 * rl;
#pragma unroll
            for (int c = 0; c < NCH; ++c)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int cg = NCH * dhf + c;
                    const float4 raw = *reinterpret_cast<const float4*>(vq + 4 * 16 * (4 * cg + e));
                    h4v bh, bl;
                    __builtin_memcpy(&bh, &raw.x, 8);
                    __builtin_memcpy(&bl, &raw.z, 8);
                    O[c][e] = __builtin_amdgcn_mfma_f32_16x16x16f16(ah, bh, O[c][e], 0, 0, 0);
                    O[c][e] = __builtin_amdgcn_mfma_f32_16x16x16f16(ah, bl, O[c][e], 0, 0, 0);
                    O[c][e] = __builtin_amdgcn_mfma_f32_16x16x16f16(al, bh, O[c][e], 0, 0, 0);
                }
            continue;
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float* vr = Vt + (4 * g + r) * DH + HD * dhf + 4 * rl;
#pragma unroll
            for (int c = 0; c < NCH; ++c) {
                const float4 vv = *reinterpret_cast<const float4*>(vr + 64 * c);
                O[c][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(pr[r], vv.x, O[c][0], 0, 0, 0);
                O[c][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(pr[r], vv.y, O[c][1], 0, 0, 0);
                O[c][2] = __builtin_amdgcn_mfma_f32_16x16x4f32(pr[r], vv.z, O[c][2], 0, 0, 0);
                O[c][3] = __builtin_amdgcn_mfma_f32_16x16x4f32(pr[r], vv.w, O[c][3], 0, 0, 0);
            }
        }
    }
    wait_vm<0>();
    __syncthreads();  // every wave is done with the tile buffers: they become the staging areas

    // ---- exact corrections for the keys still within TAU of the final maxima ----
    if (wave_valid) {
        publish_m(m_run);
        compact();
        publish_m(m_ref);
        flush_staged(smem + w * C::STAGE, pair_dots, pair_flags);
    }
    float l = l_part;
    l = g4a_col_sum4(l);
    // O row 4g + r' is query qw + row/8, head h0 + row%8; this wave's columns HD*dhf + 64c + 4rl + e
    if (!split) {
        if (!wave_valid) return;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = 4 * g + r;
            const float lr = __shfl(l, row, 64);
            const float inv = lr > 0.0f ? 1.0f / lr : 0.0f;
            const uint32_t qi = qw + (row >> 3);
            if (qi >= p.T) continue;
            float* orow = p.out + ((size_t)qi * p.Hq + h0 + (row & 7)) * DH + HD * dhf + 4 * rl;
#pragma unroll
            for (int c = 0; c < NCH; ++c)
                *reinterpret_cast<float4*>(orow + 64 * c) =
                    make_float4(O[c][0][r] * inv, O[c][1][r] * inv, O[c][2][r] * inv, O[c][3][r] * inv);
        }
        return;
    }
    // ---- one half of a split block: its partial, in the wave's register layout ----
    const uint32_t bi = kvh * p.nbig + (blk - (NB - p.nbig));  // split block of this kv head
    float* const mine = p.part + ((size_t)(bi * 2 + half_id) * 8 + w) * C::PART_WAVE;
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
            for (int r = 0; r < 4; ++r) mine[((c * 4 + e) * 4 + r) * 64 + lane] = O[c][e][r];
    if (g == 0) {
        mine[NCH * 16 * 64 + rl] = l;
        mine[NCH * 16 * 64 + 16 + rl] = m_ref;
    }
}

// Merge of the two halves of each split query block of prefill_dsplit:
// workgroup = (split block, dim half, kv head), wave w = the producing waves'
// (row block w, dim half); out = (O0 e^{m0-M} + O1 e^{m1-M}) / (l0 e^{m0-M} + l1 e^{m1-M}).
// Every load of a thread is issued before the first use (the stores to `out`
// would otherwise keep the compiler from moving later loads above them: one
// memory round trip per 8 loads).
template <int DH>
__device__ __forceinline__ void prefill_merge(const G4aPrefillParams& p) {
    using C = DsplitCfg<DH>;
    constexpr int HD = C::HD, NCH = C::NCH;
    const int tid = threadIdx.x, lane = tid & 63;
    const int rb = tid >> 6, dhf = blockIdx.x & 1;
    const int w = rb + 4 * dhf;  // the producing wave
    const int g = lane >> 4, rl = lane & 15;
    const uint32_t kvh = blockIdx.y;
    const uint32_t NB = (p.T + 7) / 8;
    const uint32_t sb = blockIdx.x >> 1;
    const uint32_t blk = NB - p.nbig + sb;
    const uint32_t qw = blk * 8 + 2 * rb;
    const uint32_t h0 = kvh * 8;
    const uint32_t bi = kvh * p.nbig + sb;
    const float* __restrict__ const p0 = p.part + ((size_t)(bi * 2 + 0) * 8 + w) * C::PART_WAVE;
    const float* __restrict__ const p1 = p.part + ((size_t)(bi * 2 + 1) * 8 + w) * C::PART_WAVE;
    float x0[4][NCH][4], x1[4][NCH][4], l0[4], m0[4], l1[4], m1[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int row = 4 * g + r;
        l0[r] = p0[NCH * 16 * 64 + row];
        m0[r] = p0[NCH * 16 * 64 + 16 + row];
        l1[r] = p1[NCH * 16 * 64 + row];
        m1[r] = p1[NCH * 16 * 64 + 16 + row];
#pragma unroll
        for (int c = 0; c < NCH; ++c)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int idx = ((c * 4 + e) * 4 + r) * 64 + lane;
                x0[r][c][e] = p0[idx];
                x1[r][c][e] = p1[idx];
            }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int row = 4 * g + r;
        const uint32_t qi = qw + (row >> 3);
        if (qi >= p.T) continue;
        const float M = fmaxf(m0[r], m1[r]);
        const float e0 = (m0[r] == NEG_INF) ? 0.0f : expf(m0[r] - M);
        const float e1 = (m1[r] == NEG_INF) ? 0.0f : expf(m1[r] - M);
        const float L = l0[r] * e0 + l1[r] * e1;
        const float inv = L > 0.0f ? 1.0f / L : 0.0f;
        const float a0 = e0 * inv, a1 = e1 * inv;
        float* orow = p.out + ((size_t)qi * p.Hq + h0 + (row & 7)) * DH + HD * dhf + 4 * rl;
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            float o[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = x0[r][c][e] * a0 + x1[r][c][e] * a1;
            *reinterpret_cast<float4*>(orow + 64 * c) = make_float4(o[0], o[1], o[2], o[3]);
        }
    }
}

}  // namespace

extern "C" {
__global__ __launch_bounds__(512) void g4a_prefill2_d256(G4aPrefillParams p) { prefill_pair<256>(p); }
__global__ __launch_bounds__(512) void g4a_prefill2_d512(G4aPrefillParams p) { prefill_dsplit<512>(p); }
__global__ __launch_bounds__(256) void g4a_prefill_merge_d512(G4aPrefillParams p) { prefill_merge<512>(p); }
__global__ __launch_bounds__(256) void g4a_split_kv(G4aSplitParams p) { split_kv(p); }
}
