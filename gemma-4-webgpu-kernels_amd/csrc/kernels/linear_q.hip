// Quantised projections for gfx950: y = x . W^T with W packed 2/4/8-bit
// (offset-binary sub-byte fields LSB-first, or native I8) and f32 scales, plus
// the two epilogues Gemma-4 fuses into a projection (GeGLU of gate and up, and
// the per-layer-input gate times a column slice), and the quantised embedding
// gather.
//
// Replaces, behind the backend trait, the WGSL MATMUL_Q / MATMUL_Q_SCALAR /
// EMBED_Q kernels (rust/src/kernels/matmul_q.wgsl, matmul_q_scalar.wgsl,
// embed_q.wgsl, dispatched by rust/src/backend_wgpu.rs:624-832); the semantics
// are the CPU backend's (rust/src/backend.rs:44-58 QuantWeight::deq,
// rust/src/backend_cpu.rs:127-145 embed_rows, :174-222 linear, :55-58
// gelu_tanh, and the trait's compositions rust/src/backend.rs:156-168).
//
// Two linear kernels:
//  * linear_q_words (rows whose packed bytes are whole 32-bit words, one scale
//    per row): decode projections are weight-streaming (HBM-bound). Lane l of a
//    wave owns words l, l + 64, ... of every row, so each wave load reads 256
//    contiguous bytes of a row. Every lane takes the same number of steps (a
//    step: one word of each of RU rows); two register sets alternate so the
//    next step's loads are in flight while a step computes. The activations
//    sit in LDS (MT rows, zero-padded to whole wave strides) and are read once
//    per word for all RU rows. Each field is turned into a sign-extended byte holding
//    value * F (F = 16 for 4-bit, 64 for 2-bit, 1 for 8-bit: an exact power of
//    two) by one mask, so one SDWA convert and one FMA handle a value; the
//    final scale is s / F. Per lane the sum runs over its words in order (an
//    FMA chain within a word), then a transposed butterfly reduces the MT*RU
//    sums across the wave. Not the CPU's summation order: results agree within
//    f32 reordering error.
//  * linear_q_elem (any K, grouped scales): one thread per output, the CPU's
//    exact order (acc += x[k] * (q * s) for k in order, separately rounded), so
//    plain projections are bit-identical to the reference.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "g4a_math.h"
#include "g4a_params.h"

namespace {

__device__ __forceinline__ float gelu_tanh(float v) { return g4a_gelu_tanh(v); }

// BITS = 32: an f32 weight per word (the unquantised linear).
template <int BITS>
struct QFmt {
    static constexpr int VPW = 32 / BITS;  // values per word
    static constexpr float INV_F = BITS == 4 ? 0.0625f : BITS == 2 ? 0.015625f : 1.0f;
};

__device__ __forceinline__ float sbyte(uint32_t v, int j) { return (float)(int8_t)(v >> (8 * j)); }

// The VPW values of a word whose fields are two's complement, each as value * F,
// in k order.
template <int BITS>
__device__ __forceinline__ void unpack(uint32_t v, float (&q)[QFmt<BITS>::VPW]) {
    if constexpr (BITS == 32) {
        q[0] = __uint_as_float(v);
    } else if constexpr (BITS == 8) {
#pragma unroll
        for (int j = 0; j < 4; ++j) q[j] = sbyte(v, j);
    } else if constexpr (BITS == 4) {
        const uint32_t a = (v << 4) & 0xF0F0F0F0u;  // field 2j at the top of byte j
        const uint32_t b = v & 0xF0F0F0F0u;         // field 2j + 1
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            q[2 * j] = sbyte(a, j);
            q[2 * j + 1] = sbyte(b, j);
        }
    } else {
        const uint32_t a0 = (v << 6) & 0xC0C0C0C0u, a1 = (v << 4) & 0xC0C0C0C0u;
        const uint32_t a2 = (v << 2) & 0xC0C0C0C0u, a3 = v & 0xC0C0C0C0u;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            q[4 * j] = sbyte(a0, j);
            q[4 * j + 1] = sbyte(a1, j);
            q[4 * j + 2] = sbyte(a2, j);
            q[4 * j + 3] = sbyte(a3, j);
        }
    }
}

// Sums v[i] over the 64 lanes for all V (a power of two <= 64) values at once:
// each butterfly step hands half of the remaining values to the partner lane,
// so log2(V) steps leave one value per lane, then plain xor steps finish it.
// Returns the total of value `idx` (set here from the lane's bits); every lane
// whose low 6 - log2(V) bits are zero holds a distinct idx.
template <int V, int LANES = 64>
__device__ __forceinline__ float wave_reduce_many(float (&v)[V], int lane, int& idx) {
    idx = 0;
    int o = LANES / 2;  // LANES = 32: each half-wave reduces on its own
#pragma unroll
    for (int n = V; n > 1; n >>= 1, o >>= 1) {
        const int half = n / 2;
        const bool hi = (lane & o) != 0;
#pragma unroll
        for (int i = 0; i < half; ++i) {
            const float lo_v = v[i], hi_v = v[i + half];  // values first: a select of addresses would go to scratch
            const float send = hi ? lo_v : hi_v;
            const float keep = hi ? hi_v : lo_v;
            v[i] = keep + __shfl_xor(send, o, 64);
        }
        idx = 2 * idx + (hi ? 1 : 0);
    }
    float s = v[0];
#pragma unroll
    for (; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
    return s;
}

// The value index wave_reduce_many<V, LANES> leaves in `lane`.
template <int V, int LANES>
__device__ __forceinline__ int reduce_slot(int lane) {
    int idx = 0, o = LANES / 2;
#pragma unroll
    for (int n = V; n > 1; n >>= 1, o >>= 1) idx = 2 * idx + ((lane & o) ? 1 : 0);
    return idx;
}

// LPR (lanes per row) = 32 splits the wave into two halves that walk different
// rows (RU each): for rows of an odd multiple of 32 words (2-bit rows of 1536
// values are 96 words) every lane then has a word on every step.
template <int BITS, int MT, int RU, int D, int MODE, int LPR = 64>
__device__ __forceinline__ void linear_q_words(const G4aLinearParams& p) {
    using F = QFmt<BITS>;
    constexpr int VPW = F::VPW;
    constexpr int V = MT * RU;
    constexpr int RC = RU * (64 / LPR);  // rows per chunk (both halves)
    extern __shared__ __attribute__((aligned(16))) float xs[];  // [MT][J * LPR * VPW], zeros past K
    const int lane = threadIdx.x & 63;
    const int ll = lane & (LPR - 1);        // lane within its row group
    const int hf = lane / LPR;              // row group (0 for LPR = 64)
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: rows in scalar registers
    const uint32_t K = p.K, W = p.W, N = p.N;
    const uint32_t J = (W + LPR - 1) / LPR;  // word steps per row chunk (lanes past W read zeros of x)
    const uint32_t KP = J * LPR * VPW;       // padded activation row
    const uint32_t m0 = blockIdx.y * MT;
    const uint32_t first = (blockIdx.x * (blockDim.x / 64) + wv) * p.rows_per_wave;
    const uint32_t last = min(first + p.rows_per_wave, N);
    const uint32_t nchunks = first < last ? (last - first + RC - 1) / RC : 0;
    const uint32_t T = nchunks * J;         // the wave's steps: chunk t / J, word step t % J

    // Step t loads word lane + 64 (t % J) (clamped to the row) of the RU rows of
    // chunk t / J (clamped to the matrix). D register sets form a ring, so the
    // loads of steps t + 1 .. t + D - 1 are in flight while step t computes,
    // with no register copies.
    // The output this lane stores after a chunk's reduction, and the epilogue
    // operands of that output (scales, the gelu-times column), which each step
    // loads with its words: a load issued at the store itself would wait for
    // every word in flight.
    const int oidx = reduce_slot<V, LPR>(ll);
    const uint32_t omt = oidx / RU, orr = oidx % RU;
    auto load = [&](uint32_t (&wd)[RU], uint32_t (&wd2)[RU], float (&ep)[2], uint32_t t) {
        const uint32_t c = t / J, j = t - c * J;
        const uint32_t w = min(ll + LPR * j, W - 1);
#pragma unroll
        for (int r = 0; r < RU; ++r) {
            const size_t row = min(first + c * RC + hf * RU + r, N - 1);
            wd[r] = p.w[row * W + w];
            if (MODE == 1) wd2[r] = p.w2[row * W + w];
        }
        const uint32_t n = min(first + c * RC + hf * RU + orr, N - 1);
        if (BITS != 32) ep[0] = p.s[n];
        if (MODE == 1) ep[1] = p.s2[n];
        if (MODE == 2) ep[1] = p.b[(size_t)min(m0 + omt, p.M - 1) * p.b_stride + p.b_off + n];
    };
    uint32_t wd[D][RU], wd2[D][RU];
    float ep[D][2];
    // the first steps' words are requested before the activations are staged
    // (mode 3: right after the loads of the partials the staging merges)
    auto prefetch = [&]() {
#pragma unroll
        for (int d = 0; d + 1 < D; ++d)
            if (T) load(wd[d], wd2[d], ep[d], min((uint32_t)d, T - 1));
    };
    if constexpr (MODE == 3) {
        // x: one attention row merged from its decode step's split partials
        // (MT = 1; workgroup 0 also stores the row)
        float* const xout = blockIdx.x == 0 ? p.xout : nullptr;
        if (p.dh == 512) combine_row_stage<512>(p.part, p.hq, p.nsplit, xs, KP, xout, prefetch);
        else combine_row_stage<256>(p.part, p.hq, p.nsplit, xs, KP, xout, prefetch);
    } else {
        prefetch();
        for (uint32_t i = threadIdx.x; i < MT * KP / 4; i += blockDim.x) {
            const uint32_t e = 4 * i, mt = e / KP, k = e - mt * KP;
            float4 xv = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (m0 + mt < p.M && k < K) xv = *reinterpret_cast<const float4*>(p.x + (size_t)(m0 + mt) * K + k);
            *reinterpret_cast<float4*>(xs + e) = xv;
        }
    }
    __syncthreads();

    float acc[V], acc2[V];
#pragma unroll
    for (int i = 0; i < V; ++i) acc[i] = acc2[i] = 0.0f;

    auto step = [&](const uint32_t (&wd)[RU], const uint32_t (&wd2)[RU], const float (&ep)[2], uint32_t t) {
        const uint32_t c = t / J, j = t - c * J;
        const uint32_t w = ll + LPR * j;
        float xv[MT][VPW];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
            if constexpr (VPW == 1) {
                xv[mt][0] = xs[mt * KP + w];
            } else {
#pragma unroll
                for (int i = 0; i < VPW; i += 4) {
                    const float4 v4 = *reinterpret_cast<const float4*>(xs + mt * KP + w * VPW + i);
                    xv[mt][i] = v4.x;
                    xv[mt][i + 1] = v4.y;
                    xv[mt][i + 2] = v4.z;
                    xv[mt][i + 3] = v4.w;
                }
            }
#pragma unroll
        for (int r = 0; r < RU; ++r) {
            float q[VPW];
            unpack<BITS>(wd[r] ^ p.xm, q);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int i = 0; i < VPW; ++i) acc[mt * RU + r] = __builtin_fmaf(xv[mt][i], q[i], acc[mt * RU + r]);
            if (MODE == 1) {
                float q2[VPW];
                unpack<BITS>(wd2[r] ^ p.xm, q2);
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                    for (int i = 0; i < VPW; ++i)
                        acc2[mt * RU + r] = __builtin_fmaf(xv[mt][i], q2[i], acc2[mt * RU + r]);
            }
        }
        if (j + 1 == J) {
            // the chunk's sums are complete: reduce across the wave and store
            int idx;
            const float a = wave_reduce_many<V, LPR>(acc, ll, idx);
            float a2 = 0.0f;
            if (MODE == 1) {
                int idx2;
                a2 = wave_reduce_many<V, LPR>(acc2, ll, idx2);
            }
            if ((ll & (LPR / V - 1)) == 0) {
                const uint32_t mt = idx / RU, r = idx % RU;
                const uint32_t n = first + c * RC + hf * RU + r, m = m0 + mt;
                if (n < last && m < p.M) {
                    const float v = BITS == 32 ? a : a * (ep[0] * F::INV_F);  // f32 weights carry no scale
                    float o = v;
                    if (MODE == 1) o = gelu_tanh(v) * (a2 * (ep[1] * F::INV_F));
                    if (MODE == 2) o = gelu_tanh(v) * ep[1];
                    p.y[(size_t)m * N + n] = o;
                }
            }
#pragma unroll
            for (int i = 0; i < V; ++i) acc[i] = acc2[i] = 0.0f;
        }
    };

    // Whole groups of D steps, with no branch between them: the loads of a step
    // never wait behind a path that skipped one. Steps past T (at most D - 1)
    // re-read the last words and store nothing: their rows lie past `last`.
    for (uint32_t t = 0; t < T; t += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            load(wd[(d + D - 1) % D], wd2[(d + D - 1) % D], ep[(d + D - 1) % D], min(t + d + D - 1, T - 1));
            // keep the loads ahead of this step's arithmetic: left alone, the
            // scheduler sinks them below it, behind a wait for every load in flight
            __builtin_amdgcn_sched_barrier(0);
            step(wd[d], wd2[d], ep[d], t + d);
        }
    }
}

// ---------------------------------------------------------------------------
// Prefill projections (M >= 16) on the matrix cores: v_mfma_f32_16x16x32_bf16
// with exact products. x = x0 + x1 + x2 exactly, each part a bf16 holding the
// next 8 significant bits (rounded splits of an f32 leave at most 8 bits for
// the last part); the quantised fields times F are small integers, exact in
// bf16. So every product x_p * q is exact in f32 and the three partial sums
// differ from the f32 sum only by accumulation rounding, like the VALU kernel.
//
// Workgroup: 64 activation rows (tokens) x 64 AB weight rows, 4 waves; wave w
// owns weight rows 16 AB w .. + 16 AB - 1 as AB 16-row A blocks (the MFMA's A
// operand, one 8-value fragment per lane: row lane % 16, k 8 (lane / 16) .. + 7
// of each 32-wide sub-step) and all 64 tokens (four 16-token B blocks), so
// each B fragment read from LDS feeds AB MFMAs. AB = 2 for large M (more MFMA
// work per staged x), 1 when the grid would otherwise be too small. Per 64-wide k step the workgroup stages
// the three bf16 parts of its x tile in LDS (double-buffered); the next step's
// x and weight fragments are loaded into registers before this step's MFMAs.
// C lane layout: weight row 4 (lane / 16) + i, token lane % 16.
typedef __bf16 bf8v __attribute__((ext_vector_type(8)));
typedef float f4v __attribute__((ext_vector_type(4)));

constexpr int LQ_BM = 64, LQ_BK = 64;
constexpr int LQ_XS = LQ_BK + 8;  // bf16 per staged x row (+16 bytes: rows start on different banks)

// The packed bytes of the 8 fields of a row at k .. k + 7 (8, 4 or 2 bytes).
template <int BITS>
__device__ __forceinline__ uint2 frag8_load(const uint8_t* __restrict__ rowp, uint32_t k) {
    if constexpr (BITS == 8) return *reinterpret_cast<const uint2*>(rowp + k);
    if constexpr (BITS == 4) return make_uint2(*reinterpret_cast<const uint32_t*>(rowp + k / 2), 0u);
    return make_uint2(*reinterpret_cast<const uint16_t*>(rowp + k / 4), 0u);
}

// Those 8 fields as value * F in bf16 (small integers: exact).
template <int BITS>
__device__ __forceinline__ bf8v frag8_bf16(uint2 w, uint32_t xm) {
    float q[8];
    if constexpr (BITS == 4) {
        unpack<4>(w.x ^ xm, q);
    } else if constexpr (BITS == 8) {
        float t0[4], t1[4];
        unpack<8>(w.x ^ xm, t0);
        unpack<8>(w.y ^ xm, t1);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            q[i] = t0[i];
            q[4 + i] = t1[i];
        }
    } else {
        float t[16];
        unpack<2>((w.x ^ xm) & 0xFFFFu, t);
#pragma unroll
        for (int i = 0; i < 8; ++i) q[i] = t[i];
    }
    bf8v a;
#pragma unroll
    for (int i = 0; i < 8; ++i) a[i] = (__bf16)q[i];
    return a;
}

template <int BITS, int AB, int MODE>
__device__ __forceinline__ void linear_q_mfma(const G4aLinearParams& p) {
    constexpr int LQ_BN = 64 * AB;
    using F = QFmt<BITS>;
    __shared__ __attribute__((aligned(16))) __bf16 xsp[2][3][LQ_BM * LQ_XS];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, rl = lane & 15;
    const uint32_t K = p.K, N = p.N, M = p.M;
    const uint32_t n0 = blockIdx.x * LQ_BN, m0 = blockIdx.y * LQ_BM;
    const uint32_t nsteps = K / LQ_BK;
    // this lane's A rows, one per 16-row block (rows past N: re-read, not stored)
    const uint8_t* wrow[AB];
    const uint8_t* wrow2[AB];
#pragma unroll
    for (int ab = 0; ab < AB; ++ab) {
        const uint32_t row = min(n0 + 16 * AB * wv + 16 * ab + rl, N - 1);
        wrow[ab] = p.wb + (size_t)row * p.row_bytes;
        wrow2[ab] = MODE == 1 ? p.wb2 + (size_t)row * p.row_bytes : nullptr;
    }

    // x tile staging: thread tid splits tokens tid / 4 (16 values at 16 (tid % 4))
    const uint32_t xt = tid >> 2, xk = 16 * (tid & 3);
    const bool xin = m0 + xt < M;
    const float* __restrict__ xrow = p.x + (size_t)min(m0 + xt, M - 1) * K;
    float4 xr[4];
    auto load_x = [&](uint32_t st) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            xr[i] = xin ? *reinterpret_cast<const float4*>(xrow + st * LQ_BK + xk + 4 * i)
                        : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    };
    auto stage_x = [&](int buf) {
        const float v[16] = {xr[0].x, xr[0].y, xr[0].z, xr[0].w, xr[1].x, xr[1].y, xr[1].z, xr[1].w,
                             xr[2].x, xr[2].y, xr[2].z, xr[2].w, xr[3].x, xr[3].y, xr[3].z, xr[3].w};
        bf8v p0[2], p1[2], p2[2];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const __bf16 a = (__bf16)v[i];
            const float r1 = v[i] - (float)a;
            const __bf16 b = (__bf16)r1;
            const __bf16 c = (__bf16)(r1 - (float)b);
            p0[i / 8][i % 8] = a;
            p1[i / 8][i % 8] = b;
            p2[i / 8][i % 8] = c;
        }
        __bf16* d0 = &xsp[buf][0][xt * LQ_XS + xk];
        __bf16* d1 = &xsp[buf][1][xt * LQ_XS + xk];
        __bf16* d2 = &xsp[buf][2][xt * LQ_XS + xk];
        *reinterpret_cast<bf8v*>(d0) = p0[0];
        *reinterpret_cast<bf8v*>(d0 + 8) = p0[1];
        *reinterpret_cast<bf8v*>(d1) = p1[0];
        *reinterpret_cast<bf8v*>(d1 + 8) = p1[1];
        *reinterpret_cast<bf8v*>(d2) = p2[0];
        *reinterpret_cast<bf8v*>(d2 + 8) = p2[1];
    };
    // A fragments of one step, packed: block ab, sub-step kk covers k 32 kk + 8 g .. + 7.
    // They are unpacked only at the start of their step, so their loads stay in
    // flight under the previous step's MFMAs.
    uint2 wr[AB][2], wr2[AB][2];
    auto load_w = [&](uint32_t st) {
#pragma unroll
        for (int ab = 0; ab < AB; ++ab)
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                const uint32_t k = st * LQ_BK + 32 * kk + 8 * g;
                wr[ab][kk] = frag8_load<BITS>(wrow[ab], k);
                if (MODE == 1) wr2[ab][kk] = frag8_load<BITS>(wrow2[ab], k);
            }
    };

    f4v acc[AB][4], acc2[AB][4];
#pragma unroll
    for (int ab = 0; ab < AB; ++ab)
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) acc[ab][tb] = acc2[ab][tb] = f4v{0.0f, 0.0f, 0.0f, 0.0f};

    if (nsteps) {
        load_x(0);
        load_w(0);
        stage_x(0);
    }
    for (uint32_t st = 0; st < nsteps; ++st) {
        __syncthreads();  // step st's x parts are staged; every wave is done with the other buffer
        bf8v a[AB][2], a2[AB][2];
#pragma unroll
        for (int ab = 0; ab < AB; ++ab)
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                a[ab][kk] = frag8_bf16<BITS>(wr[ab][kk], p.xm);
                if (MODE == 1) a2[ab][kk] = frag8_bf16<BITS>(wr2[ab][kk], p.xm);
            }
        if (st + 1 < nsteps) {
            load_x(st + 1);
            load_w(st + 1);
        }
        // the next step's loads go out before this step's MFMAs
        __builtin_amdgcn_sched_barrier(0);
        const int buf = st & 1;
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
#pragma unroll
            for (int tb = 0; tb < 4; ++tb) {
                const int off = (16 * tb + rl) * LQ_XS + 32 * kk + 8 * g;
#pragma unroll
                for (int part = 0; part < 3; ++part) {
                    const bf8v bx = *reinterpret_cast<const bf8v*>(&xsp[buf][part][off]);
#pragma unroll
                    for (int ab = 0; ab < AB; ++ab) {
                        acc[ab][tb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[ab][kk], bx, acc[ab][tb], 0, 0, 0);
                        if (MODE == 1)
                            acc2[ab][tb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2[ab][kk], bx, acc2[ab][tb], 0, 0, 0);
                    }
                }
            }
        if (st + 1 < nsteps) stage_x(buf ^ 1);
    }

    // lane (g, rl) of blocks (ab, tb) holds weight rows 16 AB wv + 16 ab + 4 g + i, token 16 tb + rl.
    // Every scale (and b value) is loaded before the first store, at indices clamped
    // into range: y may alias them as far as the compiler knows, so a load after a
    // store waited for it, one memory round trip per output.
    float sc[AB][4], sc2[AB][4], bv[AB][4][4];
#pragma unroll
    for (int ab = 0; ab < AB; ++ab)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t n = min(n0 + 16 * AB * wv + 16 * ab + 4 * g + i, N - 1);
            sc[ab][i] = p.s[n];
            if (MODE == 1) sc2[ab][i] = p.s2[n];
            if (MODE == 2) {
#pragma unroll
                for (int tb = 0; tb < 4; ++tb) {
                    const uint32_t m = min(m0 + 16 * tb + rl, M - 1);
                    bv[ab][tb][i] = p.b[(size_t)m * p.b_stride + p.b_off + n];
                }
            }
        }
    // all of them in (s_waitcnt vmcnt(0)): with no load left pending, the compiler
    // puts no wait among the stores below, which vmcnt also counts on this GPU
    __builtin_amdgcn_s_waitcnt(0x0F70);
#pragma unroll
    for (int ab = 0; ab < AB; ++ab)
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) {
            const uint32_t m = m0 + 16 * tb + rl;
            if (m >= M) continue;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t n = n0 + 16 * AB * wv + 16 * ab + 4 * g + i;
                if (n >= N) continue;
                const float v = acc[ab][tb][i] * (sc[ab][i] * F::INV_F);
                float o = v;
                if (MODE == 1) o = gelu_tanh(v) * (acc2[ab][tb][i] * (sc2[ab][i] * F::INV_F));
                if (MODE == 2) o = gelu_tanh(v) * bv[ab][tb][i];
                p.y[(size_t)m * N + n] = o;
            }
        }
}

// QuantWeight::deq (rust/src/backend.rs:44-58) of element (n, k).
__device__ __forceinline__ float deq(const uint8_t* __restrict__ wb, const float* __restrict__ s, uint32_t bits,
                                     uint32_t row_bytes, uint32_t group, uint32_t sstride, uint32_t signed_i8,
                                     uint32_t n, uint32_t k) {
    int32_t qv;
    if (signed_i8) {
        qv = (int32_t)(int8_t)wb[(size_t)n * row_bytes + k];
    } else {
        const uint32_t per_byte = 8 / bits;
        const uint32_t b = wb[(size_t)n * row_bytes + k / per_byte];
        const uint32_t shift = (k % per_byte) * bits;
        qv = (int32_t)((b >> shift) & ((1u << bits) - 1u)) - (int32_t)(1u << (bits - 1));
    }
    return (float)qv * s[(size_t)n * sstride + k / group];
}

// CpuBackend::linear with an f32 weight (rust/src/backend_cpu.rs:199-208), one
// thread per output in the CPU's order: bit-identical.
__device__ __forceinline__ void linear_f32_elem(const G4aLinearParams& p) {
    const uint32_t n = blockIdx.x * blockDim.x + threadIdx.x, m = blockIdx.y;
    if (n >= p.N) return;
    const float* __restrict__ xr = p.x + (size_t)m * p.K;
    const float* __restrict__ wr = reinterpret_cast<const float*>(p.w) + (size_t)n * p.K;
    float acc = 0.0f;
    for (uint32_t k = 0; k < p.K; ++k) acc += xr[k] * wr[k];
    p.y[(size_t)m * p.N + n] = acc;
}

template <int MODE>
__device__ __forceinline__ void linear_q_elem(const G4aLinearParams& p) {
    const uint32_t n = blockIdx.x * blockDim.x + threadIdx.x, m = blockIdx.y;
    if (n >= p.N) return;
    const float* __restrict__ xr = p.x + (size_t)m * p.K;
    float acc = 0.0f, acc2 = 0.0f;
    for (uint32_t k = 0; k < p.K; ++k) {
        acc += xr[k] * deq(p.wb, p.s, p.bits, p.row_bytes, p.group_size, p.scale_stride, p.signed_i8, n, k);
        if (MODE == 1)
            acc2 += xr[k] * deq(p.wb2, p.s2, p.bits, p.row_bytes, p.group_size, p.scale_stride, p.signed_i8, n, k);
    }
    float o = acc;
    if (MODE == 1) o = gelu_tanh(acc) * acc2;
    if (MODE == 2) o = gelu_tanh(acc) * p.b[(size_t)m * p.b_stride + p.b_off + n];
    p.y[(size_t)m * p.N + n] = o;
}

// ---------------------------------------------------------------------------
// Decode projections (M <= 2) over large weights on the int8 matrix cores
// (v_mfma_i32_16x16x64_i8), with exact integer products and sums.
//
// x is cut into LI8_NSL signed digits per element against one power of two per
// activation row: with max|x| < 2^E, u = x * 2^(6-E) has |u| < 64, and
// b_0 = rint(u), b_j = rint(128 r_(j-1)), r_j = 128 r_(j-1) - b_j (r_0 = u - b_0)
// are integers in [-64, 64] (int8), each step exact in f32. So
// x = 2^(E-6) * sum_j b_j 2^(-7j) exactly for every element within 2^-32 of the
// row's maximum (smaller ones keep all bits down to 2^(E-56)). The weight
// fields times F (the sign-extended bytes of the word kernel) are int8 too, so
// each digit column's dot product is exact in int32, and the only roundings are
// the f32 sum of the LI8_NSL column totals (largest weight 2^0, each next one
// 2^-7 of it) and the final scaling. The result is within a few f32 ulps of the
// exact sum of x_k * deq(n, k): closer to it than any f32 summation order,
// including the CPU's. A row holding an inf or NaN is computed in the CPU's
// exact order instead (the element kernel's loop), since the digits cannot hold
// it.
//
// Layout. A = 16 weight rows x 64 k, B = 64 k x 16 columns (column 8m + j: digit
// j of activation row m), D = 16 rows x 16 columns in int32. Lane l holds row /
// column l % 16 and k-group l / 16 of A / B, and rows 4 (l / 16) + v of column
// l % 16 of D. Which k sits in which byte of a lane's 16 A bytes is a choice
// here, made so that the fields come out of the loaded words with one shift and
// one mask per 4 bytes; the digits are staged in LDS in the same order, and the
// sum over k does not depend on it. A row is read in units of LPU 64-byte
// pieces (LPU = 2: whole 128-byte lines); lane (row r, group g) loads the LPU
// adjacent 16-byte pieces at byte 16 LPU g of each unit, each piece holding
// 8 / BITS MFMA steps of 64 k.
//
// Work split: chunks of 16 RB rows (RB A blocks share each B fragment read from
// LDS), dealt round-robin over the waves of the grid (wave gw takes chunks gw,
// gw + GW, ...: at any time the whole GPU reads nearby rows). Each wave streams
// its chunks unit by unit through a ring of D register sets, so the loads of the
// next D - 1 units are in flight while a unit computes (the word kernel's ring).
typedef int i4v __attribute__((ext_vector_type(4)));
constexpr int LI8_NSL = 8;      // digits per activation element
constexpr int LI8_KMAX = 4096;  // K limit: the digits of one row fill at most 64 KiB of LDS

template <int BITS>
struct I8Fmt {
    static constexpr int MPS = 8 / BITS;                                  // MFMA steps per 64-byte piece
    static constexpr int LOG2F = BITS == 2 ? 6 : BITS == 4 ? 4 : 0;     // fields are value * 2^LOG2F
};

// The k of byte 4 i + p of the A / B operand of lane group g at MFMA step s. A
// unit of LPU 64-byte pieces: lane group g loads 16-byte piece h < LPU of it at
// byte 16 (LPU g + h), i.e. words 4 (LPU g + h) .. + 3; piece v = LPU J + h of
// the row (J the unit) holds MFMA steps MPS v .. MPS v + MPS - 1.
template <int BITS, int LPU>
__device__ __forceinline__ uint32_t i8_k(uint32_t s, uint32_t g, uint32_t i, uint32_t p) {
    constexpr uint32_t MPS = 8 / BITS;
    const uint32_t v = s / MPS, t = s % MPS, h = v % LPU;
    const uint32_t wb = 16 * (v - h) + 4 * (LPU * g + h);  // the piece's first word
    if constexpr (BITS == 2) {
        return 16 * (wb + t) + 4 * p + i;  // byte p of (word << (6 - 2 i)) & 0xC0C0C0C0, word t of the piece
    } else if constexpr (BITS == 4) {
        return 8 * (wb + 2 * t + (i >> 1)) + 2 * p + (i & 1);  // i even: (word << 4) & 0xF0F0F0F0, odd: word & ..
    } else {
        return 4 * (wb + i) + p;  // register i is word i of the piece
    }
}

// The A operand of MFMA step t of a unit from the lane's 16 loaded bytes.
template <int BITS, int T>
__device__ __forceinline__ i4v i8_operand(const uint4& w, uint32_t xm) {
    if constexpr (BITS == 2) {
        const uint32_t v = (T == 0 ? w.x : T == 1 ? w.y : T == 2 ? w.z : w.w) ^ xm;
        return i4v{(int)((v << 6) & 0xC0C0C0C0u), (int)((v << 4) & 0xC0C0C0C0u), (int)((v << 2) & 0xC0C0C0C0u),
                   (int)(v & 0xC0C0C0C0u)};
    } else if constexpr (BITS == 4) {
        const uint32_t v0 = (T == 0 ? w.x : w.z) ^ xm, v1 = (T == 0 ? w.y : w.w) ^ xm;
        return i4v{(int)((v0 << 4) & 0xF0F0F0F0u), (int)(v0 & 0xF0F0F0F0u), (int)((v1 << 4) & 0xF0F0F0F0u),
                   (int)(v1 & 0xF0F0F0F0u)};
    } else {
        return i4v{(int)(w.x ^ xm), (int)(w.y ^ xm), (int)(w.z ^ xm), (int)(w.w ^ xm)};
    }
}

template <int BITS, int MT, int RB, int D, int LPU, int NW>
__device__ __forceinline__ void linear_q_i8(const G4aLinearParams& p) {
    using F = I8Fmt<BITS>;
    constexpr int MPS = F::MPS;
    constexpr int TPT = LI8_KMAX / (256 * NW);  // digit tasks per thread at most (K / 4 tasks, 64 NW threads)
    extern __shared__ __attribute__((aligned(16))) uint32_t bsh[];  // [K / 64 steps][64 lanes][4 words] digits
    __shared__ float redmax[NW][MT];
    __shared__ int redbad[NW][MT];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t K = p.K, N = p.N;
    const uint32_t NU = K * BITS / (512 * LPU);  // units per row
    const uint32_t NS = K / 64;                  // MFMA steps per row
    const uint32_t row_bytes = K * BITS / 8;
    const uint32_t nchunk = (N + 16 * RB - 1) / (16 * RB);
    const uint32_t GW = gridDim.x * NW, gw = blockIdx.x * NW + wv;
    // the wave's chunks: ordinals 0 .. nc - 1, chunk gw + i GW
    const uint32_t nc = nchunk > gw ? (nchunk - gw + GW - 1) / GW : 0;
    auto chunk = [&](uint32_t i) { return gw + i * GW; };
    const uint32_t T = nc * NU;  // the wave's units
    const int r = lane & 15, g = lane >> 4;
    // the output this lane stores at a chunk's end: digit column cc = 8 m + jj,
    // rows 4 g + v of D; lanes jj < 4 store row 4 g + jj of activation row m
    const int cc = lane & 15, om = cc >> 3, jj = cc & 7;

    // Unit loads: the chunk's row bases are set when a chunk starts (rows past N
    // clamped to the last row), then each unit adds 64 LPU bytes: one wave-uniform
    // base and a 32-bit lane offset per load. Each ring slot holds the RB 16-byte
    // loads, and at a chunk's first unit the scale of the row this lane stores.
    uint32_t li = 0, lj = 0;  // the next unit to load: chunk ordinal, unit
    uint32_t roff[RB];
    auto load = [&](uint4 (&a)[RB][LPU], float (&sc)[RB]) {
        // past the wave's last unit: that unit again (its lines are in cache), never
        // the next wave's rows
        const bool past = li >= nc;
        const uint32_t c = chunk(past ? nc - 1 : li), jl = past ? NU - 1 : lj;
        if (lj == 0 && !past) {
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                roff[rb] = (min(16 * (RB * c + rb) + r, N - 1) - 16 * RB * c) * row_bytes + 16 * LPU * g;
                sc[rb] = p.s[min(16 * (RB * c + rb) + 4 * g + (jj & 3), N - 1)];
            }
        }
        const uint8_t* __restrict__ base = p.wb + (size_t)(16 * RB * c) * row_bytes + 64 * LPU * jl;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int h = 0; h < LPU; ++h) a[rb][h] = *reinterpret_cast<const uint4*>(base + roff[rb] + 16 * h);
        if (++lj == NU) {
            lj = 0;
            ++li;
        }
    };
    // --- digits of x. Thread task (s, g, i) covers the 4 k's of bytes 4 i .. 4 i + 3
    // of lane group g at step s; the tasks partition k, so the values loaded for
    // them also give the row maxima (and a non-finite flag). The x loads go out
    // first, then the first units' weight loads (which they would otherwise queue
    // behind), then the digits are staged.
    float xv[MT][TPT][4];
    float mx[MT];
    int bad[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        mx[m] = 0.0f;
        bad[m] = 0;
    }
#pragma unroll
    for (int tt = 0; tt < TPT; ++tt) {
        const uint32_t task = tid + 64 * NW * tt;
        const bool on = task < NS * 16;
        const uint32_t s = task >> 4, tg = (task >> 2) & 3, ti = task & 3;
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int pp = 0; pp < 4; ++pp) {
                const float v = (on && m < (int)p.M) ? p.x[(size_t)m * K + i8_k<BITS, LPU>(s, tg, ti, pp)] : 0.0f;
                xv[m][tt][pp] = v;
                mx[m] = fmaxf(mx[m], fabsf(v));
                bad[m] |= !(fabsf(v) <= 3.40282347e38f);  // inf or NaN
            }
    }
    __builtin_amdgcn_sched_barrier(0);
    uint4 wa[D][RB][LPU];
    float ws[D][RB];
#pragma unroll
    for (int d = 0; d + 1 < D; ++d)
        if (T) load(wa[d], ws[d]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        mx[m] = g4a_wave_max(mx[m]);
        bad[m] = __any(bad[m]) ? 1 : 0;
        if (lane == 0) {
            redmax[wv][m] = mx[m];
            redbad[wv][m] = bad[m];
        }
    }
    __syncthreads();
    int xe[MT], xb[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        float M4 = redmax[0][m];
        xb[m] = redbad[0][m];
#pragma unroll
        for (int w = 1; w < NW; ++w) {
            M4 = fmaxf(M4, redmax[w][m]);
            xb[m] |= redbad[w][m];
        }
        xe[m] = 0;
        if (M4 > 0.0f) frexpf(M4, &xe[m]);  // M4 < 2^e
    }
#pragma unroll
    for (int tt = 0; tt < TPT; ++tt) {
        const uint32_t task = tid + 64 * NW * tt;
        if (task >= NS * 16) break;
        const uint32_t s = task >> 4, tg = (task >> 2) & 3, ti = task & 3;
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            uint32_t dg[LI8_NSL];
#pragma unroll
            for (int j = 0; j < LI8_NSL; ++j) dg[j] = 0;
            if (!xb[m]) {
#pragma unroll
                for (int pp = 0; pp < 4; ++pp) {
                    float u = ldexpf(xv[m][tt][pp], 6 - xe[m]);
#pragma unroll
                    for (int j = 0; j < LI8_NSL; ++j) {
                        const float b = rintf(u);
                        dg[j] |= ((uint32_t)(int)b & 0xFFu) << (8 * pp);
                        u = (u - b) * 128.0f;
                    }
                }
            }
#pragma unroll
            for (int j = 0; j < LI8_NSL; ++j) bsh[(s * 64 + 16 * tg + 8 * m + j) * 4 + ti] = dg[j];
        }
        if constexpr (MT == 1) {
#pragma unroll
            for (int j = 8; j < 16; ++j) bsh[(s * 64 + 16 * tg + j) * 4 + ti] = 0u;
        }
    }
    __syncthreads();
    const int my_e = xe[0] + (MT > 1 && om == 1 ? xe[MT - 1] - xe[0] : 0);
    const int my_bad = MT > 1 && om == 1 ? xb[MT - 1] : xb[0];

    i4v acc[RB];
    float cur_s[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        acc[rb] = i4v{0, 0, 0, 0};
        cur_s[rb] = 0.0f;
    }
    uint32_t si = 0, sj = 0;  // the unit to compute
    auto step = [&](const uint4 (&a)[RB][LPU], const float (&sc)[RB], bool live) {
        const uint32_t c = chunk(si), j = sj;
        if (++sj == NU) {
            sj = 0;
            ++si;
        }
        if (j == 0) {
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) cur_s[rb] = sc[rb];
        }
#pragma unroll
        for (int h = 0; h < LPU; ++h)
#pragma unroll
            for (int tt = 0; tt < MPS; ++tt) {
                const uint32_t st = (LPU * j + h) * MPS + tt;
                const uint4 bw = *reinterpret_cast<const uint4*>(bsh + (st * 64 + lane) * 4);
                const i4v bv = i4v{(int)bw.x, (int)bw.y, (int)bw.z, (int)bw.w};
#pragma unroll
                for (int rb = 0; rb < RB; ++rb) {
                    i4v av;
                    if (tt == 0) av = i8_operand<BITS, 0>(a[rb][h], p.xm);
                    if (tt == 1) av = i8_operand<BITS, (MPS > 1 ? 1 : 0)>(a[rb][h], p.xm);
                    if (tt == 2) av = i8_operand<BITS, (MPS > 2 ? 2 : 0)>(a[rb][h], p.xm);
                    if (tt == 3) av = i8_operand<BITS, (MPS > 3 ? 3 : 0)>(a[rb][h], p.xm);
                    acc[rb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bv, acc[rb], 0, 0, 0);
                }
            }
        if (j + 1 == NU) {
            // the chunk's digit-column sums are complete: weight column j by 2^(-7 j),
            // sum the LI8_NSL columns of each activation row (8 lanes), scale, store
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                float tot[4];
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    float x = ldexpf((float)acc[rb][v], -7 * jj);
                    x += g4a_dpp<G4A_DPP_XOR1>(x);
                    x += g4a_dpp<G4A_DPP_XOR2>(x);
                    x += g4a_dpp<G4A_DPP_HALF_MIRROR>(x);
                    tot[v] = x;
                }
                acc[rb] = i4v{0, 0, 0, 0};
                const uint32_t n = 16 * (RB * c + rb) + 4 * g + jj;
                if (live && jj < 4 && om < (int)p.M && n < N) {
                    const float tv = jj == 0 ? tot[0] : jj == 1 ? tot[1] : jj == 2 ? tot[2] : tot[3];
                    float o;
                    if (!my_bad) {
                        o = (float)((double)tv * (double)cur_s[rb] * ldexp(1.0, my_e - 6 - F::LOG2F));
                    } else {
                        o = 0.0f;  // the CPU's order (an inf or NaN in the row)
                        const float* __restrict__ xr = p.x + (size_t)om * K;
                        for (uint32_t k = 0; k < K; ++k)
                            o += xr[k] * deq(p.wb, p.s, p.bits, p.row_bytes, p.group_size, p.scale_stride,
                                             p.signed_i8, n, k);
                    }
                    p.y[(size_t)om * N + n] = o;
                }
            }
        }
    };

    // Whole groups of D units, no branch between them; units past T (at most
    // D - 1) re-read the wave's last unit and store nothing.
    for (uint32_t t = 0; t < T; t += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            load(wa[(d + D - 1) % D], ws[(d + D - 1) % D]);
            __builtin_amdgcn_sched_barrier(0);
            step(wa[d], ws[d], t + d < T);
        }
    }
}

// embed_rows on a quantised table (rust/src/backend_cpu.rs:127-137): one thread
// per output element.
__device__ __forceinline__ void embed_rows_q(const G4aEmbedParams& p) {
    const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= (size_t)p.T * p.D) return;
    const uint32_t i = (uint32_t)(e / p.D), d = (uint32_t)(e % p.D);
    p.out[e] = deq(p.wb, p.s, p.bits, p.row_bytes, p.group_size, p.scale_stride, p.signed_i8, p.ids[i], d) * p.scale;
}

}  // namespace

// Variants (activation rows MT, weight rows RU, loads in flight D steps):
// (1, 2, 4) short weights at M = 1, (1, 8, 2) tall weights at M = 1, (4, 4, 2) M >= 2.
#define G4A_LINEAR_WORDS(B, MT, RU, D, MODE)                                                            \
    extern "C" __global__ __launch_bounds__(256) void g4a_linear_q_b##B##_m##MT##_r##RU##_mode##MODE( \
        G4aLinearParams p) {                                                                           \
        linear_q_words<B, MT, RU, D, MODE>(p);                                                         \
    }
#define G4A_LINEAR_SET(B, MODE) \
    G4A_LINEAR_WORDS(B, 1, 2, 4, MODE) G4A_LINEAR_WORDS(B, 1, 8, 2, MODE) G4A_LINEAR_WORDS(B, 4, 4, 2, MODE)
// 32 lanes per row (two rows per wave step), M = 1, for rows of an odd multiple of 32 words
#define G4A_LINEAR_HALF(B, RU, D, MODE)                                                                  \
    extern "C" __global__ __launch_bounds__(256) void g4a_linear_q_b##B##_m1_r##RU##_h_mode##MODE(  \
        G4aLinearParams p) {                                                                           \
        linear_q_words<B, 1, RU, D, MODE, 32>(p);                                                      \
    }
G4A_LINEAR_HALF(2, 1, 4, 0)
G4A_LINEAR_HALF(2, 4, 2, 0)
G4A_LINEAR_HALF(2, 1, 4, 1)
G4A_LINEAR_HALF(2, 4, 2, 1)
G4A_LINEAR_HALF(2, 1, 4, 2)
G4A_LINEAR_HALF(2, 4, 2, 2)
G4A_LINEAR_SET(2, 0)
G4A_LINEAR_SET(2, 1)
G4A_LINEAR_SET(2, 2)
G4A_LINEAR_SET(4, 0)
G4A_LINEAR_SET(4, 1)
G4A_LINEAR_SET(4, 2)
G4A_LINEAR_SET(8, 0)
G4A_LINEAR_SET(8, 1)
G4A_LINEAR_SET(8, 2)
// mode 3: a decode step's output projection, merging the split partials while staging x
G4A_LINEAR_WORDS(2, 1, 2, 4, 3)
G4A_LINEAR_WORDS(4, 1, 2, 4, 3)
G4A_LINEAR_WORDS(8, 1, 2, 4, 3)

#define G4A_LINEAR_MFMA(B, MODE)                                                                     \
    extern "C" __global__ __launch_bounds__(256) void g4a_linear_q_mfma_b##B##_n64_mode##MODE(G4aLinearParams p) {  \
        linear_q_mfma<B, 1, MODE>(p);                                                                \
    }                                                                                                \
    extern "C" __global__ __launch_bounds__(256) void g4a_linear_q_mfma_b##B##_n128_mode##MODE(G4aLinearParams p) { \
        linear_q_mfma<B, 2, MODE>(p);                                                                \
    }
G4A_LINEAR_MFMA(2, 0)
G4A_LINEAR_MFMA(2, 1)
G4A_LINEAR_MFMA(2, 2)
G4A_LINEAR_MFMA(4, 0)
G4A_LINEAR_MFMA(4, 1)
G4A_LINEAR_MFMA(4, 2)
G4A_LINEAR_MFMA(8, 0)
G4A_LINEAR_MFMA(8, 1)
G4A_LINEAR_MFMA(8, 2)

// int8 matrix cores, M <= MT, MODE 0: (bits, MT); 2 A blocks per chunk, units of
// 128 row bytes, one unit in flight ahead of the one computing
#define G4A_LINEAR_I8(B, MT)                                                                              \
    extern "C" __global__ __launch_bounds__(G4A_LI8_THREADS) void g4a_linear_q_i8_b##B##_m##MT(             \
        G4aLinearParams p) {                                                                              \
        linear_q_i8<B, MT, 2, 2, G4A_LI8_UNIT_BYTES / 64, G4A_LI8_THREADS / 64>(p);                        \
    }
G4A_LINEAR_I8(2, 1)
G4A_LINEAR_I8(2, 2)
G4A_LINEAR_I8(4, 1)
G4A_LINEAR_I8(4, 2)
G4A_LINEAR_I8(8, 1)
G4A_LINEAR_I8(8, 2)

G4A_LINEAR_WORDS(32, 1, 2, 4, 0)
G4A_LINEAR_WORDS(32, 1, 8, 2, 0)
G4A_LINEAR_WORDS(32, 4, 4, 2, 0)
extern "C" __global__ __launch_bounds__(64) void g4a_linear_f32_elem(G4aLinearParams p) { linear_f32_elem(p); }

extern "C" __global__ __launch_bounds__(64) void g4a_linear_q_elem_mode0(G4aLinearParams p) { linear_q_elem<0>(p); }
extern "C" __global__ __launch_bounds__(64) void g4a_linear_q_elem_mode1(G4aLinearParams p) { linear_q_elem<1>(p); }
extern "C" __global__ __launch_bounds__(64) void g4a_linear_q_elem_mode2(G4aLinearParams p) { linear_q_elem<2>(p); }
extern "C" __global__ __launch_bounds__(256) void g4a_embed_rows_q(G4aEmbedParams p) { embed_rows_q(p); }
