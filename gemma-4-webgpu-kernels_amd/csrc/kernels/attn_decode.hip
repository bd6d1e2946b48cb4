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
// Work decomposition. A workgroup is 8 waves (512 threads) and owns one key
// split of one (query, kv head); the host picks the split count so the grid
// covers every CU (k_start/k_end already trimmed to the visible range). K and
// V stream from HBM straight into LDS with global->LDS copies
// (global_load_lds_dwordx4), several chunks ahead of the one in use.
//   - decode_wave (groups of 8 heads, Gemma-4's MQA): every wave streams its
//     own 16-key wave tiles through a private LDS ring and never waits for
//     another wave inside the loop; lane = (key, head pair) for the scores,
//     lane = output dims for P.V (fused multiply-adds);
//   - decode_split (groups of 4 heads): slots of waves share 64-key tiles
//     through a common ring with a barrier per chunk; P.V on the matrix cores.
// At the end the waves' partials merge through LDS and the split's (m, l, acc)
// partial is written, or the normalised output when there is a single split;
// a separate combine kernel merges the partials (log-sum-exp).
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "g4a_math.h"
#include "g4a_params.h"

namespace {

constexpr float NEG_INF = G4A_NEG_INF;

__device__ __forceinline__ float wave_max(float x) { return g4a_wave_max(x); }
__device__ __forceinline__ float wave_sum(float x) { return g4a_wave_sum(x); }

__device__ __forceinline__ float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }
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

// A decode step whose query position lives in device memory (G4aDecodeParams::dpos,
// g4a_attention_devpos): the position is read at run time and the key range follows
// from it (keys k_pos0 .. qpos, the last `window` of them), so a captured step
// replays at whatever position the counter holds. The planned k_end bounds the
// range: a counter past the plan reads no key beyond it.
__device__ __forceinline__ G4aDecodeParams at_device_pos(const G4aDecodeParams& p) {
    G4aDecodeParams r = p;
    if (p.dpos) {
        const uint32_t qp = __builtin_amdgcn_readfirstlane(*p.dpos);
        const uint32_t n = qp >= p.k_pos0 ? qp - p.k_pos0 + 1u : 0u;  // keys at or before the query
        const uint32_t lo = (p.window && n > p.window) ? n - p.window : 0u;
        r.q_pos0 = qp;
        r.k_end = min(n, p.k_end);
        r.k_start = min(lo, r.k_end);
    }
    return r;
}

// Split partials: the acc value of row ih (= query * Hq + head), split s, dim d
// sits at (ih * nsplit + s) * DH + d: a split's row of a head is one contiguous
// run of DH floats, so the decode kernels' final stores are whole 2 KiB rows
// (at hd512 @32K the workgroups' scattered 64-byte stores had cost ~0.25 us
// more at the end of the launch); the combine reads split s of a head at stride
// DH. The (m, l) pairs follow all acc values: [ih][s][2].
template <int DH>
__device__ __forceinline__ size_t part_index(size_t ih, uint32_t nsplit, uint32_t s, uint32_t d) {
    return (ih * nsplit + s) * DH + d;
}

// Sixteen dims (16B .. 16B+15 of a 64-dim stage) of the exact dots of the two
// heads of a wave, lane = key: dot = ((dot + q[d]*k[d]) + q[d+1]*k[d+1]) + ...,
// every multiply and add rounded separately, in the CPU reference's order.
// q[h][16B + j] sits in lane j of every 16-lane row of qv[h][B]; each multiply
// takes it through a DPP row broadcast (row_newbcast:j) as its first operand,
// so the hot loop issues no scalar loads. Written as one asm block so every
// multiply is a single v_mul_f32_dpp; the leading s_nop covers the 2 wait
// states a DPP read needs after a VALU write of its source.
__device__ __forceinline__ void qk_dims16(float (&s)[2], float q0, float q1, const float4 (&k)[4]) {
    // the multiplies of a dimension are issued before the adds of the one before
    // it (two rotating temporary pairs), so no add waits for its own multiply
    float t0a, t0b, t1a, t1b;
    asm volatile(
        "s_nop 1\n\t"
        "v_mul_f32_dpp %[t0a], %[q0], %[k0] row_newbcast:0 row_mask:0xf bank_mask:0xf\n\t"
        "v_mul_f32_dpp %[t0b], %[q1], %[k0] row_newbcast:0 row_mask:0xf bank_mask:0xf\n\t"
        "v_mul_f32_dpp %[t1a], %[q0], %[k1] row_newbcast:1 row_mask:0xf bank_mask:0xf\n\t"
        "v_mul_f32_dpp %[t1b], %[q1], %[k1] row_newbcast:1 row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32 %[a0], %[a0], %[t0a]\n\t"
        "v_add_f32 %[a1], %[a1], %[t0b]\n\t"
        "v_mul_f32_dpp %[t0a], %[q0], %[k2] row_newbcast:2 row_mask:0xf bank_mask:0xf\n\t"
        "v_mul_f32_dpp %[t0b], %[q1], %[k2] row_newbcast:2 row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32 %[a0], %[a0], %[t1a]\n\t"
        "v_add_f32 %[a1], %[a1], %[t1b]\n\t"
        "v_mul_f32_dpp %[t1a], %[q0], %[k3] row_newbcast:3 row_mask:0xf bank_mask:0xf\n\t"
        "v_mul_f32_dpp %[t1b], %[q1], %[k3] row_newbcast:3 row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32 %[a0], %[a0], %[t0a]\n\t"
        "v_add_f32 %[a1], %[a1], %[t0b]\n\t"
        "v_mul_f32_dpp %[t0a], %[q0], %[k4] row_newbcast:4 row_mask:0xf bank_mask:0xf\n\t"
        "v_mul_f32_dpp %[t0b], %[q1], %[k4] row_newbcast:4 row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32 %[a0], %[a0], %[t1a]\n\t"
        "v_add_f32 %[a1], %[a1], %[t1b]\n\t"
        "v_mul_f32_dpp %[t1a], %[q0], %[k5] row_newbcast:5 row_mask:0xf bank_mask:0xf\n\t"
        "v_mul_f32_dpp %[t1b], %[q1], %[k5] row_newbcast:5 row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32 %[a0], %[a0], %[t0a]\n\t"
        "v_add_f32 %[a1], %[a1], %[t0b]\n\t"
        "v_mul_f32_dpp %[t0a], %[q0], %[k6] row_newbcast:6 row_mask:0xf bank_mask:0xf\n\t"
        "v_mul_f32_dpp %[t0b], %[q1], %[k6] row_newbcast:6 row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32 %[a0], %[a0], %[t1a]\n\t"
        "v_add_f32 %[a1], %[a1], %[t1b]\n\t"
        "v_mul_f32_dpp %[t1a], %[q0], %[k7] row_newbcast:7 row_mask:0xf bank_mask:0xf\n\t"
        "v_mul_f32_dpp %[t1b], %[q1], %[k7] row_newbcast:7 row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32 %[a0], %[a0], %[t0a]\n\t"
        "v_add_f32 %[a1], %[a1], %[t0b]\n\t"
        "v_mul_f32_dpp %[t0a], %[q0], %[k8] row_newbcast:8 row_mask:0xf bank_mask:0xf\n\t"
        "v_mul_f32_dpp %[t0b], %[q1], %[k8] row_newbcast:8 row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32 %[a0], %[a0], %[t1a]\n\t"
        "v_add_f32 %[a1], %[a1], %[t1b]\n\t"
        "v_mul_f32_dpp %[t1a], %[q0], %[k9] row_newbcast:9 row_mask:0xf bank_mask:0xf\n\t"
        "v_mul_f32_dpp %[t1b], %[q1], %[k9] row_newbcast:9 row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32 %[a0], %[a0], %[t0a]\n\t"
        "v_add_f32 %[a1], %[a1], %[t0b]\n\t"
        "v_mul_f32_dpp %[t0a], %[q0], %[k10] row_newbcast:10 row_mask:0xf bank_mask:0xf\n\t"
        "v_mul_f32_dpp %[t0b], %[q1], %[k10] row_newbcast:10 row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32 %[a0], %[a0], %[t1a]\n\t"
        "v_add_f32 %[a1], %[a1], %[t1b]\n\t"
        "v_mul_f32_dpp %[t1a], %[q0], %[k11] row_newbcast:11 row_mask:0xf bank_mask:0xf\n\t"
        "v_mul_f32_dpp %[t1b], %[q1], %[k11] row_newbcast:11 row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32 %[a0], %[a0], %[t0a]\n\t"
        "v_add_f32 %[a1], %[a1], %[t0b]\n\t"
        "v_mul_f32_dpp %[t0a], %[q0], %[k12] row_newbcast:12 row_mask:0xf bank_mask:0xf\n\t"
        "v_mul_f32_dpp %[t0b], %[q1], %[k12] row_newbcast:12 row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32 %[a0], %[a0], %[t1a]\n\t"
        "v_add_f32 %[a1], %[a1], %[t1b]\n\t"
        "v_mul_f32_dpp %[t1a], %[q0], %[k13] row_newbcast:13 row_mask:0xf bank_mask:0xf\n\t"
        "v_mul_f32_dpp %[t1b], %[q1], %[k13] row_newbcast:13 row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32 %[a0], %[a0], %[t0a]\n\t"
        "v_add_f32 %[a1], %[a1], %[t0b]\n\t"
        "v_mul_f32_dpp %[t0a], %[q0], %[k14] row_newbcast:14 row_mask:0xf bank_mask:0xf\n\t"
        "v_mul_f32_dpp %[t0b], %[q1], %[k14] row_newbcast:14 row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32 %[a0], %[a0], %[t1a]\n\t"
        "v_add_f32 %[a1], %[a1], %[t1b]\n\t"
        "v_mul_f32_dpp %[t1a], %[q0], %[k15] row_newbcast:15 row_mask:0xf bank_mask:0xf\n\t"
        "v_mul_f32_dpp %[t1b], %[q1], %[k15] row_newbcast:15 row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32 %[a0], %[a0], %[t0a]\n\t"
        "v_add_f32 %[a1], %[a1], %[t0b]\n\t"
        "v_add_f32 %[a0], %[a0], %[t1a]\n\t"
        "v_add_f32 %[a1], %[a1], %[t1b]\n\t"
        : [a0] "+v"(s[0]), [a1] "+v"(s[1]), [t0a] "=&v"(t0a), [t0b] "=&v"(t0b), [t1a] "=&v"(t1a), [t1b] "=&v"(t1b)
        : [q0] "v"(q0), [q1] "v"(q1), [k0] "v"(k[0].x), [k1] "v"(k[0].y), [k2] "v"(k[0].z), [k3] "v"(k[0].w), [k4] "v"(k[1].x), [k5] "v"(k[1].y), [k6] "v"(k[1].z), [k7] "v"(k[1].w), [k8] "v"(k[2].x), [k9] "v"(k[2].y), [k10] "v"(k[2].z), [k11] "v"(k[2].w), [k12] "v"(k[3].x), [k13] "v"(k[3].y), [k14] "v"(k[3].z), [k15] "v"(k[3].w));
}

template <int DH, int GROUP>
struct DecodeCfg {
    static constexpr int KCD = 64;                       // dims per K chunk (64 keys x KCD dims)
    static constexpr int NCOL = KCD / 4;                 // 16-byte columns of a K chunk row
    static constexpr int HGW = GROUP / 2;                // waves per key-tile slot (2 heads each in the score phase)
    static constexpr int KT = 8 / HGW;                   // key-tile slots per 8-wave workgroup
    static constexpr int SLOT_THREADS = 64 * HGW;
    static constexpr int LPT = 16 * KCD / SLOT_THREADS;  // 16-byte copies per lane per chunk
    static constexpr int NB = (8 / KT) * (64 / KCD);     // chunk buffers per slot (128 KiB ring in all)
    static constexpr int AHEAD = NB - 1;                 // chunks in flight ahead of the one in use
    static constexpr int NKS = DH / KCD;                 // K chunks per tile: 64 keys x KCD dims
    static constexpr int NVC = DH / KCD;                 // V chunks per tile: KPC keys x DH dims
    static constexpr int NCH = NKS + NVC;
    static constexpr int KPC = 64 / NVC;                 // keys per V chunk
    static constexpr int BUF = 64 * KCD;                 // floats per chunk buffer
    static constexpr int WD = DH / HGW;                  // output dims per wave in the P.V phase
    static constexpr int NDG = WD / 64;                  // 64-dim MFMA groups per wave
    static constexpr int NHQ = GROUP / 4;                // head quarters (4x4x1 P.V)
    static constexpr int NACC = NHQ * NDG;               // 4-register accumulators per wave
    static constexpr int RING = KT * NB * BUF;
    static constexpr int MERGE = (KT - 1) * HGW * NACC * 256;  // slots 1.. hand their accumulators to slot 0
    static constexpr int PBUF = KT * 64 * GROUP;
    static constexpr int QS = GROUP * DH;                // the kv group's query rows
    static constexpr int SMEM = RING + PBUF + KT * GROUP + KT * 2 * GROUP + QS;
    static_assert(MERGE <= RING, "the merge buffer overlays the chunk ring");
    static_assert(NCH % NB == 0, "the ring buffer of a chunk must be static within a tile");
    static_assert(KPC * DH == BUF, "a V chunk fills a chunk buffer");
    static_assert(NDG >= 1, "a wave owns at least one 64-dim group");
    static_assert(QS % 256 == 0, "the query rows are copied in 1 KiB wave copies");
    static_assert(LPT * (AHEAD - 1) + 2 * (QS / 256 + 7) / 8 < 64, "vmcnt immediate range");
};

// Asynchronous 16-byte-per-lane copy global -> LDS (global_load_lds_dwordx4):
// lane l's 16 bytes at `src` land at lds_dst + 16*l; lds_dst must be
// wave-uniform (it goes through M0, after which the copy needs one wait state).
// Completion is tracked by vmcnt like any vector load. Written as inline asm so
// the compiler does not serialise every later LDS read behind all copies in
// flight: the kernel waits for each chunk itself (wait_vm) before a barrier.
// M0 is declared clobbered, so the compiler never keeps a value of its own in
// M0 across a copy.
// NT marks the load non-temporal: for K/V that a long-context decode streams
// once (measured 28.1 -> 27.0 us at 32K). Short contexts keep the default
// policy: a token's small caches are reread by the next token.
template <bool NT = false>
__device__ __forceinline__ void copy16_to_lds(const float* src, float* lds_dst) {
    const uint32_t m0 = (uint32_t)(uintptr_t)((__attribute__((address_space(3))) float*)lds_dst);
    if constexpr (NT)
        asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(src), "{m0}"(m0) : "memory");
    else
        asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(m0) : "memory");
}

// The same copy addressed as a wave-uniform 64-bit base (SGPRs) plus a 32-bit
// per-lane byte offset: a stream whose lanes keep fixed offsets from a moving
// base needs no per-copy vector address arithmetic (the decode loop issued ~11
// VALU instructions per copy, two of them 64-bit multiplies, before this form).
template <bool NT = false>
__device__ __forceinline__ void copy16s_to_lds(const void* sbase, uint32_t voff, float* lds_dst) {
    const uint32_t m0 = (uint32_t)(uintptr_t)((__attribute__((address_space(3))) float*)lds_dst);
    if constexpr (NT)
        asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1 nt" ::"v"(voff), "s"(sbase), "{m0}"(m0) : "memory");
    else
        asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "{m0}"(m0) : "memory");
}

// The same copy with 4 bytes per lane (global_load_lds_dword): lane l's 4 bytes
// at `src` land at lds_dst + 4*l (lanes switched off by the exec mask write nothing).
__device__ __forceinline__ void copy4_to_lds(const void* src, void* lds_dst) {
    const uint32_t m0 = (uint32_t)(uintptr_t)((__attribute__((address_space(3))) char*)lds_dst);
    asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(src), "{m0}"(m0) : "memory");
}

// Wait until at most N vector-memory operations of this wave are in flight
// (they retire in issue order, so every copy issued before the last N has landed).
template <int N>
__device__ __forceinline__ void wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// wait_vm<n>() for an n known only after loop unrolling (it folds to one
// s_waitcnt); counts above 16 wait for everything, which is always safe.
__device__ __forceinline__ void wait_vm_upto16(int n) {
    switch (n) {
#define G4A_WAIT_CASE(k) \
    case k: wait_vm<k>(); break;
        G4A_WAIT_CASE(1) G4A_WAIT_CASE(2) G4A_WAIT_CASE(3) G4A_WAIT_CASE(4) G4A_WAIT_CASE(5) G4A_WAIT_CASE(6)
        G4A_WAIT_CASE(7) G4A_WAIT_CASE(8) G4A_WAIT_CASE(9) G4A_WAIT_CASE(10) G4A_WAIT_CASE(11) G4A_WAIT_CASE(12)
        G4A_WAIT_CASE(13) G4A_WAIT_CASE(14) G4A_WAIT_CASE(15) G4A_WAIT_CASE(16)
#undef G4A_WAIT_CASE
        default: wait_vm<0>(); break;
    }
}

// Workgroup barrier for LDS hand-offs: this wave's LDS reads and writes are
// complete (lgkmcnt(0)) before it arrives. Unlike __syncthreads it does not
// wait for outstanding global->LDS copies, which keep streaming across it.
__device__ __forceinline__ void barrier_lds() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Split-K flash decode (see the file header). An 8-wave workgroup owns one key
// split of one (query, kv head); its waves form KT key-tile slots of HGW waves.
// Every slot streams, per 64-key tile, DH/64 K chunks (64 keys x 64 dims) and
// DH/64 V chunks (KPC keys x DH dims) of 16 KiB straight from HBM into a ring
// of NB LDS chunk buffers with global->LDS copies, AHEAD chunks ahead of the
// one in use, so K and V form one continuous stream across phases and tiles.
// In LDS a K chunk is stored row-major (64 floats per key) with the 16-byte
// column index XOR-swizzled by the key's low 4 bits, so the lane = key reads of
// the score phase hit distinct banks.
//   score phase: wave g of a slot owns heads 2g, 2g+1 (lane = key);
//   P.V phase:   wave g of a slot owns output dims [g*WD, (g+1)*WD) of all
//                GROUP heads, so a slot's accumulators never need summing;
//   end:         slots 1.. hand (m, l, acc) to slot 0 through LDS, which
//                merges them and writes the split's partial (or the output).
//
// KPOS selects explicit key positions (p.k_pos, a device array) over contiguous
// ones (k_pos0 + j). It is a template parameter so the contiguous kernel issues
// no vector loads of its own inside the streaming loop: every vector-memory
// wait there is one of the kernel's own chunk waits.
template <int DH, int GROUP, bool KPOS>
__device__ __forceinline__ void decode_split(const G4aDecodeParams& p) {
    static_assert(DH == 256 || DH == 512, "fast decode handles head_dim 256 / 512");
    static_assert(GROUP == 4 || GROUP == 8, "fast decode handles groups of 4 / 8 heads");
    using C = DecodeCfg<DH, GROUP>;
    constexpr int HGW = C::HGW, KT = C::KT, LPT = C::LPT, NB = C::NB, AHEAD = C::AHEAD, NKS = C::NKS,
                  KCD = C::KCD, NCOL = C::NCOL,
                  NCH = C::NCH, KPC = C::KPC, BUF = C::BUF, WD = C::WD, NDG = C::NDG, NHQ = C::NHQ,
                  NACC = C::NACC;

    __shared__ __attribute__((aligned(16))) float smem[C::SMEM];
    float* const ring = smem;                     // [KT][NB][BUF]
    float* const mrg = smem;                      // [KT-1][HGW][NACC][4][64] after the tile loop
    float* const pbuf = smem + C::RING;           // [KT][64 keys][4][NHQ]
    float* const corrbuf = pbuf + C::PBUF;        // [KT][GROUP]
    float* const mlbuf = corrbuf + KT * GROUP;    // [KT][2][GROUP]
    float* const qs = mlbuf + KT * 2 * GROUP;     // [GROUP][DH] query rows of this kv group

    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = w % HGW;   // score phase: heads 2g, 2g+1; P.V phase: dims [g*WD, (g+1)*WD)
    const int kt = w / HGW;  // key-tile slot
    const uint32_t split = blockIdx.x, qi = blockIdx.y, kvh = blockIdx.z;
    const uint32_t qpos = p.q_pos ? p.q_pos[qi] : p.q_pos0 + qi;
    const uint32_t ks = p.k_start + split * p.keys_per_split;
    const uint32_t ke = min(ks + p.keys_per_split, p.k_end);
    const uint32_t h0 = kvh * GROUP;
    const size_t row_stride = (size_t)p.Hkv * DH;
    const float* __restrict__ kbase = p.k + (size_t)kvh * DH;
    const float* __restrict__ vbase = p.v + (size_t)kvh * DH;
    float* const my_ring = ring + kt * NB * BUF;
    float* const my_pbuf = pbuf + kt * 64 * GROUP;

    // The query rows go to LDS first (copies issued before every chunk, so the
    // first chunk wait covers them).
    {
        const float* qsrc = p.q + ((size_t)qi * p.Hq + h0) * DH;
        for (int i = w; i < C::QS / 256; i += 8) copy16_to_lds(qsrc + 256 * i + 4 * lane, qs + 256 * i);
    }

    float m[2] = {NEG_INF, NEG_INF}, lpart[2] = {0.0f, 0.0f};
    // acc[NDG*hq + dg] register r of lane l is head 4*hq + r, dim g*WD + 64*dg + l.
    f4v acc[NACC];
#pragma unroll
    for (int a = 0; a < NACC; ++a) acc[a] = f4v{0.0f, 0.0f, 0.0f, 0.0f};

    const uint32_t ntiles = ke > ks ? (ke - ks + 63) / 64 : 0;
    const uint32_t niter = (ntiles + KT - 1) / KT;

    // Copies are issued for every chunk step whether or not the slot has a tile,
    // so the number in flight is the same on every path and each chunk's wait
    // count is exact; an idle slot copies from the small dummy buffer (which
    // stays in L2) into its ring instead of K/V.
    struct Tile {
        uint32_t t0, row0, nk;
        bool active;
        const float* kb;
        const float* vb;
    };
    auto tile_info = [&](uint32_t it) -> Tile {
        Tile T;
        const uint32_t t = it * KT + kt;
        T.t0 = ks + t * 64;
        T.active = it < niter && t < ntiles;
        if (T.active) {
            const uint32_t kpos_first = KPOS ? p.k_pos[T.t0] : p.k_pos0 + T.t0;
            T.active = kpos_first <= qpos;  // ascending positions: a future first key means a future tile
        }
        T.nk = T.active ? min(64u, ke - T.t0) : 1u;
        T.row0 = T.active ? phys_row(T.t0, p.ring_cap) : 0u;
        T.kb = T.active ? kbase : p.dummy;
        T.vb = T.active ? vbase : p.dummy;
        return T;
    };
    auto prow = [&](const Tile& T, uint32_t r) -> uint32_t {  // physical row of tile key r, clamped to the tile
        uint32_t x = T.row0 + min(r, T.nk - 1);
        if (p.ring_cap && x >= p.ring_cap) x -= p.ring_cap;
        return x;
    };
    // chunk c of a tile into ring buffer `bi`: K chunks c < NKS (dims 64c..64c+63 of
    // the 64 keys), V chunks c >= NKS (keys KPC*(c-NKS) .. +KPC-1, all DH dims).
    // Wave g of the slot fills float4 slots (i*HGW + g)*64 + lane, i < LPT.
    auto issue_chunk = [&](const Tile& T, int c, int bi) {
        float* const dst = my_ring + bi * BUF;
#pragma unroll
        for (int i = 0; i < LPT; ++i) {
            const int sl = (i * HGW + g) * 64 + lane;
            const float* src;
            if (c < NKS) {
                const int r = sl / NCOL;
                const int j = (sl % NCOL) ^ (r % NCOL);
                src = T.kb + (size_t)prow(T, r) * row_stride + KCD * c + 4 * j;
            } else {
                const int key = (c - NKS) * KPC + sl / (DH / 4);
                src = T.vb + (size_t)prow(T, key) * row_stride + 4 * (sl % (DH / 4));
            }
            copy16_to_lds<true>(src, dst + (i * HGW + g) * 256);
        }
    };

    Tile cur = tile_info(0);
#pragma unroll
    for (int c = 0; c < AHEAD; ++c) issue_chunk(cur, c, c % NB);

    const float* const my_q = qs + 2 * g * DH;  // heads 2g, 2g+1
    // this lane's key row in a K chunk and its swizzled float4 columns
    const float* kcol[NCOL];
#pragma unroll
    for (int j = 0; j < NCOL; ++j) kcol[j] = my_ring + lane * KCD + 4 * (j ^ (lane % NCOL));

    for (uint32_t it = 0; it < niter; ++it) {
        const bool last = it + 1 == niter;  // no copies beyond the last tile step
        const Tile nxt = tile_info(it + 1);
        float s[2] = {0.0f, 0.0f};
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            const int bi = c % NB;
            const float* const buf = my_ring + bi * BUF;
            // this wave's part of chunk c has landed (the copies issued after it are the
            // next AHEAD-1 chunks, fewer at the end of the last tile); after the barrier
            // every wave's has, and every wave is done with the buffer the next copy refills
            if (c + AHEAD > NCH && last) wait_vm_upto16(LPT * (NCH - 1 - c));
            else wait_vm<LPT * (AHEAD - 1)>();
            barrier_lds();
            if (c + AHEAD < NCH) issue_chunk(cur, c + AHEAD, (c + AHEAD) % NB);
            else if (!last) issue_chunk(nxt, c + AHEAD - NCH, (c + AHEAD) % NB);
            if (!cur.active) continue;
            if (c < NKS) {
                // exact sequential dots, lane = key, heads 2g and 2g+1, dims 64c .. 64c+63;
                // q comes from LDS, one value per lane of each 16-lane row, via DPP broadcast
#pragma unroll
                for (int b = 0; b < KCD / 16; ++b) {
                    const float q0 = my_q[KCD * c + 16 * b + (lane & 15)];
                    const float q1 = my_q[DH + KCD * c + 16 * b + (lane & 15)];
                    float4 k4[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) k4[i] = *reinterpret_cast<const float4*>(kcol[4 * b + i] + bi * BUF);
                    qk_dims16(s, q0, q1, k4);
                }
                if (c == NKS - 1) {
                    // online softmax for heads 2g, 2g+1 over the tile (lane = key)
                    const uint32_t j = cur.t0 + min((uint32_t)lane, cur.nk - 1);
                    const uint32_t kp = KPOS ? p.k_pos[j] : p.k_pos0 + j;
                    const bool vis = (uint32_t)lane < cur.nk && kp <= qpos && (p.window == 0 || qpos - kp < p.window);
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const float sc = vis ? score_epilogue(s[h], p.scale, p.softcap) : NEG_INF;
                        const float mn = fmaxf(m[h], wave_max(sc));
                        const float corr = (m[h] == NEG_INF) ? 0.0f : expf(m[h] - mn);
                        const float pr = (sc == NEG_INF) ? 0.0f : expf(sc - mn);
                        lpart[h] = lpart[h] * corr + pr;
                        m[h] = mn;
                        const int hl = 2 * g + h;  // head within the kv group
                        my_pbuf[lane * GROUP + (hl & 3) * NHQ + (hl >> 2)] = pr;
                        if (lane == 0) corrbuf[kt * GROUP + hl] = corr;
                    }
                }
            } else {
                const int vc = c - NKS;
                if (vc == 0) {
                    // rescale the running output of every head by its correction factor
#pragma unroll
                    for (int hq = 0; hq < NHQ; ++hq) {
                        const float* cb = corrbuf + kt * GROUP + hq * 4;
                        const f4v cr = f4v{cb[0], cb[1], cb[2], cb[3]};
#pragma unroll
                        for (int dg = 0; dg < NDG; ++dg) acc[NDG * hq + dg] *= cr;
                    }
                }
                // P.V on v_mfma_f32_4x4x1_16b_f32, one key per step:
                // lane l gives A = P[key][4hq + l%4] and B = V[key][g*WD + 64dg + l];
                // register r of the result is out[4hq + r][g*WD + 64dg + l]
#pragma unroll
                for (int kr = 0; kr < KPC; ++kr) {
                    const int kk = vc * KPC + kr;  // key within the tile
                    float a[NHQ];
#pragma unroll
                    for (int hq = 0; hq < NHQ; ++hq) a[hq] = my_pbuf[kk * GROUP + (lane & 3) * NHQ + hq];
#pragma unroll
                    for (int dg = 0; dg < NDG; ++dg) {
                        const float vv = buf[kr * DH + g * WD + 64 * dg + lane];
#pragma unroll
                        for (int hq = 0; hq < NHQ; ++hq)
                            acc[NDG * hq + dg] =
                                __builtin_amdgcn_mfma_f32_4x4x1f32(a[hq], vv, acc[NDG * hq + dg], 0, 0, 0);
                    }
                }
            }
        }
        cur = nxt;
    }

    wait_vm<0>();  // no copy may still be landing in the ring the merge buffer overlays
    // ---- per-slot (m, l) through LDS; slots 1.. hand their accumulators to slot 0 ----
#pragma unroll
    for (int h = 0; h < 2; ++h) lpart[h] = wave_sum(lpart[h]);
    if (lane == 0) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            mlbuf[kt * 2 * GROUP + 2 * g + h] = m[h];
            mlbuf[kt * 2 * GROUP + GROUP + 2 * g + h] = lpart[h];
        }
    }
    __syncthreads();  // every wave is done with the chunk ring: the merge buffer overlays it
    auto mslot = [&](int sl, int a, int r) -> float* {
        return mrg + ((((size_t)(sl - 1) * HGW + g) * NACC + a) * 4 + r) * 64 + lane;
    };
    if (kt > 0) {
#pragma unroll
        for (int a = 0; a < NACC; ++a)
#pragma unroll
            for (int r = 0; r < 4; ++r) *mslot(kt, a, r) = acc[a][r];
    }
    __syncthreads();
    if (kt != 0) return;
    // head h of the kv group: M = max over slots, L = sum of l * e^(m - M), es = slot weights
    auto head_stats = [&](int h, float& M, float& L, float (&es)[KT]) {
        M = NEG_INF;
#pragma unroll
        for (int sl = 0; sl < KT; ++sl) M = fmaxf(M, mlbuf[sl * 2 * GROUP + h]);
        L = 0.0f;
#pragma unroll
        for (int sl = 0; sl < KT; ++sl) {
            const float ms = mlbuf[sl * 2 * GROUP + h];
            es[sl] = (ms == NEG_INF) ? 0.0f : expf(ms - M);
            L += mlbuf[sl * 2 * GROUP + GROUP + h] * es[sl];
        }
    };
    auto merged = [&](int a, int r, const float (&es)[KT]) -> float {
        float o = acc[a][r] * es[0];
#pragma unroll
        for (int sl = 1; sl < KT; ++sl) o += *mslot(sl, a, r) * es[sl];
        return o;
    };
    auto write_ml = [&](size_t ih, float M, float L) {
        float* ml = p.part + (size_t)p.T * p.Hq * p.nsplit * DH + (ih * p.nsplit + split) * 2;
        ml[0] = M;
        ml[1] = L;
    };
#pragma unroll
    for (int hq = 0; hq < NHQ; ++hq) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int h = 4 * hq + r;
            float M, L, es[KT];
            head_stats(h, M, L, es);
            const size_t ih = (size_t)qi * p.Hq + h0 + h;
            const float inv = L > 0.0f ? 1.0f / L : 0.0f;
#pragma unroll
            for (int dg = 0; dg < NDG; ++dg) {
                const float o = merged(NDG * hq + dg, r, es);
                const int d = g * WD + 64 * dg + lane;
                if (p.nsplit == 1) p.out[ih * DH + d] = o * inv;
                else p.part[part_index<DH>(ih, p.nsplit, split, d)] = o;
            }
            if (p.nsplit > 1 && g == 0 && lane == 0) write_ml(ih, M, L);
        }
    }
}

// Per-wave streaming decode for groups of 8 query heads (Gemma-4's 8:1 MQA).
// An 8-wave workgroup owns one key split of one (query, kv head), as in
// decode_split, but its waves never synchronise inside the streaming loop:
// wave w owns the split's 16-key wave tiles u = 8*it + w (the split's tiles
// are every nsplit-th tile of the key range, see below) and streams their K
// and V rows into a private LDS ring of NB 4 KiB chunks, one chunk ahead of
// the one it computes on, so each wave waits only for its own copies (vmcnt)
// and a slow wave delays nobody. Per wave tile, DH/64 K chunks (16 keys x 64 dims, 16-byte columns
// XOR-swizzled by key) then 16/KPC V chunks (KPC keys x DH dims):
//   scores: lane l = (key l%16, head pair l/16): heads 2(l/16), 2(l/16)+1 of
//           key l%16, the exact sequential dot of qk_dims16 (each 16-lane row
//           broadcasts its own head pair's query values);
//   softmax: online, per head, over the 16 keys of a row;
//   P.V:    lane l owns dims 4l..4l+3 (+256 for DH 512) of all 8 heads, fused
//           multiply-adds with the probabilities broadcast from LDS.
// At the end the 8 wave partials (m, l, acc) merge through LDS (wave w merges
// head w) into the split's partial, or the normalised output for one split.
template <int DH>
struct WaveCfg {
    static constexpr int GROUP = 8;
    static constexpr int KEYS = 16;                   // keys per wave tile
    // 4 KiB chunks in a 4-deep ring; 8 KiB chunks in a 2-deep ring (the same LDS, twice
    // the bytes in flight, half the chunk steps) measured 25.7 against 24.9 us at 32K keys
    static constexpr int BUF = 1024;                  // floats per chunk buffer (4 KiB)
    static constexpr int NB = 4;                      // chunk buffers per wave (16 KiB: the merge's partial)
    static constexpr int KCD = BUF / KEYS;            // dims per K chunk (16 keys x KCD dims)
    static constexpr int NCOL = KCD / 4;              // 16-byte columns of a K chunk row
    // Chunks in flight beyond the one in use. One beats three (8 MB instead of
    // 24 MB outstanding over the GPU): hd512 decode at 32K keys 25.05 -> 24.69 us,
    // at 131072 keys 83.8 -> 81.4 us; only calls forced to a few splits (8 or 32
    // workgroups at 131072 keys) lose, ~1.5 %. Zero is 15 % slower.
    static constexpr int AHEAD = 1;
    static constexpr int LPT = BUF / 256;             // 16-byte copies per lane per chunk
    static constexpr int NKS = DH / KCD;              // K chunks per wave tile
    static constexpr int KPC = BUF / DH;              // keys per V chunk
    static constexpr int NVC = KEYS / KPC;            // V chunks per wave tile
    static constexpr int NCH = NKS + NVC;
    static constexpr int ND = DH / 256;               // float4 dim groups per lane in P.V
    static constexpr int RING = 8 * NB * BUF;
    static constexpr int MERGE = GROUP * DH;          // a wave's partial, in its own ring after the loop
    static constexpr int QS = GROUP * DH;
    static constexpr int PB = 8 * KEYS * GROUP;       // [wave][key][head]
    static constexpr int SMEM = RING + QS + PB + 8 * GROUP + 8 * 2 * GROUP + 8;
    static constexpr int KPB = 8 * 2 * KEYS;          // explicit positions: [wave][tile parity][key]
    static_assert(MERGE <= NB * BUF, "a wave's partial fits its ring");
    static_assert(NCOL >= KEYS && NCOL % 4 == 0, "the K column swizzle (column ^ key) stays inside a row");
    static_assert(KPC * DH == BUF && KEYS % KPC == 0, "V chunks hold whole keys of the tile");
    static_assert(QS % 2048 == 0, "the query rows are copied in 8 waves x 1 KiB copies");
    static_assert(LPT * AHEAD + QS / 2048 < 64, "vmcnt immediate range");
    static_assert(LPT * AHEAD <= 16, "tail waits go through wait_vm_upto16");
};

template <int DH, bool KPOS>
__device__ __forceinline__ void decode_wave(const G4aDecodeParams& p, uint32_t split, uint32_t qi) {
    using C = WaveCfg<DH>;
    constexpr int GROUP = C::GROUP, KEYS = C::KEYS, BUF = C::BUF, NB = C::NB, AHEAD = C::AHEAD, LPT = C::LPT,
                  NKS = C::NKS, KPC = C::KPC, NCH = C::NCH, ND = C::ND, KCD = C::KCD, NCOL = C::NCOL;

    __shared__ __attribute__((aligned(16))) float smem[C::SMEM + (KPOS ? C::KPB : 0)];
    float* const ring = smem;                   // [8 waves][NB][BUF]; after the loop wave w's
                                                // [GROUP][DH] partial in its ring
    float* const qs = smem + C::RING;           // [GROUP][DH]
    float* const pbuf = qs + C::QS;             // [8 waves][KEYS][GROUP]
    float* const corrbuf = pbuf + C::PB;        // [8 waves][GROUP]
    float* const mlbuf = corrbuf + 8 * GROUP;   // [8 waves][2][GROUP]
    int* const progress = reinterpret_cast<int*>(mlbuf + 8 * 2 * GROUP);  // [8 waves] chunk steps done

    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int key = lane & 15;  // score phase: key of the wave tile
    const int hp = lane >> 4;   // score phase: heads 2hp, 2hp+1
    const uint32_t kvh = blockIdx.z;
    const uint32_t qpos = p.q_pos ? p.q_pos[qi] : p.q_pos0 + qi;
    const uint32_t h0 = kvh * GROUP;
    const size_t row_stride = (size_t)p.Hkv * DH;
    const float* __restrict__ kbase = p.k + (size_t)kvh * DH;
    const float* __restrict__ vbase = p.v + (size_t)kvh * DH;
    float* const my_ring = ring + w * NB * BUF;
    float* const my_pbuf = pbuf + w * KEYS * GROUP;
    float* const my_corr = corrbuf + w * GROUP;
    uint32_t* const my_kp = reinterpret_cast<uint32_t*>(smem + C::SMEM) + w * 2 * KEYS;  // KPOS: [parity][key]

    // query rows: wave w copies 1 KiB pieces w, w + 8, ... (issued before any chunk)
    {
        const float* qsrc = p.q + ((size_t)qi * p.Hq + h0) * DH;
#pragma unroll
        for (int i = 0; i < C::QS / 2048; ++i)
            copy16_to_lds(qsrc + 256 * (w + 8 * i) + 4 * lane, qs + 256 * (w + 8 * i));
    }

    // This split's tiles are dealt round-robin over the whole key range: tile
    // split + u * nsplit of the ceil(nkeys / 16) tiles, u = 8 * it + w, so every
    // wave's reads spread over all of the cache's memory channels (contiguous
    // 128-key ranges per split measured ~0.8 us slower at 32K keys).
    const uint32_t ntiles_all = (p.k_end - p.k_start + KEYS - 1) / KEYS;
    const uint32_t ntiles = ntiles_all > split ? (ntiles_all - split + p.nsplit - 1) / p.nsplit : 0u;
    const uint32_t niter = (ntiles + 7) / 8;

    // As in decode_split, every chunk step issues its copies (idle tiles copy the
    // dummy buffer), so each wait count below is exact.
    struct Tile {
        uint32_t t0, row0, nk;
        bool active;
        bool whole;  // all KEYS keys in consecutive physical rows: the copies take the fixed lane offsets
        const float* kb;
        const float* vb;
    };
    auto tile_info = [&](uint32_t it) -> Tile {
        Tile T;
        const uint32_t u = it * 8 + w;
        T.t0 = p.k_start + (split + u * p.nsplit) * KEYS;
        T.active = it < niter && u < ntiles;
        // contiguous positions: a tile whose first key is past this query is skipped
        // (ascending positions). Explicit positions are not read here: the host trims
        // [k_start, k_end) to keys at or before the last query, the per-key mask covers
        // earlier queries, and a load here would hold up the tile's copies.
        if (!KPOS && T.active) T.active = p.k_pos0 + T.t0 <= qpos;
        T.nk = T.active ? min((uint32_t)KEYS, p.k_end - T.t0) : 1u;
        T.row0 = T.active ? phys_row(T.t0, p.ring_cap) : 0u;
        T.whole = T.active && T.nk == (uint32_t)KEYS && (p.ring_cap == 0u || T.row0 + KEYS <= p.ring_cap);
        T.kb = T.active ? kbase : p.dummy;
        T.vb = T.active ? vbase : p.dummy;
        return T;
    };
    // Byte offsets of lane slot 64i + lane from the first row of a whole tile (see
    // issue_chunk): K chunks add KCD c floats, V chunks KPC (c - NKS) rows, to the base.
    uint32_t koff[LPT], voff[LPT];
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
        const int sl = 64 * i + lane;
        const int r = sl / NCOL;
        koff[i] = (uint32_t)((r * row_stride + 4 * ((sl % NCOL) ^ r)) * sizeof(float));
        voff[i] = (uint32_t)(((sl / (DH / 4)) * row_stride + 4 * (sl % (DH / 4))) * sizeof(float));
    }
    auto prow = [&](const Tile& T, uint32_t r) -> uint32_t {  // physical row of tile key r, clamped to the tile
        uint32_t x = T.row0 + min(r, T.nk - 1);
        if (p.ring_cap && x >= p.ring_cap) x -= p.ring_cap;
        return x;
    };
    // chunk c of a wave tile into ring buffer bi: K chunks c < NKS hold dims
    // KCD c .. KCD c + KCD-1 of the 16 keys (key r's 16-byte column j at slot j ^ r), V chunks
    // hold keys KPC*(c-NKS) .. +KPC-1, all DH dims. Lane l fills 16-byte slot 64i + l.
    // With explicit positions chunk 0 is preceded by one more copy, the tile's 16
    // key positions into my_kp[parity] (clamped to the tile's last key; an idle tile
    // copies dummy words): waiting for chunk 0 then also covers them, and every
    // other wait below counts one copy short at most, i.e. waits a little longer.
    auto issue_chunk = [&](const Tile& T, int c, int bi, uint32_t parity) {
        if constexpr (KPOS) {
            if (c == 0 && lane < KEYS) {
                const void* src = T.active ? (const void*)(p.k_pos + T.t0 + min((uint32_t)lane, T.nk - 1))
                                           : (const void*)(p.dummy + lane);
                copy4_to_lds(src, my_kp + parity * KEYS);
            }
        }
        float* const dst = my_ring + bi * BUF;
        if (T.whole) {
            // the tile's rows are consecutive: a wave-uniform base plus each lane's fixed offset
            const float* const base = c < NKS ? kbase + (size_t)T.row0 * row_stride + KCD * c
                                              : vbase + ((size_t)T.row0 + (c - NKS) * KPC) * row_stride;
#pragma unroll
            for (int i = 0; i < LPT; ++i) copy16s_to_lds<true>(base, c < NKS ? koff[i] : voff[i], dst + 256 * i);
            return;
        }
#pragma unroll
        for (int i = 0; i < LPT; ++i) {
            const int sl = 64 * i + lane;
            const float* src;
            if (c < NKS) {
                const int r = sl / NCOL;
                const int j = (sl % NCOL) ^ r;
                src = T.kb + (size_t)prow(T, r) * row_stride + KCD * c + 4 * j;
            } else {
                const int kr = (c - NKS) * KPC + sl / (DH / 4);
                src = T.vb + (size_t)prow(T, kr) * row_stride + 4 * (sl % (DH / 4));
            }
            copy16_to_lds<true>(src, dst + 256 * i);
        }
    };

    Tile cur = tile_info(0);
#pragma unroll
    for (int c = 0; c < AHEAD; ++c) issue_chunk(cur, c, c, 0u);
    if (lane == 0) progress[w] = -1;
    wait_vm<LPT * AHEAD>();  // this wave's query pieces have landed
    barrier_lds();           // ... and every wave's

    const float* const q0row = qs + (2 * hp) * DH + key;      // head 2hp, dims d + key
    const float* const q1row = qs + (2 * hp + 1) * DH + key;  // head 2hp + 1
    // the lane's query values for every tile, read from LDS once: dims 16 i + key
    // of heads 2hp, 2hp+1 (64 VGPRs at Dh 512; 25.9 against 26.35 us at 32K keys
    // with the reads inside the dot loop)
    float qreg[2][DH / 16];
#pragma unroll
    for (int i = 0; i < DH / 16; ++i) {
        qreg[0][i] = q0row[16 * i];
        qreg[1][i] = q1row[16 * i];
    }
    const float* kcol[NCOL];
#pragma unroll
    for (int j = 0; j < NCOL; ++j) kcol[j] = my_ring + key * KCD + 4 * (j ^ key);

    float m[2] = {NEG_INF, NEG_INF}, lpart[2] = {0.0f, 0.0f};
    float4 acc[GROUP][ND];
#pragma unroll
    for (int h = 0; h < GROUP; ++h)
#pragma unroll
        for (int e = 0; e < ND; ++e) acc[h][e] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);

    int other_seen = -1;  // the partner wave's chunk count, one chunk step old
    for (uint32_t it = 0; it < niter; ++it) {
        const bool last = it + 1 == niter;  // no copies beyond the last wave tile
        const Tile nxt = tile_info(it + 1);
        float s[2] = {0.0f, 0.0f};
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            const int bi = c % NB;
            const float* const buf = my_ring + bi * BUF;
            // chunk c + AHEAD refills the buffer of chunk c + AHEAD - NB; with AHEAD + 1 == NB
            // that is chunk c - 1, whose LDS reads must have completed
            if constexpr (AHEAD + 1 >= NB) asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            if (c + AHEAD < NCH) issue_chunk(cur, c + AHEAD, (c + AHEAD) % NB, it & 1u);
            else if (!last) issue_chunk(nxt, c + AHEAD - NCH, (c + AHEAD) % NB, (it + 1) & 1u);
            // chunk c has landed: the copies issued after it are the next AHEAD chunks
            // (fewer at the end of the last wave tile)
            if (last && c + AHEAD >= NCH) wait_vm_upto16(LPT * (NCH - 1 - c));
            else wait_vm<LPT * AHEAD>();
            {
                // The two waves sharing a SIMD (w and w ^ 4) would otherwise issue oldest
                // first, starving the younger one: a wave behind its partner raises its
                // issue priority until it catches up. The partner's count is the one read
                // a chunk step earlier, so the read never holds this wave up.
                const int done = (int)(it * NCH) + c;
                progress[w] = done;
                const int other = __builtin_amdgcn_readfirstlane(other_seen);
                other_seen = progress[w ^ 4];
                if (other > done) __builtin_amdgcn_s_setprio(1);
                else __builtin_amdgcn_s_setprio(0);
                // left alone, the scheduler gathers the priority changes of all
                // chunks after the last one, where they no longer steer anything
                __builtin_amdgcn_sched_barrier(0);
            }
            if (!cur.active) continue;
            if (c < NKS) {
#pragma unroll
                for (int b = 0; b < KCD / 16; ++b) {
                    const float q0 = qreg[0][(KCD / 16) * c + b];
                    const float q1 = qreg[1][(KCD / 16) * c + b];
                    float4 k4[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) k4[i] = ld4(kcol[4 * b + i] + bi * BUF);
                    qk_dims16(s, q0, q1, k4);
                }
                if (c == NKS - 1) {
                    // online softmax of heads 2hp, 2hp+1 over the row's 16 keys
                    const uint32_t j = cur.t0 + min((uint32_t)key, cur.nk - 1);
                    const uint32_t kp = KPOS ? my_kp[(it & 1u) * KEYS + key] : p.k_pos0 + j;
                    const bool vis =
                        (uint32_t)key < cur.nk && kp <= qpos && (p.window == 0 || qpos - kp < p.window);
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const float sc = vis ? score_epilogue(s[h], p.scale, p.softcap) : NEG_INF;
                        const float mn = fmaxf(m[h], g4a_row_max16(sc));
                        const float corr = (m[h] == NEG_INF) ? 0.0f : expf(m[h] - mn);
                        const float pr = (sc == NEG_INF) ? 0.0f : expf(sc - mn);
                        lpart[h] = lpart[h] * corr + pr;
                        m[h] = mn;
                        my_pbuf[key * GROUP + 2 * hp + h] = pr;
                        if (key == 0) my_corr[2 * hp + h] = corr;
                    }
                }
            } else {
                const int vc = c - NKS;
                if (vc == 0 && it > 0) {
                    // rescale the running output of every head by its correction factor
                    // (none before the first tile: the output is still zero)
                    const float4 c0 = ld4(my_corr), c1 = ld4(my_corr + 4);
                    const float cr[GROUP] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
#pragma unroll
                    for (int h = 0; h < GROUP; ++h)
#pragma unroll
                        for (int e = 0; e < ND; ++e) {
                            acc[h][e].x *= cr[h];
                            acc[h][e].y *= cr[h];
                            acc[h][e].z *= cr[h];
                            acc[h][e].w *= cr[h];
                        }
                }
#pragma unroll
                for (int kr = 0; kr < KPC; ++kr) {
                    const float* const prow8 = my_pbuf + (vc * KPC + kr) * GROUP;
                    const float4 p0 = ld4(prow8), p1 = ld4(prow8 + 4);
                    const float pk[GROUP] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
#pragma unroll
                    for (int e = 0; e < ND; ++e) {
                        const float4 v4 = ld4(buf + kr * DH + 256 * e + 4 * lane);
#pragma unroll
                        for (int h = 0; h < GROUP; ++h) {
                            acc[h][e].x = __builtin_fmaf(pk[h], v4.x, acc[h][e].x);
                            acc[h][e].y = __builtin_fmaf(pk[h], v4.y, acc[h][e].y);
                            acc[h][e].z = __builtin_fmaf(pk[h], v4.z, acc[h][e].z);
                            acc[h][e].w = __builtin_fmaf(pk[h], v4.w, acc[h][e].w);
                        }
                    }
                }
            }
        }
        cur = nxt;
    }

    // The wave's partial goes into its own ring (free once its copies have landed),
    // so no wave waits for another before writing.
    __builtin_amdgcn_s_setprio(0);
    wait_vm<0>();
#pragma unroll
    for (int h = 0; h < 2; ++h) lpart[h] = g4a_row_sum16(lpart[h]);
    if (key == 0) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            mlbuf[w * 2 * GROUP + 2 * hp + h] = m[h];
            mlbuf[w * 2 * GROUP + GROUP + 2 * hp + h] = lpart[h];
        }
    }
    // head w stays in this wave's registers: wave w merges it (w is wave-uniform, so
    // these are scalar branches)
    float4 a[8][ND];
#pragma unroll
    for (int h = 0; h < GROUP; ++h) {
        if (h == w) {
#pragma unroll
            for (int e = 0; e < ND; ++e) a[h][e] = acc[h][e];
        } else {
#pragma unroll
            for (int e = 0; e < ND; ++e) *reinterpret_cast<float4*>(my_ring + h * DH + 256 * e + 4 * lane) = acc[h][e];
        }
    }
    __syncthreads();
    // Wave w merges head w: M = max over waves, L = sum of l * e^(m - M). The 8
    // wave partials are read first; lane x of each 8-lane group computes wave x's
    // weight e^(m_x - M) and l_x e^(m_x - M), which every lane takes in wave order.
    const int h = w;
#pragma unroll
    for (int x = 0; x < 8; ++x) {
        if (x == w) {
            // a[x] holds this wave's own head w, from the copy above (h == x == w)
        } else {
#pragma unroll
            for (int e = 0; e < ND; ++e) a[x][e] = ld4(ring + x * NB * BUF + h * DH + 256 * e + 4 * lane);
        }
    }
    const float mx = mlbuf[(lane & 7) * 2 * GROUP + h];
    const float M = g4a_max8(mx);
    const float ex = (mx == NEG_INF) ? 0.0f : expf(mx - M);
    const float lx = mlbuf[(lane & 7) * 2 * GROUP + GROUP + h] * ex;
    float L = 0.0f, es[8];
#pragma unroll
    for (int x = 0; x < 8; ++x) {
        es[x] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ex), x));
        L += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lx), x));
    }
    const size_t ih = (size_t)qi * p.Hq + h0 + h;
    const float sc = p.nsplit == 1 ? (L > 0.0f ? 1.0f / L : 0.0f) : 1.0f;
#pragma unroll
    for (int e = 0; e < ND; ++e) {
        float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
        for (int x = 0; x < 8; ++x) {
            o.x = __builtin_fmaf(a[x][e].x, es[x], o.x);
            o.y = __builtin_fmaf(a[x][e].y, es[x], o.y);
            o.z = __builtin_fmaf(a[x][e].z, es[x], o.z);
            o.w = __builtin_fmaf(a[x][e].w, es[x], o.w);
        }
        o.x *= sc;
        o.y *= sc;
        o.z *= sc;
        o.w *= sc;
        const uint32_t d = 256 * e + 4 * lane;
        float* const dst = p.nsplit == 1 ? p.out + ih * DH + d : p.part + part_index<DH>(ih, p.nsplit, split, d);
        g4a_store_nt(dst, o);
    }
    if (p.nsplit > 1 && lane == 0) {
        float* ml = p.part + (size_t)p.T * p.Hq * p.nsplit * DH + (ih * p.nsplit + split) * 2;
        ml[0] = M;
        ml[1] = L;
    }
}

// Exact dots of 16 dims (16B .. 16B+15) for ONE head per lane: lane = key,
// each 16-lane row a head. q[h][16B + j] sits in lane j of the row of head h;
// each multiply takes it through a DPP row broadcast (row_newbcast:j), then
// dot = dot + q*k, separately rounded, in the reference's order.
__device__ __forceinline__ void qk1_dims16(float& s, float q, const float4 (&k)[4]) {
    // the multiplies run 4 terms ahead of the adds (4 rotating temporaries), so an
    // add waits only for the add before it, never for its own multiply
    float t0, t1, t2, t3;
    asm volatile(
        "s_nop 1\n\t"
        "v_mul_f32_dpp %[t0], %[q], %[k0] row_newbcast:0 row_mask:0xf bank_mask:0xf\n\t"
        "v_mul_f32_dpp %[t1], %[q], %[k1] row_newbcast:1 row_mask:0xf bank_mask:0xf\n\t"
        "v_mul_f32_dpp %[t2], %[q], %[k2] row_newbcast:2 row_mask:0xf bank_mask:0xf\n\t"
        "v_mul_f32_dpp %[t3], %[q], %[k3] row_newbcast:3 row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32 %[a], %[a], %[t0]\n\t"
        "v_mul_f32_dpp %[t0], %[q], %[k4] row_newbcast:4 row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32 %[a], %[a], %[t1]\n\t"
        "v_mul_f32_dpp %[t1], %[q], %[k5] row_newbcast:5 row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32 %[a], %[a], %[t2]\n\t"
        "v_mul_f32_dpp %[t2], %[q], %[k6] row_newbcast:6 row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32 %[a], %[a], %[t3]\n\t"
        "v_mul_f32_dpp %[t3], %[q], %[k7] row_newbcast:7 row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32 %[a], %[a], %[t0]\n\t"
        "v_mul_f32_dpp %[t0], %[q], %[k8] row_newbcast:8 row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32 %[a], %[a], %[t1]\n\t"
        "v_mul_f32_dpp %[t1], %[q], %[k9] row_newbcast:9 row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32 %[a], %[a], %[t2]\n\t"
        "v_mul_f32_dpp %[t2], %[q], %[k10] row_newbcast:10 row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32 %[a], %[a], %[t3]\n\t"
        "v_mul_f32_dpp %[t3], %[q], %[k11] row_newbcast:11 row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32 %[a], %[a], %[t0]\n\t"
        "v_mul_f32_dpp %[t0], %[q], %[k12] row_newbcast:12 row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32 %[a], %[a], %[t1]\n\t"
        "v_mul_f32_dpp %[t1], %[q], %[k13] row_newbcast:13 row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32 %[a], %[a], %[t2]\n\t"
        "v_mul_f32_dpp %[t2], %[q], %[k14] row_newbcast:14 row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32 %[a], %[a], %[t3]\n\t"
        "v_mul_f32_dpp %[t3], %[q], %[k15] row_newbcast:15 row_mask:0xf bank_mask:0xf\n\t"
        "v_add_f32 %[a], %[a], %[t0]\n\t"
        "v_add_f32 %[a], %[a], %[t1]\n\t"
        "v_add_f32 %[a], %[a], %[t2]\n\t"
        "v_add_f32 %[a], %[a], %[t3]\n\t"
        : [a] "+v"(s), [t0] "=&v"(t0), [t1] "=&v"(t1), [t2] "=&v"(t2), [t3] "=&v"(t3)
        : [q] "v"(q), [k0] "v"(k[0].x), [k1] "v"(k[0].y), [k2] "v"(k[0].z), [k3] "v"(k[0].w), [k4] "v"(k[1].x),
          [k5] "v"(k[1].y), [k6] "v"(k[1].z), [k7] "v"(k[1].w), [k8] "v"(k[2].x), [k9] "v"(k[2].y), [k10] "v"(k[2].z),
          [k11] "v"(k[2].w), [k12] "v"(k[3].x), [k13] "v"(k[3].y), [k14] "v"(k[3].z), [k15] "v"(k[3].w));
}

// Short-context decode for groups of 8 query heads: the sliding layers' 512-key
// window and global layers up to 8K keys, where a call is bound by latency
// rather than by HBM bandwidth.
//
// A 4-wave workgroup owns a key split of 32 keys = two 16-key tiles; wave
// w = 2 * tile + half takes heads 4 * half .. +3 of its tile. Every copy of
// the workgroup is issued up front (one memory round trip): query rows, K rows
// and V rows go global -> LDS, each wave copying half of its tile's rows.
//   scores: lane = (head: 16-lane row, key: lane % 16), ONE exact dot per lane
//           (((0 + q0*k0) + q1*k1) + ..., separately rounded), q held in
//           registers and broadcast along each row with DPP, K read from LDS
//           (rows padded to DH + 4 floats: the 16 keys of a read sit on
//           distinct banks), one 16-dim block ahead of its use;
//   softmax: per head over the tile's 16 keys (row max and sum by DPP);
//   P.V:    lane l owns dims 4l..4l+3 (+256 for DH 512) of its 4 heads, fused
//           multiply-adds over the tile's V rows in LDS;
//   end:    the two tiles merge through LDS (wave w merges heads 2w, 2w+1)
//           into the split's partial (m, l, acc), or the output for one split;
//           the combine kernel merges the split partials.
// With DS = 2 or 4, DS workgroups share a split: all compute the same scores,
// and each copies, accumulates, merges and stores 1 / DS of the output dims
// (workgroup dh: dims dh * DH / DS ..), which shortens the P.V and the merge
// when the GPU has CUs to spare (a sliding call's 16 splits). Every output
// dim sees the same sequence of operations either way, so the results are
// bit-identical to DS = 1.
template <int DH, int DS = 1>
struct ShortCfg {
    static constexpr int GROUP = 8;
    static constexpr int HD = DH / DS;           // output dims of a workgroup (V, P.V, merge, stores)
    static constexpr int DPL = HD / 64;          // output dims per lane: 1, 2, 4 or 8
    static constexpr int VC = HD >= 256 ? HD / 256 : 1;  // copies per V row (a 512-byte row: 32 lanes)
    static constexpr int KEYS = 16;              // keys per tile
    static constexpr int TILES = 2;              // tiles per workgroup (4 waves)
    static constexpr int RS = DH + 4;            // K row stride in LDS (floats)
    static constexpr int QRS = DH + 16;          // query row stride in LDS: 4 rows x 16 floats on distinct banks
    static constexpr int NRC = DH / 256;         // 1 KiB copies per row
    static constexpr int NB = DH / 16;           // 16-dim blocks of a dot
    static constexpr int QS = GROUP * QRS;
    static constexpr int KS = TILES * KEYS * RS;
    static constexpr int VS = TILES * KEYS * HD;
    static constexpr int PB = 4 * KEYS * 4;      // [wave][key][4 heads]
    static constexpr int ML = 4 * 2 * 4;         // [wave][m, l][4 heads]
    static constexpr int MERGE = 4 * 4 * HD;     // [wave][4 heads][HD], over the K rows after the scores
    static constexpr int SMEM = QS + KS + VS + PB + ML;
    static constexpr int COPIES = 2 * NRC + (KEYS / 2) * (NRC + VC);  // per wave: query, K and V rows
    static_assert(MERGE <= KS, "the wave partials fit over the K rows");
    static_assert(SMEM * 4 <= 160 * 1024, "LDS budget of a CU");
    static_assert(COPIES < 64, "vmcnt range");
    static_assert(DPL <= 2 || DPL % 4 == 0, "P.V lanes hold a float, a float2 or whole float4 groups");
};

template <int DH, int DS = 1>
__device__ __forceinline__ void decode_short(const G4aDecodeParams& p, uint32_t split, uint32_t qi, uint32_t dh = 0) {
    using C = ShortCfg<DH, DS>;
    constexpr int GROUP = C::GROUP, KEYS = C::KEYS, RS = C::RS, QRS = C::QRS, NRC = C::NRC, NB = C::NB;
    constexpr int HD = C::HD, DPL = C::DPL, VC = C::VC;

    __shared__ __attribute__((aligned(16))) float smem[C::SMEM];
    float* const qs = smem;              // [GROUP][QRS]
    float* const kbuf = qs + C::QS;      // [TILES][KEYS][RS]; after the scores: [4 waves][4 heads][DH]
    float* const vbuf = kbuf + C::KS;    // [TILES][KEYS][HD]
    float* const pbuf = vbuf + C::VS;    // [4 waves][KEYS][4]
    float* const mlbuf = pbuf + C::PB;   // [4 waves][2][4]

    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int tile = w >> 1, half = w & 1;
    const int r = lane >> 4;     // score phase: head 4 * half + r
    const int key = lane & 15;   // score phase: key of the tile
    const uint32_t kvh = blockIdx.z;
    const uint32_t qpos = p.q_pos ? p.q_pos[qi] : p.q_pos0 + qi;
    const uint32_t t0 = p.k_start + split * p.keys_per_split + tile * KEYS;
    const uint32_t nk = t0 < p.k_end ? min((uint32_t)KEYS, p.k_end - t0) : 0u;
    // contiguous key positions: a tile whose first key is in the future is idle
    const bool active = nk > 0 && p.k_pos0 + t0 <= qpos;
    const uint32_t h0 = kvh * GROUP;
    const size_t row_stride = (size_t)p.Hkv * DH;
    float* const tk = kbuf + tile * KEYS * RS;
    float* const tv = vbuf + tile * KEYS * HD;
    float* const my_p = pbuf + w * KEYS * 4;
    float* const my_ml = mlbuf + w * 8;

    // query rows: copy i (row i / NRC, 1 KiB piece i % NRC); wave w takes i = w, w + 4, ...
    {
        const float* qsrc = p.q + ((size_t)qi * p.Hq + h0) * DH;
#pragma unroll
        for (int c = 0; c < 2 * NRC; ++c) {
            const int i = w + 4 * c;
            copy16_to_lds(qsrc + (i / NRC) * DH + 256 * (i % NRC) + 4 * lane, qs + (i / NRC) * QRS + 256 * (i % NRC));
        }
    }
    // this wave's half of its tile: rows 8 * half .. +7, clamped to the tile's last key
    if (active) {
        const float* const kb = p.k + (size_t)kvh * DH;
        const float* const vb = p.v + (size_t)kvh * DH;
        // one modulo per wave: the host sends a ring here only when it holds at least
        // 64 rows, so base + (offset < KEYS) passes the ring's end at most once
        const uint32_t base = phys_row(t0, p.ring_cap);
        uint32_t rows[KEYS / 2];
#pragma unroll
        for (int i = 0; i < KEYS / 2; ++i) {
            uint32_t x = base + min((uint32_t)(8 * half + i), nk - 1);
            if (p.ring_cap && x >= p.ring_cap) x -= p.ring_cap;
            rows[i] = x;
        }
#pragma unroll
        for (int i = 0; i < KEYS / 2; ++i)
#pragma unroll
            for (int c = 0; c < NRC; ++c)
                copy16_to_lds(kb + rows[i] * row_stride + 256 * c + 4 * lane, tk + (8 * half + i) * RS + 256 * c);
        // V: this workgroup's dims dh * HD .. + HD - 1 of each row
        if (HD >= 256 || lane < HD / 4) {
#pragma unroll
            for (int i = 0; i < KEYS / 2; ++i)
#pragma unroll
                for (int c = 0; c < VC; ++c)
                    copy16_to_lds(vb + rows[i] * row_stride + dh * HD + 256 * c + 4 * lane,
                                  tv + (8 * half + i) * HD + 256 * c);
        }
        wait_vm<(KEYS / 2) * VC>();  // this wave's query pieces and K rows have landed
    } else {
        wait_vm<0>();
    }
    barrier_lds();  // ... and every wave's

    float s = NEG_INF;  // score of (head 4 * half + r, key)
    if (active) {
        float qreg[NB];  // q[h][16b + key]: lane `key` of the head's row holds the block's value
#pragma unroll
        for (int b = 0; b < NB; ++b) qreg[b] = qs[(4 * half + r) * QRS + 16 * b + key];
        const float* const krow = tk + key * RS;
        float4 kc[4], kn[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) kc[i] = ld4(krow + 4 * i);
        float dot = 0.0f;
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            if (b + 1 < NB) {
#pragma unroll
                for (int i = 0; i < 4; ++i) kn[i] = ld4(krow + 16 * (b + 1) + 4 * i);
            }
            qk1_dims16(dot, qreg[b], kc);
#pragma unroll
            for (int i = 0; i < 4; ++i) kc[i] = kn[i];
        }
        const uint32_t kp = p.k_pos0 + t0 + key;
        const bool vis = (uint32_t)key < nk && kp <= qpos && (p.window == 0 || qpos - kp < p.window);
        if (vis) s = score_epilogue(dot, p.scale, p.softcap);
    }
    // row max and sum over the tile's 16 keys by DPP (the additions of an xor
    // 1, 2, 4, 8 butterfly, without LDS round trips)
    const float m = g4a_row_max16(s);
    const float pr = (s == NEG_INF) ? 0.0f : expf(s - m);
    const float l = g4a_row_sum16(pr);
    my_p[key * 4 + r] = pr;
    if (key == 0) {
        my_ml[r] = m;
        my_ml[4 + r] = l;
    }

    wait_vm<0>();   // this wave's V rows have landed
    barrier_lds();  // ... and its partner's; every wave is done with the K rows
    float* const merge = kbuf;  // the two tiles' partials, over the K rows
    float* const mlp = p.part + (size_t)p.T * p.Hq * p.nsplit * DH;  // (m, l) pairs of the partials
    if constexpr (DPL % 4 == 0) {
        // lanes hold whole float4 groups (dims 4l + 256 e)
        constexpr int NG = DPL / 4;
        float4 acc[4][NG];
#pragma unroll
        for (int h = 0; h < 4; ++h)
#pragma unroll
            for (int e = 0; e < NG; ++e) acc[h][e] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (active) {
#pragma unroll
            for (int k0 = 0; k0 < KEYS; k0 += 8) {
                float4 pk[8], vk[8][NG];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    pk[j] = ld4(my_p + (k0 + j) * 4);
#pragma unroll
                    for (int e = 0; e < NG; ++e) vk[j][e] = ld4(tv + (k0 + j) * HD + 256 * e + 4 * lane);
                }
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float pw[4] = {pk[j].x, pk[j].y, pk[j].z, pk[j].w};
#pragma unroll
                    for (int e = 0; e < NG; ++e)
#pragma unroll
                        for (int h = 0; h < 4; ++h) {
                            acc[h][e].x = __builtin_fmaf(pw[h], vk[j][e].x, acc[h][e].x);
                            acc[h][e].y = __builtin_fmaf(pw[h], vk[j][e].y, acc[h][e].y);
                            acc[h][e].z = __builtin_fmaf(pw[h], vk[j][e].z, acc[h][e].z);
                            acc[h][e].w = __builtin_fmaf(pw[h], vk[j][e].w, acc[h][e].w);
                        }
                }
            }
        }
        // merge the two tiles: wave w merges heads 2w, 2w + 1 (waves half and 2 + half hold them)
#pragma unroll
        for (int h = 0; h < 4; ++h)
#pragma unroll
            for (int e = 0; e < NG; ++e)
                *reinterpret_cast<float4*>(merge + (w * 4 + h) * HD + 256 * e + 4 * lane) = acc[h][e];
        barrier_lds();
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int h = 2 * w + i;  // head of the group
            const int x0 = h >> 2, x1 = 2 + (h >> 2), hr = h & 3;
            const float m0 = mlbuf[x0 * 8 + hr], m1 = mlbuf[x1 * 8 + hr];
            const float l0 = mlbuf[x0 * 8 + 4 + hr], l1 = mlbuf[x1 * 8 + 4 + hr];
            float4 a0[NG], a1[NG];
#pragma unroll
            for (int e = 0; e < NG; ++e) {
                a0[e] = ld4(merge + (x0 * 4 + hr) * HD + 256 * e + 4 * lane);
                a1[e] = ld4(merge + (x1 * 4 + hr) * HD + 256 * e + 4 * lane);
            }
            const float M = fmaxf(m0, m1);
            const float e0 = (m0 == NEG_INF) ? 0.0f : expf(m0 - M);
            const float e1 = (m1 == NEG_INF) ? 0.0f : expf(m1 - M);
            const float L = l0 * e0 + l1 * e1;
            const size_t ih = (size_t)qi * p.Hq + h0 + h;
            const float sc = p.nsplit == 1 ? (L > 0.0f ? 1.0f / L : 0.0f) : 1.0f;
#pragma unroll
            for (int e = 0; e < NG; ++e) {
                float4 o;
                o.x = (a0[e].x * e0 + a1[e].x * e1) * sc;
                o.y = (a0[e].y * e0 + a1[e].y * e1) * sc;
                o.z = (a0[e].z * e0 + a1[e].z * e1) * sc;
                o.w = (a0[e].w * e0 + a1[e].w * e1) * sc;
                const uint32_t d = dh * HD + 256 * e + 4 * lane;
                float* const dst = p.nsplit == 1 ? p.out + ih * DH + d : p.part + part_index<DH>(ih, p.nsplit, split, d);
                g4a_store_nt(dst, o);
            }
            if (p.nsplit > 1 && lane == 0 && dh == 0) {
                float* const ml = mlp + (ih * p.nsplit + split) * 2;
                ml[0] = M;
                ml[1] = L;
            }
        }
    } else {
        // 1 or 2 dims per lane (dims l, or 2l and 2l + 1): the split parts of head_dim 256
        float acc[4][DPL];
#pragma unroll
        for (int h = 0; h < 4; ++h)
#pragma unroll
            for (int d = 0; d < DPL; ++d) acc[h][d] = 0.0f;
        auto ld_dims = [&](const float* row, float (&x)[DPL]) {
            if constexpr (DPL == 1) {
                x[0] = row[lane];
            } else {
                const float2 v = *reinterpret_cast<const float2*>(row + 2 * lane);
                x[0] = v.x;
                x[1] = v.y;
            }
        };
        if (active) {
#pragma unroll
            for (int k0 = 0; k0 < KEYS; k0 += 8) {
                float4 pk[8];
                float vk[8][DPL];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    pk[j] = ld4(my_p + (k0 + j) * 4);
                    ld_dims(tv + (k0 + j) * HD, vk[j]);
                }
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float pw[4] = {pk[j].x, pk[j].y, pk[j].z, pk[j].w};
#pragma unroll
                    for (int d = 0; d < DPL; ++d)
#pragma unroll
                        for (int h = 0; h < 4; ++h) acc[h][d] = __builtin_fmaf(pw[h], vk[j][d], acc[h][d]);
                }
            }
        }
#pragma unroll
        for (int h = 0; h < 4; ++h)
#pragma unroll
            for (int d = 0; d < DPL; ++d) merge[(w * 4 + h) * HD + DPL * lane + d] = acc[h][d];
        barrier_lds();
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int h = 2 * w + i;
            const int x0 = h >> 2, x1 = 2 + (h >> 2), hr = h & 3;
            const float m0 = mlbuf[x0 * 8 + hr], m1 = mlbuf[x1 * 8 + hr];
            const float l0 = mlbuf[x0 * 8 + 4 + hr], l1 = mlbuf[x1 * 8 + 4 + hr];
            float a0[DPL], a1[DPL];
            ld_dims(merge + (x0 * 4 + hr) * HD, a0);
            ld_dims(merge + (x1 * 4 + hr) * HD, a1);
            const float M = fmaxf(m0, m1);
            const float e0 = (m0 == NEG_INF) ? 0.0f : expf(m0 - M);
            const float e1 = (m1 == NEG_INF) ? 0.0f : expf(m1 - M);
            const float L = l0 * e0 + l1 * e1;
            const size_t ih = (size_t)qi * p.Hq + h0 + h;
            const float sc = p.nsplit == 1 ? (L > 0.0f ? 1.0f / L : 0.0f) : 1.0f;
#pragma unroll
            for (int d = 0; d < DPL; ++d) {
                const float o = (a0[d] * e0 + a1[d] * e1) * sc;
                const uint32_t dd = dh * HD + DPL * lane + d;
                float* const dst =
                    p.nsplit == 1 ? p.out + ih * DH + dd : p.part + part_index<DH>(ih, p.nsplit, split, dd);
                __builtin_nontemporal_store(o, dst);
            }
            if (p.nsplit > 1 && lane == 0 && dh == 0) {
                float* const ml = mlp + (ih * p.nsplit + split) * 2;
                ml[0] = M;
                ml[1] = L;
            }
        }
    }
}

// out = sum_s acc_s * e^(m_s - M) / sum_s l_s * e^(m_s - M), M = max_s m_s; 0 when the
// denominator is 0 (the semantics of rust/src/kernels/attention_combine.wgsl:1-28).
// One block of COMBINE_THREADS per (32 output dims, head, query): the block
// reads one whole 128-byte piece of each split's row (part_index), so every
// fetched line is used by the block that fetched it (blocks of 16 dims each
// used half of every line, and the other half came in again on another XCD).
// Every wave computes the maximum M and the weighted sum of l itself from all
// (m, l) pairs and keeps its own copy of the split weights e^(m_s - M) in LDS,
// so no barrier stands between the loads and the sums. Thread (group g, dim i)
// sums splits s = g, g + 16, ... in split order, and the 16 groups reduce
// through LDS. The first COMBINE_EARLY splits of each thread (all of them up
// to 256 splits) are loaded together with the (m, l) pairs, before the weights
// are known, so a step pays one memory round trip for them instead of two.
constexpr int COMBINE_MAX_SPLITS = 1024;
constexpr int COMBINE_EARLY = 16;
constexpr int COMBINE_DIMS = 32;
constexpr int COMBINE_THREADS = 512;

template <int DH>
__device__ __forceinline__ void combine(const G4aCombineParams& p, uint32_t qi) {
    static_assert(DH % COMBINE_DIMS == 0, "whole blocks of dims");
    __shared__ float wgt[COMBINE_THREADS / 64][COMBINE_MAX_SPLITS];  // one copy per wave
    __shared__ float red[16][COMBINE_DIMS + 1];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = tid >> 6;
    const int i = tid & (COMBINE_DIMS - 1), grp = tid / COMBINE_DIMS;  // 16 groups
    const size_t ih = (size_t)qi * p.Hq + blockIdx.y;
    const uint32_t d = blockIdx.x * COMBINE_DIMS + i;
    const float2* __restrict__ ml =
        reinterpret_cast<const float2*>(p.part + (size_t)p.T * p.Hq * p.nsplit * DH + ih * p.nsplit * 2);
    // this block's 32 dims: a 128-byte run in each split's row, DH floats apart
    const float* __restrict__ acc = p.part + part_index<DH>(ih, p.nsplit, 0, blockIdx.x * COMBINE_DIMS) + i;
    const uint32_t ns = p.nsplit;
    float* const wg = wgt[w];
    // (m, l) of splits lane, lane + 64, ... first (their wait then leaves the partials in flight)
    float2 mls[COMBINE_MAX_SPLITS / 64];
#pragma unroll
    for (int r = 0; r < COMBINE_MAX_SPLITS / 64; ++r) {
        const uint32_t s = lane + 64 * r;
        mls[r] = s < ns ? ml[s] : make_float2(NEG_INF, 0.0f);
    }
    // splits grp + 16 u, u < COMBINE_EARLY (clamped: loads past the last split repeat it and are not summed)
    float x0[COMBINE_EARLY];
#pragma unroll
    for (int u = 0; u < COMBINE_EARLY; ++u) {
        const uint32_t s = grp + 16 * u;
        x0[u] = acc[(size_t)(s < ns ? s : ns - 1) * DH];
    }
    float M = NEG_INF;
#pragma unroll
    for (int r = 0; r < COMBINE_MAX_SPLITS / 64; ++r) M = fmaxf(M, mls[r].x);
    M = wave_max(M);
    float L = 0.0f;
#pragma unroll
    for (int r = 0; r < COMBINE_MAX_SPLITS / 64; ++r) {
        const uint32_t s = lane + 64 * r;
        if (s < ns) {
            const float e = (mls[r].x == NEG_INF) ? 0.0f : expf(mls[r].x - M);
            wg[s] = e;
            L += mls[r].y * e;
        }
    }
    L = wave_sum(L);
    // the wave's own LDS writes above are read below by other lanes of the same
    // wave: a wave's LDS instructions execute in order, so only the compiler
    // must keep them in place
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float A = 0.0f;
#pragma unroll
    for (int u = 0; u < COMBINE_EARLY; ++u) {
        const uint32_t s = grp + 16 * u;
        if (s < ns) A += x0[u] * wg[s];
    }
    constexpr int U = 8;
    uint32_t s = grp + 16 * COMBINE_EARLY;
    for (; s + 16 * (U - 1) < ns; s += 16 * U) {
        float x[U];
#pragma unroll
        for (int u = 0; u < U; ++u) x[u] = acc[(size_t)(s + 16 * u) * DH];
#pragma unroll
        for (int u = 0; u < U; ++u) A += x[u] * wg[s + 16 * u];
    }
    for (; s < ns; s += 16) A += acc[(size_t)s * DH] * wg[s];
    red[grp][i] = A;
    __syncthreads();
    if (tid < COMBINE_DIMS) {
        A = 0.0f;
#pragma unroll
        for (int g = 0; g < 16; ++g) A += red[g][tid];
        p.out[ih * DH + d] = L > 0.0f ? A / L : 0.0f;
    }
}

// The same merge for up to COMBINE_ROW_SPLITS splits (the host sends no more),
// one block per (head, query); thread t sums dims t (+256) over the splits in
// split order. Every wave loads the (m, l) pairs beside its partial loads and
// computes the split weights itself (lane s holds split s's), taking split s's
// by a readlane: the wave reductions end in readlanes, so each wave's weights
// and sum have the same bits, and no LDS hand-off or barrier sits between the
// loads' one memory round trip and the sums.
constexpr uint32_t COMBINE_ROW_SPLITS = 16;

template <int DH>
__device__ __forceinline__ void combine_rows(const G4aCombineParams& p, uint32_t h, uint32_t qi) {
    const int tid = threadIdx.x, lane = tid & 63;
    const size_t ih = (size_t)qi * p.Hq + h;
    const uint32_t ns = p.nsplit;  // 1 .. COMBINE_ROW_SPLITS: the clamped loads stay in the split range
    const bool on = (uint32_t)lane < ns;
    const float2 ml = reinterpret_cast<const float2*>(p.part + (size_t)p.T * p.Hq * ns * DH +
                                                      ih * ns * 2)[min((uint32_t)lane, ns - 1)];
    float x[DH / 256][COMBINE_ROW_SPLITS];
#pragma unroll
    for (int e = 0; e < DH / 256; ++e) {
        const float* __restrict__ acc = p.part + part_index<DH>(ih, ns, 0, 256 * e + tid);  // split s at acc[DH s]
#pragma unroll
        for (uint32_t u = 0; u < COMBINE_ROW_SPLITS; ++u)
            x[e][u] = acc[(size_t)(u < ns ? u : ns - 1) * DH];
    }
    __builtin_amdgcn_sched_barrier(0);  // every load issued before the weights' arithmetic
    const float mx = on ? ml.x : NEG_INF;
    const float M = wave_max(mx);
    const float wt = (mx == NEG_INF) ? 0.0f : expf(mx - M);
    const float L = wave_sum(on ? ml.y * wt : 0.0f);
#pragma unroll
    for (int e = 0; e < DH / 256; ++e) {
        float A = 0.0f;
#pragma unroll
        for (uint32_t u = 0; u < COMBINE_ROW_SPLITS; ++u) {  // a select, not a branch: a branch would
            const float t = A + x[e][u] * g4a_lane(wt, u);  // take each load into it, one round trip each
            A = u < ns ? t : A;
        }
        p.out[ih * DH + 256 * e + tid] = L > 0.0f ? A / L : 0.0f;
    }
}

// combine_rows' merge of every head of one query (T = 1, 1 .. G4A_FUSE_MAX_SPLITS
// splits) done by one 256-thread workgroup into LDS: xs[h * DH + d] is the
// merged attention row (the activation row of the output projection that
// follows), zeros from Hq * DH up to KP; xout, if set, receives the row too.
// Each wave computes the split weights of heads wave, wave + 4, ... exactly as
// each wave of combine_rows does; each dim then sums its splits in order from 0,
// multiplies and adds rounded separately, so every value has combine_rows'
// bits. Thread t merges four adjacent dims (one float4 of a split's 16-dim
// row) in each 1024-dim group; the loads of two groups (every split) are in
// flight at once, the first two groups' issued before the split weights are
// known. `after_issue` runs right after those first loads are issued (the
// projection requests its first weight words there).
template <int DH, typename F>
__device__ __forceinline__ void combine_row_stage(const float* __restrict__ part, uint32_t Hq, uint32_t ns, float* xs,
                                                  uint32_t KP, float* xout, F&& after_issue) {
    constexpr int FS = G4A_FUSE_MAX_SPLITS;
    __shared__ float cw[G4A_FUSE_MAX_HEADS][FS];
    __shared__ float cl[G4A_FUSE_MAX_HEADS];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t K = Hq * DH;
    float4 x[2][FS];
    auto issue = [&](int g, uint32_t k) {
        const uint32_t kk = k < K ? k : K - 4;
        const uint32_t h = kk / DH, d = kk - h * DH;
        const float* __restrict__ acc = part + part_index<DH>(h, ns, 0, d);  // split s at acc[DH s]
#pragma unroll
        for (int s = 0; s < FS; ++s)  // ns >= 1: the clamped loads stay in the split range
            x[g][s] = *reinterpret_cast<const float4*>(acc + (size_t)((uint32_t)s < ns ? s : ns - 1) * DH);
    };
    issue(0, 4 * tid);
    issue(1, 1024 + 4 * tid);
    after_issue();
    const float2* __restrict__ ml = reinterpret_cast<const float2*>(part + (size_t)Hq * ns * DH);
    for (uint32_t h = wv; h < Hq; h += 4) {
        const bool on = (uint32_t)lane < ns;
        const float2 m = on ? ml[h * ns + lane] : make_float2(NEG_INF, 0.0f);
        const float M = wave_max(m.x);
        const float e = (m.x == NEG_INF) ? 0.0f : expf(m.x - M);
        if (on) cw[h][lane] = e;
        const float L = wave_sum(on ? m.y * e : 0.0f);
        if (lane == 0) cl[h] = L;
    }
    __syncthreads();
    for (uint32_t k0 = 0; k0 < KP; k0 += 2048) {
        if (k0 && k0 < K) {
            issue(0, k0 + 4 * tid);
            issue(1, k0 + 1024 + 4 * tid);
        }
#pragma unroll
        for (int g = 0; g < 2; ++g) {
            const uint32_t k = k0 + 1024 * g + 4 * tid;
            if (k < K) {
                const uint32_t h = k / DH;
                float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
#pragma unroll
                for (int s = 0; s < FS; ++s)
                    if ((uint32_t)s < ns) {
                        const float w = cw[h][s];
                        a0 += x[g][s].x * w;
                        a1 += x[g][s].y * w;
                        a2 += x[g][s].z * w;
                        a3 += x[g][s].w * w;
                    }
                const float L = cl[h];
                const float4 o =
                    L > 0.0f ? make_float4(a0 / L, a1 / L, a2 / L, a3 / L) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                *reinterpret_cast<float4*>(xs + k) = o;
                if (xout) *reinterpret_cast<float4*>(xout + k) = o;
            } else if (k < KP) {
                *reinterpret_cast<float4*>(xs + k) = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            }
        }
    }
}

// Batched decode: one launch over the independent single-query steps of
// b.seq[]; grid (largest split count, sequences, Hkv). The decode parameters of
// sequence blockIdx.y are rebuilt from its descriptor (T = 1; key positions
// relative to its first cache key, or explicit ones from b.kpos); a workgroup
// past the sequence's split count exits at once.
__device__ __forceinline__ bool batch_params(const G4aBatchParams& b, uint32_t si, G4aDecodeParams& p) {
    const G4aSeqDesc& sd = b.seq[si];
    p = G4aDecodeParams{};
    p.nsplit = (sd.k_end - sd.k_start + b.keys_per_split - 1) / b.keys_per_split;
    p.q = sd.q;
    p.k = sd.k;
    p.v = sd.v;
    p.out = sd.out;
    p.part = b.part + sd.part;
    p.dummy = b.dummy;
    p.q_pos0 = sd.q_pos;
    p.k_pos0 = 0;
    // explicit positions (the KPOS kernel): sd.kpos locates the position of key k_start
    if (sd.kpos != G4A_NO_KPOS) p.k_pos = b.kpos + sd.kpos - sd.k_start;
    p.T = 1;
    p.Hq = b.Hq;
    p.Hkv = b.Hkv;
    p.k_start = sd.k_start;
    p.k_end = sd.k_end;
    p.keys_per_split = b.keys_per_split;
    p.ring_cap = b.ring_cap;
    p.window = b.window;
    p.scale = b.scale;
    p.softcap = b.softcap;
    return p.nsplit > 0;
}

template <int DH>
__device__ __forceinline__ void decode_short_batch(const G4aBatchParams& b) {
    G4aDecodeParams p;
    if (!batch_params(b, blockIdx.y, p) || blockIdx.x >= p.nsplit) return;
    decode_short<DH>(p, blockIdx.x, 0u);
}

template <int DH, bool KPOS>
__device__ __forceinline__ void decode_wave_batch(const G4aBatchParams& b) {
    G4aDecodeParams p;
    if (!batch_params(b, blockIdx.y, p) || blockIdx.x >= p.nsplit) return;
    decode_wave<DH, KPOS>(p, blockIdx.x, 0u);
}

// The LSE combines of a batched decode, each sequence merged by the kernel a
// single call with its split count uses: more than COMBINE_ROW_SPLITS splits
// here, grid (DH/COMBINE_DIMS, Hq, sequences) of COMBINE_THREADS ...
template <int DH>
__device__ __forceinline__ void combine_batch(const G4aBatchParams& b) {
    G4aDecodeParams p;
    if (!batch_params(b, blockIdx.z, p) || p.nsplit <= COMBINE_ROW_SPLITS) return;
    const G4aCombineParams cp{p.part, p.out, 1u, b.Hq, p.nsplit, (uint32_t)DH};
    combine<DH>(cp, 0u);
}

// ... and 2 .. COMBINE_ROW_SPLITS splits here, grid (Hq, sequences).
template <int DH>
__device__ __forceinline__ void combine_rows_batch(const G4aBatchParams& b) {
    G4aDecodeParams p;
    if (!batch_params(b, blockIdx.y, p) || p.nsplit < 2 || p.nsplit > COMBINE_ROW_SPLITS) return;
    const G4aCombineParams cp{p.part, p.out, 1u, b.Hq, p.nsplit, (uint32_t)DH};
    combine_rows<DH>(cp, blockIdx.x, 0u);
}

// Generic masked attention, one wave per (query, head) row, for any head dims
// (Dh <= 1024, Dv <= 1024) and group sizes: the shapes the fast kernels do not
// take. It follows the CPU backend's row in its order (rust/src/backend_cpu.rs:
// 286-331) rather than an online softmax, so that nothing but expf / tanhf
// separates it from the reference: (1) the row maximum of the scores, (2) e_j =
// exp(s_j - max) and their sum in key order, inv = 1 / sum (0 when the sum is
// 0), (3) out += (e_j * inv) * v_j in key order, multiply and add rounded
// separately, weights of 0 skipped. The scores (the exact sequential dot, the
// scale, the soft-cap of rust/src/backend_cpu.rs:303-305) are recomputed in
// each pass instead of being stored, so any key count runs without a buffer;
// the key-order sum and accumulation are dependent chains over the row's keys.
// The reference GPU's fallback (rust/src/kernels/attention.wgsl) has the same
// masking semantics with an online softmax.
__device__ __forceinline__ void generic_attention(const G4aGenericParams& p) {
    constexpr int MAXV = 16;  // Dv <= 64 * MAXV
    __shared__ float qs[1024];
    __shared__ float eb[64];
    const int lane = threadIdx.x;
    const uint32_t h = blockIdx.x, qi = blockIdx.y;
    const uint32_t group = p.Hq / p.Hkv;
    const uint32_t kvh = h / group;
    const uint32_t qpos = p.q_pos ? p.q_pos[qi] : p.q_pos0 + qi;
    const float* __restrict__ qr = p.q + ((size_t)qi * p.Hq + h) * p.Dh;
    for (uint32_t d = lane; d < p.Dh; d += 64) qs[d] = qr[d];
    __syncthreads();

    // the score of this lane's key of the 64-key tile at t0 (NEG_INF when masked
    // or past the tile's nk keys)
    auto score = [&](uint32_t t0, uint32_t nk) -> float {
        const bool inr = (uint32_t)lane < nk;
        const uint32_t j = inr ? t0 + lane : t0;
        const float* __restrict__ kr = p.k + ((size_t)phys_row(j, p.ring_cap) * p.Hkv + kvh) * p.Dh;
        float dot = 0.0f;
        for (uint32_t d = 0; d < p.Dh; ++d) dot = dot + qs[d] * kr[d];
        const uint32_t kp = p.k_pos ? p.k_pos[j] : p.k_pos0 + j;
        const bool vis = inr && kp <= qpos && (p.window == 0 || qpos - kp < p.window);
        return vis ? score_epilogue(dot, p.scale, p.softcap) : NEG_INF;
    };
    // e_j of this lane's key into eb (0 for a masked key: it adds nothing to the sum)
    auto weights = [&](uint32_t t0, uint32_t nk, float maxv) {
        const float s = score(t0, nk);
        eb[lane] = s == NEG_INF ? 0.0f : expf(s - maxv);
        __syncthreads();
    };

    // 1: the row maximum (the order of a maximum does not matter)
    float maxv = NEG_INF;
    for (uint32_t t0 = p.k_start; t0 < p.k_end; t0 += 64)
        maxv = fmaxf(maxv, wave_max(score(t0, min(64u, p.k_end - t0))));
    // 2: the sum of the e_j in key order (every lane runs the same chain)
    float sum = 0.0f;
    for (uint32_t t0 = p.k_start; t0 < p.k_end; t0 += 64) {
        const uint32_t nk = min(64u, p.k_end - t0);
        weights(t0, nk, maxv);
        for (uint32_t jj = 0; jj < nk; ++jj) sum = sum + eb[jj];
        __syncthreads();
    }
    const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
    // 3: out += (e_j * inv) * v_j in key order; lane l owns dims l, l + 64, ...
    float acc[MAXV];
#pragma unroll
    for (int e = 0; e < MAXV; ++e) acc[e] = 0.0f;
    for (uint32_t t0 = p.k_start; t0 < p.k_end; t0 += 64) {
        const uint32_t nk = min(64u, p.k_end - t0);
        weights(t0, nk, maxv);
        for (uint32_t jj = 0; jj < nk; ++jj) {
            const float w = eb[jj] * inv;
            if (w == 0.0f) continue;  // the same for every lane
            const float* __restrict__ vr = p.v + ((size_t)phys_row(t0 + jj, p.ring_cap) * p.Hkv + kvh) * p.Dv;
#pragma unroll
            for (int e = 0; e < MAXV; ++e) {
                const uint32_t d = lane + 64 * e;
                if (d < p.Dv) acc[e] = acc[e] + w * vr[d];
            }
        }
        __syncthreads();
    }
    float* o = p.out + ((size_t)qi * p.Hq + h) * p.Dv;
#pragma unroll
    for (int e = 0; e < MAXV; ++e) {
        const uint32_t d = lane + 64 * e;
        if (d < p.Dv) o[d] = acc[e];
    }
}

}  // namespace

extern "C" {
// the contiguous-position single-call kernels also take a device position (at_device_pos)
__global__ __launch_bounds__(512) void g4a_decode_d256_g8(G4aDecodeParams p) {
    decode_wave<256, false>(at_device_pos(p), blockIdx.x, blockIdx.y);
}
__global__ __launch_bounds__(512) void g4a_decode_d512_g8(G4aDecodeParams p) {
    decode_wave<512, false>(at_device_pos(p), blockIdx.x, blockIdx.y);
}
__global__ __launch_bounds__(512) void g4a_decode_d256_g4(G4aDecodeParams p) {
    decode_split<256, 4, false>(at_device_pos(p));
}
__global__ __launch_bounds__(512) void g4a_decode_d512_g4(G4aDecodeParams p) {
    decode_split<512, 4, false>(at_device_pos(p));
}
__global__ __launch_bounds__(512) void g4a_decode_d256_g8_kpos(G4aDecodeParams p) {
    decode_wave<256, true>(p, blockIdx.x, blockIdx.y);
}
__global__ __launch_bounds__(512) void g4a_decode_d512_g8_kpos(G4aDecodeParams p) {
    decode_wave<512, true>(p, blockIdx.x, blockIdx.y);
}
__global__ __launch_bounds__(512) void g4a_decode_d256_g4_kpos(G4aDecodeParams p) { decode_split<256, 4, true>(p); }
__global__ __launch_bounds__(512) void g4a_decode_d512_g4_kpos(G4aDecodeParams p) { decode_split<512, 4, true>(p); }
__global__ __launch_bounds__(256) void g4a_decode_short_d256(G4aDecodeParams p) {
    decode_short<256>(at_device_pos(p), blockIdx.x, blockIdx.y);
}
__global__ __launch_bounds__(256) void g4a_decode_short_d512(G4aDecodeParams p) {
    decode_short<512>(at_device_pos(p), blockIdx.x, blockIdx.y);
}
// DS workgroups per split (grid x = DS * splits): workgroup DS s + dh owns output dims part dh
__global__ __launch_bounds__(256) void g4a_decode_short2_d256(G4aDecodeParams p) {
    decode_short<256, 2>(at_device_pos(p), blockIdx.x >> 1, blockIdx.y, blockIdx.x & 1u);
}
__global__ __launch_bounds__(256) void g4a_decode_short2_d512(G4aDecodeParams p) {
    decode_short<512, 2>(at_device_pos(p), blockIdx.x >> 1, blockIdx.y, blockIdx.x & 1u);
}
__global__ __launch_bounds__(256) void g4a_decode_short4_d256(G4aDecodeParams p) {
    decode_short<256, 4>(at_device_pos(p), blockIdx.x >> 2, blockIdx.y, blockIdx.x & 3u);
}
__global__ __launch_bounds__(256) void g4a_decode_short4_d512(G4aDecodeParams p) {
    decode_short<512, 4>(at_device_pos(p), blockIdx.x >> 2, blockIdx.y, blockIdx.x & 3u);
}
// The same with a split's DS workgroups on one XCD: workgroups are dealt to the
// XCDs round-robin by index, and x = (split mod 8) + 8 (DS (split div 8) + part)
// gives the DS workgroups of a split the same x mod 8, so one L2 fill of the
// split's K rows (which all of them read) serves them all. The host launches
// these only with a split count that is a multiple of 8. Placement only: the
// results are the split-major kernels' bit for bit.
__global__ __launch_bounds__(256) void g4a_decode_short2x_d256(G4aDecodeParams p) {
    decode_short<256, 2>(at_device_pos(p), (blockIdx.x & 7u) + 8u * (blockIdx.x >> 4), blockIdx.y, (blockIdx.x >> 3) & 1u);
}
__global__ __launch_bounds__(256) void g4a_decode_short2x_d512(G4aDecodeParams p) {
    decode_short<512, 2>(at_device_pos(p), (blockIdx.x & 7u) + 8u * (blockIdx.x >> 4), blockIdx.y, (blockIdx.x >> 3) & 1u);
}
__global__ __launch_bounds__(256) void g4a_decode_short4x_d256(G4aDecodeParams p) {
    decode_short<256, 4>(at_device_pos(p), (blockIdx.x & 7u) + 8u * (blockIdx.x >> 5), blockIdx.y, (blockIdx.x >> 3) & 3u);
}
__global__ __launch_bounds__(256) void g4a_decode_short4x_d512(G4aDecodeParams p) {
    decode_short<512, 4>(at_device_pos(p), (blockIdx.x & 7u) + 8u * (blockIdx.x >> 5), blockIdx.y, (blockIdx.x >> 3) & 3u);
}
__global__ __launch_bounds__(256) void g4a_decode_short_batch_d256(G4aBatchParams b) { decode_short_batch<256>(b); }
__global__ __launch_bounds__(256) void g4a_decode_short_batch_d512(G4aBatchParams b) { decode_short_batch<512>(b); }
__global__ __launch_bounds__(512) void g4a_decode_wave_batch_d256(G4aBatchParams b) { decode_wave_batch<256, false>(b); }
__global__ __launch_bounds__(512) void g4a_decode_wave_batch_d512(G4aBatchParams b) { decode_wave_batch<512, false>(b); }
// sequences with explicit key positions (every descriptor of the launch has kpos set)
__global__ __launch_bounds__(512) void g4a_decode_wave_batch_kpos_d256(G4aBatchParams b) {
    decode_wave_batch<256, true>(b);
}
__global__ __launch_bounds__(512) void g4a_decode_wave_batch_kpos_d512(G4aBatchParams b) {
    decode_wave_batch<512, true>(b);
}
__global__ __launch_bounds__(COMBINE_THREADS) void g4a_combine_batch_d256(G4aBatchParams b) { combine_batch<256>(b); }
__global__ __launch_bounds__(COMBINE_THREADS) void g4a_combine_batch_d512(G4aBatchParams b) { combine_batch<512>(b); }
__global__ __launch_bounds__(256) void g4a_combine_rows_batch_d256(G4aBatchParams b) { combine_rows_batch<256>(b); }
__global__ __launch_bounds__(256) void g4a_combine_rows_batch_d512(G4aBatchParams b) { combine_rows_batch<512>(b); }
__global__ __launch_bounds__(256) void g4a_combine_rows_d256(G4aCombineParams p) {
    combine_rows<256>(p, blockIdx.x, blockIdx.y);
}
__global__ __launch_bounds__(256) void g4a_combine_rows_d512(G4aCombineParams p) {
    combine_rows<512>(p, blockIdx.x, blockIdx.y);
}
__global__ __launch_bounds__(COMBINE_THREADS) void g4a_combine_d256(G4aCombineParams p) { combine<256>(p, blockIdx.z); }
__global__ __launch_bounds__(COMBINE_THREADS) void g4a_combine_d512(G4aCombineParams p) { combine<512>(p, blockIdx.z); }
__global__ __launch_bounds__(64) void g4a_generic_attention(G4aGenericParams p) { generic_attention(p); }
}
