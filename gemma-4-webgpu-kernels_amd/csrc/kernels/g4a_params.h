// Kernel argument blocks shared by the gfx950 code objects and the host
// dispatcher (libg4a.so). Plain C layout: each kernel takes one of these by
// value, passed through hipModuleLaunchKernel's kernelParams.
#pragma once
#include <stdint.h>

// Split-K flash-decode over the MQA group of one kv head.
// Logical key j (k_start <= j < k_end) lives in physical row
//   row(j) = ring_cap ? j % ring_cap : j
// of k/v, whose rows are [Hkv][Dh] f32 (row-major, like the reference's
// [S, Hkv, Dh] tensors). Key j has absolute position
//   kpos(j) = k_pos ? k_pos[j] : k_pos0 + j
// and query i has qpos(i) = q_pos ? q_pos[i] : q_pos0 + i.
// Visibility follows rust/src/backend_cpu.rs:293:
//   kpos <= qpos && (window == 0 || qpos - kpos < window).
struct G4aDecodeParams {
    const float* q;        // [T, Hq, Dh]
    const float* k;        // [rows, Hkv, Dh]
    const float* v;        // [rows, Hkv, Dh]
    float* out;            // [T, Hq*Dh]
    float* part;           // nsplit > 1: acc [T*Hq][nsplit][Dh] then (m,l) [T*Hq][nsplit][2]
    const float* dummy;    // >= 4 KiB of readable device memory: the load target of idle tiles
    const uint32_t* q_pos; // device [T] or null
    const uint32_t* k_pos; // device [S] or null
    uint32_t q_pos0, k_pos0;
    uint32_t T, Hq, Hkv;
    uint32_t k_start, k_end;
    uint32_t keys_per_split, nsplit;  // the 8-head streaming kernel deals tiles round-robin over nsplit instead
    uint32_t ring_cap;
    uint32_t window;
    float scale, softcap;
    // Device position (g4a_attention_devpos), or null. When set (T = 1, contiguous
    // positions), the query's position is read from it at run time and the key
    // range follows: keys k_pos0 .. qpos (the last `window` of them), k_end never
    // past the planned k_end; q_pos0, k_start and k_end above are then the plan's.
    const uint32_t* dpos;
};

// One sequence of a batched decode launch (g4a_decode_*_batch_*,
// g4a_combine_batch_*): a single query over the cache rows k / v, keys
// [k_start, k_end) in splits of G4aBatchParams::keys_per_split. Positions are
// relative to the sequence's first cache key: key j sits at position j
// (physical row j % ring_cap for a ring), the query at q_pos; or, with kpos set,
// key j at G4aBatchParams::kpos[kpos + j - k_start] and the query at q_pos, both
// absolute (only the positions of the visible keys k_start .. k_end are staged).
constexpr uint32_t G4A_NO_KPOS = 0xFFFFFFFFu;
struct G4aSeqDesc {
    const float* q;        // [1, Hq, Dh]
    const float* k;        // [rows, Hkv, Dh]
    const float* v;        // [rows, Hkv, Dh]
    float* out;            // [1, Hq*Dh]
    uint32_t k_start, k_end;
    uint32_t q_pos;
    uint32_t part;         // offset of its partials in G4aBatchParams::part, in floats
    uint32_t kpos;         // offset of its key positions in G4aBatchParams::kpos, or G4A_NO_KPOS
};

// Sequences per batched decode launch: their descriptors travel in the kernel
// arguments (56 bytes each), so a launch needs no upload of its own.
constexpr uint32_t G4A_BATCH_SEQ = 64;

// Arguments of a batched decode launch: sequences seq[0 .. gridDim.y) (decode)
// or seq[0 .. gridDim.z) (combine) and the shape they share. A sequence's
// partials are laid out as G4aDecodeParams::part for T = 1 and its split count.
struct G4aBatchParams {
    G4aSeqDesc seq[G4A_BATCH_SEQ];
    float* part;
    const float* dummy;
    const uint32_t* kpos;  // the explicit key positions of the launch's sequences (device)
    uint32_t Hq, Hkv;
    uint32_t keys_per_split;
    uint32_t ring_cap;
    uint32_t window;
    float scale, softcap;
};

static_assert(sizeof(G4aBatchParams) <= 4096, "batched decode arguments fit the kernel argument segment");

// Log-sum-exp merge of the split partials written by the decode kernel.
struct G4aCombineParams {
    const float* part;
    float* out;
    uint32_t T, Hq, nsplit, Dh;
};

// Generic per-(query, head) attention for shapes outside the fast paths
// (any Hq/Hkv/Dh/Dv). Positions as in G4aDecodeParams: device arrays, or
// q_pos0 + i / k_pos0 + j when the array is null.
struct G4aGenericParams {
    const float* q;        // [T, Hq, Dh]
    const float* k;        // [rows, Hkv, Dh]
    const float* v;        // [rows, Hkv, Dv]
    float* out;            // [T, Hq*Dv]
    const uint32_t* q_pos; // device [T] or null
    const uint32_t* k_pos; // device [S] or null
    uint32_t q_pos0, k_pos0;
    uint32_t T, S, Hq, Hkv, Dh, Dv;
    uint32_t k_start, k_end;
    uint32_t ring_cap;
    uint32_t window;
    float scale, softcap;
};

// Query-tiled causal / sliding-window prefill over contiguous positions:
// query i has position q_pos0 + i, key j has position k_pos0 + j; group of 8
// query heads per kv head; Dh == Dv in {256, 512}; no soft-cap.
struct G4aPrefillParams {
    const float* q;        // [T, Hq, Dh]
    const float* k;        // [rows, Hkv, Dh]
    const float* v;        // [rows, Hkv, Dh]
    float* out;            // [T, Hq*Dh]
    // keys [split0, split0 + split_n) pre-split by g4a_split_kv (G4aSplitParams)
    const float* ksplit;   // K rows, scaled by their kscale^-1, as fp16 hi/lo pairs
    const float* kscale;   // [Hkv][split_n / 16]: the power of two each split 16-key tile was divided by
    const float* vsplit;   // V key quads as fp16 hi/lo pairs
    const uint32_t* vflag; // == epoch: some V value is outside the fp16 split's range
    uint32_t T, S, Hq, Hkv;
    uint32_t q_pos0, k_pos0;
    uint32_t ring_cap, window;
    uint32_t split0, split_n, epoch;
    float scale;
    float tau;             // rescoring band: keys whose estimated score is within tau of the row maximum are rescored exactly
    // head_dim 512 causal balance: the last `nbig` query blocks (8 queries each)
    // run as two workgroups over the two halves of their key tiles; each half
    // writes its partial (O, l, m) to `part` and g4a_prefill_merge_d512 merges
    // them. Workgroup i runs the split halves first, then the other blocks,
    // heaviest first (so heavy work starts first).
    float* part;
    uint32_t nbig;
};

// Pre-split keys for the head_dim 256 prefill: keys [k0, k0 + nkeys) (logical,
// read through the ring; keys past the cache re-read its last row), k0 and
// nkeys multiples of 16.
//   kout: key j -> row j - k0 (Hkv * Dh 4-byte slots); each 8-dim block of a
//         head is 8 slots: 8 fp16 hi parts, then 8 fp16 lo parts of x' = x * 2^-a
//         (hi = fp16(x'), lo = fp16(x' - hi), both rounded to nearest even),
//         with a per (16-key tile, head) chosen so the tile's largest |x'| lies in
//         [2^14, 2^15): no fp16 overflow, and only values below 2^-17 of the
//         tile's largest reach fp16's subnormals (an absolute error of 2^-39 of
//         that largest);
//   kscale: [Hkv][nkeys / 16] the factor 2^a of tile i (keys k0 + 16i ..) of
//         head h at h * (nkeys / 16) + i;
//   vout: keys 4i .. 4i+3 (relative to k0) of head h form a 4*Dh-slot block at
//         (i * Hkv + h) * 4 * Dh; dim 64c + 4n + e of it sits at slots
//         4 * ((4c + e) * 16 + n) .. +3: the 4 keys' fp16 hi parts, then their
//         fp16 lo parts (hi = fp16(x), lo = fp16(x - hi));
//   vflag: set to epoch if some V value of a key in [vis_lo, vis_hi) is not
//          finite or beyond +-32768.
// Keys outside [vis_lo, vis_hi) (the call's trimmed key range; the tiles round
// it out to multiples of 16) are seen by no query: their K and V splits are
// written as zeros, so P = 0 times such a key's V is 0 whatever its slot holds
// (an unwritten ring slot may hold NaN).
struct G4aSplitParams {
    const float* k;        // [rows, Hkv, Dh]
    const float* v;        // [rows, Hkv, Dh]
    float* kout;
    float* kscale;
    float* vout;
    uint32_t* vflag;
    uint32_t k0, nkeys, S, Hkv, Dh;
    uint32_t ring_cap, epoch;
    uint32_t vis_lo, vis_hi;
};

// Per-head RMSNorm + half-split partial RoPE over rows of Dh values (the
// attention producer, g4a_norm_rope). Up to three segments (q, k, v) run in
// one launch; segment s covers T * heads_s rows, segment-major.
struct G4aNormRopeSeg {
    const float* x;     // [T, heads, Dh]
    const float* w;     // [Dh] RMSNorm weight, or null (unweighted)
    float* y;           // [T, heads, Dh], or a KV cache [rows, heads, Dh] when `cache`
    uint32_t heads;
    uint32_t norm;      // 1: RMSNorm the row
    uint32_t rope;      // 1: rotate its first rotary_dim dims
    uint32_t cache;     // 1: token t goes to logical cache row cache_row + t (slot % ring_cap)
    uint32_t first_t;   // tokens below it are skipped (their ring slots are rewritten by later tokens)
};

struct G4aNormRopeParams {
    G4aNormRopeSeg seg[3];
    const float* freq;      // [rotary_dim / 2]: theta^(-2j/rotary_dim), computed on the host
    const float2* sc;       // [sc_rows][rotary_dim / 2]: (sinf, cosf) of pos * freq[j], computed on the host
    uint32_t sc_rows;       // positions the table covers; later positions use sincosf on the device
    uint32_t any_norm;      // some segment is normalised: the workgroup runs the sequential sums
    const uint32_t* pos;    // device [T], or null: position pos0 + t
    uint32_t pos0;
    uint32_t T, Dh, rotary_dim;
    uint32_t nseg, total_rows;
    uint32_t cache_row, ring_cap;
    float eps;
    // Device position (g4a_attn_producer_devpos), or null. When set (T = 1): the
    // token's position and its logical cache row are *dpos, read at run time; a
    // position past max_pos (the table's and the cache's bound) writes nothing.
    const uint32_t* dpos;
    uint32_t max_pos;
};

// The int8 matrix-core projection (M <= 2): threads per workgroup, and the row
// bytes each 16-row block streams per unit (K * bits / 8 must be a multiple).
constexpr uint32_t G4A_LI8_THREADS = 256;
constexpr uint32_t G4A_LI8_UNIT_BYTES = 128;

// Quantised projection y[M, N] = epilogue(x[M, K] . W^T) (g4a_linear_q_*).
// W rows are packed fields of `bits` bits, LSB-first (offset binary, or native
// I8 when bits = 8 and xm = 0), each row starting on a 32-bit word for the
// word-parallel kernel. mode 0: y = acc * s[n]; mode 1: gelu(acc * s[n]) *
// (acc2 * s2[n]) with the second weight w2/s2; mode 2: gelu(acc * s[n]) *
// b[m * b_stride + b_off + n].
struct G4aLinearParams {
    const uint32_t* w;      // word-parallel kernel: [N, W] words
    const uint8_t* wb;      // element kernel: [N, row_bytes] bytes
    const float* s;         // [N, scale_stride]
    const uint32_t* w2;     // mode 1
    const uint8_t* wb2;
    const float* s2;
    const float* b;         // mode 2: [M, b_stride]
    const float* x;         // [M, K]
    float* y;               // [M, N]
    uint32_t M, N, K, W;
    uint32_t rows_per_wave;
    uint32_t b_stride, b_off;
    uint32_t xm;            // word mask turning each field into two's complement
    uint32_t bits, row_bytes, group_size, scale_stride, signed_i8;
    // mode 3 (x is one attention row merged from a decode step's split partials
    // while it is staged): the partials (T = 1: acc, then (m, l)), their split
    // count, head dim and query heads; xout, if set, receives the merged row
    const float* part;
    float* xout;
    uint32_t nsplit, dh, hq;
};

// Split counts up to which a decode step's output projection merges the split
// partials itself (mode 3), and the query heads it takes.
constexpr uint32_t G4A_FUSE_MAX_SPLITS = 16;
constexpr uint32_t G4A_FUSE_MAX_HEADS = 64;

// Quantised embedding rows: out[i, d] = deq(ids[i], d) * scale.
struct G4aEmbedParams {
    const uint8_t* wb;      // [V, row_bytes]
    const float* s;         // [V, scale_stride]
    const uint32_t* ids;    // [T]
    float* out;             // [T, D]
    uint32_t T, D;
    uint32_t bits, row_bytes, group_size, scale_stride, signed_i8;
    float scale;
};


// Elementwise ops (g4a_ew): y = op(a, b) over n elements.
enum G4aEwOp : uint32_t {
    G4A_EW_ADD = 0,
    G4A_EW_MUL = 1,
    G4A_EW_SCALE = 2,     // a * s
    G4A_EW_SCALE_BY = 3,  // a * sp[0]
    G4A_EW_GELU = 4,
    G4A_EW_GEGLU = 5,     // gelu(a) * b
    G4A_EW_SOFTCAP = 6,   // s * tanh(a / s)
    G4A_EW_FILL = 7,      // s (a is not read): the clear that graph capture can hold
};

struct G4aEwParams {
    const float* a;
    const float* b;
    const float* sp;
    float* y;
    size_t n;
    float s;
    uint32_t op;
};

// counters[i] += inc for i < n (u32, wrapping): advances device positions between
// replays of a captured decode step (g4a_u32_add).
struct G4aCounterParams {
    uint32_t* c;
    uint32_t n;
    uint32_t inc;
};

struct G4aSliceColsParams {
    const float* x;  // [rows, stride]
    float* y;        // [rows, width]
    uint32_t rows, stride, offset, width;
};

// y = (res + x * inv * w) * scale_by[0] per row of D values; res, w, scale_by optional.
struct G4aRmsRowsParams {
    const float* x;
    const float* w;
    const float* res;
    const float* scale_by;
    float* y;
    uint32_t rows, D;
    float eps;
};

struct G4aEmbedF32Params {
    const float* table;     // [V, D]
    const uint32_t* ids;    // [T]
    float* out;             // [T, D]
    uint32_t T, D;
    float scale;
};
