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
    uint32_t keys_per_split, nsplit;
    uint32_t ring_cap;
    uint32_t window;
    float scale, softcap;
};

// Log-sum-exp merge of the split partials written by the decode kernel.
struct G4aCombineParams {
    const float* part;
    float* out;
    uint32_t T, Hq, nsplit, Dh;
};

// Generic per-(query, head) attention for shapes outside the fast paths
// (any Hq/Hkv/Dh/Dv). Positions are always device arrays here.
struct G4aGenericParams {
    const float* q;        // [T, Hq, Dh]
    const float* k;        // [rows, Hkv, Dh]
    const float* v;        // [rows, Hkv, Dv]
    float* out;            // [T, Hq*Dv]
    const uint32_t* q_pos; // [T]
    const uint32_t* k_pos; // [S]
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
    const float* ksplit;   // head_dim 256: keys ksplit0.. as bf16 hi/lo pairs (g4a_split_k_bf16 layout)
    uint32_t T, S, Hq, Hkv;
    uint32_t q_pos0, k_pos0;
    uint32_t ring_cap, window;
    uint32_t ksplit0, ksplit_n;
    float scale;
};

// K rows split into bf16 pairs for the matrix-core score estimate: key j of
// [k0, k0 + nkeys) (logical, read through the ring) becomes row j - k0 of
// `out`, same row stride as k (Hkv * Dh 4-byte slots); each 8-dim block of a
// head occupies 8 slots: the 8 bf16 hi parts, then the 8 bf16 lo parts, with
// hi = bf16(x) and lo = bf16(x - hi), both rounded to nearest even.
struct G4aSplitParams {
    const float* k;        // [rows, Hkv, Dh]
    float* out;            // [nkeys, Hkv, Dh] slots
    uint32_t k0, nkeys, Hkv, Dh;
    uint32_t ring_cap;
};
