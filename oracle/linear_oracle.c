/*
 * TEST INFRASTRUCTURE ONLY — the CPU oracle for the quantised projections
 * around the attention path (q/k/v/o projections, the GeGLU MLP input and the
 * per-layer-input gate).
 *
 * Nothing in the product path links, loads or calls this file. Only tests/,
 * __graft_entry__.smoke() and the cpu_baseline leg of bench.py use it, and
 * only as the checker / the CPU baseline.
 *
 * It restates the reference's CPU backend with its exact arithmetic order:
 *
 *   oracle_deq          <- rust/src/backend.rs:44-58    (QuantWeight::deq: offset-binary
 *                                                        sub-byte fields packed LSB-first,
 *                                                        or native I8; times the (row,
 *                                                        group) scale)
 *   oracle_linear_q     <- rust/src/backend_cpu.rs:174-222 (CpuBackend::linear on a
 *                                                        quantised weight: each weight row
 *                                                        dequantised once, then
 *                                                        acc += x[k] * w[k] for k in order)
 *   oracle_gelu_tanh    <- rust/src/backend_cpu.rs:55-58 (gelu_tanh_scalar, libm tanhf as
 *                                                        Rust's f32::tanh)
 *   oracle_embed_rows_q <- rust/src/backend_cpu.rs:127-145 (embed_rows on a quantised
 *                                                        table: deq(id, d) * scale)
 *   oracle_linear_f32   <- rust/src/backend_cpu.rs:174-222 (linear on an f32 weight)
 *   oracle_softcap_n    <- rust/src/backend_cpu.rs:242-244 (cap * tanhf(v / cap))
 *   oracle_embed_rows_f32 <- rust/src/backend_cpu.rs:138-144 (table[id, d] * scale)
 *
 * Build with -ffp-contract=off and without -ffast-math: every f32 operation is
 * a separately rounded IEEE single operation, as in the Rust code.
 *
 * Parity pinning (tests/test_linear_oracle.py): hand-packed bytes with known
 * values (zero points, field order, sign of I8), one-hot inputs that read one
 * dequantised weight exactly, an f64 brute force, grouped against per-row
 * scales, and the Lcg-regenerated inputs of the reference's own test
 * (rust/tests/gpu.rs:150-190).
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>

/* QuantWeight::per_byte / row_bytes / scale_stride (rust/src/backend.rs:28-41) */
static size_t per_byte(uint32_t bits, int signed_i8) { return signed_i8 ? 1 : (size_t)(8 / bits); }
static size_t row_bytes(size_t K, uint32_t bits, int signed_i8) { return signed_i8 ? K : K / per_byte(bits, signed_i8); }
static size_t scale_stride(size_t K, size_t group) { return (K + group - 1) / group; }

/* QuantWeight::deq (rust/src/backend.rs:44-58) */
float oracle_deq(const uint8_t *qb, const float *scales, size_t K, uint32_t bits, int signed_i8, size_t group,
                 size_t n, size_t k) {
    const size_t rb = row_bytes(K, bits, signed_i8);
    int32_t qv;
    if (signed_i8) {
        qv = (int32_t)(int8_t)qb[n * rb + k];
    } else {
        const size_t pb = per_byte(bits, signed_i8);
        const uint32_t b = qb[n * rb + k / pb];
        const uint32_t shift = (uint32_t)(k % pb) * bits;
        qv = (int32_t)((b >> shift) & ((1u << bits) - 1u)) - (int32_t)(1u << (bits - 1));
    }
    return (float)qv * scales[n * scale_stride(K, group) + k / group];
}

/* CpuBackend::linear with a quantised weight (rust/src/backend_cpu.rs:174-222):
 * y[i, n] = sum over k in order of x[i, k] * deq(n, k), one f32 accumulator per
 * output. The reference splits rows across threads without changing any sum. */
void oracle_linear_q(const uint8_t *qb, const float *scales, size_t N, size_t K, uint32_t bits, int signed_i8,
                     size_t group, const float *x, size_t M, float *y) {
    float *row = (float *)malloc((K ? K : 1) * sizeof(float));
    for (size_t n = 0; n < N; ++n) {
        for (size_t k = 0; k < K; ++k) row[k] = oracle_deq(qb, scales, K, bits, signed_i8, group, n, k);
        for (size_t i = 0; i < M; ++i) {
            const float *xb = x + i * K;
            float acc = 0.0f;
            for (size_t k = 0; k < K; ++k) acc += xb[k] * row[k];
            y[i * N + n] = acc;
        }
    }
    free(row);
}

/* gelu_tanh_scalar (rust/src/backend_cpu.rs:55-58):
 * c = sqrt(2/pi) in f32; 0.5 * v * (1 + tanh(c * (v + 0.044715 * v * v * v))). */
float oracle_gelu_tanh(float v) {
    const float c = sqrtf(2.0f / 3.14159265358979323846f);
    return 0.5f * v * (1.0f + tanhf(c * (v + 0.044715f * v * v * v)));
}

void oracle_gelu_tanh_n(const float *x, float *y, size_t n) {
    for (size_t i = 0; i < n; ++i) y[i] = oracle_gelu_tanh(x[i]);
}

/* CpuBackend::embed_rows on a quantised table (rust/src/backend_cpu.rs:127-137):
 * out[i, d] = deq(ids[i], d) * scale. */
void oracle_embed_rows_q(const uint8_t *qb, const float *scales, size_t V, size_t D, uint32_t bits, int signed_i8,
                         size_t group, const uint32_t *ids, size_t T, float scale, float *out) {
    (void)V;
    for (size_t i = 0; i < T; ++i)
        for (size_t d = 0; d < D; ++d)
            out[i * D + d] = oracle_deq(qb, scales, D, bits, signed_i8, group, ids[i], d) * scale;
}

/* CpuBackend::linear with an f32 weight (rust/src/backend_cpu.rs:174-222):
 * y[i, n] = sum over k in order of x[i, k] * w[n, k]. */
void oracle_linear_f32(const float *w, size_t N, size_t K, const float *x, size_t M, float *y) {
    for (size_t n = 0; n < N; ++n) {
        const float *wb = w + n * K;
        for (size_t i = 0; i < M; ++i) {
            const float *xb = x + i * K;
            float acc = 0.0f;
            for (size_t k = 0; k < K; ++k) acc += xb[k] * wb[k];
            y[i * N + n] = acc;
        }
    }
}

/* CpuBackend::softcap (rust/src/backend_cpu.rs:242-244): cap * tanh(v / cap). */
void oracle_softcap_n(const float *x, float cap, float *y, size_t n) {
    for (size_t i = 0; i < n; ++i) y[i] = cap * tanhf(x[i] / cap);
}

/* CpuBackend::embed_rows on an f32 table (rust/src/backend_cpu.rs:138-144). */
void oracle_embed_rows_f32(const float *table, size_t D, const uint32_t *ids, size_t T, float scale, float *out) {
    for (size_t i = 0; i < T; ++i)
        for (size_t d = 0; d < D; ++d) out[i * D + d] = table[(size_t)ids[i] * D + d] * scale;
}
