/*
 * TEST INFRASTRUCTURE ONLY — the CPU oracle for the attention hot path.
 *
 * Nothing in the product path (the HIP kernels, libg4a.so, the C++ backend)
 * links, loads or calls this file. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py use it, and only as the checker / the CPU
 * baseline.
 *
 * It restates, in C, the reference's CPU backend for the functions on the
 * attention path, keeping the exact arithmetic order so results are
 * bit-identical to the Rust code on the same inputs:
 *
 *   oracle_attention   <- rust/src/backend_cpu.rs:270-336 (CpuBackend::attention)
 *   par_ranges         <- rust/src/backend_cpu.rs:63-91   (row-parallel scoped threads,
 *                                                          GEMMA_CPU_THREADS, PAR_MIN_WORK)
 *   oracle_rms_norm    <- rust/src/backend_cpu.rs:149-172 (CpuBackend::rms_norm)
 *   oracle_concat_rows <- rust/src/backend_cpu.rs:352-364 (concat_rows / kv_append)
 *   oracle_rope        <- rust/src/backend_cpu.rs:248-268 (CpuBackend::rope: half-split
 *                                                          partial RoPE; libm powf/sinf/cosf
 *                                                          as Rust's f32::powf / sin_cos)
 *
 * Arithmetic contract (what makes it bit-identical to the Rust oracle):
 *   - every f32 op is a separately rounded IEEE single op: this file must be
 *     built with -ffp-contract=off and without -ffast-math (Rust never
 *     contracts a*b+c into an FMA and never reassociates);
 *   - the q.k dot runs d = 0..Dh-1 in order, then `*= scale`, then the
 *     optional soft-cap `cap*tanhf(dot/cap)`;
 *   - exp is libm expf (Rust's f32::exp calls the platform expf);
 *   - the probability sum runs j = 0..S-1 in order, inv = 1/sum (0 if sum==0);
 *   - the output accumulates (e*inv)*v over j in order, skipping w == 0.
 *
 * Parity pinning (what checks this restatement, see tests/test_oracle.py):
 *   closed forms (single visible key, q = 0 -> mean of visible v, all-future
 *   keys -> 0, window isolation), an f64 brute force, key-permutation and
 *   thread-count invariance, and the Lcg-regenerated inputs of the reference's
 *   own parity tests (rust/tests/gpu.rs:122-142, :262-293).
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

/* rust/src/backend_cpu.rs:64 */
#define PAR_MIN_WORK ((size_t)1 << 14)

typedef struct {
    const float *q, *k, *v;
    float *out;
    size_t T, S, Hq, Hkv, Dh, Dv;
    const uint32_t *q_pos, *k_pos;
    float scale;
    uint32_t window;
    float softcap;
} attn_job;

typedef struct {
    const attn_job *job;
    size_t start, end;
} attn_range;

/* One contiguous chunk of (query, head) rows: rust/src/backend_cpu.rs:280-333. */
static void attn_rows(const attn_job *o, size_t start, size_t end) {
    const size_t hq = o->Hq, dh = o->Dh, dv = o->Dv, s = o->S, hkv = o->Hkv;
    const size_t group = hq / hkv;
    float *scores = (float *)malloc((s ? s : 1) * sizeof(float));
    float *dst = o->out + start * dv;
    for (size_t r = start; r < end; ++r) {
        const size_t i = r / hq, h = r % hq;
        const uint32_t qpos = o->q_pos[i];
        const size_t kvh = h / group;
        const size_t qb = (i * hq + h) * dh;
        float maxv = -INFINITY;
        for (size_t j = 0; j < s; ++j) {
            const uint32_t kpos = o->k_pos[j];
            /* causal + optional sliding-window mask (u32 arithmetic, kpos <= qpos here) */
            if (kpos > qpos || (o->window > 0 && qpos - kpos >= o->window)) {
                scores[j] = -INFINITY;
                continue;
            }
            const size_t kb = (j * hkv + kvh) * dh;
            float dot = 0.0f;
            for (size_t d = 0; d < dh; ++d) dot += o->q[qb + d] * o->k[kb + d];
            dot *= o->scale;
            if (o->softcap > 0.0f) dot = o->softcap * tanhf(dot / o->softcap);
            scores[j] = dot;
            if (dot > maxv) maxv = dot;
        }
        float sum = 0.0f;
        for (size_t j = 0; j < s; ++j) {
            if (scores[j] == -INFINITY) {
                scores[j] = 0.0f;
            } else {
                const float e = expf(scores[j] - maxv);
                scores[j] = e;
                sum += e;
            }
        }
        const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
        float *ob = dst + (r - start) * dv;
        for (size_t j = 0; j < s; ++j) {
            const float w = scores[j] * inv;
            if (w == 0.0f) continue;
            const float *vb = o->v + (j * hkv + kvh) * dv;
            for (size_t d = 0; d < dv; ++d) ob[d] += w * vb[d];
        }
    }
    free(scores);
}

static void *attn_thread(void *p) {
    const attn_range *r = (const attn_range *)p;
    attn_rows(r->job, r->start, r->end);
    return NULL;
}

/* Thread count rule of par_ranges (rust/src/backend_cpu.rs:70-78): the
 * GEMMA_CPU_THREADS override if it parses to >= 1, else the core count;
 * capped at n rows, at least 1. `requested` > 0 replaces the env/core lookup
 * (the harness uses it to time a fixed thread count). */
size_t oracle_thread_count(size_t n, int requested) {
    size_t threads = 0;
    if (requested > 0) {
        threads = (size_t)requested;
    } else {
        const char *env = getenv("GEMMA_CPU_THREADS");
        if (env && *env) {
            char *endp = NULL;
            unsigned long long t = strtoull(env, &endp, 10);
            if (endp && *endp == '\0' && t >= 1) threads = (size_t)t;
        }
        if (threads == 0) {
            long c = sysconf(_SC_NPROCESSORS_ONLN);
            threads = c > 0 ? (size_t)c : 1;
        }
    }
    if (threads > n) threads = n;
    if (threads < 1) threads = 1;
    return threads;
}

/*
 * CpuBackend::attention. q [T,Hq,Dh], k [S,Hkv,Dh], v [S,Hkv,Dv] row-major f32;
 * out [T, Hq*Dv] is fully written. q_pos[T], k_pos[S] are absolute positions.
 * Returns the number of threads used.
 */
int oracle_attention(const float *q, const float *k, const float *v, float *out, size_t T, size_t S,
                     size_t Hq, size_t Hkv, size_t Dh, size_t Dv, const uint32_t *q_pos, const uint32_t *k_pos,
                     float scale, uint32_t window, float softcap, int requested_threads) {
    attn_job job = {q, k, v, out, T, S, Hq, Hkv, Dh, Dv, q_pos, k_pos, scale, window, softcap};
    const size_t n = T * Hq;
    memset(out, 0, n * Dv * sizeof(float));
    if (n == 0) return 1;
    const size_t work = T * Hq * S * (Dh + Dv);
    const size_t threads = oracle_thread_count(n, requested_threads);
    if (threads == 1 || work < PAR_MIN_WORK) {
        attn_rows(&job, 0, n);
        return 1;
    }
    const size_t chunk = (n + threads - 1) / threads;
    size_t nt = (n + chunk - 1) / chunk;
    pthread_t *tids = (pthread_t *)malloc(nt * sizeof(pthread_t));
    attn_range *rg = (attn_range *)malloc(nt * sizeof(attn_range));
    for (size_t t = 0; t < nt; ++t) {
        rg[t].job = &job;
        rg[t].start = t * chunk;
        rg[t].end = (t + 1) * chunk < n ? (t + 1) * chunk : n;
        pthread_create(&tids[t], NULL, attn_thread, &rg[t]);
    }
    for (size_t t = 0; t < nt; ++t) pthread_join(tids[t], NULL);
    free(tids);
    free(rg);
    return (int)nt;
}

/* CpuBackend::rms_norm (rust/src/backend_cpu.rs:149-172): per row of d values,
 * ss = sequential sum of x*x, inv = 1/sqrt(ss/d + eps), y = x*inv (*w if given). */
void oracle_rms_norm(const float *x, const float *w, float *y, size_t rows, size_t d, float eps) {
    for (size_t i = 0; i < rows; ++i) {
        const float *xr = x + i * d;
        float ss = 0.0f;
        for (size_t j = 0; j < d; ++j) ss += xr[j] * xr[j];
        const float inv = 1.0f / sqrtf(ss / (float)d + eps);
        float *o = y + i * d;
        if (w) {
            for (size_t j = 0; j < d; ++j) o[j] = xr[j] * inv * w[j];
        } else {
            for (size_t j = 0; j < d; ++j) o[j] = xr[j] * inv;
        }
    }
}

/* CpuBackend::rope (rust/src/backend_cpu.rs:248-268): x, y [T, heads, head_dim];
 * for each row and j < rotary_dim/2: freq = theta^(-(2j)/rotary_dim) (powf),
 * ang = pos * freq, a = x[j], b = x[j + half]: y[j] = a*cos - b*sin,
 * y[j + half] = b*cos + a*sin; every other dim is copied. */
void oracle_rope(const float *x, float *y, size_t T, size_t heads, size_t head_dim, size_t rotary_dim,
                 const uint32_t *positions, float theta) {
    memcpy(y, x, T * heads * head_dim * sizeof(float));
    const size_t half = rotary_dim / 2;
    for (size_t i = 0; i < T; ++i) {
        const float pos = (float)positions[i];
        for (size_t h = 0; h < heads; ++h) {
            const size_t base = (i * heads + h) * head_dim;
            for (size_t j = 0; j < half; ++j) {
                const float freq = powf(theta, -(2.0f * (float)j) / (float)rotary_dim);
                const float ang = pos * freq;
                const float sn = sinf(ang), cs = cosf(ang);
                const float a = x[base + j];
                const float b = x[base + j + half];
                y[base + j] = a * cs - b * sn;
                y[base + j + half] = b * cs + a * sn;
            }
        }
    }
}

/* CpuBackend::concat_rows / kv_append (rust/src/backend_cpu.rs:352-364):
 * out = a ++ b along rows (a may be NULL). */
void oracle_concat_rows(const float *a, size_t a_elems, const float *b, size_t b_elems, float *out) {
    if (a && a_elems) memcpy(out, a, a_elems * sizeof(float));
    memcpy(out + a_elems, b, b_elems * sizeof(float));
}

/* f64 brute force of the same masked softmax attention (no f32 rounding in the
 * scores, probabilities or accumulation): the independent reference the f32
 * restatement is measured against. */
void oracle_attention_f64(const float *q, const float *k, const float *v, double *out, size_t T, size_t S,
                          size_t Hq, size_t Hkv, size_t Dh, size_t Dv, const uint32_t *q_pos,
                          const uint32_t *k_pos, double scale, uint32_t window, double softcap) {
    const size_t group = Hq / Hkv;
    double *sc = (double *)malloc((S ? S : 1) * sizeof(double));
    for (size_t i = 0; i < T; ++i) {
        for (size_t h = 0; h < Hq; ++h) {
            const size_t kvh = h / group;
            const float *qr = q + (i * Hq + h) * Dh;
            double m = -INFINITY;
            for (size_t j = 0; j < S; ++j) {
                const uint32_t kp = k_pos[j], qp = q_pos[i];
                if (kp > qp || (window > 0 && qp - kp >= window)) {
                    sc[j] = -INFINITY;
                    continue;
                }
                const float *kr = k + (j * Hkv + kvh) * Dh;
                double dot = 0.0;
                for (size_t d = 0; d < Dh; ++d) dot += (double)qr[d] * (double)kr[d];
                dot *= scale;
                if (softcap > 0.0) dot = softcap * tanh(dot / softcap);
                sc[j] = dot;
                if (dot > m) m = dot;
            }
            double sum = 0.0;
            for (size_t j = 0; j < S; ++j) {
                sc[j] = (sc[j] == -INFINITY) ? 0.0 : exp(sc[j] - m);
                sum += sc[j];
            }
            double *o = out + (i * Hq + h) * Dv;
            for (size_t d = 0; d < Dv; ++d) o[d] = 0.0;
            if (sum > 0.0) {
                for (size_t j = 0; j < S; ++j) {
                    if (sc[j] == 0.0) continue;
                    const double w = sc[j] / sum;
                    const float *vr = v + (j * Hkv + kvh) * Dv;
                    for (size_t d = 0; d < Dv; ++d) o[d] += w * (double)vr[d];
                }
            }
        }
    }
    free(sc);
}
