// Host code under AddressSanitizer + UndefinedBehaviorSanitizer, no GPU needed:
// libg4a.so built with -fsanitize on its host side (tests/test_sanitize.py) and
// the CPU oracle built the same way, driven over the paths that run on the host:
//   - g4a_attention_plan with no context over a sweep of shapes, windows, rings,
//     explicit position arrays and forced splits (the key-range trim of
//     rust/src/backend_wgpu.rs:924-936, the split choice, workspace sizing),
//     checking the plan's invariants;
//   - argument errors (also of the device-position entry points), g4a_create
//     without a device, and option validation;
//   - the oracle's attention, rms_norm, rope, projections and embeddings on
//     small inputs, including empty ones.
// Any sanitizer report aborts the process (halt_on_error); exit status 0 = clean.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <vector>

#include "g4a.h"

extern "C" {
int oracle_attention(const float* q, const float* k, const float* v, float* out, size_t T, size_t S, size_t Hq,
                     size_t Hkv, size_t Dh, size_t Dv, const uint32_t* q_pos, const uint32_t* k_pos, float scale,
                     uint32_t window, float softcap, int requested_threads);
void oracle_rms_norm(const float* x, const float* w, float* y, size_t rows, size_t d, float eps);
void oracle_rope(const float* x, float* y, size_t T, size_t heads, size_t head_dim, size_t rotary_dim,
                 const uint32_t* positions, float theta);
void oracle_linear_q(const uint8_t* qb, const float* scales, size_t N, size_t K, uint32_t bits, int signed_i8,
                     size_t group, const float* x, size_t M, float* y);
void oracle_linear_f32(const float* w, size_t N, size_t K, const float* x, size_t M, float* y);
void oracle_embed_rows_q(const uint8_t* qb, const float* scales, size_t V, size_t D, uint32_t bits, int signed_i8,
                         size_t group, const uint32_t* ids, size_t T, float scale, float* out);
}

namespace {

int g_failures = 0;
long g_plans = 0;

void check(bool ok, const char* what) {
    if (!ok) {
        std::printf("FAIL %s\n", what);
        ++g_failures;
    }
}

std::vector<uint32_t> ascending(std::mt19937& rng, size_t n, uint32_t first) {
    std::vector<uint32_t> v(n);
    uint32_t p = first;
    for (size_t i = 0; i < n; ++i) {
        v[i] = p;
        p += 1 + (rng() % 7 == 0 ? rng() % 5 : 0);  // mostly contiguous, with holes
    }
    return v;
}

void plan_sweep() {
    std::mt19937 rng(7);
    const uint32_t Ts[] = {0, 1, 2, 3, 15, 16, 17, 100, 2048};
    const uint32_t Ss[] = {0, 1, 7, 16, 63, 64, 65, 512, 520, 1000, 8192, 32768, 131072};
    const uint32_t Dhs[] = {8, 64, 256, 512, 1024};
    const uint32_t windows[] = {0, 1, 3, 512};
    const uint32_t group_heads[][2] = {{8, 1}, {4, 1}, {16, 2}, {8, 8}, {6, 3}};
    for (uint32_t T : Ts)
        for (uint32_t S : Ss)
            for (uint32_t Dh : Dhs)
                for (uint32_t W : windows)
                    for (auto& hh : group_heads)
                        for (int mode = 0; mode < 4; ++mode) {
                            g4a_attn_args a{};
                            a.T = T;
                            a.S = S;
                            a.Hq = hh[0];
                            a.Hkv = hh[1];
                            a.Dh = a.Dv = Dh;
                            a.scale = 1.0f;
                            a.sliding_window = W;
                            a.q_pos0 = S > T ? S - T : 0;
                            std::vector<uint32_t> qp, kp;
                            if (mode == 1 && S && T) {  // explicit positions with holes
                                kp = ascending(rng, S, rng() % 3);
                                qp.resize(T);
                                for (uint32_t i = 0; i < T; ++i) qp[i] = kp.back() + 1 - (T - 1 - i) + (rng() % 2);
                                a.k_pos = kp.data();
                                a.q_pos = qp.data();
                            }
                            if (mode == 2) a.splits = 1 + rng() % 1100;
                            if (mode == 3 && W) a.kv_ring_cap = W + T + (rng() % 3) - 1;
                            g4a_attn_plan p{};
                            const int rc = g4a_attention_plan(nullptr, &a, &p);
                            ++g_plans;
                            if (rc != G4A_OK) continue;  // refused shapes are fine; only accepted plans are checked
                            check(p.k_start <= p.k_end && p.k_end <= S, "plan: 0 <= k_start <= k_end <= S");
                            if (p.k_end > p.k_start && p.kernel != 0) {
                                check(p.splits >= 1, "plan: at least one split");
                                check(uint64_t(p.splits) * (p.keys_per_split ? p.keys_per_split : 1) >=
                                          uint64_t(p.k_end - p.k_start) ||
                                          p.keys_per_split == 0,
                                      "plan: the splits cover the key range");
                            }
                        }
}

void error_paths() {
    g4a_attn_args a{};
    g4a_attn_plan p{};
    check(g4a_attention_plan(nullptr, nullptr, &p) != G4A_OK, "null args refused");
    a.T = 1;
    a.S = 10;
    a.Hq = 8;
    a.Hkv = 3;  // 8 heads over 3 kv heads
    a.Dh = a.Dv = 256;
    check(g4a_attention_plan(nullptr, &a, &p) != G4A_OK, "Hq % Hkv != 0 refused");
    check(g4a_attention_plan(nullptr, &a, nullptr) != G4A_OK, "null plan refused");
    g4a_options o;
    g4a_default_options(&o);
    check(o.size == sizeof(g4a_options) && o.short_decode == 1 && o.linear_i8 == -1, "default options");
    g4a_ctx* ctx = nullptr;
    o.batch_kernel = 7;
    check(g4a_create_with(0, nullptr, &o, &ctx) == G4A_E_ARG && !ctx, "an option out of range is refused");
    g4a_default_options(&o);
    o.size = 4;
    check(g4a_create_with(0, nullptr, &o, &ctx) == G4A_E_ARG && !ctx, "an options struct of another size");
    check(std::strlen(g4a_last_error(nullptr)) > 0, "the failed create left a message");
    const int rc = g4a_create(0, nullptr, &ctx);  // no device in a CPU-only container
    if (rc == G4A_OK) {
        g4a_destroy(ctx);
    } else {
        check(ctx == nullptr, "a failed create returns no context");
    }
    check(g4a_create(0, nullptr, nullptr) != G4A_OK, "null out refused");
    // the device-position entry points refuse a missing context or arguments before any device work
    g4a_attn_args d{};
    d.T = 1;
    d.S = 100;
    d.Hq = 8;
    d.Hkv = 1;
    d.Dh = d.Dv = 256;
    check(g4a_attention_devpos(nullptr, &d, nullptr) != G4A_OK, "devpos attention without a context refused");
    g4a_producer_args pa{};
    check(g4a_attn_producer_devpos(nullptr, &pa, nullptr, 0) != G4A_OK, "devpos producer without a context refused");
    check(g4a_u32_add(nullptr, nullptr, 1, 1) != G4A_OK, "counter add without a context refused");
    void* stream = nullptr;
    check(g4a_stream(nullptr, &stream) != G4A_OK && stream == nullptr, "stream query without a context refused");
}

void oracle_paths() {
    std::mt19937 rng(3);
    std::normal_distribution<float> nd;
    for (size_t T : {0, 1, 3})
        for (size_t S : {0, 1, 5, 70})
            for (size_t Dh : {8, 64}) {
                const size_t Hq = 4, Hkv = 2;
                std::vector<float> q(T * Hq * Dh + 1), k(S * Hkv * Dh + 1), v(S * Hkv * Dh + 1), out(T * Hq * Dh + 1);
                for (auto& x : q) x = nd(rng);
                for (auto& x : k) x = nd(rng);
                for (auto& x : v) x = nd(rng);
                std::vector<uint32_t> qp(T + 1), kp(S + 1);
                for (size_t j = 0; j < S; ++j) kp[j] = uint32_t(j);
                for (size_t i = 0; i < T; ++i) qp[i] = uint32_t(S ? S - T + i : i);
                for (uint32_t W : {0u, 2u})
                    for (float cap : {0.0f, 5.0f}) {
                        oracle_attention(q.data(), k.data(), v.data(), out.data(), T, S, Hq, Hkv, Dh, Dh, qp.data(),
                                         kp.data(), 0.5f, W, cap, 2);
                        for (size_t i = 0; i < T * Hq * Dh; ++i) check(std::isfinite(out[i]), "oracle attention finite");
                    }
            }
    std::vector<float> x(5 * 16), y(5 * 16), w(16, 1.0f);
    for (auto& e : x) e = nd(rng);
    oracle_rms_norm(x.data(), w.data(), y.data(), 5, 16, 1e-6f);
    oracle_rms_norm(x.data(), nullptr, y.data(), 5, 16, 1e-6f);
    const uint32_t pos[5] = {0, 1, 2, 100000, 4000000000u};
    oracle_rope(x.data(), y.data(), 5, 1, 16, 10, pos, 1e4f);
    for (uint32_t bits : {2u, 4u, 8u})
        for (int sg : {0, 1}) {
            if (sg && bits != 8) continue;
            const size_t N = 9, K = 40, per_byte = sg ? 1 : 8 / bits, rb = K / per_byte;
            std::vector<uint8_t> qb(N * rb);
            for (auto& b : qb) b = uint8_t(rng());
            for (size_t group : {K, size_t(8)}) {
                const size_t groups = (K + group - 1) / group;
                std::vector<float> sc(N * groups, 0.01f), xi(3 * K), yo(3 * N);
                for (auto& e : xi) e = nd(rng);
                oracle_linear_q(qb.data(), sc.data(), N, K, bits, sg, group, xi.data(), 3, yo.data());
                const uint32_t ids[2] = {0, 8};
                std::vector<float> emb(2 * K);
                oracle_embed_rows_q(qb.data(), sc.data(), N, K, bits, sg, group, ids, 2, 1.5f, emb.data());
            }
        }
    std::vector<float> wf(6 * 7), xf(2 * 7), yf(2 * 6);
    oracle_linear_f32(wf.data(), 6, 7, xf.data(), 2, yf.data());
}

}  // namespace

int main() {
    plan_sweep();
    error_paths();
    oracle_paths();
    std::printf("%ld plans checked\n%s: %d failure(s)\n", g_plans, g_failures ? "FAILED" : "PASSED", g_failures);
    return g_failures ? 1 : 0;
}
