// Parity driver for the C++ HipBackend (gemma-4-webgpu-kernels_amd/csrc/hip_backend.hpp):
// the reference's backend tests for this path, run through the op surface a
// Rust HipBackend would call, checked against the CPU oracle
// (oracle/attn_oracle.c, a restatement of rust/src/backend_cpu.rs:270-336).
//
//   grouped_attention_parity   rust/tests/gpu.rs:262-293 (same cases, Lcg seed 21)
//   slice/concat/kv_append     rust/tests/gpu.rs:96-120 (three 200-row appends: growth)
//   norm_rope_parity           kernel_parity's rmsNorm and rope(partial) (rust/tests/gpu.rs:53-59,
//                              :84-90, Lcg seed 7) and fused_op_parity's head_norm_rope cases
//                              (rust/tests/gpu.rs:322-334, Lcg seed 33)
//   quantized_kernel_parity    rust/tests/gpu.rs:146-190 (Lcg seed 9): q4/q2 linear at M = 5
//                              and 1, q4 with K = 52, I8, the grouped-scale q4 embedding,
//                              plus the fused GeGLU and gelu-times-columns projections,
//                              against oracle/linear_oracle.c
//   kernel_parity_ops          rust/tests/gpu.rs:37-100 (Lcg seed 7): f32 linear (tiled and
//                              gemv), add, mul, scale, geluTanh, geglu, softcap,
//                              scaleByTensor, embedRows, sliceCols; fused_op_parity's
//                              add_rms_norm (rust/tests/gpu.rs:310-321, Lcg seed 33)
//   kv_cache_decode            prefill chunks + decode steps through KvCache, with a
//                              sliding layer on a ring (incl. regrowth and wrap-around)
//                              and a global layer on the growing buffer, every step
//                              checked against the oracle over the full history
//
// The bar is the north star's: max-abs <= 1e-5 and mean-abs <= 1e-6 (f32),
// exact equality for the copies. Exit status 0 = all passed.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "hip_backend.hpp"

extern "C" int oracle_attention(const float* q, const float* k, const float* v, float* out, size_t T, size_t S,
                                size_t Hq, size_t Hkv, size_t Dh, size_t Dv, const uint32_t* q_pos,
                                const uint32_t* k_pos, float scale, uint32_t window, float softcap,
                                int requested_threads);

extern "C" void oracle_linear_q(const uint8_t* qb, const float* scales, size_t N, size_t K, uint32_t bits,
                                int signed_i8, size_t group, const float* x, size_t M, float* y);
extern "C" float oracle_gelu_tanh(float v);
extern "C" void oracle_linear_f32(const float* w, size_t N, size_t K, const float* x, size_t M, float* y);
extern "C" void oracle_softcap_n(const float* x, float cap, float* y, size_t n);
extern "C" void oracle_embed_rows_f32(const float* table, size_t D, const uint32_t* ids, size_t T, float scale,
                                      float* out);
extern "C" float oracle_deq(const uint8_t* qb, const float* scales, size_t K, uint32_t bits, int signed_i8,
                            size_t group, size_t n, size_t k);
extern "C" void oracle_embed_rows_q(const uint8_t* qb, const float* scales, size_t V, size_t D, uint32_t bits,
                                    int signed_i8, size_t group, const uint32_t* ids, size_t T, float scale,
                                    float* out);
extern "C" void oracle_rms_norm(const float* x, const float* w, float* y, size_t rows, size_t d, float eps);
extern "C" void oracle_rope(const float* x, float* y, size_t T, size_t heads, size_t head_dim, size_t rotary_dim,
                            const uint32_t* positions, float theta);

namespace {

int g_failures = 0;

// rust/tests/common/mod.rs:30-42
struct Lcg {
    uint32_t s;
    explicit Lcg(uint32_t seed) : s(seed) {}
    float next() {
        s = (s * 1103515245u + 12345u) & 0x7fffffffu;
        return float(s) / float(0x7fffffff);
    }
    std::vector<float> rand(size_t n, float scale) {
        std::vector<float> out(n);
        for (auto& x : out) x = (next() * 2.0f - 1.0f) * scale;
        return out;
    }
};

void expect(bool ok, const std::string& label) {
    std::printf("  %s %s\n", ok ? "ok  " : "FAIL", label.c_str());
    std::fflush(stdout);
    if (!ok) ++g_failures;
}

void close(const std::string& label, const std::vector<float>& got, const std::vector<float>& want) {
    if (got.size() != want.size()) {
        expect(false, label + ": size " + std::to_string(got.size()) + " != " + std::to_string(want.size()));
        return;
    }
    double mx = 0.0, sum = 0.0;
    for (size_t i = 0; i < got.size(); ++i) {
        double d = std::fabs(double(got[i]) - double(want[i]));
        if (!(d <= mx)) mx = d;  // NaN-propagating
        sum += d;
    }
    double mean = got.empty() ? 0.0 : sum / double(got.size());
    char buf[160];
    std::snprintf(buf, sizeof buf, " (max-abs %.3e mean-abs %.3e)", mx, mean);
    expect(mx <= 1e-5 && mean <= 1e-6, label + buf);
}

std::vector<float> oracle(const std::vector<float>& q, const std::vector<float>& k, const std::vector<float>& v,
                          size_t T, size_t S, size_t Hq, size_t Hkv, size_t Dh, const std::vector<uint32_t>& qp,
                          const std::vector<uint32_t>& kp, float scale, uint32_t window) {
    std::vector<float> out(T * Hq * Dh);
    oracle_attention(q.data(), k.data(), v.data(), out.data(), T, S, Hq, Hkv, Dh, Dh, qp.data(), kp.data(), scale,
                     window, 0.0f, 0);
    return out;
}

std::vector<uint32_t> iota(uint32_t from, uint32_t to) {
    std::vector<uint32_t> r;
    for (uint32_t i = from; i < to; ++i) r.push_back(i);
    return r;
}

void grouped_attention_parity(g4a::HipBackend& b) {
    std::printf("grouped_attention_parity\n");
    Lcg r(21);
    struct Case { size_t t, s, hq, hkv, dh; uint32_t window; };
    const Case cases[] = {{3, 300, 8, 1, 256, 0}, {3, 300, 8, 1, 256, 150}, {1, 700, 8, 1, 512, 0},
                          {1, 900, 8, 1, 256, 512}, {5, 5, 8, 1, 256, 0},     {6, 70, 8, 1, 256, 3},
                          {2, 200, 4, 1, 256, 0},   {1, 64, 8, 2, 512, 0}};
    for (const Case& c : cases) {
        auto q = r.rand(c.t * c.hq * c.dh, 0.5f);
        auto k = r.rand(c.s * c.hkv * c.dh, 0.5f);
        auto v = r.rand(c.s * c.hkv * c.dh, 0.5f);
        auto kpos = iota(0, uint32_t(c.s));
        auto qpos = iota(uint32_t(c.s - c.t), uint32_t(c.s));
        const float scale = 1.0f / std::sqrt(float(c.dh));
        g4a::AttnOpts o;
        o.q_pos = qpos.data();
        o.n_q_pos = qpos.size();
        o.k_pos = kpos.data();
        o.n_k_pos = kpos.size();
        o.scale = scale;
        o.sliding_window = c.window;
        auto out = b.attention(b.tensor(q.data(), {c.t, c.hq, c.dh}), b.tensor(k.data(), {c.s, c.hkv, c.dh}),
                               b.tensor(v.data(), {c.s, c.hkv, c.dh}), o);
        if (out.shape != std::vector<size_t>{c.t, c.hq * c.dh}) expect(false, "attention output shape");
        char label[128];
        std::snprintf(label, sizeof label, "grouped attention (T=%zu, S=%zu, Hq=%zu, Hkv=%zu, Dh=%zu, window=%u)", c.t,
                      c.s, c.hq, c.hkv, c.dh, c.window);
        close(label, b.readback(out), oracle(q, k, v, c.t, c.s, c.hq, c.hkv, c.dh, qpos, kpos, scale, c.window));
    }
}

void copies_and_kv_append(g4a::HipBackend& b) {
    std::printf("slice_rows / concat_rows / kv_append\n");
    Lcg r(7);
    const size_t rows = 4, stride = 13;
    auto x = r.rand(rows * stride, 1.0f);
    auto sl = b.readback(b.slice_rows(b.tensor(x.data(), {rows, stride}), 2, 2));
    expect(sl == std::vector<float>(x.begin() + 2 * stride, x.begin() + 4 * stride), "slice_rows");
    auto a = r.rand(2 * stride, 1.0f);
    auto c = r.rand(3 * stride, 1.0f);
    auto ta = b.tensor(a.data(), {2, stride});
    auto tc = b.tensor(c.data(), {3, stride});
    auto cat = b.concat_rows(&ta, tc);
    std::vector<float> want = a;
    want.insert(want.end(), c.begin(), c.end());
    expect(cat.shape == std::vector<size_t>{5, stride} && b.readback(cat) == want, "concat_rows");
    expect(b.readback(b.concat_rows(nullptr, tc)) == c, "concat_rows (None)");

    // three appends of 200 rows: capacity 256 -> 512 -> 1024 (rust/tests/gpu.rs:108-120)
    const size_t dim = 8;
    std::optional<g4a::HipTensor> t;
    std::vector<float> host;
    const size_t caps[] = {256, 512, 1024};
    const bool dead[] = {false, true, true};
    for (int i = 0; i < 3; ++i) {
        auto chunk = r.rand(200 * dim, 1.0f);
        host.insert(host.end(), chunk.begin(), chunk.end());
        auto res = b.kv_append(t ? &*t : nullptr, b.tensor(chunk.data(), {200, dim}));
        expect(res.tensor.cap_rows == caps[i] && res.dead.has_value() == dead[i],
               "kv_append step " + std::to_string(i) + ": capacity " + std::to_string(res.tensor.cap_rows));
        t = res.tensor;
    }
    expect(t->shape == std::vector<size_t>{600, dim}, "kv_append shape [600, 8]");
    expect(b.readback(*t) == host, "kv_append (growth) contents");
    // an append that fits reuses the buffer in place
    auto extra = r.rand(10 * dim, 1.0f);
    auto res = b.kv_append(&*t, b.tensor(extra.data(), {10, dim}));
    host.insert(host.end(), extra.begin(), extra.end());
    expect(!res.dead && res.tensor.buffer == t->buffer && b.readback(res.tensor) == host, "kv_append in place");
}

// A two-layer stack: layer 0 slides (window 512, Dh 256, ring), layer 1 is
// global (Dh 512, growing buffer). Chunk sizes force a ring regrowth (a chunk
// wider than the ring allows) and wrap-around (history longer than the ring).
void kv_cache_decode(g4a::HipBackend& b) {
    std::printf("kv_cache_decode (ring sliding layer + growing global layer)\n");
    const uint32_t W = 512;
    const size_t Hq = 8, Hkv = 1, D0 = 256, D1 = 512;
    std::vector<size_t> chunks = {100};
    for (int i = 0; i < 20; ++i) chunks.push_back(1);
    chunks.push_back(450);
    for (int i = 0; i < 10; ++i) chunks.push_back(1);
    chunks.push_back(64);
    for (int i = 0; i < 420; ++i) chunks.push_back(1);
    chunks.push_back(33);
    for (int i = 0; i < 4; ++i) chunks.push_back(1);

    Lcg r(99);
    g4a::KvCache cache(2);
    std::vector<float> k0, v0, k1, v1;  // full host history per layer
    uint32_t pos = 0;
    size_t step = 0, checked = 0;
    uint32_t last_ring = 0;
    for (size_t rows : chunks) {
        auto qpos = iota(pos, pos + uint32_t(rows));
        cache.push_positions(qpos.data(), qpos.size());
        const auto& kpos = cache.positions;
        const size_t S = kpos.size();
        for (int layer = 0; layer < 2; ++layer) {
            const size_t D = layer ? D1 : D0;
            const uint32_t window = layer ? 0 : W;
            const float scale = layer ? 1.0f : 1.0f / 16.0f;
            auto q = r.rand(rows * Hq * D, 1.0f);
            auto kn = r.rand(rows * Hkv * D, 1.0f);
            auto vn = r.rand(rows * Hkv * D, 1.0f);
            auto& kh = layer ? k1 : k0;
            auto& vh = layer ? v1 : v0;
            kh.insert(kh.end(), kn.begin(), kn.end());
            vh.insert(vh.end(), vn.begin(), vn.end());
            auto [k, v] = cache.append_and_read(b, layer, b.tensor(kn.data(), {rows, Hkv, D}),
                                                b.tensor(vn.data(), {rows, Hkv, D}), window);
            if (k.shape[0] != S) expect(false, "cache rows != positions");
            g4a::AttnOpts o;
            o.q_pos = qpos.data();
            o.n_q_pos = qpos.size();
            o.k_pos = kpos.data();
            o.n_k_pos = S;
            o.scale = scale;
            o.sliding_window = window;
            auto out = b.attention(b.tensor(q.data(), {rows, Hq, D}), k, v, o);
            // every chunk, and every 16th decode step, is checked against the oracle
            if (rows > 1 || step % 16 == 0 || step + 1 == chunks.size()) {
                char label[160];
                std::snprintf(label, sizeof label, "layer %d step %zu: T=%zu S=%zu%s", layer, step, rows, S,
                              layer ? "" : (" ring " + std::to_string(k.ring_cap)).c_str());
                close(label, b.readback(out), oracle(q, kh, vh, rows, S, Hq, Hkv, D, qpos, kpos, scale, window));
                ++checked;
            }
            if (layer == 0) {
                if (k.ring_cap != last_ring) std::printf("  ring capacity %u at S=%zu\n", k.ring_cap, S);
                last_ring = k.ring_cap;
                if (k.ring_cap < W + rows - 1) expect(false, "ring smaller than window + chunk - 1");
            }
        }
        pos += uint32_t(rows);
        ++step;
        auto dead = cache.take_dead();
        b.end_frame({}, std::move(dead));
    }
    // the ring reads back its resident rows in logical order
    const auto* slot = cache.read(0);
    const size_t S = cache.positions.size();
    const size_t live = std::min<size_t>(S, slot->first.ring_cap);
    auto got = b.readback(slot->first);
    std::vector<float> want(k0.end() - live * D0, k0.end());
    expect(S > slot->first.ring_cap && got == want, "ring wrapped and holds the last " + std::to_string(live) + " keys");
    const auto* g = cache.read(1);
    expect(b.readback(g->second) == v1, "global layer holds the whole history");
    std::printf("  %zu attention calls checked over %zu tokens\n", checked, S);
    cache.reset(b);
}

void norm_rope_parity(g4a::HipBackend& b) {
    std::printf("norm_rope_parity\n");
    {
        Lcg r(7);
        r.rand(17 * 40 + 23 * 40 + 40, 1.0f);  // kernel_parity's linear draws
        const size_t t = 5, d = 48;
        const auto x = r.rand(t * d, 1.0f);
        const auto w = r.rand(d, 0.1f);
        std::vector<float> want(t * d);
        oracle_rms_norm(x.data(), w.data(), want.data(), t, d, 1e-6f);
        auto gx = b.tensor(x.data(), {t, d});
        auto gw = b.tensor(w.data(), {d});
        close("rmsNorm", b.readback(b.rms_norm(gx, &gw, 1e-6f)), want);
        oracle_rms_norm(x.data(), nullptr, want.data(), t, d, 1e-6f);
        close("rmsNorm (unweighted)", b.readback(b.rms_norm(gx, nullptr, 1e-6f)), want);
        r.rand(100 + 100 + 30 * 16, 1.0f);  // elementwise and embed draws
        const size_t T = 4, heads = 2, dh = 16, rot = 8;
        const uint32_t pos[4] = {0, 1, 5, 9};
        const auto xr = r.rand(T * heads * dh, 1.0f);
        std::vector<float> wr(T * heads * dh);
        oracle_rope(xr.data(), wr.data(), T, heads, dh, rot, pos, 1e4f);
        close("rope(partial)", b.readback(b.rope(b.tensor(xr.data(), {T, heads, dh}), pos, T, 1e4f, dh, heads, rot)), wr);
    }
    Lcg r(33);
    r.rand(5 * 48 + 5 * 48 + 48, 1.0f);  // fused_op_parity's add_rms_norm draws
    const size_t cases[3][4] = {{3, 4, 16, 8}, {2, 8, 256, 256}, {2, 1, 512, 128}};
    for (const auto& c : cases) {
        const size_t t = c[0], heads = c[1], dh = c[2], rot = c[3];
        const auto x = r.rand(t * heads * dh, 1.0f);
        const auto w = r.rand(dh, 0.1f);
        std::vector<uint32_t> pos(t);
        for (size_t i = 0; i < t; ++i) pos[i] = uint32_t(i * 7 + 3);
        std::vector<float> normed(x.size()), want(x.size());
        oracle_rms_norm(x.data(), w.data(), normed.data(), t * heads, dh, 1e-6f);
        oracle_rope(normed.data(), want.data(), t, heads, dh, rot, pos.data(), 1e4f);
        auto got = b.head_norm_rope(b.tensor(x.data(), {t, heads, dh}), b.tensor(w.data(), {dh}), 1e-6f, pos.data(),
                                    t, 1e4f, dh, heads, rot);
        close("head_norm_rope (heads=" + std::to_string(heads) + ", Dh=" + std::to_string(dh) + ", rot=" +
                  std::to_string(rot) + ")",
              b.readback(got), want);
    }
}

// rust/src/dequant.rs:53-63 (pack_unsigned): raw fields LSB-first
std::vector<uint8_t> pack_unsigned(const std::vector<uint32_t>& v, uint32_t bits) {
    const size_t per = 8 / bits;
    std::vector<uint8_t> out((v.size() + per - 1) / per, 0);
    for (size_t i = 0; i < v.size(); ++i)
        out[i / per] |= uint8_t((v[i] & ((1u << bits) - 1)) << ((i % per) * bits));
    return out;
}

// The word-parallel kernel sums in another order than the CPU: per output
// |gpu - oracle| <= 2e-6 * sum_k |x_k w_nk| + 1e-7 (the reference's own test
// allows 2e-3 absolute, rust/tests/gpu.rs:156-190).
void close_linear(const std::string& label, const std::vector<float>& got, const std::vector<float>& want,
                  const g4a::QuantWeight& q, const std::vector<float>& x, size_t m) {
    const size_t N = q.shape[0], K = q.shape[1];
    double worst = 0.0, max_abs = 0.0;
    bool ok = got.size() == want.size();
    for (size_t i = 0; ok && i < m; ++i)
        for (size_t n = 0; n < N; ++n) {
            double bound = 0.0;
            for (size_t k = 0; k < K; ++k)
                bound += std::fabs(double(x[i * K + k])) *
                         std::fabs(double(oracle_deq(q.qbytes.data(), q.scales.data(), K, q.bits, q.signed_i8 ? 1 : 0,
                                                     q.group_size, n, k)));
            const double err = std::fabs(double(got[i * N + n]) - double(want[i * N + n]));
            const double tol = 2e-6 * bound + 1e-7;
            worst = std::max(worst, err / tol);
            max_abs = std::max(max_abs, err);
        }
    char buf[128];
    std::snprintf(buf, sizeof buf, " (max-abs %.3e, worst err/tol %.3f)", max_abs, worst);
    expect(ok && worst <= 1.0, label + buf);
}

// sum_k |x_ik w_nk| per output [m, N]
std::vector<double> abs_bound(const g4a::QuantWeight& q, const std::vector<float>& x, size_t m) {
    const size_t N = q.shape[0], K = q.shape[1];
    std::vector<double> out(m * N, 0.0);
    for (size_t i = 0; i < m; ++i)
        for (size_t n = 0; n < N; ++n)
            for (size_t k = 0; k < K; ++k)
                out[i * N + n] += std::fabs(double(x[i * K + k])) *
                                  std::fabs(double(oracle_deq(q.qbytes.data(), q.scales.data(), K, q.bits,
                                                              q.signed_i8 ? 1 : 0, q.group_size, n, k)));
    return out;
}

// gelu(g) * u with g, u reordered sums: the bound of each carried through
// (|gelu'| < 1.13), plus 2e-6 relative for tanhf
void close_fused(const std::string& label, const std::vector<float>& got, const std::vector<float>& want,
                 const std::vector<float>& g, const std::vector<double>& bg, const std::vector<float>& u,
                 const std::vector<double>* bu) {
    double worst = 0.0, max_abs = 0.0;
    bool ok = got.size() == want.size();
    for (size_t i = 0; ok && i < want.size(); ++i) {
        double tol = 1.13 * (2e-6 * bg[i] + 1e-7) * std::fabs(double(u[i]));
        if (bu) tol += std::fabs(double(oracle_gelu_tanh(g[i]))) * (2e-6 * (*bu)[i] + 1e-7);
        tol += 2e-6 * std::fabs(double(want[i])) + 1e-7;
        const double err = std::fabs(double(got[i]) - double(want[i]));
        worst = std::max(worst, err / tol);
        max_abs = std::max(max_abs, err);
    }
    char buf[128];
    std::snprintf(buf, sizeof buf, " (max-abs %.3e, worst err/tol %.3f)", max_abs, worst);
    expect(ok && worst <= 1.0, label + buf);
}

std::vector<float> oracle_linear(const g4a::QuantWeight& q, const std::vector<float>& x, size_t m) {
    std::vector<float> y(m * q.shape[0]);
    oracle_linear_q(q.qbytes.data(), q.scales.data(), q.shape[0], q.shape[1], q.bits, q.signed_i8 ? 1 : 0,
                    q.group_size, x.data(), m, y.data());
    return y;
}

void quantized_kernel_parity(g4a::HipBackend& b) {
    std::printf("quantized_kernel_parity\n");
    Lcg r(9);
    auto scales = [&](size_t n) {
        std::vector<float> s(n);
        for (auto& v : s) v = 0.01f + r.next() * 0.05f;
        return s;
    };
    auto randu = [&](size_t n, uint32_t bits) {
        std::vector<uint32_t> v(n);
        for (auto& x : v) x = uint32_t(std::floor(r.next() * float(1u << bits))) % (1u << bits);
        return v;
    };
    for (uint32_t bits : {4u, 2u}) {
        const size_t n = 40, k = 64;
        g4a::QuantWeight q;
        q.qbytes = pack_unsigned(randu(n * k, bits), bits);
        q.scales = scales(n);
        q.shape[0] = n;
        q.shape[1] = k;
        q.bits = bits;
        q.group_size = k;
        const auto gw = b.quant_tensor(q);
        for (size_t m : {size_t(5), size_t(1)}) {
            const auto x = r.rand(m * k, 1.0f);
            close_linear("linear q" + std::to_string(bits) + " M=" + std::to_string(m),
                         b.readback(b.linear(b.tensor(x.data(), {m, k}), gw)), oracle_linear(q, x, m), q, x, m);
        }
    }
    {
        const uint32_t bits = 4;
        const size_t n = 21, k = 52, m = 3;
        g4a::QuantWeight q;
        q.qbytes = pack_unsigned(randu(n * k, bits), bits);
        q.scales = scales(n);
        q.shape[0] = n;
        q.shape[1] = k;
        q.bits = bits;
        q.group_size = k;
        const auto x = r.rand(m * k, 1.0f);
        const auto got = b.readback(b.linear(b.tensor(x.data(), {m, k}), b.quant_tensor(q)));
        expect(got == oracle_linear(q, x, m), "linear q4 oddK (element kernel, bit-exact)");
    }
    {
        const size_t n = 30, k = 48, m = 4;
        g4a::QuantWeight q;
        q.qbytes.resize(n * k);
        for (auto& v : q.qbytes) v = uint8_t(uint32_t(std::floor(r.next() * 256.0f)));
        q.scales.resize(n);
        for (auto& v : q.scales) v = 0.01f + r.next() * 0.03f;
        q.shape[0] = n;
        q.shape[1] = k;
        q.bits = 8;
        q.signed_i8 = true;
        q.group_size = k;
        const auto x = r.rand(m * k, 1.0f);
        close_linear("linear i8", b.readback(b.linear(b.tensor(x.data(), {m, k}), b.quant_tensor(q))),
                     oracle_linear(q, x, m), q, x, m);
    }
    {
        const size_t v = 50, d = 32, group = 16;
        const uint32_t bits = 4;
        g4a::QuantWeight q;
        q.qbytes = pack_unsigned(randu(v * d, bits), bits);
        q.scales.resize(v * (d / group));
        for (auto& s : q.scales) s = 0.02f + r.next() * 0.04f;
        q.shape[0] = v;
        q.shape[1] = d;
        q.bits = bits;
        q.group_size = group;
        const uint32_t ids[5] = {3, 7, 49, 0, 21};
        const float sc = std::sqrt(float(d));
        std::vector<float> want(5 * d);
        oracle_embed_rows_q(q.qbytes.data(), q.scales.data(), v, d, bits, 0, group, ids, 5, sc, want.data());
        expect(b.readback(b.embed_rows(b.quant_tensor(q), ids, 5, sc)) == want, "embed q4 grouped (bit-exact)");
    }
    // the fused projections (rust/src/backend.rs:156-168 compositions)
    {
        const size_t n = 96, k = 256, m = 3;
        const uint32_t bits = 4;
        g4a::QuantWeight qg, qu;
        for (auto* q : {&qg, &qu}) {
            q->qbytes = pack_unsigned(randu(n * k, bits), bits);
            q->scales = scales(n);
            q->shape[0] = n;
            q->shape[1] = k;
            q->bits = bits;
            q->group_size = k;
        }
        const auto x = r.rand(m * k, 1.0f);
        const auto g = oracle_linear(qg, x, m), u = oracle_linear(qu, x, m);
        std::vector<float> want(m * n);
        for (size_t i = 0; i < want.size(); ++i) want[i] = oracle_gelu_tanh(g[i]) * u[i];
        const auto gx = b.tensor(x.data(), {m, k});
        const auto bg = abs_bound(qg, x, m), bu = abs_bound(qu, x, m);
        close_fused("linear_geglu q4", b.readback(b.linear_geglu(gx, b.quant_tensor(qg), b.quant_tensor(qu))), want,
                    g, bg, u, &bu);
        const size_t stride = 5 * n, off = 2 * n;
        const auto bs = r.rand(m * stride, 1.0f);
        std::vector<float> cols(m * n);
        for (size_t i = 0; i < m; ++i)
            for (size_t j = 0; j < n; ++j) {
                cols[i * n + j] = bs[i * stride + off + j];
                want[i * n + j] = oracle_gelu_tanh(g[i * n + j]) * cols[i * n + j];
            }
        close_fused("linear_gelu_mul_cols q4",
                    b.readback(b.linear_gelu_mul_cols(gx, b.quant_tensor(qg), b.tensor(bs.data(), {m, stride}), off)),
                    want, g, bg, cols, nullptr);
    }
}

void kernel_parity_ops(g4a::HipBackend& b) {
    std::printf("kernel_parity_ops\n");
    Lcg r(7);
    {
        const size_t m = 17, k = 40, n = 23;
        const auto x = r.rand(m * k, 1.0f), w = r.rand(n * k, 1.0f);
        std::vector<float> want(m * n);
        oracle_linear_f32(w.data(), n, k, x.data(), m, want.data());
        const auto gw = b.tensor(w.data(), {n, k});
        close("linear (tiled)", b.readback(b.linear(b.tensor(x.data(), {m, k}), gw)), want);
        const auto x1 = r.rand(k, 1.0f);
        std::vector<float> want1(n);
        oracle_linear_f32(w.data(), n, k, x1.data(), 1, want1.data());
        close("linear (gemv)", b.readback(b.linear(b.tensor(x1.data(), {1, k}), gw)), want1);
    }
    r.rand(5 * 48 + 48, 1.0f);  // rmsNorm (norm_rope_parity covers it)
    {
        const size_t n = 100;
        const auto a = r.rand(n, 1.0f), c = r.rand(n, 1.0f);
        const auto ga = b.tensor(a.data(), {n}), gc = b.tensor(c.data(), {n});
        std::vector<float> want(n);
        for (size_t i = 0; i < n; ++i) want[i] = a[i] + c[i];
        expect(b.readback(b.add(ga, gc)) == want, "add (bit-exact)");
        for (size_t i = 0; i < n; ++i) want[i] = a[i] * c[i];
        expect(b.readback(b.mul(ga, gc)) == want, "mul (bit-exact)");
        for (size_t i = 0; i < n; ++i) want[i] = a[i] * 3.5f;
        expect(b.readback(b.scale(ga, 3.5f)) == want, "scale (bit-exact)");
        for (size_t i = 0; i < n; ++i) want[i] = oracle_gelu_tanh(a[i]);
        close("geluTanh", b.readback(b.gelu_tanh(ga)), want);
        for (size_t i = 0; i < n; ++i) want[i] = oracle_gelu_tanh(a[i]) * c[i];
        close("geglu", b.readback(b.geglu(ga, gc)), want);
        std::vector<float> a50(n);
        for (size_t i = 0; i < n; ++i) a50[i] = a[i] * 50.0f;
        oracle_softcap_n(a50.data(), 30.0f, want.data(), n);
        close("softcap", b.readback(b.softcap(b.scale(ga, 50.0f), 30.0f)), want);
        const float s = 0.37f;
        for (size_t i = 0; i < n; ++i) want[i] = a[i] * s;
        expect(b.readback(b.scale_by_tensor(ga, b.tensor(&s, {1}))) == want, "scaleByTensor (bit-exact)");
        const float big[3] = {1000.0f, -1000.0f, 50.0f};
        const auto gv = b.readback(b.gelu_tanh(b.tensor(big, {3})));
        expect(std::isfinite(gv[0]) && std::isfinite(gv[1]) && std::isfinite(gv[2]), "gelu finite on large inputs");
        const auto z = b.readback(b.zeros({37}));
        bool zero = true;
        for (float v : z) zero &= v == 0.0f;
        expect(zero, "zeros");
    }
    {
        const size_t v = 30, d = 16;
        const auto table = r.rand(v * d, 1.0f);
        const uint32_t ids[5] = {3, 7, 0, 29, 12};
        std::vector<float> want(5 * d);
        oracle_embed_rows_f32(table.data(), d, ids, 5, 4.0f, want.data());
        expect(b.readback(b.embed_rows(b.tensor(table.data(), {v, d}), ids, 5, 4.0f)) == want, "embedRows (bit-exact)");
    }
    r.rand(4 * 2 * 16, 1.0f);  // rope(partial)
    {
        const size_t rows = 4, stride = 20;
        const auto x = r.rand(rows * stride, 1.0f);
        std::vector<float> want;
        for (size_t i = 0; i < rows; ++i) want.insert(want.end(), x.begin() + i * stride + 5, x.begin() + i * stride + 12);
        expect(b.readback(b.slice_cols(b.tensor(x.data(), {rows, stride}), 5, 7)) == want, "sliceCols (bit-exact)");
    }
    {
        Lcg q(33);
        const size_t t = 5, d = 48;
        const auto x = q.rand(t * d, 1.0f), res = q.rand(t * d, 1.0f), w = q.rand(d, 0.1f);
        const float s = 1.37f;
        std::vector<float> normed(t * d), want(t * d);
        oracle_rms_norm(x.data(), w.data(), normed.data(), t, d, 1e-6f);
        for (size_t i = 0; i < t * d; ++i) want[i] = res[i] + normed[i];
        const auto gx = b.tensor(x.data(), {t, d}), gr = b.tensor(res.data(), {t, d}), gw = b.tensor(w.data(), {d});
        close("add_rms_norm", b.readback(b.add_rms_norm(gr, gx, gw, 1e-6f, nullptr)), want);
        for (auto& v : want) v = v * s;
        const auto gs = b.tensor(&s, {1});
        close("add_rms_norm (layer_scalar)", b.readback(b.add_rms_norm(gr, gx, gw, 1e-6f, &gs)), want);
    }
}

}  // namespace

int main() {
    std::unique_ptr<g4a::HipBackend> b;
    try {
        b = g4a::HipBackend::create(0);
    } catch (const std::exception& e) {
        std::fprintf(stderr, "test_backend: %s\n", e.what());
        return 2;
    }
    try {
        grouped_attention_parity(*b);
        copies_and_kv_append(*b);
        norm_rope_parity(*b);
        quantized_kernel_parity(*b);
        kernel_parity_ops(*b);
        kv_cache_decode(*b);
    } catch (const std::exception& e) {
        std::fprintf(stderr, "test_backend: exception: %s\n", e.what());
        return 1;
    }
    std::printf("%s: %d failure(s)\n", g_failures ? "FAILED" : "PASSED", g_failures);
    return g_failures ? 1 : 0;
}
