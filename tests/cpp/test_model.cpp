// Whole-model parity on the reference's tiny config: Gemma4Model::forward
// (rust/src/model.rs:142-313) composed over two backends,
//   - the C++ HipBackend (gemma-4-webgpu-kernels_amd/csrc/hip_backend.hpp), the
//     op surface a Rust HipBackend calls, with its KvCache (a ring for sliding
//     layers, the reference's growing kv_append buffer for global ones), and
//   - a CPU backend made of the oracle's restatements of CpuBackend's ops
//     (oracle/attn_oracle.c, oracle/linear_oracle.c) and the trait's default
//     compositions (rust/src/backend.rs:130-168),
// as the reference's own tests run it (rust/tests/gpu.rs:190-227 full_model_parity,
// rust/tests/model.rs:38-51 incremental_decode_matches_full_sequence):
//   tiny config (rust/tests/common/mod.rs:44-56): 6 layers [S,F,S,S,S,S], the last 2
//   reading layer 3's KV (rust/src/config.rs:152-159), hidden 32, 4 query heads over 1 kv
//   head, head_dim 8 / global 16 (partial rotary 0.25), window 3, per-layer inputs 12;
//   f32 weights from SyntheticWeights (Mulberry seed 123, drawn in the model's request
//   order, rust/tests/common/mod.rs:15-27, :95-127).
// Checks (bar: the reference's 5e-3 max |d| on logits, rust/tests/gpu.rs:200, :213; the
// achieved difference is printed):
//   1. a 5-token prefill, GPU against CPU;
//   2. five single-token decode steps, GPU against CPU, and against the prefill
//      (incremental == full sequence, rust/tests/model.rs:38-51, bar 1e-3);
//   3. 300 decode steps (the global layer's kv_append buffer grows past its first
//      256-row capacity; the cache holds 300 positions), GPU against CPU at every 25th
//      step and the last, all logits finite.
// With --cpu-only (no GPU), the reference's CPU model tests on the oracle composition:
// incremental == full sequence, a 20-token sliding sequence stays finite, and a reset
// cache reproduces the same logits (rust/tests/model.rs:24-90).
// Exit status 0 = all passed.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "hip_backend.hpp"

extern "C" int oracle_attention(const float* q, const float* k, const float* v, float* out, size_t T, size_t S,
                                size_t Hq, size_t Hkv, size_t Dh, size_t Dv, const uint32_t* q_pos,
                                const uint32_t* k_pos, float scale, uint32_t window, float softcap,
                                int requested_threads);
extern "C" void oracle_rms_norm(const float* x, const float* w, float* y, size_t rows, size_t d, float eps);
extern "C" void oracle_rope(const float* x, float* y, size_t T, size_t heads, size_t head_dim, size_t rotary_dim,
                            const uint32_t* positions, float theta);
extern "C" void oracle_linear_f32(const float* w, size_t N, size_t K, const float* x, size_t M, float* y);
extern "C" void oracle_gelu_tanh_n(const float* x, float* y, size_t n);
extern "C" void oracle_embed_rows_f32(const float* table, size_t D, const uint32_t* ids, size_t T, float scale,
                                      float* out);

namespace {

int g_failures = 0;

void expect(bool ok, const std::string& label) {
    std::printf("  %s %s\n", ok ? "ok  " : "FAIL", label.c_str());
    std::fflush(stdout);
    if (!ok) ++g_failures;
}

// rust/tests/common/mod.rs:15-27 (mulberry32)
struct Mulberry {
    uint32_t s;
    explicit Mulberry(uint32_t seed) : s(seed) {}
    double next() {
        s += 0x6d2b79f5u;
        uint32_t t = s;
        t = (t ^ (t >> 15)) * (1u | t);
        t = (t + (t ^ (t >> 7)) * (61u | t)) ^ t;
        return double(t ^ (t >> 14)) / 4294967296.0;
    }
};

// rust/tests/common/mod.rs:44-56 parsed as rust/src/config.rs does
struct Config {
    size_t vocab = 48, hidden = 32, inter = 64, layers = 6, hq = 4, hkv = 1, head_dim = 8, global_head_dim = 16,
           dple = 12, kv_shared = 2;
    uint32_t window = 3;
    float eps = 1e-6f;
    std::vector<bool> global = {false, true, false, false, false, false};
    bool is_global(size_t i) const { return global[i]; }
    size_t dh(size_t i) const { return is_global(i) ? global_head_dim : head_dim; }
    // rust/src/config.rs:152-159
    size_t kv_source_layer(size_t i) const {
        const size_t first_shared = layers > kv_shared ? layers - kv_shared : 0;
        if (i < first_shared) return i;
        for (size_t j = first_shared; j-- > 0;)
            if (global[j] == global[i]) return j;
        return i;
    }
    float theta(size_t i) const { return is_global(i) ? 1e6f : 1e4f; }
    // rust/src/model.rs:257: (dh as f32 * partial_rotary_factor).round()
    size_t rotary_dim(size_t i) const { return size_t(std::lround(float(dh(i)) * (is_global(i) ? 0.25f : 1.0f))); }
};

// rust/tests/common/mod.rs:59-92
std::vector<size_t> shape_of(const std::string& name, const Config& c, size_t layer) {
    const size_t h = c.hidden, i_ = c.inter, v = c.vocab, p = c.dple, l = c.layers, hq = c.hq, hkv = c.hkv;
    if (name == "language_model.embed_tokens.weight") return {v, h};
    if (name == "language_model.embed_tokens_per_layer.weight") return {v, l * p};
    if (name == "language_model.per_layer_model_projection.weight") return {l * p, h};
    if (name == "language_model.per_layer_projection_norm.weight") return {p};
    if (name == "language_model.norm.weight") return {h};
    if (name == "lm_head.weight") return {v, h};
    const size_t dh = c.dh(layer);
    const std::string sub = name.substr(name.find('.', std::string("language_model.layers.").size()) + 1);
    if (sub == "input_layernorm.weight" || sub == "post_attention_layernorm.weight" ||
        sub == "pre_feedforward_layernorm.weight" || sub == "post_feedforward_layernorm.weight" ||
        sub == "post_per_layer_input_norm.weight")
        return {h};
    if (sub == "self_attn.q_proj.weight") return {hq * dh, h};
    if (sub == "self_attn.k_proj.weight" || sub == "self_attn.v_proj.weight") return {hkv * dh, h};
    if (sub == "self_attn.o_proj.weight") return {h, hq * dh};
    if (sub == "self_attn.q_norm.weight" || sub == "self_attn.k_norm.weight") return {dh};
    if (sub == "mlp.gate_proj.weight" || sub == "mlp.up_proj.weight") return {i_, h};
    if (sub == "mlp.down_proj.weight") return {h, i_};
    if (sub == "per_layer_input_gate.weight") return {p, h};
    if (sub == "per_layer_projection.weight") return {h, p};
    if (sub == "layer_scalar") return {1};
    std::fprintf(stderr, "unknown weight %s\n", name.c_str());
    std::exit(2);
}

struct HostWeight {
    std::vector<float> data;
    std::vector<size_t> shape;
};

bool ends_with(const std::string& s, const char* suf) {
    const size_t n = std::strlen(suf);
    return s.size() >= n && s.compare(s.size() - n, n, suf) == 0;
}

// SyntheticWeights (rust/tests/common/mod.rs:95-127) drawn in the order Gemma4Model
// requests them: resolve_top (rust/src/model.rs:91-105), then resolve_layer(i) for
// every layer in LayerWeights' field order (:107-132; a shared layer has no k/v weights)
std::map<std::string, HostWeight> synthetic_weights(const Config& c, uint32_t seed) {
    Mulberry rng(seed);
    std::map<std::string, HostWeight> w;
    auto draw = [&](const std::string& name, size_t layer) {
        const auto shape = shape_of(name, c, layer);
        size_t n = 1;
        for (size_t d : shape) n *= d;
        const bool is_norm = ends_with(name, "norm.weight") || ends_with(name, "layernorm.weight");
        const bool is_scalar = ends_with(name, "layer_scalar");
        const double base = (is_norm || is_scalar) ? 1.0 : 0.0, scale = (is_norm || is_scalar) ? 0.05 : 0.04;
        HostWeight hw{std::vector<float>(n), shape};
        for (auto& x : hw.data) x = float(base + (rng.next() * 2.0 - 1.0) * scale);
        w[name] = std::move(hw);
    };
    for (const char* n : {"language_model.embed_tokens.weight", "language_model.embed_tokens_per_layer.weight",
                          "language_model.per_layer_model_projection.weight",
                          "language_model.per_layer_projection_norm.weight", "language_model.norm.weight",
                          "lm_head.weight"})
        draw(n, 0);
    for (size_t i = 0; i < c.layers; ++i) {
        const std::string p = "language_model.layers." + std::to_string(i) + ".";
        const bool owns_kv = c.kv_source_layer(i) == i;
        draw(p + "input_layernorm.weight", i);
        draw(p + "self_attn.q_proj.weight", i);
        draw(p + "self_attn.q_norm.weight", i);
        if (owns_kv) {
            draw(p + "self_attn.k_proj.weight", i);
            draw(p + "self_attn.v_proj.weight", i);
            draw(p + "self_attn.k_norm.weight", i);
        }
        for (const char* s : {"self_attn.o_proj.weight", "post_attention_layernorm.weight",
                              "pre_feedforward_layernorm.weight", "mlp.gate_proj.weight", "mlp.up_proj.weight",
                              "mlp.down_proj.weight", "post_feedforward_layernorm.weight",
                              "per_layer_input_gate.weight", "per_layer_projection.weight",
                              "post_per_layer_input_norm.weight", "layer_scalar"})
            draw(p + s, i);
    }
    return w;
}

// ---- the CPU backend: CpuBackend's ops through the oracle (rust/src/backend_cpu.rs) ----

struct CpuT {
    std::vector<float> d;
    std::vector<size_t> shape;
    size_t rows() const { return shape[0]; }
    size_t cols() const { return d.size() / (shape.empty() ? 1 : shape[0]); }
};

struct CpuBackend {
    using Tensor = CpuT;
    Tensor tensor(const std::vector<float>& d, std::vector<size_t> shape) { return {d, std::move(shape)}; }
    Tensor reshape(const Tensor& x, std::vector<size_t> shape) { return {x.d, std::move(shape)}; }
    Tensor embed_rows(const Tensor& table, const uint32_t* ids, size_t n, float scale) {
        const size_t D = table.shape[1];
        Tensor y{std::vector<float>(n * D), {n, D}};
        oracle_embed_rows_f32(table.d.data(), D, ids, n, scale, y.d.data());
        return y;
    }
    Tensor linear(const Tensor& x, const Tensor& w) {
        const size_t N = w.shape[0], K = w.shape[1], M = x.d.size() / K;
        Tensor y{std::vector<float>(M * N), {M, N}};
        oracle_linear_f32(w.d.data(), N, K, x.d.data(), M, y.d.data());
        return y;
    }
    Tensor rms_norm(const Tensor& x, const Tensor* w, float eps) {
        const size_t d = x.shape.back(), rows = x.d.size() / d;
        Tensor y{std::vector<float>(x.d.size()), x.shape};
        oracle_rms_norm(x.d.data(), w ? w->d.data() : nullptr, y.d.data(), rows, d, eps);
        return y;
    }
    // rust/src/backend_cpu.rs:224-241
    Tensor add(const Tensor& a, const Tensor& b) {
        Tensor y = a;
        for (size_t i = 0; i < y.d.size(); ++i) y.d[i] = a.d[i] + b.d[i];
        return y;
    }
    Tensor mul(const Tensor& a, const Tensor& b) {
        Tensor y = a;
        for (size_t i = 0; i < y.d.size(); ++i) y.d[i] = a.d[i] * b.d[i];
        return y;
    }
    Tensor scale(const Tensor& a, float s) {
        Tensor y = a;
        for (auto& v : y.d) v = v * s;
        return y;
    }
    Tensor scale_by_tensor(const Tensor& a, const Tensor& s) { return scale(a, s.d[0]); }
    Tensor gelu_tanh(const Tensor& a) {
        Tensor y = a;
        oracle_gelu_tanh_n(a.d.data(), y.d.data(), a.d.size());
        return y;
    }
    Tensor geglu(const Tensor& g, const Tensor& u) { return mul(gelu_tanh(g), u); }
    Tensor slice_cols(const Tensor& x, size_t offset, size_t width) {
        const size_t rows = x.shape[0], stride = x.shape[1];
        Tensor y{std::vector<float>(rows * width), {rows, width}};
        for (size_t r = 0; r < rows; ++r)
            std::copy_n(x.d.begin() + r * stride + offset, width, y.d.begin() + r * width);
        return y;
    }
    Tensor slice_rows(const Tensor& x, size_t start, size_t count) {
        const size_t dim = x.shape[1];
        return {std::vector<float>(x.d.begin() + start * dim, x.d.begin() + (start + count) * dim), {count, dim}};
    }
    // rust/src/backend.rs:136-168: the trait's default compositions
    Tensor add_rms_norm(const Tensor& res, const Tensor& x, const Tensor& w, float eps, const Tensor* scale_by) {
        Tensor h = add(res, rms_norm(x, &w, eps));
        return scale_by ? scale_by_tensor(h, *scale_by) : h;
    }
    Tensor linear_geglu(const Tensor& x, const Tensor& wg, const Tensor& wu) { return geglu(linear(x, wg), linear(x, wu)); }
    Tensor linear_gelu_mul_cols(const Tensor& x, const Tensor& w, const Tensor& b, size_t offset) {
        return geglu(linear(x, w), slice_cols(b, offset, w.shape[0]));
    }
    Tensor rope(const Tensor& x, const uint32_t* pos, float theta, size_t head_dim, size_t heads, size_t rot) {
        Tensor y{std::vector<float>(x.d.size()), x.shape};
        oracle_rope(x.d.data(), y.d.data(), x.shape[0], heads, head_dim, rot, pos, theta);
        return y;
    }
    Tensor head_norm_rope(const Tensor& x, const Tensor& w, float eps, const uint32_t* pos, size_t n_pos, float theta,
                          size_t head_dim, size_t heads, size_t rot) {
        (void)n_pos;
        const size_t t = x.shape[0];
        Tensor n = reshape(rms_norm(reshape(x, {t * heads, head_dim}), &w, eps), {t, heads, head_dim});
        return rope(n, pos, theta, head_dim, heads, rot);
    }
    Tensor attention(const Tensor& q, const Tensor& k, const Tensor& v, const g4a::AttnOpts& o) {
        const size_t T = q.shape[0], Hq = q.shape[1], Dh = q.shape[2], S = k.shape[0], Hkv = k.shape[1];
        const size_t Dv = v.shape[2];
        Tensor y{std::vector<float>(T * Hq * Dv), {T, Hq * Dv}};
        oracle_attention(q.d.data(), k.d.data(), v.d.data(), y.d.data(), T, S, Hq, Hkv, Dh, Dv, o.q_pos, o.k_pos,
                         o.scale, o.sliding_window, o.attn_softcap, 0);
        return y;
    }
    std::vector<float> readback(const Tensor& t) { return t.d; }

    // KVCache (rust/src/kvcache.rs) over CpuBackend::kv_append = concat_rows (:352-364)
    struct Cache {
        std::vector<uint32_t> positions;
        std::vector<std::pair<Tensor, Tensor>> slots;
        std::vector<bool> has;
        explicit Cache(size_t layers) : slots(layers), has(layers, false) {}
        void push_positions(const uint32_t* p, size_t n) { positions.insert(positions.end(), p, p + n); }
        std::pair<Tensor, Tensor> append_and_read(CpuBackend&, size_t src, const Tensor& k, const Tensor& v, uint32_t) {
            if (!has[src]) {
                slots[src] = {k, v};
                has[src] = true;
            } else {
                for (int which = 0; which < 2; ++which) {
                    Tensor& old = which ? slots[src].second : slots[src].first;
                    const Tensor& add = which ? v : k;
                    old.d.insert(old.d.end(), add.d.begin(), add.d.end());
                    old.shape[0] += add.shape[0];
                }
            }
            return slots[src];
        }
        const std::pair<Tensor, Tensor>& read(size_t src) const { return slots[src]; }
        void end_frame(CpuBackend&) {}
        void reset() {
            positions.clear();
            std::fill(has.begin(), has.end(), false);
            slots.assign(slots.size(), {});
        }
    };
};

// ---- the GPU backend: the C++ HipBackend mirror ----

struct HipBackendAdapter {
    using Tensor = g4a::HipTensor;
    g4a::HipBackend& b;
    Tensor tensor(const std::vector<float>& d, std::vector<size_t> shape) { return b.tensor(d.data(), std::move(shape)); }
    Tensor reshape(const Tensor& x, std::vector<size_t> shape) { return b.reshape(x, std::move(shape)); }
    Tensor embed_rows(const Tensor& table, const uint32_t* ids, size_t n, float scale) {
        return b.embed_rows(table, ids, n, scale);
    }
    Tensor linear(const Tensor& x, const Tensor& w) { return b.linear(x, w); }
    Tensor rms_norm(const Tensor& x, const Tensor* w, float eps) { return b.rms_norm(x, w, eps); }
    Tensor add(const Tensor& a, const Tensor& c) { return b.add(a, c); }
    Tensor scale(const Tensor& a, float s) { return b.scale(a, s); }
    Tensor scale_by_tensor(const Tensor& a, const Tensor& s) { return b.scale_by_tensor(a, s); }
    Tensor slice_rows(const Tensor& x, size_t start, size_t count) { return b.slice_rows(x, start, count); }
    Tensor add_rms_norm(const Tensor& res, const Tensor& x, const Tensor& w, float eps, const Tensor* s) {
        return b.add_rms_norm(res, x, w, eps, s);
    }
    Tensor linear_geglu(const Tensor& x, const Tensor& wg, const Tensor& wu) { return b.linear_geglu(x, wg, wu); }
    Tensor linear_gelu_mul_cols(const Tensor& x, const Tensor& w, const Tensor& c, size_t off) {
        return b.linear_gelu_mul_cols(x, w, c, off);
    }
    Tensor rope(const Tensor& x, const uint32_t* pos, float theta, size_t head_dim, size_t heads, size_t rot) {
        return b.rope(x, pos, x.shape[0], theta, head_dim, heads, rot);
    }
    Tensor head_norm_rope(const Tensor& x, const Tensor& w, float eps, const uint32_t* pos, size_t n_pos, float theta,
                          size_t head_dim, size_t heads, size_t rot) {
        return b.head_norm_rope(x, w, eps, pos, n_pos, theta, head_dim, heads, rot);
    }
    Tensor attention(const Tensor& q, const Tensor& k, const Tensor& v, const g4a::AttnOpts& o) {
        return b.attention(q, k, v, o);
    }
    std::vector<float> readback(const Tensor& t) { return b.readback(t); }

    struct Cache {
        g4a::KvCache kv;
        explicit Cache(size_t layers) : kv(layers) {}
        std::vector<uint32_t>& positions_ref() { return kv.positions; }
        void push_positions(const uint32_t* p, size_t n) { kv.push_positions(p, n); }
        std::pair<Tensor, Tensor> append_and_read(HipBackendAdapter& a, size_t src, const Tensor& k, const Tensor& v,
                                                  uint32_t window) {
            return kv.append_and_read(a.b, src, k, v, window);
        }
        const std::pair<Tensor, Tensor>& read(size_t src) const { return *kv.read(src); }
        // rust/src/model.rs:196-201: after the readback, free what growth superseded
        void end_frame(HipBackendAdapter& a) { a.b.end_frame({}, kv.take_dead()); }
        void reset_with(HipBackendAdapter& a) { kv.reset(a.b); }
    };
};

template <class C>
const std::vector<uint32_t>& cache_positions(const C& c) {
    return c.positions;
}
template <>
const std::vector<uint32_t>& cache_positions(const HipBackendAdapter::Cache& c) {
    return c.kv.positions;
}

// Gemma4Model (rust/src/model.rs:62-313) over backend B.
template <class B>
struct Model {
    using T = typename B::Tensor;
    B& b;
    const Config& c;
    std::map<std::string, T> w;
    typename B::Cache cache;

    Model(B& backend, const Config& cfg, const std::map<std::string, HostWeight>& hw)
        : b(backend), c(cfg), cache(cfg.layers) {
        for (const auto& [name, x] : hw) w.emplace(name, b.tensor(x.data, x.shape));  // Mirrored (common/mod.rs:130-156)
    }
    const T& W(const std::string& name) const { return w.at(name); }
    const T& L(size_t i, const char* sub) const { return w.at("language_model.layers." + std::to_string(i) + "." + sub); }

    // rust/src/model.rs:142-205
    std::vector<float> forward(const std::vector<uint32_t>& ids, const std::vector<uint32_t>& positions) {
        const size_t t = ids.size(), dple = c.dple, l = c.layers;
        T h = b.embed_rows(W("language_model.embed_tokens.weight"), ids.data(), t, std::sqrt(float(c.hidden)));
        T emb = b.embed_rows(W("language_model.embed_tokens_per_layer.weight"), ids.data(), t, std::sqrt(float(dple)));
        T proj = b.linear(h, W("language_model.per_layer_model_projection.weight"));
        proj = b.reshape(proj, {t * l, dple});
        proj = b.rms_norm(proj, &W("language_model.per_layer_projection_norm.weight"), c.eps);
        proj = b.reshape(proj, {t, l * dple});
        const T ple = b.scale(b.add(proj, emb), float(M_SQRT1_2));
        cache.push_positions(positions.data(), positions.size());
        for (size_t i = 0; i < l; ++i) h = decoder_layer(i, h, positions, ple);
        h = b.rms_norm(h, &W("language_model.norm.weight"), c.eps);
        T last = b.slice_rows(h, t - 1, 1);
        T logits = b.linear(last, W("lm_head.weight"));
        auto out = b.readback(logits);
        cache.end_frame(b);
        return out;
    }

    // rust/src/model.rs:207-245
    T decoder_layer(size_t i, const T& residual, const std::vector<uint32_t>& positions, const T& ple) {
        T attn = attention(i, b.rms_norm(residual, &L(i, "input_layernorm.weight"), c.eps), positions);
        T h = b.add_rms_norm(residual, attn, L(i, "post_attention_layernorm.weight"), c.eps, nullptr);
        T x = b.rms_norm(h, &L(i, "pre_feedforward_layernorm.weight"), c.eps);
        T ff = b.linear_geglu(x, L(i, "mlp.gate_proj.weight"), L(i, "mlp.up_proj.weight"));
        ff = b.linear(ff, L(i, "mlp.down_proj.weight"));
        h = b.add_rms_norm(h, ff, L(i, "post_feedforward_layernorm.weight"), c.eps, nullptr);
        T inj = b.linear_gelu_mul_cols(h, L(i, "per_layer_input_gate.weight"), ple, i * c.dple);
        inj = b.linear(inj, L(i, "per_layer_projection.weight"));
        return b.add_rms_norm(h, inj, L(i, "post_per_layer_input_norm.weight"), c.eps, &L(i, "layer_scalar"));
    }

    // rust/src/model.rs:247-304
    T attention(size_t i, const T& x, const std::vector<uint32_t>& positions) {
        const size_t hq = c.hq, hkv = c.hkv, dh = c.dh(i), t = x.shape[0], rot = c.rotary_dim(i);
        const float theta = c.theta(i);
        T q = b.reshape(b.linear(x, L(i, "self_attn.q_proj.weight")), {t, hq, dh});
        q = b.head_norm_rope(q, L(i, "self_attn.q_norm.weight"), c.eps, positions.data(), positions.size(), theta, dh,
                             hq, rot);
        const size_t src = c.kv_source_layer(i);
        const uint32_t window = c.is_global(i) ? 0u : c.window;
        std::pair<T, T> kv;
        if (src == i) {
            T k = b.reshape(b.linear(x, L(i, "self_attn.k_proj.weight")), {t, hkv, dh});
            T v = b.reshape(b.linear(x, L(i, "self_attn.v_proj.weight")), {t, hkv, dh});
            k = b.head_norm_rope(k, L(i, "self_attn.k_norm.weight"), c.eps, positions.data(), positions.size(), theta,
                                 dh, hkv, rot);
            v = b.reshape(b.rms_norm(b.reshape(v, {t * hkv, dh}), nullptr, c.eps), {t, hkv, dh});  // head_norm
            kv = cache.append_and_read(b, src, k, v, window);
        } else {
            kv = cache.read(src);
        }
        const auto& kpos = cache_positions(cache);
        g4a::AttnOpts o;
        o.q_pos = positions.data();
        o.n_q_pos = positions.size();
        o.k_pos = kpos.data();
        o.n_k_pos = kpos.size();
        o.scale = 1.0f;
        o.sliding_window = window;
        o.attn_softcap = 0.0f;
        T out = b.attention(q, kv.first, kv.second, o);
        return b.linear(out, L(i, "self_attn.o_proj.weight"));
    }
};

float max_abs_diff(const std::vector<float>& a, const std::vector<float>& b) {
    float d = 0.0f;
    for (size_t i = 0; i < a.size(); ++i) d = std::max(d, std::fabs(a[i] - b[i]));
    return a.size() == b.size() ? d : INFINITY;
}

bool all_finite(const std::vector<float>& a) {
    return std::all_of(a.begin(), a.end(), [](float x) { return std::isfinite(x); });
}

void report(const char* what, float d, float bar) {
    char label[200];
    std::snprintf(label, sizeof label, "%s: max |d| %.3e (bar %.0e)", what, d, bar);
    expect(d < bar, label);
}

const std::vector<uint32_t> IDS = {2, 5, 11, 19, 30};

std::vector<uint32_t> iota(uint32_t a, uint32_t n) {
    std::vector<uint32_t> v(n);
    for (uint32_t i = 0; i < n; ++i) v[i] = a + i;
    return v;
}

// rust/tests/model.rs:24-90 on the oracle composition
void cpu_model_tests(const Config& cfg) {
    std::printf("[model] CPU (oracle) composition, tiny config, SyntheticWeights seed 42\n");
    const auto hw = synthetic_weights(cfg, 42);
    CpuBackend cb;
    Model<CpuBackend> full(cb, cfg, hw), inc(cb, cfg, hw);
    const auto lf = full.forward(IDS, iota(0, 5));
    expect(lf.size() == cfg.vocab && all_finite(lf), "forward: vocab-length finite logits");
    std::vector<float> li;
    for (uint32_t i = 0; i < IDS.size(); ++i) li = inc.forward({IDS[i]}, {i});
    report("incremental decode matches the full sequence", max_abs_diff(lf, li), 1e-3f);
    Model<CpuBackend> longm(cb, cfg, hw);
    std::vector<uint32_t> ids20;
    for (uint32_t i = 0; i < 20; ++i) ids20.push_back((i * 7) % 48);
    expect(all_finite(longm.forward(ids20, iota(0, 20))), "20-token sliding-window sequence stays finite");
    Model<CpuBackend> rm(cb, cfg, hw);
    const auto a = rm.forward(IDS, iota(0, 5));
    rm.cache.reset();
    const auto a2 = rm.forward(IDS, iota(0, 5));
    expect(a == a2, "a reset cache reproduces the logits exactly");
}

// rust/tests/gpu.rs:190-227 (and more: the long decode compared step by step)
void gpu_model_tests(const Config& cfg) {
    std::printf("[model] HipBackend against the oracle composition, tiny config, SyntheticWeights seed 123\n");
    auto backend = g4a::HipBackend::create(0);
    HipBackendAdapter gb{*backend};
    CpuBackend cb;
    const auto hw = synthetic_weights(cfg, 123);
    {
        Model<CpuBackend> cm(cb, cfg, hw);
        Model<HipBackendAdapter> gm(gb, cfg, hw);
        report("full prefill forward parity (5 tokens)", max_abs_diff(cm.forward(IDS, iota(0, 5)),
                                                                      gm.forward(IDS, iota(0, 5))), 5e-3f);
    }
    std::vector<float> lfull;
    {
        Model<HipBackendAdapter> gm(gb, cfg, hw);
        lfull = gm.forward(IDS, iota(0, 5));
    }
    {
        Model<CpuBackend> ic(cb, cfg, hw);
        Model<HipBackendAdapter> ig(gb, cfg, hw);
        std::vector<float> lc, lg;
        for (uint32_t i = 0; i < IDS.size(); ++i) {
            lc = ic.forward({IDS[i]}, {i});
            lg = ig.forward({IDS[i]}, {i});
        }
        report("incremental decode parity (5 single-token steps)", max_abs_diff(lc, lg), 5e-3f);
        report("GPU incremental decode matches the GPU full sequence", max_abs_diff(lfull, lg), 1e-3f);
    }
    {
        Model<CpuBackend> lc(cb, cfg, hw);
        Model<HipBackendAdapter> lg(gb, cfg, hw);
        float worst = 0.0f;
        bool finite = true;
        size_t cap_seen = 0;
        for (uint32_t i = 0; i < 300; ++i) {
            const uint32_t id = (i * 7) % 48;
            const auto g = lg.forward({id}, {i});
            finite &= all_finite(g);
            if (i % 25 == 0 || i == 299) {
                const auto want = lc.forward({id}, {i});
                worst = std::max(worst, max_abs_diff(want, g));
            } else {
                lc.forward({id}, {i});
            }
            const auto* gl = lg.cache.kv.read(1);  // the global layer's growing buffer
            if (gl && gl->first.cap_rows != cap_seen) {
                std::printf("  global layer K capacity %zu rows at %u cached positions\n", gl->first.cap_rows, i + 1);
                cap_seen = gl->first.cap_rows;
            }
        }
        expect(finite, "300-step decode with KV growth stays finite");
        expect(lg.cache.kv.positions.size() == 300, "the cache holds 300 positions");
        expect(cap_seen > 256, "the global layer's kv_append buffer grew past its first 256-row capacity");
        report("300-step decode parity (every 25th step and the last)", worst, 5e-3f);
    }
}

}  // namespace

int main(int argc, char** argv) {
    const bool cpu_only = argc > 1 && std::strcmp(argv[1], "--cpu-only") == 0;
    const Config cfg;
    try {
        cpu_model_tests(cfg);
        if (!cpu_only) gpu_model_tests(cfg);
    } catch (const std::exception& e) {
        std::printf("  FAIL exception: %s\n", e.what());
        ++g_failures;
    }
    std::printf("%s: %d failure(s)\n", g_failures ? "FAILED" : "PASSED", g_failures);
    return g_failures ? 1 : 0;
}
