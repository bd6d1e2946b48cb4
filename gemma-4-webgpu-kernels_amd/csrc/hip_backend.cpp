// HipBackend: the attention-path subset of the reference's Backend trait over
// libg4a.so's C-ABI. Declarations and conventions are in hip_backend.hpp.
#include "hip_backend.hpp"

#include <algorithm>
#include <cstring>

namespace g4a {

namespace {

// Recycled buffers kept per backend (the reference keeps 128 MiB,
// rust/src/backend_wgpu.rs:191; a 288 GB device affords more).
constexpr size_t kPoolMaxBytes = size_t(2) << 30;
constexpr size_t kKvMinRows = 256;  // first KV allocation (rust/src/backend_wgpu.rs:1024)

size_t product(const std::vector<size_t>& s) {
    size_t n = 1;
    for (size_t d : s) n *= d;
    return n;
}

// pow2 bucket of at least 256 bytes (rust/src/backend_wgpu.rs:384-389)
size_t bucket(size_t bytes) {
    size_t size = 256;
    while (size < std::max<size_t>(bytes, 16)) size <<= 1;
    return size;
}

std::string shape_str(const std::vector<size_t>& s) {
    std::string r = "[";
    for (size_t i = 0; i < s.size(); ++i) r += (i ? ", " : "") + std::to_string(s[i]);
    return r + "]";
}

[[noreturn]] void bad(const std::string& msg) { throw std::runtime_error("hip backend: " + msg); }

}  // namespace

DeviceBuffer::~DeviceBuffer() {
    if (owner_) owner_->release(ptr_, bytes_);
}

std::unique_ptr<HipBackend> HipBackend::create(int device) {
    g4a_ctx* ctx = nullptr;
    if (int rc = g4a_create(device, nullptr, &ctx))
        bad("g4a_create failed (" + std::to_string(rc) + "): " + g4a_last_error(nullptr));
    return std::unique_ptr<HipBackend>(new HipBackend(ctx));
}

HipBackend::~HipBackend() {
    if (!ctx_) return;
    g4a_sync(ctx_);
    for (auto& [size, p] : pool_) g4a_free(ctx_, p);
    pool_.clear();
    g4a_destroy(ctx_);
}

void HipBackend::check(int rc, const char* what) const {
    if (rc != G4A_OK) bad(std::string(what) + " failed (" + std::to_string(rc) + "): " + g4a_last_error(ctx_));
}

std::shared_ptr<DeviceBuffer> HipBackend::alloc(size_t bytes) {
    size_t size = bucket(bytes);
    void* p = nullptr;
    auto it = pool_.find(size);
    if (it != pool_.end()) {
        p = it->second;
        pool_.erase(it);
        pooled_bytes_ -= size;
    } else {
        check(g4a_malloc(ctx_, size, &p), "g4a_malloc");
    }
    return std::make_shared<DeviceBuffer>(this, p, size);
}

// Stream order makes reuse safe: an op that later receives this buffer is
// enqueued after every op that used it (rust/src/backend_wgpu.rs:403-412 keeps
// the same bound on pooled bytes, destroying the rest).
void HipBackend::release(void* ptr, size_t bytes) {
    if (pooled_bytes_ + bytes > kPoolMaxBytes) {
        g4a_sync(ctx_);  // the GPU may still read it
        g4a_free(ctx_, ptr);
        return;
    }
    pool_.emplace(bytes, ptr);
    pooled_bytes_ += bytes;
}

HipTensor HipBackend::alloc_tensor(std::vector<size_t> shape) {
    HipTensor t;
    t.buffer = alloc(product(shape) * sizeof(float));
    t.shape = std::move(shape);
    return t;
}

HipTensor HipBackend::tensor(const float* data, std::vector<size_t> shape) {
    HipTensor t = alloc_tensor(std::move(shape));
    check(g4a_h2d(ctx_, t.data(), data, t.size() * sizeof(float)), "g4a_h2d");
    return t;
}

HipTensor HipBackend::zeros(std::vector<size_t> shape) {
    HipTensor t = alloc_tensor(std::move(shape));
    check(g4a_zero(ctx_, t.data(), t.size() * sizeof(float)), "g4a_zero");
    return t;
}

// rust/src/backend_wgpu.rs:730-732: a view; a growing KV buffer's spare
// capacity is not carried over. A ring view keeps its ring when the row count
// (dim 0) is unchanged, since the rows are the same.
HipTensor HipBackend::reshape(const HipTensor& x, std::vector<size_t> shape) {
    if (product(shape) != x.size()) bad("reshape " + shape_str(x.shape) + " -> " + shape_str(shape));
    if (x.ring_cap && (shape.empty() || shape[0] != x.shape[0])) bad("reshape of a KV ring must keep its row count");
    HipTensor t;
    t.buffer = x.buffer;
    t.ring_cap = x.ring_cap;
    t.scales = x.scales;
    t.quant = x.quant;
    t.shape = std::move(shape);
    return t;
}

// rust/src/backend_wgpu.rs:895-969 (the attention dispatch) and
// rust/src/backend.rs:119-120 (the contract).
HipTensor HipBackend::quant_tensor(const QuantWeight& q) {
    const size_t N = q.shape[0], K = q.shape[1];
    const size_t group = q.group_size ? q.group_size : K;
    const size_t per_byte = q.signed_i8 ? 1 : 8 / q.bits;
    const size_t row_bytes = q.signed_i8 ? K : K / per_byte;
    const size_t stride = (K + group - 1) / group;
    if (q.qbytes.size() < N * row_bytes || q.scales.size() < N * stride)
        throw std::runtime_error("quant_tensor: payload smaller than the shape needs");
    HipTensor t;
    t.shape = {N, K};
    t.buffer = alloc(std::max<size_t>(q.qbytes.size(), 4));
    check(g4a_h2d(ctx_, t.buffer->ptr(), q.qbytes.data(), q.qbytes.size()), "quant_tensor (bytes)");
    t.scales = alloc(q.scales.size() * sizeof(float));
    check(g4a_h2d(ctx_, t.scales->ptr(), q.scales.data(), q.scales.size() * sizeof(float)), "quant_tensor (scales)");
    g4a_qweight d{};
    d.qbytes = t.buffer->ptr();
    d.scales = static_cast<const float*>(t.scales->ptr());
    d.N = uint32_t(N);
    d.K = uint32_t(K);
    d.bits = q.signed_i8 ? 8 : q.bits;
    d.signed_i8 = q.signed_i8 ? 1 : 0;
    d.group_size = uint32_t(group);
    t.quant = d;
    return t;
}

HipTensor HipBackend::embed_rows(const HipTensor& table, const uint32_t* ids, size_t n_ids, float scale) {
    if (table.shape.size() != 2) throw std::runtime_error("embed_rows: the table must be [V, D]");
    HipTensor out = alloc_tensor({n_ids, table.shape[1]});
    if (table.quant)
        check(g4a_embed_rows_q(ctx_, &*table.quant, ids, uint32_t(n_ids), scale, out.data()), "embed_rows");
    else
        check(g4a_embed_rows(ctx_, table.data(), uint32_t(table.shape[0]), uint32_t(table.shape[1]), ids,
                             uint32_t(n_ids), scale, out.data()),
              "embed_rows");
    return out;
}

HipTensor HipBackend::linear(const HipTensor& x, const HipTensor& w) {
    if (x.shape.size() != 2 || w.shape.size() != 2 || x.shape[1] != w.shape[1])
        throw std::runtime_error("linear: x [T, K] and W [N, K] required, got " + shape_str(x.shape) + " and " +
                                 shape_str(w.shape));
    HipTensor y = alloc_tensor({x.shape[0], w.shape[0]});
    if (w.quant)
        check(g4a_linear_q(ctx_, &*w.quant, x.data(), y.data(), uint32_t(x.shape[0])), "linear");
    else
        check(g4a_linear(ctx_, w.data(), uint32_t(w.shape[0]), uint32_t(w.shape[1]), x.data(), y.data(),
                         uint32_t(x.shape[0])),
              "linear");
    return y;
}

namespace {
void same_size(const HipTensor& a, const HipTensor& b, const char* op) {
    if (a.size() != b.size()) throw std::runtime_error(std::string(op) + ": operands differ in size");
}
}  // namespace

HipTensor HipBackend::add(const HipTensor& a, const HipTensor& b) {
    same_size(a, b, "add");
    HipTensor y = alloc_tensor(a.shape);
    check(g4a_add(ctx_, a.data(), b.data(), y.data(), a.size()), "add");
    return y;
}
HipTensor HipBackend::mul(const HipTensor& a, const HipTensor& b) {
    same_size(a, b, "mul");
    HipTensor y = alloc_tensor(a.shape);
    check(g4a_mul(ctx_, a.data(), b.data(), y.data(), a.size()), "mul");
    return y;
}
HipTensor HipBackend::scale(const HipTensor& a, float s) {
    HipTensor y = alloc_tensor(a.shape);
    check(g4a_scale(ctx_, a.data(), s, y.data(), a.size()), "scale");
    return y;
}
HipTensor HipBackend::scale_by_tensor(const HipTensor& a, const HipTensor& s) {
    HipTensor y = alloc_tensor(a.shape);
    check(g4a_scale_by_tensor(ctx_, a.data(), s.data(), y.data(), a.size()), "scale_by_tensor");
    return y;
}
HipTensor HipBackend::gelu_tanh(const HipTensor& a) {
    HipTensor y = alloc_tensor(a.shape);
    check(g4a_gelu_tanh(ctx_, a.data(), y.data(), a.size()), "gelu_tanh");
    return y;
}
HipTensor HipBackend::geglu(const HipTensor& gate, const HipTensor& up) {
    same_size(gate, up, "geglu");
    HipTensor y = alloc_tensor(gate.shape);
    check(g4a_geglu(ctx_, gate.data(), up.data(), y.data(), gate.size()), "geglu");
    return y;
}
HipTensor HipBackend::softcap(const HipTensor& a, float cap) {
    HipTensor y = alloc_tensor(a.shape);
    check(g4a_softcap(ctx_, a.data(), cap, y.data(), a.size()), "softcap");
    return y;
}

HipTensor HipBackend::slice_cols(const HipTensor& x, size_t offset, size_t width) {
    if (x.shape.size() != 2) throw std::runtime_error("slice_cols: x must be [rows, stride]");
    HipTensor y = alloc_tensor({x.shape[0], width});
    check(g4a_slice_cols(ctx_, x.data(), uint32_t(x.shape[0]), uint32_t(x.shape[1]), uint32_t(offset),
                         uint32_t(width), y.data()),
          "slice_cols");
    return y;
}

HipTensor HipBackend::add_rms_norm(const HipTensor& residual, const HipTensor& x, const HipTensor& w, float eps,
                                   const HipTensor* scale_by) {
    same_size(residual, x, "add_rms_norm");
    const size_t d = x.shape.back();
    HipTensor y = alloc_tensor(x.shape);
    check(g4a_add_rms_norm(ctx_, residual.data(), x.data(), w.data(), scale_by ? scale_by->data() : nullptr, y.data(),
                           uint32_t(x.size() / d), uint32_t(d), eps),
          "add_rms_norm");
    return y;
}

HipTensor HipBackend::linear_geglu(const HipTensor& x, const HipTensor& w_gate, const HipTensor& w_up) {
    if (w_gate.quant && w_up.quant) {
        const g4a_qweight &g = *w_gate.quant, &u = *w_up.quant;
        if (g.N == u.N && g.K == u.K && g.bits == u.bits && g.signed_i8 == u.signed_i8 && g.group_size == u.group_size) {
            if (x.shape.size() != 2 || x.shape[1] != g.K) throw std::runtime_error("linear_geglu: x must be [T, K]");
            HipTensor y = alloc_tensor({x.shape[0], size_t(g.N)});
            check(g4a_linear_q_geglu(ctx_, &g, &u, x.data(), y.data(), uint32_t(x.shape[0])), "linear_geglu");
            return y;
        }
    }
    return geglu(linear(x, w_gate), linear(x, w_up));
}

HipTensor HipBackend::linear_gelu_mul_cols(const HipTensor& x, const HipTensor& w, const HipTensor& b, size_t offset) {
    if (w.quant && b.shape.size() == 2 && b.shape[0] == x.shape[0]) {
        const g4a_qweight& q = *w.quant;
        if (x.shape.size() != 2 || x.shape[1] != q.K)
            throw std::runtime_error("linear_gelu_mul_cols: x must be [M, K]");
        HipTensor y = alloc_tensor({x.shape[0], size_t(q.N)});
        check(g4a_linear_q_gelu_mul_cols(ctx_, &q, x.data(), b.data(), uint32_t(b.shape[1]), uint32_t(offset),
                                         y.data(), uint32_t(x.shape[0])),
              "linear_gelu_mul_cols");
        return y;
    }
    return geglu(linear(x, w), slice_cols(b, offset, w.shape[0]));
}

HipTensor HipBackend::attention(const HipTensor& q, const HipTensor& k, const HipTensor& v, const AttnOpts& o) {
    if (q.shape.size() != 3 || k.shape.size() != 3 || v.shape.size() != 3)
        bad("attention wants q [T,Hq,Dh], k [S,Hkv,Dh], v [S,Hkv,Dv]; got " + shape_str(q.shape) + " " +
            shape_str(k.shape) + " " + shape_str(v.shape));
    const size_t T = q.shape[0], Hq = q.shape[1], Dh = q.shape[2];
    const size_t S = k.shape[0], Hkv = k.shape[1], Dv = v.shape[2];
    if (k.shape[2] != Dh || v.shape[0] != S || v.shape[1] != Hkv) bad("attention: k/v shapes disagree");
    if (o.n_q_pos != T || o.n_k_pos != S)
        bad("attention: " + std::to_string(o.n_q_pos) + " q positions for " + std::to_string(T) + " queries, " +
            std::to_string(o.n_k_pos) + " k positions for " + std::to_string(S) + " keys");
    if (k.ring_cap != v.ring_cap) bad("attention: k and v use different KV layouts");
    HipTensor out = alloc_tensor({T, Hq * Dv});
    g4a_attn_args a{};
    a.q = q.data();
    a.k = k.data();
    a.v = v.data();
    a.out = out.data();
    a.T = uint32_t(T);
    a.S = uint32_t(S);
    a.Hq = uint32_t(Hq);
    a.Hkv = uint32_t(Hkv);
    a.Dh = uint32_t(Dh);
    a.Dv = uint32_t(Dv);
    a.q_pos = o.q_pos;
    a.k_pos = o.k_pos;
    a.scale = o.scale;
    a.sliding_window = o.sliding_window;
    a.attn_softcap = o.attn_softcap;
    a.kv_ring_cap = k.ring_cap;
    check(g4a_attention(ctx_, &a), "g4a_attention");
    return out;
}

HipTensor HipBackend::rms_norm(const HipTensor& x, const HipTensor* w, float eps) {
    if (x.shape.empty() || x.ring_cap) bad("rms_norm wants a plain tensor");
    const size_t d = x.shape.back(), rows = x.size() / std::max<size_t>(d, 1);
    if (w && w->size() != d) bad("rms_norm: weight of " + std::to_string(w->size()) + " for rows of " + std::to_string(d));
    HipTensor out = alloc_tensor(x.shape);
    check(g4a_rms_norm(ctx_, x.data(), w ? w->data() : nullptr, out.data(), uint32_t(rows), uint32_t(d), eps),
          "g4a_rms_norm");
    return out;
}

namespace {
void check_rows(const HipTensor& x, size_t n_positions, size_t head_dim, size_t heads, const char* op) {
    if (x.shape.size() != 3 || x.shape[1] != heads || x.shape[2] != head_dim)
        bad(std::string(op) + " wants x [T, heads, head_dim]; got " + shape_str(x.shape));
    if (n_positions != x.shape[0]) bad(std::string(op) + ": one position per token");
}
}  // namespace

HipTensor HipBackend::rope(const HipTensor& x, const uint32_t* positions, size_t n_positions, float theta,
                           size_t head_dim, size_t heads, size_t rotary_dim) {
    check_rows(x, n_positions, head_dim, heads, "rope");
    HipTensor out = alloc_tensor(x.shape);
    check(g4a_rope(ctx_, x.data(), out.data(), uint32_t(x.shape[0]), uint32_t(heads), uint32_t(head_dim),
                   uint32_t(rotary_dim), positions, 0, theta),
          "g4a_rope");
    return out;
}

HipTensor HipBackend::head_norm_rope(const HipTensor& x, const HipTensor& w, float eps, const uint32_t* positions,
                                     size_t n_positions, float theta, size_t head_dim, size_t heads,
                                     size_t rotary_dim) {
    check_rows(x, n_positions, head_dim, heads, "head_norm_rope");
    if (w.size() != head_dim) bad("head_norm_rope: weight of " + std::to_string(w.size()) + " for head_dim " +
                                  std::to_string(head_dim));
    HipTensor out = alloc_tensor(x.shape);
    check(g4a_head_norm_rope(ctx_, x.data(), w.data(), out.data(), uint32_t(x.shape[0]), uint32_t(heads),
                             uint32_t(head_dim), uint32_t(rotary_dim), positions, 0, theta, eps),
          "g4a_head_norm_rope");
    return out;
}

HipTensor HipBackend::slice_rows(const HipTensor& x, size_t start, size_t count) {
    if (x.ring_cap) bad("slice_rows of a KV ring");
    if (x.shape.empty() || start + count > x.shape[0]) bad("slice_rows out of range");
    const size_t dim = x.size() / std::max<size_t>(x.shape[0], 1);
    HipTensor out = alloc_tensor({count, dim});
    check(g4a_d2d(ctx_, out.data(), x.data() + start * dim, count * dim * sizeof(float)), "g4a_d2d");
    return out;
}

HipTensor HipBackend::concat_rows(const HipTensor* a, const HipTensor& b) {
    if (b.ring_cap || (a && a->ring_cap)) bad("concat_rows of a KV ring");
    if (!a) {
        HipTensor out = alloc_tensor(b.shape);
        check(g4a_d2d(ctx_, out.data(), b.data(), b.size() * sizeof(float)), "g4a_d2d");
        return out;
    }
    if (a->shape.size() != b.shape.size() || !std::equal(a->shape.begin() + 1, a->shape.end(), b.shape.begin() + 1))
        bad("concat_rows " + shape_str(a->shape) + " + " + shape_str(b.shape));
    std::vector<size_t> shape = a->shape;
    shape[0] += b.shape[0];
    HipTensor out = alloc_tensor(shape);
    check(g4a_d2d(ctx_, out.data(), a->data(), a->size() * sizeof(float)), "g4a_d2d");
    check(g4a_d2d(ctx_, out.data() + a->size(), b.data(), b.size() * sizeof(float)), "g4a_d2d");
    return out;
}

// rust/src/backend_wgpu.rs:1014-1055: a capacity buffer of max(rows, 256) rows
// that doubles (or grows to fit) when full; the old buffer is reported dead.
KvAppend<HipTensor> HipBackend::kv_append(const HipTensor* existing, const HipTensor& add) {
    if (add.shape.empty() || add.shape[0] == 0) bad("kv_append of an empty tensor");
    if (existing && existing->ring_cap) bad("kv_append on a KV ring (use kv_append_ring)");
    const size_t rows = add.shape[0];
    const size_t dim = add.size() / rows;
    auto make_buffer = [&](size_t cap) {
        HipTensor t;
        t.buffer = alloc(cap * dim * sizeof(float));
        t.cap_rows = cap;
        return t;
    };
    if (!existing) {
        HipTensor t = make_buffer(std::max(rows, kKvMinRows));
        check(g4a_d2d(ctx_, t.data(), add.data(), add.size() * sizeof(float)), "g4a_d2d");
        t.shape = add.shape;
        return {t, std::nullopt};
    }
    if (existing->size() / std::max<size_t>(existing->shape[0], 1) != dim) bad("kv_append row size mismatch");
    const size_t len = existing->shape[0];
    const size_t cap_rows = existing->cap_rows ? existing->cap_rows : len;
    HipTensor dst = *existing;
    dst.cap_rows = cap_rows;
    std::optional<HipTensor> dead;
    if (len + rows > cap_rows) {
        dst = make_buffer(std::max(cap_rows * 2, len + rows));
        check(g4a_d2d(ctx_, dst.data(), existing->data(), len * dim * sizeof(float)), "g4a_d2d");
        dead = *existing;
    }
    check(g4a_kv_write(ctx_, dst.data(), 0, uint32_t(dim), uint32_t(len), add.data(), uint32_t(rows)), "g4a_kv_write");
    HipTensor view;
    view.buffer = dst.buffer;
    view.shape = add.shape;
    view.shape[0] = len + rows;
    view.cap_rows = dst.cap_rows;
    return {view, dead};
}

// Copy logical rows [first, first+count) between two KV layouts: a ring keeps
// row j in slot j % cap, a linear buffer (cap 0) keeps row j at j - base.
void HipBackend::copy_rows_ring(const HipTensor& src, uint32_t src_cap, HipTensor& dst, uint32_t dst_cap,
                                uint64_t first, uint64_t count, size_t row_elems) {
    const uint64_t end = first + count;
    uint64_t j = first;
    while (j < end) {
        uint64_t s = src_cap ? j % src_cap : j;
        uint64_t d = dst_cap ? j % dst_cap : j - first;
        uint64_t run = end - j;
        if (src_cap) run = std::min<uint64_t>(run, src_cap - s);
        if (dst_cap) run = std::min<uint64_t>(run, dst_cap - d);
        check(g4a_d2d(ctx_, dst.data() + d * row_elems, src.data() + s * row_elems, run * row_elems * sizeof(float)),
              "g4a_d2d");
        j += run;
    }
}

// A sliding-window layer needs, for a chunk of `rows` new queries, the last
// window + rows - 1 keys; older keys are never visible again. The ring holds
// exactly that many slots (slot = logical row % ring_cap), so the cache stays
// O(window) for any context length. A later, larger chunk re-lays the live
// rows into a bigger ring, which is reported dead like kv_append's growth.
KvAppend<HipTensor> HipBackend::kv_append_ring(const HipTensor* existing, const HipTensor& add, uint32_t window) {
    if (window == 0) bad("kv_append_ring needs a sliding window");
    if (add.shape.empty() || add.shape[0] == 0) bad("kv_append_ring of an empty tensor");
    const size_t rows = add.shape[0];
    const size_t dim = add.size() / rows;
    const uint64_t need = uint64_t(window) + rows - 1;
    if (need > UINT32_MAX) bad("kv_append_ring: ring too large");
    auto make_ring = [&](uint64_t cap) {
        HipTensor t;
        t.buffer = alloc(cap * dim * sizeof(float));
        t.ring_cap = uint32_t(cap);
        return t;
    };
    HipTensor dst;
    std::optional<HipTensor> dead;
    uint64_t len = 0;
    if (!existing) {
        dst = make_ring(need);
    } else {
        if (!existing->ring_cap) bad("kv_append_ring on a linear KV tensor");
        if (existing->size() / existing->shape[0] != dim) bad("kv_append_ring row size mismatch");
        len = existing->shape[0];
        dst = *existing;
        if (existing->ring_cap < need) {
            dst = make_ring(need);
            const uint64_t live = std::min<uint64_t>(len, existing->ring_cap);
            copy_rows_ring(*existing, existing->ring_cap, dst, dst.ring_cap, len - live, live, dim);
            dead = *existing;
        }
    }
    if (len + rows > UINT32_MAX) bad("kv_append_ring: position overflow");
    check(g4a_kv_write(ctx_, dst.data(), dst.ring_cap, uint32_t(dim), uint32_t(len), add.data(), uint32_t(rows)),
          "g4a_kv_write");
    HipTensor view;
    view.buffer = dst.buffer;
    view.ring_cap = dst.ring_cap;
    view.shape = add.shape;
    view.shape[0] = len + rows;
    return {view, dead};
}

// rust/src/backend_wgpu.rs:1057-1089: blocking read. A ring reads back its
// resident rows (the last min(rows, ring_cap)) in logical order.
std::vector<float> HipBackend::readback(const HipTensor& t) {
    if (!t.ring_cap) {
        std::vector<float> out(t.size());
        check(g4a_d2h(ctx_, out.data(), t.data(), out.size() * sizeof(float)), "g4a_d2h");
        return out;
    }
    const size_t dim = t.size() / t.shape[0];
    const uint64_t live = std::min<uint64_t>(t.shape[0], t.ring_cap);
    HipTensor lin = alloc_tensor({size_t(live), dim});
    copy_rows_ring(t, t.ring_cap, lin, 0, t.shape[0] - live, live, dim);
    std::vector<float> out(live * dim);
    check(g4a_d2h(ctx_, out.data(), lin.data(), out.size() * sizeof(float)), "g4a_d2h");
    return out;
}

// Launches are already submitted to the stream when an op returns.
void HipBackend::flush() {}

// rust/src/backend_wgpu.rs:1100-1124. Buffers return to the pool when their
// last handle drops, so keep-sets need no bookkeeping here: dropping the
// retired tensors is the whole job.
void HipBackend::end_frame(const std::vector<HipTensor>& keep, std::vector<HipTensor> also_free) {
    (void)keep;
    also_free.clear();
}

void HipBackend::free_tensor(HipTensor t) { t.buffer.reset(); }

std::pair<HipTensor, HipTensor> KvCache::append_and_read(HipBackend& b, size_t src_layer, const HipTensor& k_new,
                                                        const HipTensor& v_new, uint32_t window) {
    auto& slot = slots_.at(src_layer);
    const HipTensor* k_old = slot ? &slot->first : nullptr;
    const HipTensor* v_old = slot ? &slot->second : nullptr;
    KvAppend<HipTensor> rk = window ? b.kv_append_ring(k_old, k_new, window) : b.kv_append(k_old, k_new);
    KvAppend<HipTensor> rv = window ? b.kv_append_ring(v_old, v_new, window) : b.kv_append(v_old, v_new);
    if (rk.dead) dead_.push_back(*rk.dead);
    if (rv.dead) dead_.push_back(*rv.dead);
    slot = std::make_pair(rk.tensor, rv.tensor);
    return *slot;
}

void KvCache::reset(HipBackend& b) {
    for (auto& s : slots_) {
        if (s) {
            b.free_tensor(s->first);
            b.free_tensor(s->second);
            s.reset();
        }
    }
    for (auto& t : dead_) b.free_tensor(t);
    dead_.clear();
    positions.clear();
}

}  // namespace g4a
