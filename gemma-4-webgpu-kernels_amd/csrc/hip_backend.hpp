// C++ mirror of the reference's backend-agnostic op surface for the attention
// path (rust/src/backend.rs:59-180), implemented over the C-ABI of libg4a.so.
// It does what a Rust `HipBackend` would do over the same calls through FFI:
// same op names, same argument meaning, same conventions:
//   - ops are infallible: a failing g4a call throws std::runtime_error (the
//     Rust backend panics, rust/src/backend_wgpu.rs:1077-1078); only
//     construction reports failure as a value to handle (here: create() throws
//     before any op can run, matching WgpuBackend::create -> Result);
//   - ops are stream-ordered and return before the GPU runs them; readback()
//     blocks (rust/src/backend_wgpu.rs:1-6);
//   - tensors are cheap shared handles (rust/src/backend_wgpu.rs:69-75) and
//     must not outlive the backend that made them;
//   - position slices are borrowed for the duration of the call
//     (rust/src/backend.rs:61-64).
// Beyond the reference: kv_append_ring() keeps a sliding-window layer's cache
// as a ring of window + chunk - 1 slots (slot = position % capacity) instead of
// a growing buffer, and KvCache uses it for sliding layers.
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <memory>
#include <optional>
#include <stdexcept>
#include <string>
#include <vector>

#include "g4a.h"

namespace g4a {

// rust/src/backend.rs:59-69
struct AttnOpts {
    const uint32_t* q_pos = nullptr;
    size_t n_q_pos = 0;
    const uint32_t* k_pos = nullptr;
    size_t n_k_pos = 0;
    float scale = 1.0f;
    uint32_t sliding_window = 0;  // 0 = no sliding window (full causal attention)
    float attn_softcap = 0.0f;    // 0 = no attention soft-capping
};

class HipBackend;

// rust/src/backend.rs:12-58 (QuantWeight): packed rows (sub-byte offset-binary
// fields LSB-first, or I8), one scale per (row, group), logical shape [N, K].
struct QuantWeight {
    std::vector<uint8_t> qbytes;
    std::vector<float> scales;
    size_t shape[2] = {0, 0};
    uint32_t bits = 4;
    bool signed_i8 = false;
    size_t group_size = 0;
};

// A pooled device allocation; released to its backend's pool when the last
// handle drops. Reuse is safe without a sync: every op runs on the backend's
// single stream, so a later op that reuses the memory runs after every earlier
// op that read it.
class DeviceBuffer {
public:
    DeviceBuffer(HipBackend* owner, void* ptr, size_t bytes) : owner_(owner), ptr_(ptr), bytes_(bytes) {}
    ~DeviceBuffer();
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    void* ptr() const { return ptr_; }
    size_t bytes() const { return bytes_; }

private:
    HipBackend* owner_;
    void* ptr_;
    size_t bytes_;
};

// rust/src/backend_wgpu.rs:69-75 (GpuTensor): buffer + logical shape, plus the
// KV-cache metadata: cap_rows for the reference's growing capacity buffer,
// ring_cap for a sliding-window ring.
struct HipTensor {
    std::shared_ptr<DeviceBuffer> buffer;
    std::vector<size_t> shape;
    size_t cap_rows = 0;
    uint32_t ring_cap = 0;
    // a quantised weight (rust/src/backend_wgpu.rs:78-86, GpuQuant): `buffer` holds
    // the packed rows, `scales` the per-(row, group) scales
    std::shared_ptr<DeviceBuffer> scales;
    std::optional<g4a_qweight> quant;

    const std::vector<size_t>& dims() const { return shape; }
    size_t size() const {
        size_t n = 1;
        for (size_t d : shape) n *= d;
        return n;
    }
    float* data() const { return buffer ? static_cast<float*>(buffer->ptr()) : nullptr; }
};

// rust/src/backend.rs:72-77
template <class T>
struct KvAppend {
    T tensor;
    std::optional<T> dead;
};

class HipBackend {
public:
    // WgpuBackend::create (rust/src/backend_wgpu.rs:283).
    static std::unique_ptr<HipBackend> create(int device = 0);
    ~HipBackend();
    HipBackend(const HipBackend&) = delete;
    HipBackend& operator=(const HipBackend&) = delete;

    const char* name() const { return "hip"; }
    g4a_ctx* ctx() const { return ctx_; }

    // --- construction (rust/src/backend.rs:93-98) ---
    HipTensor tensor(const float* data, std::vector<size_t> shape);
    HipTensor zeros(std::vector<size_t> shape);
    HipTensor reshape(const HipTensor& x, std::vector<size_t> shape);
    // the packed weight kept in its quantised form (rust/src/backend.rs:94)
    HipTensor quant_tensor(const QuantWeight& q);

    // --- ops ---
    // out[i, :] = table[ids[i], :] * scale; table [V, D] f32 or quantised (rust/src/backend.rs:100-101)
    HipTensor embed_rows(const HipTensor& table, const uint32_t* ids, size_t n_ids, float scale);
    // y = x . W^T; x [T, K], W [N, K] f32 or quantised (rust/src/backend.rs:105-106)
    HipTensor linear(const HipTensor& x, const HipTensor& w);
    // elementwise (rust/src/backend.rs:107-116)
    HipTensor add(const HipTensor& a, const HipTensor& b);
    HipTensor mul(const HipTensor& a, const HipTensor& b);
    HipTensor scale(const HipTensor& a, float s);
    HipTensor scale_by_tensor(const HipTensor& a, const HipTensor& s);  // a * s[0]
    HipTensor gelu_tanh(const HipTensor& a);
    HipTensor geglu(const HipTensor& gate, const HipTensor& up);  // gelu(gate) * up
    HipTensor softcap(const HipTensor& a, float cap);              // cap * tanh(a / cap)
    // [:, offset : offset + width] of a [rows, stride] tensor (rust/src/backend.rs:123-124)
    HipTensor slice_cols(const HipTensor& x, size_t offset, size_t width);
    // (residual + rms_norm(x, w)) * scale_by[0], one launch (rust/src/backend.rs:136-145)
    HipTensor add_rms_norm(const HipTensor& residual, const HipTensor& x, const HipTensor& w, float eps,
                           const HipTensor* scale_by);
    // gelu(x . Wg^T) * (x . Wu^T): one launch for two quantised weights of one format,
    // else the trait's composition (rust/src/backend.rs:156-161)
    HipTensor linear_geglu(const HipTensor& x, const HipTensor& w_gate, const HipTensor& w_up);
    // gelu(x . W^T) * b[:, offset : offset + N], b [M, stride]: one launch for a quantised
    // weight, else the trait's composition (rust/src/backend.rs:162-168)
    HipTensor linear_gelu_mul_cols(const HipTensor& x, const HipTensor& w, const HipTensor& b, size_t offset);
    // q [T,Hq,Dh], k [S,Hkv,Dh], v [S,Hkv,Dv] -> [T, Hq*Dv] (rust/src/backend.rs:119-120)
    HipTensor attention(const HipTensor& q, const HipTensor& k, const HipTensor& v, const AttnOpts& o);
    // y = x / sqrt(mean(x^2) + eps) * w per row of the last dim; w == nullptr for the
    // unweighted variant (rust/src/backend.rs:103-104)
    HipTensor rms_norm(const HipTensor& x, const HipTensor* w, float eps);
    // half-split partial RoPE on [T, heads, head_dim], rotating the first rotary_dim
    // dims (rust/src/backend.rs:117-118)
    HipTensor rope(const HipTensor& x, const uint32_t* positions, size_t n_positions, float theta, size_t head_dim,
                   size_t heads, size_t rotary_dim);
    // per-head weighted RMSNorm then RoPE, one launch (rust/src/backend.rs:146-154)
    HipTensor head_norm_rope(const HipTensor& x, const HipTensor& w, float eps, const uint32_t* positions,
                             size_t n_positions, float theta, size_t head_dim, size_t heads, size_t rotary_dim);
    // rows [start, start+count) of a [rows, dim] tensor (rust/src/backend.rs:122)
    HipTensor slice_rows(const HipTensor& x, size_t start, size_t count);
    // concatenate along dim 0; a == nullptr copies b (rust/src/backend.rs:125-126)
    HipTensor concat_rows(const HipTensor* a, const HipTensor& b);
    // append rows to a KV tensor, growing a capacity buffer x2 when full
    // (rust/src/backend.rs:127-128, rust/src/backend_wgpu.rs:1014-1055)
    KvAppend<HipTensor> kv_append(const HipTensor* existing, const HipTensor& add);
    // append rows to a sliding-window KV ring that keeps the last `window` keys
    // visible to every query of the appended chunk
    KvAppend<HipTensor> kv_append_ring(const HipTensor* existing, const HipTensor& add, uint32_t window);

    // --- sync / lifecycle (rust/src/backend.rs:171-179) ---
    std::vector<float> readback(const HipTensor& t);
    void flush();
    void begin_frame() {}
    void end_frame(const std::vector<HipTensor>& keep, std::vector<HipTensor> also_free);
    void free_tensor(HipTensor t);

    // pool bookkeeping (DeviceBuffer's destructor)
    void release(void* ptr, size_t bytes);

private:
    explicit HipBackend(g4a_ctx* ctx) : ctx_(ctx) {}
    std::shared_ptr<DeviceBuffer> alloc(size_t bytes);
    void check(int rc, const char* what) const;
    HipTensor alloc_tensor(std::vector<size_t> shape);
    void copy_rows_ring(const HipTensor& src, uint32_t src_cap, HipTensor& dst, uint32_t dst_cap, uint64_t first,
                        uint64_t count, size_t row_elems);

    g4a_ctx* ctx_ = nullptr;
    std::multimap<size_t, void*> pool_;  // pow2-bucketed free buffers (rust/src/backend_wgpu.rs:384-412)
    size_t pooled_bytes_ = 0;
};

// rust/src/kvcache.rs: per-source-layer K/V slots and the absolute positions
// of cached tokens. Sliding layers (window > 0) keep rings; global layers keep
// the reference's growing buffer.
class KvCache {
public:
    explicit KvCache(size_t num_layers) : slots_(num_layers) {}
    void push_positions(const uint32_t* p, size_t n) { positions.insert(positions.end(), p, p + n); }
    // rust/src/kvcache.rs:49-62, with the layer's window choosing the layout
    std::pair<HipTensor, HipTensor> append_and_read(HipBackend& b, size_t src_layer, const HipTensor& k_new,
                                                   const HipTensor& v_new, uint32_t window);
    const std::pair<HipTensor, HipTensor>* read(size_t src_layer) const {
        return slots_[src_layer] ? &*slots_[src_layer] : nullptr;
    }
    std::vector<HipTensor> take_dead() { return std::move(dead_); }
    void reset(HipBackend& b);

    std::vector<uint32_t> positions;

private:
    std::vector<std::optional<std::pair<HipTensor, HipTensor>>> slots_;
    std::vector<HipTensor> dead_;
};

}  // namespace g4a
