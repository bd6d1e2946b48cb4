// libg4a.so — host side of the MI355X attention path behind the C-ABI in
// include/g4a.h. Loads the gfx950 code object (g4a_kernels.hsaco) with
// hipModuleLoad and launches its kernels with hipModuleLaunchKernel on one
// stream per context. Replaces the wgpu host dispatch of the reference
// (WgpuBackend::attention / kv_append, rust/src/backend_wgpu.rs:895-1055).
#include "g4a.h"

#include <dlfcn.h>
#include <math.h>
#include <hip/hip_ext.h>
#include <hip/hip_runtime_api.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "kernels/g4a_params.h"

namespace {

// Keys per decode tile; the split-K granularity (a multiple of it).
constexpr uint32_t TILE = 64;
// Query tokens from which the query-tiled prefill kernel replaces decode.
constexpr uint32_t PREFILL_MIN_T = 16;
// The prefill's exact-rescoring band: tau = max(MIN, ln(N) + LOGN) for N keys per
// row, so the keys left with their estimated scores hold at most a weight share
// ~e^-LOGN of a row: their score errors (~5e-6 rms, 6e-5 max, from the scaled
// fp16 splits and the matrix cores' summation order) then move the row's output
// by ~1e-5 * e^-LOGN * max|v - out| even when all of them push the same way.
constexpr float PREFILL_TAU_MIN = 7.0f;
constexpr float PREFILL_TAU_LOGN = 2.0f;
// Largest split-K count the LSE combine kernel takes (its LDS weight table).
constexpr uint32_t MAX_SPLITS = 1024;
// Split counts merged by the one-block-per-head combine kernel (combine_rows).
constexpr uint32_t COMBINE_ROW_SPLITS = 16;
// Output dims and threads per block of the wide combine kernel (combine).
constexpr uint32_t kCombineDims = 32;
constexpr uint32_t kCombineThreads = 512;
// Keys per 4-wave workgroup of the short-context decode kernel (two 16-key tiles).
constexpr uint32_t SHORT_KEYS = 32;
// Most visible keys of a batched decode step (1024 splits of the short kernel).
constexpr uint32_t BATCH_MAX_KEYS = SHORT_KEYS * MAX_SPLITS;

// The message of the last failure that had no context (g4a_create, or a call
// given a NULL context), per thread: two threads that fail at once each read
// their own.
thread_local std::string g_create_error;

// Bytes of the static scratch array a call that allocates nothing may use.
constexpr size_t NOALLOC_SCRATCH_BYTES = G4A_NOALLOC_SCRATCH_BYTES;

// Tags each K/V pre-split's V range flag (G4aSplitParams::epoch). Process-wide,
// so no two pre-splits of any context share a tag.
std::atomic<uint32_t> g_split_epoch{0};

uint32_t next_split_epoch() {
    uint32_t e = g_split_epoch.fetch_add(1, std::memory_order_relaxed) + 1;
    while (e == 0) e = g_split_epoch.fetch_add(1, std::memory_order_relaxed) + 1;
    return e;
}

}  // namespace

// Scratch of g4a_attention_noalloc: split partials and pre-split K/V of calls
// that may not allocate. Each GPU the library runs on holds its own copy of the
// array, at its own address, from the first context on it until the process
// ends. In host code `scratch` names a host-side stand-in, not device memory:
// kernels get the device address from scratch_setup, never the name itself.
static __device__ __align__(256) unsigned char scratch[G4A_NOALLOC_SCRATCH_BYTES];

// The graphs captured on a context, shared by the context and each of its
// graphs. A graph replays with the workspace it was captured with, so while
// any graph is live a workspace the context outgrows is kept (retired), not
// freed, until the last graph is destroyed.
struct g4a_graph_book {
    g4a_ctx* ctx = nullptr;      // null once the context is destroyed
    uint32_t live = 0;           // graphs not yet destroyed
    std::vector<void*> retired;  // workspaces replaced while graphs were live
};

struct g4a_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    hipModule_t module = nullptr;
    hipFunction_t decode[2][2][2] = {};  // [dh512][group8][explicit key positions]
    hipFunction_t combine[2] = {nullptr, nullptr};                          // [dh512]
    hipFunction_t decode_short[2] = {nullptr, nullptr};  // [dh512]
    hipFunction_t decode_short2[2] = {nullptr, nullptr};  // [dh512] two workgroups per split (output dim halves)
    hipFunction_t decode_short4[2] = {nullptr, nullptr};  // [dh512] four workgroups per split (quarters)
    hipFunction_t decode_short2x[2] = {nullptr, nullptr};  // the same two / four with a split's
    hipFunction_t decode_short4x[2] = {nullptr, nullptr};  // workgroups on one XCD
    hipFunction_t decode_batch[2] = {nullptr, nullptr};   // [dh512] short decode over many sequences
    hipFunction_t decode_wave_batch[2] = {nullptr, nullptr};  // [dh512] streaming decode over many sequences
    hipFunction_t decode_wave_batch_kpos[2] = {nullptr, nullptr};  // [dh512] the same, explicit key positions
    hipFunction_t combine_batch[2] = {nullptr, nullptr};  // [dh512]
    hipFunction_t combine_rows[2] = {nullptr, nullptr};        // [dh512] combine of <= 16 splits
    hipFunction_t combine_rows_batch[2] = {nullptr, nullptr};  // [dh512]
    // batched decode tuning (G4A_BATCH_KERNEL=short|wave, G4A_BATCH_KEYS_PER_SPLIT=n): for comparisons
    int batch_kernel = 0;  // 0 auto, 1 short, 2 streaming
    uint32_t batch_kps = 0;  // streaming split size; 0 auto
    bool short_decode = true;  // g4a_options::short_decode
    uint32_t short_ds = 4;     // g4a_options::short_max_wgs: most workgroups per short split
    hipFunction_t generic = nullptr;
    hipFunction_t prefill[2] = {nullptr, nullptr};                          // [dh512]
    hipFunction_t split_kv = nullptr;  // K/V pre-split for the head_dim 256 prefill
    hipFunction_t norm_rope = nullptr;        // the attention producer (RMSNorm + RoPE + KV write)
    hipFunction_t norm_rope_short = nullptr;  // the same with its loads issued together (<= 1 workgroup per CU)
    hipFunction_t linear_words[3][3][3] = {};  // [bits 2/4/8][(MT, RU) = (1, 2), (1, 8), (4, 4)][mode]
    hipFunction_t linear_elem[3] = {};         // [mode]
    hipFunction_t linear_mfma[3][2][3] = {};   // [bits 2/4/8][64 / 128 weight rows per tile][mode]: M >= 16
    hipFunction_t linear_i8[3][2] = {};        // [bits 2/4/8][M = 1, 2]: int8 matrix cores, mode 0
    // G4A_LINEAR_I8=0 keeps M <= 2 projections off the int8 matrix-core kernel,
    // =1 sends every eligible one there (for comparisons); unset: by weight size
    int linear_i8_use = -1;
    hipFunction_t linear_fused[3] = {};  // [bits 2/4/8]: a decode step's split partials merged into x
    // G4A_FUSE_PROJECTION=1: g4a_attention_linear_q merges eligible decode steps'
    // partials in the projection (measured slower than the separate combine on
    // MI355X, so off by default)
    bool fuse_projection = false;
    hipFunction_t embed_q = nullptr;
    hipFunction_t linear_half[2][3] = {};       // 2-bit, M = 1, 32 lanes per row: [RU = 1, 4][mode]
    hipFunction_t linear_f32_words[3] = {};  // f32 weights: (MT, RU) = (1, 2), (1, 8), (4, 4)
    hipFunction_t linear_f32_elem = nullptr;
    hipFunction_t ew = nullptr;              // elementwise ops
    hipFunction_t u32_add = nullptr;         // device counters (positions of replayed decode steps)
    hipFunction_t slice_cols = nullptr;
    hipFunction_t rms_rows = nullptr;        // (residual +) RMSNorm (* scalar) over rows of any width
    hipFunction_t embed_f32 = nullptr;
    // RoPE frequency tables theta^(-2j/rot), one per (theta, rotary_dim) seen
    struct FreqTable {
        float theta;
        uint32_t rot;
        std::vector<float> host;
        float* dev;
    };
    std::vector<FreqTable> freq_tables;
    // RoPE (sinf, cosf) tables of pos * freq[j], one per (theta, rotary_dim) seen,
    // covering positions [0, rows); grown on demand. A grown table's old buffer is
    // kept until the context ends: a captured graph may still read it.
    struct SinCosTable {
        float theta;
        uint32_t rot;
        uint32_t rows;
        float2* dev;
    };
    std::vector<SinCosTable> sc_tables;
    std::vector<void*> sc_retired;
    hipEvent_t ev_start = nullptr, ev_stop = nullptr;
    hipEvent_t ev_staging = nullptr;  // last use of the pinned staging buffer
    void* workspace = nullptr;
    size_t workspace_bytes = 0;
    size_t prev_workspace_bytes = 0;  // the size of the buffer the last growth replaced
    int query_depth = 0;              // > 0 inside a query entry point (g4a_attention_plan)
    void* scratch = nullptr;  // this device's static scratch array (the allocation-free entry point)
    hipFunction_t prefill_merge = nullptr;  // merge of the split hd512 prefill blocks
    float* dummy = nullptr;  // 4 KiB of zeros: the load target of idle decode tiles
    uint32_t* pos_dev = nullptr;  // device copies of non-contiguous positions
    size_t pos_dev_cap = 0;       // in u32
    uint32_t* pos_host = nullptr;  // pinned staging for those copies
    size_t pos_host_cap = 0;
    int cu_count = 0;
    // per-kernel event pairs (g4a_kernel_timing)
    bool timing = false;
    bool capturing = false;  // between g4a_capture_begin and g4a_capture_end
    int capture_code = 0;    // the first failure inside the open capture (sticky until g4a_capture_end)
    std::string capture_msg;
    std::shared_ptr<g4a_graph_book> book;
    std::vector<hipEvent_t> kev;  // 2 * kMaxTimed
    uint32_t kev_used = 0;
    std::string err;
};

namespace {

int fail(g4a_ctx* ctx, int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    if (ctx) {
        ctx->err = buf;
        // a refused call inside a capture leaves a graph without it: remembered, so
        // g4a_capture_end reports it instead of returning that graph (a failing
        // query, which enqueues nothing, leaves the capture alone)
        if (ctx->capturing && ctx->capture_code == 0 && ctx->query_depth == 0) {
            ctx->capture_code = code;
            ctx->capture_msg = buf;
        }
    } else {
        g_create_error = buf;
    }
    return code;
}

#define HIP_TRY(ctx, call)                                                                          \
    do {                                                                                            \
        hipError_t e_ = (call);                                                                     \
        if (e_ != hipSuccess) return fail((ctx), G4A_E_HIP, "%s: %s", #call, hipGetErrorString(e_)); \
    } while (0)

std::string default_hsaco_path() {
    Dl_info info;
    if (dladdr(reinterpret_cast<void*>(&g4a_create), &info) && info.dli_fname) {
        std::string p(info.dli_fname);
        size_t slash = p.rfind('/');
        std::string dir = slash == std::string::npos ? "." : p.substr(0, slash);
        return dir + "/g4a_kernels.hsaco";
    }
    return "g4a_kernels.hsaco";
}

// The device address of this device's scratch array, looked up once per device
// (with that device current) and kept for every later context on it.
int scratch_setup(g4a_ctx* ctx) {
    static std::mutex mu;
    static std::vector<void*> per_device;
    std::lock_guard<std::mutex> lock(mu);
    if (per_device.size() <= size_t(ctx->device)) per_device.resize(size_t(ctx->device) + 1, nullptr);
    if (!per_device[ctx->device]) {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr)
            return fail(ctx, G4A_E_HIP, "hipGetSymbolAddress(scratch) on device %d: %s", ctx->device,
                        hipGetErrorString(e));
        per_device[ctx->device] = ptr;
    }
    ctx->scratch = per_device[ctx->device];
    return G4A_OK;
}

int get_fn(g4a_ctx* ctx, hipFunction_t* f, const char* name) {
    hipError_t e = hipModuleGetFunction(f, ctx->module, name);
    if (e != hipSuccess) return fail(ctx, G4A_E_MODULE, "kernel %s missing from code object: %s", name, hipGetErrorString(e));
    return G4A_OK;
}

int ensure_workspace(g4a_ctx* ctx, size_t bytes) {
    if (bytes <= ctx->workspace_bytes) return G4A_OK;
    if (ctx->capturing)
        return fail(ctx, G4A_E_ARG, "the workspace must grow to %zu bytes, which a graph capture cannot do: "
                    "run the calls once before capturing them", bytes);
    if (ctx->workspace) {
        if (ctx->book->live) {
            // live graphs replay with this buffer: keep it until the last one is destroyed
            ctx->book->retired.push_back(ctx->workspace);
        } else {
            // the old buffer may still be read by queued kernels
            HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
            HIP_TRY(ctx, hipFree(ctx->workspace));
        }
        ctx->prev_workspace_bytes = ctx->workspace_bytes;
        ctx->workspace = nullptr;
        ctx->workspace_bytes = 0;
    }
    if (!ctx->book->live && !ctx->book->retired.empty()) {
        HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
        for (void* p : ctx->book->retired) HIP_TRY(ctx, hipFree(p));
        ctx->book->retired.clear();
    }
    // geometric growth: a run of slightly larger calls retires a bounded number of buffers
    size_t want = std::max<size_t>({bytes, 2 * ctx->prev_workspace_bytes, size_t(8) << 20});
    hipError_t e = hipMalloc(&ctx->workspace, want);
    if (e != hipSuccess) return fail(ctx, G4A_E_NOMEM, "workspace of %zu bytes: %s", want, hipGetErrorString(e));
    ctx->workspace_bytes = want;
    return G4A_OK;
}

// Query blocks of the head_dim 512 prefill that run as two workgroups, one per
// half of their key tiles: the trailing blocks (causal masks give later queries
// more keys) whose tile count exceeds the average over all blocks. Mirrors the
// kernel's tile range of a block of 8 queries (prefill_dsplit).
uint32_t prefill_split_blocks(const g4a_attn_args* a, uint32_t q_pos0, uint32_t k_pos0) {
    const uint32_t NB = (a->T + 7) / 8;
    if (NB == 0) return 0;
    auto key_hi = [&](int64_t i) -> int64_t {
        const int64_t lim = (int64_t)q_pos0 + i - (int64_t)k_pos0 + 1;
        return lim <= 0 ? 0 : std::min<int64_t>(lim, a->S);
    };
    auto key_lo = [&](int64_t i) -> int64_t {
        if (a->sliding_window == 0) return 0;
        const int64_t lo = (int64_t)q_pos0 + i - (int64_t)k_pos0 - (int64_t)a->sliding_window + 1;
        return lo <= 0 ? 0 : std::min<int64_t>(lo, a->S);
    };
    auto tiles = [&](uint32_t b) -> int64_t {  // 16-key tiles of query block b
        const int64_t lo = key_lo(8 * int64_t(b)), hi = key_hi(std::min<int64_t>(8 * int64_t(b) + 7, a->T - 1));
        const int64_t base = lo & ~int64_t(15);
        return hi > lo ? (hi - base + 15) / 16 : 0;
    };
    int64_t total = 0;
    for (uint32_t b = 0; b < NB; ++b) total += tiles(b);
    uint32_t nbig = 0;
    while (nbig < NB && tiles(NB - 1 - nbig) * int64_t(NB) > total) ++nbig;
    return nbig;
}

// Stages up to two host position arrays into device memory (stream-ordered).
// The pinned staging buffer is reused only after its previous copy finished.
int upload_positions(g4a_ctx* ctx, const uint32_t* a, size_t na, const uint32_t* b, size_t nb, const uint32_t** da,
                     const uint32_t** db) {
    const size_t n = na + nb;
    if (n == 0) return G4A_OK;
    if (ctx->capturing)
        return fail(ctx, G4A_E_ARG, "explicit positions or ids are staged from host memory, which a graph capture "
                    "cannot hold: capture calls with contiguous positions (q_pos0 / k_pos0)");
    if (n > ctx->pos_dev_cap) {
        if (ctx->pos_dev) {
            HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
            HIP_TRY(ctx, hipFree(ctx->pos_dev));
            ctx->pos_dev = nullptr;
        }
        size_t cap = std::max<size_t>(n, 1 << 16);
        if (hipMalloc(&ctx->pos_dev, cap * sizeof(uint32_t)) != hipSuccess)
            return fail(ctx, G4A_E_NOMEM, "position buffer of %zu entries", cap);
        ctx->pos_dev_cap = cap;
    }
    HIP_TRY(ctx, hipEventSynchronize(ctx->ev_staging));
    if (n > ctx->pos_host_cap) {
        if (ctx->pos_host) HIP_TRY(ctx, hipHostFree(ctx->pos_host));
        ctx->pos_host = nullptr;
        size_t cap = std::max<size_t>(n, 1 << 16);
        if (hipHostMalloc(reinterpret_cast<void**>(&ctx->pos_host), cap * sizeof(uint32_t), hipHostMallocDefault) != hipSuccess)
            return fail(ctx, G4A_E_NOMEM, "pinned staging of %zu entries", cap);
        ctx->pos_host_cap = cap;
    }
    if (na) memcpy(ctx->pos_host, a, na * sizeof(uint32_t));
    if (nb) memcpy(ctx->pos_host + na, b, nb * sizeof(uint32_t));
    HIP_TRY(ctx, hipMemcpyAsync(ctx->pos_dev, ctx->pos_host, n * sizeof(uint32_t), hipMemcpyHostToDevice, ctx->stream));
    HIP_TRY(ctx, hipEventRecord(ctx->ev_staging, ctx->stream));
    if (da) *da = na ? ctx->pos_dev : nullptr;
    if (db) *db = nb ? ctx->pos_dev + na : nullptr;
    return G4A_OK;
}

constexpr uint32_t kMaxTimed = 4096;

// Launches one kernel; `timed` brackets it with an event pair when per-kernel
// timing is on (the main kernel of an attention call).
template <typename P>
int launch(g4a_ctx* ctx, hipFunction_t f, dim3 grid, dim3 block, const P& params, const char* what,
           bool timed = false, unsigned lds_bytes = 0) {
    P copy = params;
    void* args[] = {&copy};
    const bool rec = timed && ctx->timing && ctx->kev_used < kMaxTimed;
    hipError_t e;
    if (rec) {
        // events attached to the dispatch itself: they bracket the kernel's execution,
        // not the host-side enqueue, so they agree with a profiler's kernel duration
        e = hipExtModuleLaunchKernel(f, grid.x * block.x, grid.y * block.y, grid.z * block.z, block.x, block.y,
                                     block.z, lds_bytes, ctx->stream, args, nullptr, ctx->kev[2 * ctx->kev_used],
                                     ctx->kev[2 * ctx->kev_used + 1], 0);
        if (e == hipSuccess) ++ctx->kev_used;
    } else {
        e = hipModuleLaunchKernel(f, grid.x, grid.y, grid.z, block.x, block.y, block.z, lds_bytes, ctx->stream, args,
                                  nullptr);
    }
    if (e != hipSuccess) return fail(ctx, G4A_E_HIP, "launch %s: %s", what, hipGetErrorString(e));
    return G4A_OK;
}

// Host-side analysis shared by g4a_attention and g4a_attention_plan.
struct Analysis {
    g4a_attn_plan plan{};
    bool q_contig = true, k_contig = true, k_ascending = true;
    uint32_t qmin = 0, qmax = 0;
    bool fast_shape = false;
};

uint32_t kpos_at(const g4a_attn_args* a, uint32_t j) { return a->k_pos ? a->k_pos[j] : a->k_pos0 + j; }

// First index j in [0, S) for which pred(kpos(j)) is false, for a predicate
// that is true on a prefix (Rust's slice::partition_point).
template <typename Pred>
uint32_t partition_point(const g4a_attn_args* a, Pred pred) {
    uint32_t lo = 0, hi = a->S;
    while (lo < hi) {
        uint32_t mid = lo + (hi - lo) / 2;
        if (pred(kpos_at(a, mid))) lo = mid + 1;
        else hi = mid;
    }
    return lo;
}

int analyse(g4a_ctx* ctx, const g4a_attn_args* a, Analysis* an, bool check_pointers) {
    if (!a) return fail(ctx, G4A_E_ARG, "null args");
    if (a->Hq == 0 || a->Hkv == 0 || a->Dh == 0 || a->Dv == 0)
        return fail(ctx, G4A_E_SHAPE, "zero dimension (Hq=%u Hkv=%u Dh=%u Dv=%u)", a->Hq, a->Hkv, a->Dh, a->Dv);
    if (a->Hq % a->Hkv != 0) return fail(ctx, G4A_E_SHAPE, "Hq=%u is not a multiple of Hkv=%u", a->Hq, a->Hkv);
    if (!(a->attn_softcap >= 0.0f)) return fail(ctx, G4A_E_ARG, "attn_softcap must be >= 0");
    Analysis& r = *an;
    r = Analysis{};
    if (a->T == 0) return G4A_OK;
    if (check_pointers) {
        if (!a->q || !a->out) return fail(ctx, G4A_E_ARG, "null q/out");
        if (a->S > 0 && (!a->k || !a->v)) return fail(ctx, G4A_E_ARG, "null k/v");
    }
    // query positions
    if (a->q_pos) {
        r.qmin = r.qmax = a->q_pos[0];
        for (uint32_t i = 0; i < a->T; ++i) {
            uint32_t p = a->q_pos[i];
            r.qmin = std::min(r.qmin, p);
            r.qmax = std::max(r.qmax, p);
            if (p != a->q_pos[0] + i) r.q_contig = false;
        }
    } else {
        r.qmin = a->q_pos0;
        r.qmax = a->q_pos0 + (a->T - 1);
    }
    if (a->k_pos) {
        for (uint32_t j = 0; j < a->S; ++j) {
            if (a->k_pos[j] != a->k_pos[0] + j) r.k_contig = false;
            if (j && a->k_pos[j] < a->k_pos[j - 1]) r.k_ascending = false;
        }
    }
    // active key range shared by every query (rust/src/backend_wgpu.rs:929-936)
    uint32_t k_start = 0, k_end = a->S;
    if (r.k_ascending) {
        const uint64_t qmax = r.qmax, qmin = r.qmin, win = a->sliding_window;
        k_end = partition_point(a, [&](uint32_t kp) { return uint64_t(kp) <= qmax; });
        if (win > 0 && qmin >= win)
            k_start = std::min(k_end, partition_point(a, [&](uint32_t kp) { return uint64_t(kp) + win <= qmin; }));
    }
    r.plan.k_start = k_start;
    r.plan.k_end = k_end;
    if (a->kv_ring_cap && k_end - k_start > a->kv_ring_cap)
        return fail(ctx, G4A_E_SHAPE, "visible key range [%u, %u) exceeds the KV ring of %u rows", k_start, k_end,
                    a->kv_ring_cap);
    const uint32_t group = a->Hq / a->Hkv;
    r.fast_shape = (group == 4 || group == 8) && a->Dh == a->Dv && (a->Dh == 256 || a->Dh == 512) &&
                   r.k_ascending && (a->kv_ring_cap == 0 || a->kv_ring_cap >= TILE);
    const uint32_t nkeys = k_end - k_start;
    if (nkeys == 0) {
        r.plan.kernel = G4A_KERNEL_NONE;  // every row sees no key: zero output
        return G4A_OK;
    }
    if (!r.fast_shape) {
        if (a->Dh > 1024 || a->Dv > 1024)
            return fail(ctx, G4A_E_UNSUPPORTED, "generic attention handles Dh, Dv <= 1024 (got %u, %u)", a->Dh, a->Dv);
        r.plan.kernel = G4A_KERNEL_GENERIC;
        r.plan.splits = 1;
        r.plan.keys_per_split = nkeys;
        return G4A_OK;
    }
    if (a->T >= PREFILL_MIN_T && group == 8 && r.q_contig && r.k_contig && a->attn_softcap == 0.0f &&
        a->S < (1u << 28)) {
        // query-tiled prefill: 8 queries x 8 heads per workgroup, keys in 16-key tiles
        r.plan.kernel = G4A_KERNEL_PREFILL;
        r.plan.splits = 1;
        r.plan.keys_per_split = nkeys;
        return G4A_OK;
    }
    if (group == 8 && r.k_contig && a->splits == 0) {
        // short context: 32-key splits with every load issued up front, when they
        // fit one workgroup per CU
        const uint64_t cus = uint64_t(std::max(ctx ? ctx->cu_count : 256, 1));
        const uint64_t splits = (nkeys + SHORT_KEYS - 1) / SHORT_KEYS;
        if ((ctx ? ctx->short_decode : true) && splits * a->T * a->Hkv <= cus) {
            r.plan.kernel = G4A_KERNEL_DECODE_SHORT;
            r.plan.splits = uint32_t(splits);
            r.plan.keys_per_split = SHORT_KEYS;
            r.plan.workspace_bytes = splits > 1 ? size_t(a->T) * a->Hq * splits * (a->Dh + 2) * sizeof(float) : 0;
            return G4A_OK;
        }
    }
    r.plan.kernel = G4A_KERNEL_DECODE;
    const uint32_t tiles = (nkeys + TILE - 1) / TILE;
    uint32_t splits;
    if (a->splits) {
        splits = std::min(a->splits, tiles);
    } else {
        // fill the GPU with one sequence: one 8-wave workgroup per CU (the LDS ring
        // allows one per CU), at least one 64-key tile each. Below 2 tiles per CU a
        // workgroup's second key-tile slot idles, which still beats idle CUs.
        const uint64_t target = uint64_t(std::max(ctx ? ctx->cu_count : 256, 1));
        const uint64_t per_query = std::max<uint64_t>(1, target / (uint64_t(a->T) * a->Hkv));
        splits = uint32_t(std::min<uint64_t>(per_query, tiles));
    }
    splits = std::min(std::max(splits, 1u), MAX_SPLITS);
    uint32_t kps = (nkeys + splits - 1) / splits;
    kps = (kps + TILE - 1) / TILE * TILE;
    splits = (nkeys + kps - 1) / kps;
    r.plan.splits = splits;
    r.plan.keys_per_split = kps;
    r.plan.workspace_bytes = splits > 1 ? size_t(a->T) * a->Hq * splits * (a->Dh + 2) * sizeof(float) : 0;
    return G4A_OK;
}

}  // namespace

extern "C" {

void g4a_default_options(g4a_options* o) {
    if (!o) return;
    *o = g4a_options{};
    o->size = sizeof(g4a_options);
    o->short_decode = 1;
    o->short_max_wgs = 4;
    o->batch_kernel = 0;
    o->batch_keys_per_split = 0;
    o->linear_i8 = -1;
    o->fuse_projection = 0;
}

int g4a_create(int device, const char* hsaco_path, g4a_ctx** out) {
    return g4a_create_with(device, hsaco_path, nullptr, out);
}

int g4a_create_with(int device, const char* hsaco_path, const g4a_options* opts, g4a_ctx** out) {
    if (!out) return fail(nullptr, G4A_E_ARG, "null out");
    *out = nullptr;
    g4a_options o;
    g4a_default_options(&o);
    if (opts) {
        if (opts->size != sizeof(g4a_options))
            return fail(nullptr, G4A_E_ARG, "g4a_options of %u bytes; this library's has %zu", opts->size,
                        sizeof(g4a_options));
        o = *opts;
        if ((o.short_decode != 0 && o.short_decode != 1) ||
            (o.short_max_wgs != 1 && o.short_max_wgs != 2 && o.short_max_wgs != 4) || o.batch_kernel < 0 ||
            o.batch_kernel > 2 || o.linear_i8 < -1 || o.linear_i8 > 1 ||
            (o.fuse_projection != 0 && o.fuse_projection != 1))
            return fail(nullptr, G4A_E_ARG, "g4a_options: an option is out of range");
    }
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n == 0) return fail(nullptr, G4A_E_HIP, "no HIP device (%s)", hipGetErrorString(e));
    if (device < 0 || device >= n) return fail(nullptr, G4A_E_ARG, "device %d out of range [0, %d)", device, n);
    g4a_ctx* ctx = new g4a_ctx();
    ctx->device = device;
    ctx->book = std::make_shared<g4a_graph_book>();
    ctx->book->ctx = ctx;
    auto bail = [&](int code) {
        g_create_error = ctx->err;
        g4a_destroy(ctx);
        return code;
    };
    if (hipSetDevice(device) != hipSuccess) {
        fail(ctx, G4A_E_HIP, "hipSetDevice(%d) failed", device);
        return bail(G4A_E_HIP);
    }
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess) {
        fail(ctx, G4A_E_HIP, "hipGetDeviceProperties failed");
        return bail(G4A_E_HIP);
    }
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        fail(ctx, G4A_E_UNSUPPORTED, "device %d is %s; this build targets gfx950 (MI355X)", device, prop.gcnArchName);
        return bail(G4A_E_UNSUPPORTED);
    }
    ctx->cu_count = prop.multiProcessorCount;
    ctx->short_decode = o.short_decode != 0;
    ctx->short_ds = o.short_max_wgs;
    ctx->batch_kernel = o.batch_kernel;
    ctx->batch_kps = o.batch_keys_per_split;
    ctx->linear_i8_use = o.linear_i8;
    ctx->fuse_projection = o.fuse_projection != 0;
    std::string path = hsaco_path ? std::string(hsaco_path) : default_hsaco_path();
    e = hipModuleLoad(&ctx->module, path.c_str());
    if (e != hipSuccess) {
        fail(ctx, G4A_E_MODULE, "hipModuleLoad(%s): %s", path.c_str(), hipGetErrorString(e));
        return bail(G4A_E_MODULE);
    }
    for (int d = 0; d < 2; ++d)
        for (int g = 0; g < 2; ++g)
            for (int kp = 0; kp < 2; ++kp) {
                char name[64];
                snprintf(name, sizeof name, "g4a_decode_d%d_g%d%s", d ? 512 : 256, g ? 8 : 4, kp ? "_kpos" : "");
                if (int rc = get_fn(ctx, &ctx->decode[d][g][kp], name)) return bail(rc);
            }
    if (int rc = get_fn(ctx, &ctx->decode_short[0], "g4a_decode_short_d256")) return bail(rc);
    if (int rc = get_fn(ctx, &ctx->decode_short[1], "g4a_decode_short_d512")) return bail(rc);
    if (int rc = get_fn(ctx, &ctx->decode_short2[0], "g4a_decode_short2_d256")) return bail(rc);
    if (int rc = get_fn(ctx, &ctx->decode_short2[1], "g4a_decode_short2_d512")) return bail(rc);
    if (int rc = get_fn(ctx, &ctx->decode_short4[0], "g4a_decode_short4_d256")) return bail(rc);
    if (int rc = get_fn(ctx, &ctx->decode_short4[1], "g4a_decode_short4_d512")) return bail(rc);
    if (int rc = get_fn(ctx, &ctx->decode_short2x[0], "g4a_decode_short2x_d256")) return bail(rc);
    if (int rc = get_fn(ctx, &ctx->decode_short2x[1], "g4a_decode_short2x_d512")) return bail(rc);
    if (int rc = get_fn(ctx, &ctx->decode_short4x[0], "g4a_decode_short4x_d256")) return bail(rc);
    if (int rc = get_fn(ctx, &ctx->decode_short4x[1], "g4a_decode_short4x_d512")) return bail(rc);
    if (int rc = get_fn(ctx, &ctx->decode_batch[0], "g4a_decode_short_batch_d256")) return bail(rc);
    if (int rc = get_fn(ctx, &ctx->decode_batch[1], "g4a_decode_short_batch_d512")) return bail(rc);
    if (int rc = get_fn(ctx, &ctx->decode_wave_batch[0], "g4a_decode_wave_batch_d256")) return bail(rc);
    if (int rc = get_fn(ctx, &ctx->decode_wave_batch[1], "g4a_decode_wave_batch_d512")) return bail(rc);
    if (int rc = get_fn(ctx, &ctx->decode_wave_batch_kpos[0], "g4a_decode_wave_batch_kpos_d256")) return bail(rc);
    if (int rc = get_fn(ctx, &ctx->decode_wave_batch_kpos[1], "g4a_decode_wave_batch_kpos_d512")) return bail(rc);
    if (int rc = get_fn(ctx, &ctx->combine_batch[0], "g4a_combine_batch_d256")) return bail(rc);
    if (int rc = get_fn(ctx, &ctx->combine_batch[1], "g4a_combine_batch_d512")) return bail(rc);
    if (int rc = get_fn(ctx, &ctx->combine_rows[0], "g4a_combine_rows_d256")) return bail(rc);
    if (int rc = get_fn(ctx, &ctx->combine_rows[1], "g4a_combine_rows_d512")) return bail(rc);
    if (int rc = get_fn(ctx, &ctx->combine_rows_batch[0], "g4a_combine_rows_batch_d256")) return bail(rc);
    if (int rc = get_fn(ctx, &ctx->combine_rows_batch[1], "g4a_combine_rows_batch_d512")) return bail(rc);
    if (int rc = get_fn(ctx, &ctx->combine[0], "g4a_combine_d256")) return bail(rc);
    if (int rc = get_fn(ctx, &ctx->combine[1], "g4a_combine_d512")) return bail(rc);
    if (int rc = get_fn(ctx, &ctx->generic, "g4a_generic_attention")) return bail(rc);
    if (int rc = get_fn(ctx, &ctx->prefill[0], "g4a_prefill2_d256")) return bail(rc);
    if (int rc = get_fn(ctx, &ctx->prefill[1], "g4a_prefill2_d512")) return bail(rc);
    if (int rc = get_fn(ctx, &ctx->prefill_merge, "g4a_prefill_merge_d512")) return bail(rc);
    if (int rc = get_fn(ctx, &ctx->split_kv, "g4a_split_kv")) return bail(rc);
    if (int rc = get_fn(ctx, &ctx->norm_rope, "g4a_norm_rope")) return bail(rc);
    if (int rc = get_fn(ctx, &ctx->norm_rope_short, "g4a_norm_rope_short")) return bail(rc);
    {
        static const int bits[3] = {2, 4, 8};
        static const int mt_ru[3][2] = {{1, 2}, {1, 8}, {4, 4}};
        for (int b = 0; b < 3; ++b)
            for (int v = 0; v < 3; ++v)
                for (int m = 0; m < 3; ++m) {
                    char name[64];
                    snprintf(name, sizeof name, "g4a_linear_q_b%d_m%d_r%d_mode%d", bits[b], mt_ru[v][0], mt_ru[v][1], m);
                    if (int rc = get_fn(ctx, &ctx->linear_words[b][v][m], name)) return bail(rc);
                }
        for (int m = 0; m < 3; ++m) {
            char name[64];
            for (int v = 0; v < 2; ++v) {
                snprintf(name, sizeof name, "g4a_linear_q_b2_m1_r%d_h_mode%d", v ? 4 : 1, m);
                if (int rc = get_fn(ctx, &ctx->linear_half[v][m], name)) return bail(rc);
            }
            snprintf(name, sizeof name, "g4a_linear_q_elem_mode%d", m);
            if (int rc = get_fn(ctx, &ctx->linear_elem[m], name)) return bail(rc);
            for (int b = 0; b < 3; ++b)
                for (int t = 0; t < 2; ++t) {
                    snprintf(name, sizeof name, "g4a_linear_q_mfma_b%d_n%d_mode%d", bits[b], t ? 128 : 64, m);
                    if (int rc = get_fn(ctx, &ctx->linear_mfma[b][t][m], name)) return bail(rc);
                }
        }
        for (int b = 0; b < 3; ++b)
            for (int m = 0; m < 2; ++m) {
                char name[64];
                snprintf(name, sizeof name, "g4a_linear_q_i8_b%d_m%d", bits[b], m + 1);
                if (int rc = get_fn(ctx, &ctx->linear_i8[b][m], name)) return bail(rc);
            }
        for (int b = 0; b < 3; ++b) {
            char name[64];
            snprintf(name, sizeof name, "g4a_linear_q_b%d_m1_r2_mode3", bits[b]);
            if (int rc = get_fn(ctx, &ctx->linear_fused[b], name)) return bail(rc);
        }
        if (int rc = get_fn(ctx, &ctx->embed_q, "g4a_embed_rows_q")) return bail(rc);
        static const char* f32_words[3] = {"g4a_linear_q_b32_m1_r2_mode0", "g4a_linear_q_b32_m1_r8_mode0",
                                           "g4a_linear_q_b32_m4_r4_mode0"};
        for (int v = 0; v < 3; ++v)
            if (int rc = get_fn(ctx, &ctx->linear_f32_words[v], f32_words[v])) return bail(rc);
        if (int rc = get_fn(ctx, &ctx->linear_f32_elem, "g4a_linear_f32_elem")) return bail(rc);
        if (int rc = get_fn(ctx, &ctx->ew, "g4a_ew")) return bail(rc);
        if (int rc = get_fn(ctx, &ctx->u32_add, "g4a_u32_add")) return bail(rc);
        if (int rc = get_fn(ctx, &ctx->slice_cols, "g4a_slice_cols")) return bail(rc);
        if (int rc = get_fn(ctx, &ctx->rms_rows, "g4a_rms_rows")) return bail(rc);
        if (int rc = get_fn(ctx, &ctx->embed_f32, "g4a_embed_rows_f32")) return bail(rc);
    }
    if (hipMalloc(reinterpret_cast<void**>(&ctx->dummy), 4096) != hipSuccess ||
        hipMemset(ctx->dummy, 0, 4096) != hipSuccess) {
        fail(ctx, G4A_E_NOMEM, "dummy buffer allocation failed");
        return bail(G4A_E_NOMEM);
    }

    if (hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreate(&ctx->ev_start) != hipSuccess || hipEventCreate(&ctx->ev_stop) != hipSuccess ||
        hipEventCreateWithFlags(&ctx->ev_staging, hipEventDisableTiming) != hipSuccess) {
        fail(ctx, G4A_E_HIP, "stream/event creation failed");
        return bail(G4A_E_HIP);
    }
    *out = ctx;
    return G4A_OK;
}

void g4a_destroy(g4a_ctx* ctx) {
    if (!ctx) return;
    if (ctx->stream) hipStreamSynchronize(ctx->stream);
    for (hipEvent_t ev : ctx->kev) hipEventDestroy(ev);
    if (ctx->workspace) hipFree(ctx->workspace);
    if (ctx->book) {
        // graphs that outlive the context can no longer be launched (g4a_graph_launch
        // takes the context); they only need destroying
        for (void* p : ctx->book->retired) hipFree(p);
        ctx->book->retired.clear();
        ctx->book->ctx = nullptr;
    }
    if (ctx->dummy) hipFree(ctx->dummy);
    if (ctx->pos_dev) hipFree(ctx->pos_dev);
    for (auto& ft : ctx->freq_tables) hipFree(ft.dev);
    for (auto& st : ctx->sc_tables) hipFree(st.dev);
    for (void* p : ctx->sc_retired) hipFree(p);
    if (ctx->pos_host) hipHostFree(ctx->pos_host);
    if (ctx->ev_start) hipEventDestroy(ctx->ev_start);
    if (ctx->ev_stop) hipEventDestroy(ctx->ev_stop);
    if (ctx->ev_staging) hipEventDestroy(ctx->ev_staging);
    if (ctx->stream) hipStreamDestroy(ctx->stream);
    if (ctx->module) hipModuleUnload(ctx->module);
    delete ctx;
}

const char* g4a_last_error(const g4a_ctx* ctx) { return ctx ? ctx->err.c_str() : g_create_error.c_str(); }

int g4a_malloc(g4a_ctx* ctx, size_t bytes, void** dptr) {
    if (!ctx || !dptr) return fail(ctx, G4A_E_ARG, "null ctx/dptr");
    hipError_t e = hipMalloc(dptr, std::max<size_t>(bytes, 16));
    if (e != hipSuccess) return fail(ctx, G4A_E_NOMEM, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
    return G4A_OK;
}

int g4a_free(g4a_ctx* ctx, void* dptr) {
    if (!ctx) return fail(ctx, G4A_E_ARG, "null ctx");
    if (dptr) HIP_TRY(ctx, hipFree(dptr));
    return G4A_OK;
}

namespace {
int refuse_in_capture(g4a_ctx* ctx, const char* what) {
    return ctx->capturing ? fail(ctx, G4A_E_ARG, "%s cannot be captured in a graph", what) : G4A_OK;
}
}  // namespace

int g4a_h2d(g4a_ctx* ctx, void* dst, const void* src, size_t bytes) {
    if (!ctx || (bytes && (!dst || !src))) return fail(ctx, G4A_E_ARG, "null pointer");
    if (int rc = refuse_in_capture(ctx, "g4a_h2d (a host copy)")) return rc;
    if (bytes) HIP_TRY(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
    // the caller may reuse `src` on return: make the copy complete
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    return G4A_OK;
}

int g4a_d2h(g4a_ctx* ctx, void* dst, const void* src, size_t bytes) {
    if (!ctx || (bytes && (!dst || !src))) return fail(ctx, G4A_E_ARG, "null pointer");
    if (int rc = refuse_in_capture(ctx, "g4a_d2h (a host copy)")) return rc;
    if (bytes) HIP_TRY(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    return G4A_OK;
}

int g4a_d2d(g4a_ctx* ctx, void* dst, const void* src, size_t bytes) {
    if (!ctx || (bytes && (!dst || !src))) return fail(ctx, G4A_E_ARG, "null pointer");
    if (bytes) HIP_TRY(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, ctx->stream));
    return G4A_OK;
}

int g4a_zero(g4a_ctx* ctx, void* dst, size_t bytes) {
    if (!ctx || (bytes && !dst)) return fail(ctx, G4A_E_ARG, "null pointer");
    if (int rc = refuse_in_capture(ctx, "g4a_zero (a memset)")) return rc;
    if (bytes) HIP_TRY(ctx, hipMemsetAsync(dst, 0, bytes, ctx->stream));
    return G4A_OK;
}

int g4a_sync(g4a_ctx* ctx) {
    if (!ctx) return fail(ctx, G4A_E_ARG, "null ctx");
    if (int rc = refuse_in_capture(ctx, "g4a_sync")) return rc;
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    return G4A_OK;
}

int g4a_stream(g4a_ctx* ctx, void** stream) {
    if (!ctx) return fail(ctx, G4A_E_ARG, "null ctx");
    if (!stream) return fail(ctx, G4A_E_ARG, "null stream out");
    *stream = static_cast<void*>(ctx->stream);
    return G4A_OK;
}

int g4a_attention_plan(g4a_ctx* ctx, const g4a_attn_args* a, g4a_attn_plan* plan) {
    // a query: its failures do not discard an open graph capture
    struct Query {
        g4a_ctx* c;
        explicit Query(g4a_ctx* x) : c(x) { if (c) ++c->query_depth; }
        ~Query() { if (c) --c->query_depth; }
    } q(ctx);
    if (!plan) return fail(ctx, G4A_E_ARG, "null plan");
    Analysis an;
    if (int rc = analyse(ctx, a, &an, false)) return rc;
    *plan = an.plan;
    return G4A_OK;
}

}  // extern "C"

namespace {

// Device memory for a call's split partials or pre-split K/V: the context's
// workspace, grown on demand, or with `noalloc` the library's static scratch
// array (g4a_attention_noalloc), which never grows.
int call_workspace(g4a_ctx* ctx, size_t bytes, bool noalloc, void** ws) {
    if (noalloc) {
        if (bytes > NOALLOC_SCRATCH_BYTES || !ctx->scratch)
            return fail(ctx, G4A_E_UNSUPPORTED, "the call needs %zu bytes of scratch; the static array holds %zu",
                        bytes, ctx->scratch ? NOALLOC_SCRATCH_BYTES : size_t(0));
        *ws = ctx->scratch;
        return G4A_OK;
    }
    if (int rc = ensure_workspace(ctx, bytes)) return rc;
    *ws = ctx->workspace;
    return G4A_OK;
}

// Explicit positions that are not contiguous go to the device through buffers
// the library allocates, which g4a_attention_noalloc never does.
int stage_positions(g4a_ctx* ctx, const g4a_attn_args* a, const Analysis& an, bool noalloc, const uint32_t** qd,
                    const uint32_t** kd) {
    *qd = *kd = nullptr;
    if (an.q_contig && an.k_contig) return G4A_OK;
    if (noalloc)
        return fail(ctx, G4A_E_UNSUPPORTED, "explicit non-contiguous positions are staged through buffers the "
                    "library allocates; g4a_attention_noalloc takes contiguous positions only");
    return upload_positions(ctx, an.q_contig ? nullptr : a->q_pos, an.q_contig ? 0 : a->T,
                            an.k_contig ? nullptr : a->k_pos, an.k_contig ? 0 : a->S, qd, kd);
}

// Enqueues an analysed attention call. With combine == false a multi-split
// decode leaves its partials in the workspace (the caller merges them). With
// noalloc the call allocates nothing: its scratch is the static array.
int attention_run(g4a_ctx* ctx, const g4a_attn_args* a, const Analysis& an, bool combine, bool noalloc = false,
                  const uint32_t* dpos = nullptr) {
    const g4a_attn_plan& pl = an.plan;
    if (a->T == 0) return G4A_OK;
    const size_t out_bytes = size_t(a->T) * a->Hq * a->Dv * sizeof(float);
    if (pl.kernel == G4A_KERNEL_NONE) {
        // no visible key: zero rows, written by a kernel (a memset node in a
        // captured graph is not replayed reliably)
        const size_t n = out_bytes / sizeof(float);
        G4aEwParams p{a->out, nullptr, nullptr, a->out, n, 0.0f, uint32_t(G4A_EW_FILL)};
        const uint32_t blocks = uint32_t(std::min<size_t>((n + 255) / 256, 4096));
        return launch(ctx, ctx->ew, dim3(blocks, 1, 1), dim3(256, 1, 1), p, "zero rows");
    }
    const uint32_t group = a->Hq / a->Hkv;
    const uint32_t q_pos0 = a->q_pos ? a->q_pos[0] : a->q_pos0;
    const uint32_t k_pos0 = a->k_pos ? (a->S ? a->k_pos[0] : 0) : a->k_pos0;
    if (pl.kernel == G4A_KERNEL_GENERIC) {
        // contiguous positions travel as q_pos0 / k_pos0; only the others are staged
        const uint32_t *qd = nullptr, *kd = nullptr;
        if (int rc = stage_positions(ctx, a, an, noalloc, &qd, &kd)) return rc;
        G4aGenericParams gp{a->q, a->k, a->v, a->out, qd, kd, q_pos0, k_pos0, a->T, a->S, a->Hq, a->Hkv, a->Dh,
                            a->Dv, pl.k_start, pl.k_end, a->kv_ring_cap, a->sliding_window, a->scale,
                            a->attn_softcap};
        return launch(ctx, ctx->generic, dim3(a->Hq, a->T, 1), dim3(64, 1, 1), gp, "generic attention", true);
    }
    if (pl.kernel == G4A_KERNEL_PREFILL) {
        G4aPrefillParams pp{};
        pp.q = a->q;
        pp.k = a->k;
        pp.v = a->v;
        pp.out = a->out;
        pp.T = a->T;
        pp.S = a->S;
        pp.Hq = a->Hq;
        pp.Hkv = a->Hkv;
        pp.q_pos0 = q_pos0;
        pp.k_pos0 = k_pos0;
        pp.ring_cap = a->kv_ring_cap;
        pp.window = a->sliding_window;
        pp.scale = a->scale;
        // rescoring band: the keys left with their estimated score (N of them in a row at
        // most) carry a weight share of at most N e^-tau / (1 + N e^-tau)
        {
            uint32_t n_row = pl.k_end - pl.k_start;
            if (a->sliding_window) n_row = std::min(n_row, a->sliding_window);
            pp.tau = std::max(PREFILL_TAU_MIN, logf(float(std::max(n_row, 1u))) + PREFILL_TAU_LOGN);
        }
        // 8-wave workgroups over 8 queries; scores estimated from fp16 hi/lo splits of K
        // (each 16-key tile scaled by a power of two), P.V from fp16 hi/lo splits of V,
        // both made by a pre-pass into the workspace.
        // head_dim 256: two waves per 16-row block take the even / odd key tiles;
        // 512: two waves per 16-row block split the head dim
        const bool d512 = a->Dh == 512;
        {
            // keys [k_start, k_end) widened to multiples of 16 (the kernel's tile grid);
            // workspace: the V range flag (first 256 bytes), then the K and V splits,
            // the K rows' scale factors, then (head_dim 512) the partials of the split
            // query blocks
            const uint32_t k0 = pl.k_start & ~15u, nkeys = ((pl.k_end + 15u) & ~15u) - k0;
            const size_t half = size_t(nkeys) * a->Hkv * a->Dh * sizeof(float);
            const size_t kscale_bytes = size_t(a->Hkv) * (nkeys / 16) * sizeof(float);
            if (d512) pp.nbig = prefill_split_blocks(a, pp.q_pos0, pp.k_pos0);
            // a split block's partial: 8 waves x (O of 16 rows x 256 dims, then l and m of the rows)
            const size_t part_bytes = size_t(pp.nbig) * a->Hkv * 2 * 8 * (4 * 16 * 64 + 32) * sizeof(float);
            const size_t part_off = (256 + 2 * half + kscale_bytes + 255) & ~size_t(255);
            void* wsp = nullptr;
            if (int rc = call_workspace(ctx, part_off + part_bytes, noalloc, &wsp)) return rc;
            char* const ws = static_cast<char*>(wsp);
            G4aSplitParams sp{};
            sp.k = a->k;
            sp.v = a->v;
            sp.kout = reinterpret_cast<float*>(ws + 256);
            sp.vout = reinterpret_cast<float*>(ws + 256 + half);
            sp.kscale = reinterpret_cast<float*>(ws + 256 + 2 * half);
            sp.vflag = reinterpret_cast<uint32_t*>(ws);
            sp.k0 = k0;
            sp.nkeys = nkeys;
            sp.S = a->S;
            sp.Hkv = a->Hkv;
            sp.Dh = a->Dh;
            sp.ring_cap = a->kv_ring_cap;
            sp.epoch = next_split_epoch();
            sp.vis_lo = pl.k_start;
            sp.vis_hi = pl.k_end;
            // one block per (16-key tile, kv head) for K, then one thread per 4 dims of a V key quad
            const uint64_t vthreads = uint64_t(nkeys / 4) * a->Hkv * (a->Dh / 64) * 16;
            const uint64_t blocks = uint64_t(nkeys / 16) * a->Hkv + (vthreads + 255) / 256;
            if (int rc = launch(ctx, ctx->split_kv, dim3(uint32_t(blocks), 1, 1), dim3(256, 1, 1), sp,
                                "split K/V"))
                return rc;
            pp.ksplit = sp.kout;
            pp.kscale = sp.kscale;
            pp.vsplit = sp.vout;
            pp.vflag = sp.vflag;
            pp.split0 = k0;
            pp.split_n = nkeys;
            pp.epoch = sp.epoch;
            pp.part = reinterpret_cast<float*>(ws + part_off);
        }
        if (int rc = launch(ctx, ctx->prefill[d512 ? 1 : 0], dim3((a->T + 7) / 8 + pp.nbig, a->Hkv, 1),
                            dim3(512, 1, 1), pp, "prefill", true))
            return rc;
        if (pp.nbig == 0) return G4A_OK;
        // one 4-wave workgroup per (split block, dim half, kv head)
        return launch(ctx, ctx->prefill_merge, dim3(2 * pp.nbig, a->Hkv, 1), dim3(256, 1, 1), pp, "prefill merge");
    }
    // split-K flash-decode (+ combine)
    const uint32_t *qd = nullptr, *kd = nullptr;
    if (int rc = stage_positions(ctx, a, an, noalloc, &qd, &kd)) return rc;
    void* part = nullptr;
    if (pl.splits > 1)
        if (int rc = call_workspace(ctx, pl.workspace_bytes, noalloc, &part)) return rc;
    G4aDecodeParams dp{};
    dp.q = a->q;
    dp.k = a->k;
    dp.v = a->v;
    dp.out = a->out;
    dp.part = static_cast<float*>(part);
    dp.dummy = ctx->dummy;
    dp.q_pos = qd;
    dp.k_pos = kd;
    dp.q_pos0 = q_pos0;
    dp.k_pos0 = k_pos0;
    dp.T = a->T;
    dp.Hq = a->Hq;
    dp.Hkv = a->Hkv;
    dp.k_start = pl.k_start;
    dp.k_end = pl.k_end;
    dp.keys_per_split = pl.keys_per_split;
    dp.nsplit = pl.splits;
    dp.ring_cap = a->kv_ring_cap;
    dp.window = a->sliding_window;
    dp.scale = a->scale;
    dp.softcap = a->attn_softcap;
    dp.dpos = dpos;
    const int d512 = a->Dh == 512 ? 1 : 0;
    const int g8 = group == 8 ? 1 : 0;
    if (pl.kernel == G4A_KERNEL_DECODE_SHORT) {
        // up to four workgroups per split (each a part of the output dims) while they
        // fit the CUs: a shorter P.V and merge per workgroup, bit-identical results
        const uint64_t wg = uint64_t(pl.splits) * a->T * a->Hkv, cus = uint64_t(std::max(ctx->cu_count, 1));
        const uint32_t ds = ctx->short_ds >= 4 && 4 * wg <= cus ? 4u : ctx->short_ds >= 2 && 2 * wg <= cus ? 2u : 1u;
        // the ds workgroups of a split on one XCD (one L2 fill of its K rows for all
        // of them) when the split count is a multiple of 8, which the mapping needs
        const bool grouped = ds > 1 && pl.splits % 8 == 0;
        hipFunction_t fn = ds == 4 ? (grouped ? ctx->decode_short4x[d512] : ctx->decode_short4[d512])
                           : ds == 2 ? (grouped ? ctx->decode_short2x[d512] : ctx->decode_short2[d512])
                                     : ctx->decode_short[d512];
        if (int rc = launch(ctx, fn, dim3(pl.splits * ds, a->T, a->Hkv), dim3(256, 1, 1), dp, "short decode", true))
            return rc;
    } else if (int rc = launch(ctx, ctx->decode[d512][g8][kd ? 1 : 0], dim3(pl.splits, a->T, a->Hkv),
                               dim3(512, 1, 1), dp, "decode", true)) {
        return rc;
    }
    if (pl.splits > 1 && combine) {
        G4aCombineParams cp{dp.part, a->out, a->T, a->Hq, pl.splits, a->Dh};
        if (pl.splits <= COMBINE_ROW_SPLITS) {
            if (int rc = launch(ctx, ctx->combine_rows[d512], dim3(a->Hq, a->T, 1), dim3(256, 1, 1), cp, "combine"))
                return rc;
        } else if (int rc = launch(ctx, ctx->combine[d512], dim3(a->Dh / kCombineDims, a->Hq, a->T),
                                   dim3(kCombineThreads, 1, 1), cp, "combine")) {
            return rc;
        }
    }
    return G4A_OK;
}

}  // namespace

extern "C" {

int g4a_attention(g4a_ctx* ctx, const g4a_attn_args* a) {
    if (!ctx) return fail(ctx, G4A_E_ARG, "null ctx");
    Analysis an;
    if (int rc = analyse(ctx, a, &an, true)) return rc;
    return attention_run(ctx, a, an, true);
}

int g4a_attention_noalloc(g4a_ctx* ctx, const g4a_attn_args* a) {
    if (!ctx) return fail(ctx, G4A_E_ARG, "null ctx");
    // the static scratch array is looked up (and so loaded onto the GPU) by the first
    // no-alloc call on a device, not by g4a_create: a process that never calls this
    // entry point does not hold it
    if (!ctx->scratch) {
        HIP_TRY(ctx, hipSetDevice(ctx->device));
        if (int rc = scratch_setup(ctx)) return rc;
    }
    Analysis an;
    if (int rc = analyse(ctx, a, &an, true)) return rc;
    return attention_run(ctx, a, an, true, /*noalloc=*/true);
}

int g4a_attention_devpos(g4a_ctx* ctx, const g4a_attn_args* a, const uint32_t* pos) {
    if (!ctx) return fail(ctx, G4A_E_ARG, "null ctx");
    if (!a || !pos) return fail(ctx, G4A_E_ARG, "null args / device position");
    if (a->T != 1) return fail(ctx, G4A_E_UNSUPPORTED, "a device-position decode step has one query (T = %u)", a->T);
    if (a->q_pos || a->k_pos)
        return fail(ctx, G4A_E_ARG, "a device-position decode step takes contiguous positions (q_pos, k_pos NULL)");
    if (a->S == 0) return fail(ctx, G4A_E_ARG, "S (the most keys a replay sees) must be at least 1");
    if (uint64_t(a->k_pos0) + a->S - 1 >= (uint64_t(1) << 32))
        return fail(ctx, G4A_E_ARG, "k_pos0 %u + S %u passes 2^32", a->k_pos0, a->S);
    // planned for the largest key range: the query at the last of the S keys
    g4a_attn_args m = *a;
    m.q_pos0 = a->k_pos0 + a->S - 1;
    Analysis an;
    if (int rc = analyse(ctx, &m, &an, true)) return rc;
    if (an.plan.kernel != G4A_KERNEL_DECODE && an.plan.kernel != G4A_KERNEL_DECODE_SHORT)
        return fail(ctx, G4A_E_UNSUPPORTED, "a device-position decode step runs on the decode kernels (groups of 4 "
                    "or 8 heads, head_dim 256 or 512); this shape plans kernel %u", an.plan.kernel);
    return attention_run(ctx, &m, an, true, false, pos);
}

int g4a_u32_add(g4a_ctx* ctx, uint32_t* counters, uint32_t n, uint32_t inc) {
    if (!ctx) return fail(ctx, G4A_E_ARG, "null ctx");
    if (n == 0) return G4A_OK;
    if (!counters) return fail(ctx, G4A_E_ARG, "null counters");
    G4aCounterParams p{counters, n, inc};
    return launch(ctx, ctx->u32_add, dim3((n + 255) / 256, 1, 1), dim3(256, 1, 1), p, "counter add");
}

int g4a_attention_batch(g4a_ctx* ctx, const g4a_attn_args* args, uint32_t n) {
    if (!ctx) return fail(ctx, G4A_E_ARG, "null ctx");
    if (n && !args) return fail(ctx, G4A_E_ARG, "null args");
    for (uint32_t i = 0; i < n; ++i)
        if (int rc = g4a_attention(ctx, &args[i])) return rc;
    return G4A_OK;
}

int g4a_attention_decode_batch(g4a_ctx* ctx, const g4a_attn_args* args, uint32_t n, uint32_t* n_batched) {
    if (!ctx) return fail(ctx, G4A_E_ARG, "null ctx");
    if (n_batched) *n_batched = 0;
    if (n == 0) return G4A_OK;
    if (!args) return fail(ctx, G4A_E_ARG, "null args");
    // every call is checked before anything is enqueued
    std::vector<Analysis> an(n);
    for (uint32_t i = 0; i < n; ++i)
        if (int rc = analyse(ctx, &args[i], &an[i], true)) return fail(ctx, rc, "call %u: %s", i, ctx->err.c_str());
    // the batched calls: single-query decode steps of the first such call's
    // shape; those with explicit, non-contiguous key positions (staged from host
    // memory, so not while a graph is captured) go to launches of their own
    const g4a_attn_args* ref = nullptr;
    std::vector<uint32_t> batch, batch_kpos;
    for (uint32_t i = 0; i < n; ++i) {
        const g4a_attn_args& a = args[i];
        const Analysis& r = an[i];
        if (a.T != 1 || !r.fast_shape || a.splits != 0 || a.Hq != 8 * a.Hkv) continue;
        if (!r.k_contig && ctx->capturing) continue;
        if (r.plan.kernel != G4A_KERNEL_DECODE && r.plan.kernel != G4A_KERNEL_DECODE_SHORT) continue;
        if (r.plan.k_end - r.plan.k_start > BATCH_MAX_KEYS) continue;
        if (!ref) ref = &a;
        if (a.Hq != ref->Hq || a.Hkv != ref->Hkv || a.Dh != ref->Dh || a.sliding_window != ref->sliding_window ||
            a.kv_ring_cap != ref->kv_ring_cap || memcmp(&a.scale, &ref->scale, sizeof(float)) != 0 ||
            memcmp(&a.attn_softcap, &ref->attn_softcap, sizeof(float)) != 0)
            continue;
        (r.k_contig ? batch : batch_kpos).push_back(i);
    }
    // the visible keys' positions of the explicit-position calls, staged in one upload
    std::vector<uint32_t> kpos_host, kpos_off(batch_kpos.size());
    for (size_t j = 0; j < batch_kpos.size(); ++j) {
        const g4a_attn_args& a = args[batch_kpos[j]];
        const g4a_attn_plan& pl = an[batch_kpos[j]].plan;
        if (kpos_host.size() + (pl.k_end - pl.k_start) >= G4A_NO_KPOS)
            return fail(ctx, G4A_E_SHAPE, "batched decode key positions exceed 2^32 entries");
        kpos_off[j] = uint32_t(kpos_host.size());
        kpos_host.insert(kpos_host.end(), a.k_pos + pl.k_start, a.k_pos + pl.k_end);
    }
    const uint32_t* kpos_dev = nullptr;
    if (!kpos_host.empty())
        if (int rc = upload_positions(ctx, kpos_host.data(), kpos_host.size(), nullptr, 0, &kpos_dev, nullptr))
            return rc;
    const uint32_t n_contig = uint32_t(batch.size());
    batch.insert(batch.end(), batch_kpos.begin(), batch_kpos.end());
    const uint64_t cus = uint64_t(std::max(ctx->cu_count, 1));
    // Launches of up to G4A_BATCH_SEQ sequences, the contiguous-position calls
    // (batch[0 .. n_contig)) apart from the explicit-position ones. A launch
    // whose 32-key splits fit one short-kernel workgroup per CU runs the short
    // kernel; otherwise (and always for explicit positions) the streaming kernel
    // with 64-key-multiple splits sized for one 8-wave workgroup per CU over the
    // launch's keys.
    struct Launch {
        uint32_t first, count, kps, max_split;
        bool wave, rows, wide;  // streaming kernel; combines of <= COMBINE_ROW_SPLITS / more splits
        bool kpos;              // explicit key positions
        size_t part;  // floats
    };
    std::vector<Launch> launches;
    size_t part_floats = 0;
    for (uint32_t c0 = 0; c0 < batch.size();) {
        const uint32_t c1 = c0 < n_contig ? n_contig : uint32_t(batch.size());
        Launch L{c0, std::min<uint32_t>(G4A_BATCH_SEQ, c1 - c0), SHORT_KEYS, 0, false, false, false, c0 >= n_contig,
                 part_floats};
        c0 += L.count;
        uint64_t short_wgs = 0, keys = 0;
        uint32_t max_keys = 0;
        for (uint32_t j = L.first; j < L.first + L.count; ++j) {
            const uint32_t nk = an[batch[j]].plan.k_end - an[batch[j]].plan.k_start;
            short_wgs += (nk + SHORT_KEYS - 1) / SHORT_KEYS;
            keys += nk;
            max_keys = std::max(max_keys, nk);
        }
        if (L.kpos || ctx->batch_kernel == 2 || (ctx->batch_kernel == 0 && short_wgs * ref->Hkv > cus)) {
            L.wave = true;
            uint64_t kps = ctx->batch_kps ? ctx->batch_kps : (keys * ref->Hkv + cus - 1) / cus;
            kps = std::max<uint64_t>(kps, (max_keys + MAX_SPLITS - 1) / MAX_SPLITS);
            L.kps = uint32_t((std::max<uint64_t>(kps, 1) + TILE - 1) / TILE * TILE);
        }
        for (uint32_t j = L.first; j < L.first + L.count; ++j) {
            const uint32_t nk = an[batch[j]].plan.k_end - an[batch[j]].plan.k_start;
            const uint32_t ns = (nk + L.kps - 1) / L.kps;
            L.max_split = std::max(L.max_split, ns);
            if (ns > 1) {
                (ns <= COMBINE_ROW_SPLITS ? L.rows : L.wide) = true;
                part_floats += (size_t(ref->Hq) * ns * (ref->Dh + 2) + 63) & ~size_t(63);
            }
        }
        launches.push_back(L);
    }
    if (part_floats > 0xFFFFFFFFull) return fail(ctx, G4A_E_SHAPE, "batched decode partials exceed 2^32 floats");
    if (part_floats)
        if (int rc = ensure_workspace(ctx, part_floats * sizeof(float))) return rc;
    const int d512 = ref && ref->Dh == 512 ? 1 : 0;
    for (const Launch& L : launches) {
        G4aBatchParams bp{};
        bp.part = static_cast<float*>(ctx->workspace);
        bp.dummy = ctx->dummy;
        bp.Hq = ref->Hq;
        bp.Hkv = ref->Hkv;
        bp.keys_per_split = L.kps;
        bp.ring_cap = ref->kv_ring_cap;
        bp.window = ref->sliding_window;
        bp.scale = ref->scale;
        bp.softcap = ref->attn_softcap;
        bp.kpos = kpos_dev;
        size_t off = L.part;
        for (uint32_t j = 0; j < L.count; ++j) {
            const g4a_attn_args& a = args[batch[L.first + j]];
            const g4a_attn_plan& pl = an[batch[L.first + j]].plan;
            G4aSeqDesc& d = bp.seq[j];
            d.q = a.q;
            d.k = a.k;
            d.v = a.v;
            d.out = a.out;
            d.k_start = pl.k_start;
            d.k_end = pl.k_end;
            if (L.kpos) {
                // explicit positions: absolute, key j's at kpos[kpos_off - k_start + j]
                d.q_pos = a.q_pos ? a.q_pos[0] : a.q_pos0;
                d.kpos = kpos_off[L.first + j - n_contig];
            } else {
                // key j sits at position k_pos0 + j; the kernel takes positions relative to k_pos0
                // (the visible keys end at or before the query, so q_pos >= k_pos0)
                d.q_pos = (a.q_pos ? a.q_pos[0] : a.q_pos0) - (a.k_pos ? a.k_pos[0] : a.k_pos0);
                d.kpos = G4A_NO_KPOS;
            }
            const uint32_t ns = (pl.k_end - pl.k_start + L.kps - 1) / L.kps;
            d.part = uint32_t(ns > 1 ? off : 0);
            if (ns > 1) off += (size_t(ref->Hq) * ns * (ref->Dh + 2) + 63) & ~size_t(63);
        }
        hipFunction_t f = L.kpos ? ctx->decode_wave_batch_kpos[d512]
                          : L.wave ? ctx->decode_wave_batch[d512] : ctx->decode_batch[d512];
        if (int rc = launch(ctx, f, dim3(L.max_split, L.count, bp.Hkv), dim3(L.wave ? 512 : 256, 1, 1), bp,
                            "batched decode", true))
            return rc;
        if (L.rows)
            if (int rc = launch(ctx, ctx->combine_rows_batch[d512], dim3(bp.Hq, L.count, 1), dim3(256, 1, 1), bp,
                                "batched combine", true))
                return rc;
        if (L.wide)
            if (int rc = launch(ctx, ctx->combine_batch[d512], dim3(ref->Dh / kCombineDims, bp.Hq, L.count),
                                dim3(kCombineThreads, 1, 1), bp, "batched combine", true))
                return rc;
    }
    // the rest, one call at a time
    std::vector<bool> in_batch(n, false);
    for (uint32_t i : batch) in_batch[i] = true;
    for (uint32_t i = 0; i < n; ++i)
        if (!in_batch[i])
            if (int rc = g4a_attention(ctx, &args[i])) return rc;
    if (n_batched) *n_batched = uint32_t(batch.size());
    return G4A_OK;
}

int g4a_kv_write(g4a_ctx* ctx, float* cache, uint32_t ring_cap, uint32_t row_elems, uint32_t dst_row, const float* src,
                 uint32_t n_rows) {
    if (!ctx) return fail(ctx, G4A_E_ARG, "null ctx");
    if (n_rows == 0) return G4A_OK;
    if (!cache || !src || row_elems == 0) return fail(ctx, G4A_E_ARG, "null cache/src or zero row size");
    const size_t row_bytes = size_t(row_elems) * sizeof(float);
    if (ring_cap == 0) {
        HIP_TRY(ctx, hipMemcpyAsync(cache + size_t(dst_row) * row_elems, src, n_rows * row_bytes,
                                    hipMemcpyDeviceToDevice, ctx->stream));
        return G4A_OK;
    }
    // only the last ring_cap rows survive
    uint32_t skip = n_rows > ring_cap ? n_rows - ring_cap : 0;
    uint64_t first = uint64_t(dst_row) + skip;
    uint32_t n = n_rows - skip;
    uint32_t slot = uint32_t(first % ring_cap);
    uint32_t n1 = std::min(n, ring_cap - slot);
    HIP_TRY(ctx, hipMemcpyAsync(cache + size_t(slot) * row_elems, src + size_t(skip) * row_elems, n1 * row_bytes,
                                hipMemcpyDeviceToDevice, ctx->stream));
    if (n1 < n)
        HIP_TRY(ctx, hipMemcpyAsync(cache, src + size_t(skip + n1) * row_elems, size_t(n - n1) * row_bytes,
                                    hipMemcpyDeviceToDevice, ctx->stream));
    return G4A_OK;
}

namespace {

// Device table of the RoPE frequencies freq[j] = theta^(-2j/rot), j < rot/2,
// computed with libm powf exactly as the reference computes them
// (rust/src/backend_cpu.rs:257: theta.powf(-(2.0 * j as f32) / rotary_dim as f32)).
int freq_table(g4a_ctx* ctx, float theta, uint32_t rot, const float** out) {
    for (auto& ft : ctx->freq_tables)
        if (ft.rot == rot && memcmp(&ft.theta, &theta, sizeof theta) == 0) {
            *out = ft.dev;
            return G4A_OK;
        }
    if (ctx->capturing)
        return fail(ctx, G4A_E_ARG, "a RoPE table (theta %g, rotary_dim %u) is built on first use, which a graph "
                    "capture cannot do: run the call once before capturing it", theta, rot);
    g4a_ctx::FreqTable ft{theta, rot, std::vector<float>(std::max<uint32_t>(rot / 2, 1)), nullptr};
    for (uint32_t j = 0; j < rot / 2; ++j) ft.host[j] = powf(theta, -(2.0f * (float)j) / (float)rot);
    if (hipMalloc(reinterpret_cast<void**>(&ft.dev), ft.host.size() * sizeof(float)) != hipSuccess)
        return fail(ctx, G4A_E_NOMEM, "RoPE frequency table");
    ctx->freq_tables.push_back(std::move(ft));
    auto& t = ctx->freq_tables.back();
    HIP_TRY(ctx, hipMemcpyAsync(t.dev, t.host.data(), t.host.size() * sizeof(float), hipMemcpyHostToDevice,
                                ctx->stream));
    *out = t.dev;
    return G4A_OK;
}

// Positions the (sinf, cosf) tables cover at most: 2^20 (1 GiB at rotary_dim 256).
// Later positions take the device's sincosf (within a few ulps of libm).
constexpr uint32_t SC_TABLE_MAX_ROWS = 1u << 20;

// Device table of (sinf(ang), cosf(ang)), ang = (float)pos * freq[j] in f32, for
// j < rot/2 and every position below `rows`: the reference's rope takes
// ang.sin_cos() (rust/src/backend_cpu.rs:255-259), i.e. libm's sinf and cosf,
// and the device's sincosf is an ulp away in places. Grown (at least doubled)
// when a call's largest position is past it; the host computes the new rows.
int sincos_table(g4a_ctx* ctx, float theta, uint32_t rot, const float* freq_host, uint32_t max_pos,
                 const float2** out, uint32_t* rows_out) {
    const uint32_t half = rot / 2;
    g4a_ctx::SinCosTable* tab = nullptr;
    for (auto& st : ctx->sc_tables)
        if (st.rot == rot && memcmp(&st.theta, &theta, sizeof theta) == 0) tab = &st;
    if (!tab) {
        ctx->sc_tables.push_back({theta, rot, 0u, nullptr});
        tab = &ctx->sc_tables.back();
    }
    const uint32_t want = std::min<uint64_t>(uint64_t(max_pos) + 1, SC_TABLE_MAX_ROWS);
    if (want > tab->rows) {
        if (ctx->capturing)
            return fail(ctx, G4A_E_ARG, "the RoPE sin/cos table (theta %g, rotary_dim %u) grows to position %u on "
                        "this call, which a graph capture cannot do: run the call once before capturing it",
                        theta, rot, max_pos);
        uint64_t rows = std::max<uint64_t>({uint64_t(want), 2 * uint64_t(tab->rows), 4096});
        rows = std::min<uint64_t>((rows + 4095) / 4096 * 4096, SC_TABLE_MAX_ROWS);
        float2* dev = nullptr;
        if (hipMalloc(reinterpret_cast<void**>(&dev), rows * half * sizeof(float2)) != hipSuccess)
            return fail(ctx, G4A_E_NOMEM, "RoPE sin/cos table of %llu positions", (unsigned long long)rows);
        std::vector<float2> host((rows - tab->rows) * half);
        for (uint64_t pos = tab->rows; pos < rows; ++pos)
            for (uint32_t j = 0; j < half; ++j) {
                const float ang = (float)pos * freq_host[j];
                host[(pos - tab->rows) * half + j] = make_float2(sinf(ang), cosf(ang));
            }
        if (tab->rows)
            HIP_TRY(ctx, hipMemcpyAsync(dev, tab->dev, size_t(tab->rows) * half * sizeof(float2),
                                        hipMemcpyDeviceToDevice, ctx->stream));
        HIP_TRY(ctx, hipMemcpyAsync(dev + size_t(tab->rows) * half, host.data(), host.size() * sizeof(float2),
                                    hipMemcpyHostToDevice, ctx->stream));
        // the copy from pageable memory must finish before `host` goes away
        HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
        if (tab->dev) ctx->sc_retired.push_back(tab->dev);
        tab->dev = dev;
        tab->rows = uint32_t(rows);
    }
    *out = tab->dev;
    *rows_out = tab->rows;
    return G4A_OK;
}

// One g4a_norm_rope launch over up to three row segments.
int norm_rope_launch(g4a_ctx* ctx, G4aNormRopeSeg* segs, uint32_t nseg, uint32_t T, uint32_t Dh, uint32_t rot,
                     const uint32_t* positions, uint32_t pos0, float theta, float eps, uint32_t cache_row,
                     uint32_t ring_cap, const uint32_t* dpos = nullptr, uint32_t dpos_max = 0) {
    if (Dh == 0 || Dh % 4 != 0 || Dh > 1024)
        return fail(ctx, G4A_E_UNSUPPORTED, "head_dim %u: RMSNorm/RoPE rows need head_dim %% 4 == 0 and <= 1024", Dh);
    if (rot % 2 != 0 || rot > Dh) return fail(ctx, G4A_E_ARG, "rotary_dim %u must be even and <= head_dim %u", rot, Dh);
    uint64_t rows = 0;
    for (uint32_t i = 0; i < nseg; ++i) {
        if (!segs[i].x || !segs[i].y) return fail(ctx, G4A_E_ARG, "null input/output rows");
        rows += uint64_t(T) * segs[i].heads;
    }
    if (rows == 0) return G4A_OK;
    if (rows >= (uint64_t(1) << 32)) return fail(ctx, G4A_E_SHAPE, "too many rows (%llu)", (unsigned long long)rows);
    G4aNormRopeParams p{};
    for (uint32_t i = 0; i < nseg; ++i) p.seg[i] = segs[i];
    p.nseg = nseg;
    p.total_rows = uint32_t(rows);
    p.T = T;
    p.Dh = Dh;
    p.rotary_dim = rot;
    p.eps = eps;
    p.cache_row = cache_row;
    p.ring_cap = ring_cap;
    p.pos0 = pos0;
    p.dpos = dpos;
    p.max_pos = dpos_max;
    bool needs_rope = false;
    for (uint32_t i = 0; i < nseg; ++i) {
        needs_rope |= segs[i].rope != 0;
        p.any_norm |= segs[i].norm;
    }
    if (needs_rope && rot) {
        if (int rc = freq_table(ctx, theta, rot, &p.freq)) return rc;
        uint32_t max_pos = dpos ? dpos_max : pos0 + (T ? T - 1 : 0);
        if (positions) {
            bool contig = true;
            max_pos = 0;
            for (uint32_t i = 0; i < T; ++i) {
                contig &= positions[i] == positions[0] + i;
                max_pos = std::max(max_pos, positions[i]);
            }
            if (contig) p.pos0 = positions[0];
            else if (int rc = upload_positions(ctx, positions, T, nullptr, 0, &p.pos, nullptr)) return rc;
        } else if (uint64_t(pos0) + T > (uint64_t(1) << 32)) {
            return fail(ctx, G4A_E_ARG, "positions pos0 %u + %u tokens pass 2^32", pos0, T);
        }
        const float* freq_host = nullptr;
        for (auto& ft : ctx->freq_tables)
            if (ft.rot == rot && memcmp(&ft.theta, &theta, sizeof theta) == 0) freq_host = ft.host.data();
        if (int rc = sincos_table(ctx, theta, rot, freq_host, max_pos, &p.sc, &p.sc_rows)) return rc;
    }
    const uint32_t blocks = uint32_t((rows + 3) / 4);
    // launches of at most one workgroup per CU (decode steps) wait on latency: their
    // kernel issues the norm weights and sin/cos together; longer ones keep registers
    // free for occupancy (the same rows either way)
    hipFunction_t fn = blocks <= uint32_t(std::max(ctx->cu_count, 1)) ? ctx->norm_rope_short : ctx->norm_rope;
    return launch(ctx, fn, dim3(blocks, 1, 1), dim3(256, 1, 1), p, "norm/rope rows", true);
}

// ---- quantised projections -------------------------------------------------

// Activation rows of the word-parallel kernel kept in LDS per workgroup.
constexpr size_t LINEAR_LDS_BYTES = 64 << 10;
// Activation rows from which a projection runs on the matrix cores.
constexpr uint32_t LINEAR_MFMA_MIN_M = 16;
// Packed weight bytes from which an M <= 2 projection runs on the int8 matrix
// cores (below it the word kernel's shorter start wins; both are at the
// dispatch floor there).
constexpr uint64_t LINEAR_I8_MIN_BYTES = 16ull << 20;

// Grid of a grid-stride elementwise launch over n items.
dim3 ew_grid(g4a_ctx* ctx, size_t n) {
    const size_t want = (n + 255) / 256, cap = size_t(std::max(ctx->cu_count, 1)) * 16;
    return dim3(uint32_t(std::max<size_t>(1, std::min(want, cap))), 1, 1);
}

int ew_launch(g4a_ctx* ctx, G4aEwOp op, const float* a, const float* b, const float* sp, float s, float* y, size_t n) {
    if (!ctx) return fail(ctx, G4A_E_ARG, "null ctx");
    if (n == 0) return G4A_OK;
    const bool binary = op == G4A_EW_ADD || op == G4A_EW_MUL || op == G4A_EW_GEGLU;
    if (!a || !y || (binary && !b) || (op == G4A_EW_SCALE_BY && !sp)) return fail(ctx, G4A_E_ARG, "null operand");
    G4aEwParams p{a, b, sp, y, n, s, uint32_t(op)};
    return launch(ctx, ctx->ew, ew_grid(ctx, n), dim3(256, 1, 1), p, "elementwise", true);
}

int rms_rows_launch(g4a_ctx* ctx, const float* res, const float* x, const float* w, const float* scale_by, float* y,
                    uint32_t rows, uint32_t dim, float eps) {
    if (!ctx) return fail(ctx, G4A_E_ARG, "null ctx");
    if (rows == 0) return G4A_OK;
    if (!x || !y || dim == 0) return fail(ctx, G4A_E_ARG, "null x/y or zero width");
    G4aRmsRowsParams p{x, w, res, scale_by, y, rows, dim, eps};
    return launch(ctx, ctx->rms_rows, dim3(rows, 1, 1), dim3(256, 1, 1), p, "rms rows", true);
}

int check_qweight(g4a_ctx* ctx, const g4a_qweight* w, const char* what) {
    if (!w) return fail(ctx, G4A_E_ARG, "%s: null weight", what);
    if (!w->qbytes || !w->scales) return fail(ctx, G4A_E_ARG, "%s: null qbytes/scales", what);
    if (w->N == 0 || w->K == 0) return fail(ctx, G4A_E_SHAPE, "%s: empty weight [%u, %u]", what, w->N, w->K);
    if (w->bits != 2 && w->bits != 4 && w->bits != 8)
        return fail(ctx, G4A_E_ARG, "%s: bits must be 2, 4 or 8 (got %u)", what, w->bits);
    if (w->signed_i8 && w->bits != 8) return fail(ctx, G4A_E_ARG, "%s: signed_i8 needs bits = 8", what);
    if (w->group_size == 0) return fail(ctx, G4A_E_ARG, "%s: group_size must be > 0", what);
    const uint32_t per_byte = w->signed_i8 ? 1 : 8 / w->bits;
    if (w->K % per_byte != 0)
        return fail(ctx, G4A_E_UNSUPPORTED, "%s: K = %u is not a whole number of bytes at %u bits", what, w->K, w->bits);
    return G4A_OK;
}

// y[M, N] = epilogue(x . W^T); mode 0 plain, 1 GeGLU with w2, 2 gelu times b's columns.
// Which projection kernel linear_q_launch runs for a call: the one place that
// decides it (g4a_attention_linear_q asks it too, so the projection it merges a
// decode step's partials into is the one the plain call would run).
struct LinearChoice {
    enum Kind { MFMA, I8, ELEM, WORDS } kind = ELEM;
    int wide = 0;       // MFMA: 128-row tiles
    int variant = 0;    // WORDS: (MT, RU) = (1, 2), (1, 8), (4, 4)
    int MT = 1, RU = 2;
    bool half = false;  // WORDS: 2-bit rows of an odd multiple of 32 words, two rows per wave
    uint64_t kpad = 0;  // WORDS: activation floats per row in LDS
};

LinearChoice choose_linear(const g4a_ctx* ctx, int mode, const g4a_qweight* w, const g4a_qweight* w2, const float* x,
                           uint32_t M) {
    LinearChoice c;
    const uint32_t row_bytes = w->signed_i8 ? w->K : w->K / (8 / w->bits);
    const uint32_t scale_stride = (w->K + w->group_size - 1) / w->group_size;
    const uintptr_t qa = reinterpret_cast<uintptr_t>(w->qbytes);
    const uintptr_t qa2 = mode == 1 ? reinterpret_cast<uintptr_t>(w2->qbytes) : 0;
    const bool aligned = (qa & 3) == 0 && (qa2 & 3) == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0;
    const bool aligned8 = aligned && (qa & 7) == 0 && (qa2 & 7) == 0;
    const uint64_t cus = uint64_t(std::max(ctx->cu_count, 1));
    if (M >= LINEAR_MFMA_MIN_M && w->K % 64 == 0 && scale_stride == 1 && aligned8) {
        c.kind = LinearChoice::MFMA;
        const uint64_t tiles128 = uint64_t((w->N + 127) / 128) * ((M + 63) / 64);
        c.wide = tiles128 >= 2 * cus ? 1 : 0;
        return c;
    }
    const uint64_t weight_bytes = uint64_t(w->N) * row_bytes;
    const bool i8_ok = mode == 0 && M <= 2 && scale_stride == 1 && row_bytes % G4A_LI8_UNIT_BYTES == 0 &&
                       w->K % 64 == 0 && uint64_t(w->K / 64) * 1024 <= LINEAR_LDS_BYTES && (qa & 15) == 0;
    if (i8_ok && (ctx->linear_i8_use == 1 || (ctx->linear_i8_use < 0 && weight_bytes >= LINEAR_I8_MIN_BYTES))) {
        c.kind = LinearChoice::I8;
        return c;
    }
    const uint64_t vpw = 32 / w->bits, words_per_row = uint64_t(w->K) * w->bits / 32;
    c.kpad = (words_per_row + 63) / 64 * 64 * vpw;
    const bool words = (uint64_t(w->K) * w->bits) % 32 == 0 && scale_stride == 1 && aligned &&
                       c.kpad * 4 <= LINEAR_LDS_BYTES;
    if (!words) {
        c.kind = LinearChoice::ELEM;
        return c;
    }
    c.kind = LinearChoice::WORDS;
    // 4 activation rows per workgroup when they fit its LDS share, else 1; 8 weight
    // rows in flight per wave for tall weights, 2 for short ones (more waves)
    if (M >= 2 && 4 * c.kpad * 4 <= LINEAR_LDS_BYTES) {
        c.variant = 2, c.MT = 4, c.RU = 4;
    } else if (w->N >= cus * 64) {
        c.variant = 1, c.MT = 1, c.RU = 8;
    } else {
        c.variant = 0, c.MT = 1, c.RU = 2;
    }
    // 2-bit rows of an odd multiple of 32 words (K = 1536 is 96 words): half-waves
    // walk two rows at once, so no lane idles on the row's last word step
    c.half = c.MT == 1 && w->bits == 2 && words_per_row % 64 == 32;
    return c;
}

int linear_q_launch(g4a_ctx* ctx, int mode, const g4a_qweight* w, const g4a_qweight* w2, const float* x,
                    const float* b, uint32_t b_stride, uint32_t b_off, float* y, uint32_t M) {
    if (!ctx) return fail(ctx, G4A_E_ARG, "null ctx");
    if (int rc = check_qweight(ctx, w, "weight")) return rc;
    if (mode == 1) {
        if (int rc = check_qweight(ctx, w2, "up weight")) return rc;
        if (w2->N != w->N || w2->K != w->K || w2->bits != w->bits || w2->signed_i8 != w->signed_i8 ||
            w2->group_size != w->group_size)
            return fail(ctx, G4A_E_UNSUPPORTED, "gate and up weights differ in shape or format");
    }
    if (mode == 2) {
        if (!b) return fail(ctx, G4A_E_ARG, "null column source");
        if (uint64_t(b_off) + w->N > b_stride)
            return fail(ctx, G4A_E_SHAPE, "columns [%u, %u) exceed the row stride %u", b_off, b_off + w->N, b_stride);
    }
    if (M == 0) return G4A_OK;
    if (!x || !y) return fail(ctx, G4A_E_ARG, "null x/y");
    G4aLinearParams p{};
    p.s = w->scales;
    p.s2 = mode == 1 ? w2->scales : nullptr;
    p.b = b;
    p.x = x;
    p.y = y;
    p.M = M;
    p.N = w->N;
    p.K = w->K;
    p.b_stride = b_stride;
    p.b_off = b_off;
    p.bits = w->bits;
    p.signed_i8 = w->signed_i8 ? 1 : 0;
    p.row_bytes = w->signed_i8 ? w->K : w->K / (8 / w->bits);
    p.group_size = w->group_size;
    p.scale_stride = (w->K + w->group_size - 1) / w->group_size;
    const LinearChoice ch = choose_linear(ctx, mode, w, w2, x, M);
    // sub-byte fields are offset binary: flipping each field's top bit makes it two's complement
    p.xm = w->signed_i8 ? 0u : w->bits == 4 ? 0x88888888u : w->bits == 2 ? 0xAAAAAAAAu : 0x80808080u;
    const int bi = w->bits == 2 ? 0 : w->bits == 4 ? 1 : 2;
    if (ch.kind == LinearChoice::MFMA) {
        // 64 activation rows x 128 weight rows per workgroup on the matrix cores,
        // or x 64 rows when the larger tile would leave fewer than 2 workgroups per CU
        p.wb = static_cast<const uint8_t*>(w->qbytes);
        p.wb2 = mode == 1 ? static_cast<const uint8_t*>(w2->qbytes) : nullptr;
        const int wide = ch.wide;
        const uint32_t gx = wide ? (w->N + 127) / 128 : (w->N + 63) / 64;
        for (uint32_t m0 = 0; m0 < M; m0 += 65535u * 64) {
            G4aLinearParams q = p;
            q.x = x + size_t(m0) * w->K;
            q.y = y + size_t(m0) * w->N;
            q.b = b ? b + size_t(m0) * b_stride : nullptr;
            q.M = std::min<uint32_t>(65535u * 64, M - m0);
            if (int rc = launch(ctx, ctx->linear_mfma[bi][wide][mode], dim3(gx, (q.M + 63) / 64, 1), dim3(256, 1, 1), q,
                                "quantised linear (matrix cores)", true))
                return rc;
        }
        return G4A_OK;
    }
    // M <= 2, large weights: int8 matrix cores with x cut into exact digits (mode 0)
    if (ch.kind == LinearChoice::I8) {
        p.wb = static_cast<const uint8_t*>(w->qbytes);
        // chunks of 32 weight rows, one per wave at a time; 16 waves per CU (four
        // workgroups, whose x digit staging then overlaps the others' streams)
        const uint64_t waves = G4A_LI8_THREADS / 64, chunks = (uint64_t(w->N) + 31) / 32;
        const uint64_t cap = uint64_t(std::max(ctx->cu_count, 1)) * (16 / waves);
        const uint32_t gx = uint32_t(std::max<uint64_t>(1, std::min(cap, (chunks + waves - 1) / waves)));
        return launch(ctx, ctx->linear_i8[bi][M - 1], dim3(gx, 1, 1), dim3(G4A_LI8_THREADS, 1, 1), p,
                      "quantised linear (int8 matrix cores)", true, unsigned(w->K / 64 * 1024));
    }
    // the word kernel's activation rows, zero-padded to whole wave strides of words
    const uint64_t vpw = 32 / w->bits, words_per_row = uint64_t(w->K) * w->bits / 32;
    const uint64_t kpad = ch.kpad;
    if (ch.kind == LinearChoice::ELEM) {
        // one thread per output in the CPU's order: any K, grouped scales
        p.wb = static_cast<const uint8_t*>(w->qbytes);
        p.wb2 = mode == 1 ? static_cast<const uint8_t*>(w2->qbytes) : nullptr;
        for (uint32_t m0 = 0; m0 < M; m0 += 65535) {
            G4aLinearParams q = p;
            q.x = x + size_t(m0) * w->K;
            q.y = y + size_t(m0) * w->N;
            q.b = b ? b + size_t(m0) * b_stride : nullptr;
            q.M = std::min<uint32_t>(65535, M - m0);
            if (int rc = launch(ctx, ctx->linear_elem[mode], dim3((w->N + 63) / 64, q.M, 1), dim3(64, 1, 1), q,
                                "quantised linear (element)", true))
                return rc;
        }
        return G4A_OK;
    }
    p.w = static_cast<const uint32_t*>(w->qbytes);
    p.w2 = mode == 1 ? static_cast<const uint32_t*>(w2->qbytes) : nullptr;
    p.W = uint32_t(words_per_row);
    const uint64_t cus = uint64_t(std::max(ctx->cu_count, 1));
    const int variant = ch.variant, MT = ch.MT, RU = ch.RU;
    // about 16 waves per CU over the rows (four 4-wave workgroups): weight
    // streaming needs many loads in flight
    const uint64_t target = cus * 16;
    uint64_t rpw = (w->N + target - 1) / target;
    rpw = std::max<uint64_t>(RU, (rpw + RU - 1) / RU * RU);
    p.rows_per_wave = uint32_t(rpw);
    const uint32_t gx = uint32_t((w->N + 4 * rpw - 1) / (4 * rpw));
    const bool half = ch.half;
    hipFunction_t fn = half ? ctx->linear_half[variant][mode] : ctx->linear_words[bi][variant][mode];
    const unsigned lds = unsigned(MT * (half ? (words_per_row + 31) / 32 * 32 * vpw : kpad) * 4);
    for (uint32_t m0 = 0; m0 < M; m0 += 65535u * MT) {
        G4aLinearParams q = p;
        q.x = x + size_t(m0) * w->K;
        q.y = y + size_t(m0) * w->N;
        q.b = b ? b + size_t(m0) * b_stride : nullptr;
        q.M = std::min<uint32_t>(65535u * MT, M - m0);
        if (int rc = launch(ctx, fn, dim3(gx, (q.M + MT - 1) / MT, 1), dim3(256, 1, 1), q, "quantised linear", true,
                            lds))
            return rc;
    }
    return G4A_OK;
}

}  // namespace

int g4a_linear_q(g4a_ctx* ctx, const g4a_qweight* w, const float* x, float* y, uint32_t M) {
    return linear_q_launch(ctx, 0, w, nullptr, x, nullptr, 0, 0, y, M);
}

int g4a_linear_q_geglu(g4a_ctx* ctx, const g4a_qweight* w_gate, const g4a_qweight* w_up, const float* x, float* y,
                       uint32_t M) {
    return linear_q_launch(ctx, 1, w_gate, w_up, x, nullptr, 0, 0, y, M);
}

int g4a_linear_q_gelu_mul_cols(g4a_ctx* ctx, const g4a_qweight* w, const float* x, const float* b, uint32_t b_stride,
                               uint32_t b_off, float* y, uint32_t M) {
    return linear_q_launch(ctx, 2, w, nullptr, x, b, b_stride, b_off, y, M);
}

}  // extern "C"

namespace {

// Whether linear_q_launch takes (w, M = 1, mode 0) to the word kernel's
// (MT, RU) = (1, 2) form with 64 lanes per row: the form whose mode 3 merges a
// decode step's split partials while staging x, with the same sums.
bool projection_on_short_words(const g4a_ctx* ctx, const g4a_qweight* w, const float* x) {
    const LinearChoice c = choose_linear(ctx, 0, w, nullptr, x, 1);
    return c.kind == LinearChoice::WORDS && c.variant == 0 && !c.half;
}

}  // namespace

extern "C" {

int g4a_attention_linear_q(g4a_ctx* ctx, const g4a_attn_args* a, const g4a_qweight* w, float* y) {
    if (!ctx) return fail(ctx, G4A_E_ARG, "null ctx");
    if (!a) return fail(ctx, G4A_E_ARG, "null args");
    if (int rc = check_qweight(ctx, w, "projection")) return rc;
    if (uint64_t(a->Hq) * a->Dv != w->K)
        return fail(ctx, G4A_E_SHAPE, "projection K = %u, attention rows are %u x %u", w->K, a->Hq, a->Dv);
    Analysis an;
    if (int rc = analyse(ctx, a, &an, true)) return rc;
    if (a->T == 0) return G4A_OK;
    if (!y) return fail(ctx, G4A_E_ARG, "null y");
    const g4a_attn_plan& pl = an.plan;
    // one decode step with a few splits and a projection on the short word
    // kernel, on a context that asks for it: the projection merges the
    // partials while it stages its x row
    const bool fuse = ctx->fuse_projection && a->T == 1 && (pl.kernel == G4A_KERNEL_DECODE || pl.kernel == G4A_KERNEL_DECODE_SHORT) &&
                      pl.splits >= 2 && pl.splits <= G4A_FUSE_MAX_SPLITS && pl.splits <= COMBINE_ROW_SPLITS &&
                      a->Hq <= G4A_FUSE_MAX_HEADS && (a->Dh == 256 || a->Dh == 512) && a->Dv == a->Dh &&
                      (reinterpret_cast<uintptr_t>(a->out) & 15) == 0 && projection_on_short_words(ctx, w, a->out);
    if (int rc = attention_run(ctx, a, an, !fuse)) return rc;
    if (!fuse) return linear_q_launch(ctx, 0, w, nullptr, a->out, nullptr, 0, 0, y, a->T);
    G4aLinearParams p{};
    p.w = static_cast<const uint32_t*>(w->qbytes);
    p.s = w->scales;
    p.y = y;
    p.M = 1;
    p.N = w->N;
    p.K = w->K;
    p.W = uint32_t(uint64_t(w->K) * w->bits / 32);
    p.bits = w->bits;
    p.signed_i8 = w->signed_i8 ? 1 : 0;
    p.xm = w->signed_i8 ? 0u : w->bits == 4 ? 0x88888888u : w->bits == 2 ? 0xAAAAAAAAu : 0x80808080u;
    p.part = static_cast<const float*>(ctx->workspace);  // where attention_run left the partials
    p.xout = a->out;
    p.nsplit = pl.splits;
    p.dh = a->Dh;
    p.hq = a->Hq;
    // the plain projection's grid (about 16 waves per CU over the rows): fewer,
    // taller workgroups, each merging the whole row, measured slower
    const uint64_t target = uint64_t(std::max(ctx->cu_count, 1)) * 16;
    uint64_t rpw = (uint64_t(w->N) + target - 1) / target;
    rpw = std::max<uint64_t>(2, (rpw + 1) / 2 * 2);
    p.rows_per_wave = uint32_t(rpw);
    const uint64_t vpw = 32 / w->bits, kpad = (uint64_t(p.W) + 63) / 64 * 64 * vpw;
    const int bi = w->bits == 2 ? 0 : w->bits == 4 ? 1 : 2;
    return launch(ctx, ctx->linear_fused[bi], dim3(uint32_t((w->N + 4 * rpw - 1) / (4 * rpw)), 1, 1),
                  dim3(256, 1, 1), p, "attention row + projection", true, unsigned(kpad * 4));
}

int g4a_embed_rows_q(g4a_ctx* ctx, const g4a_qweight* table, const uint32_t* ids, uint32_t T, float scale,
                     float* out) {
    if (!ctx) return fail(ctx, G4A_E_ARG, "null ctx");
    if (int rc = check_qweight(ctx, table, "table")) return rc;
    if (T == 0) return G4A_OK;
    if (!ids || !out) return fail(ctx, G4A_E_ARG, "null ids/out");
    for (uint32_t i = 0; i < T; ++i)
        if (ids[i] >= table->N) return fail(ctx, G4A_E_ARG, "id %u at %u is outside the table's %u rows", ids[i], i, table->N);
    if (uint64_t(T) * table->K >= (uint64_t(1) << 32)) return fail(ctx, G4A_E_SHAPE, "embedding output too large");
    G4aEmbedParams p{};
    p.wb = static_cast<const uint8_t*>(table->qbytes);
    p.s = table->scales;
    p.out = out;
    p.T = T;
    p.D = table->K;
    p.bits = table->bits;
    p.signed_i8 = table->signed_i8 ? 1 : 0;
    p.row_bytes = table->signed_i8 ? table->K : table->K / (8 / table->bits);
    p.group_size = table->group_size;
    p.scale_stride = (table->K + table->group_size - 1) / table->group_size;
    p.scale = scale;
    if (int rc = upload_positions(ctx, ids, T, nullptr, 0, &p.ids, nullptr)) return rc;
    const uint64_t n = uint64_t(T) * table->K;
    return launch(ctx, ctx->embed_q, dim3(uint32_t((n + 255) / 256), 1, 1), dim3(256, 1, 1), p,
                  "quantised embedding", true);
}

int g4a_head_norm_rope(g4a_ctx* ctx, const float* x, const float* w, float* y, uint32_t T, uint32_t heads,
                       uint32_t head_dim, uint32_t rotary_dim, const uint32_t* positions, uint32_t pos0, float theta,
                       float eps) {
    if (!ctx) return fail(ctx, G4A_E_ARG, "null ctx");
    G4aNormRopeSeg seg{x, w, y, heads, 1u, 1u, 0u, 0u};
    return norm_rope_launch(ctx, &seg, 1, T, head_dim, rotary_dim, positions, pos0, theta, eps, 0, 0);
}

int g4a_rms_norm(g4a_ctx* ctx, const float* x, const float* w, float* y, uint32_t rows, uint32_t dim, float eps) {
    if (!ctx) return fail(ctx, G4A_E_ARG, "null ctx");
    if (dim % 4 != 0 || dim > 1024)  // wide or ragged rows: a workgroup per row
        return rms_rows_launch(ctx, nullptr, x, w, nullptr, y, rows, dim, eps);
    G4aNormRopeSeg seg{x, w, y, rows, 1u, 0u, 0u, 0u};
    return norm_rope_launch(ctx, &seg, 1, 1, dim, 0, nullptr, 0, 0.0f, eps, 0, 0);
}

int g4a_add_rms_norm(g4a_ctx* ctx, const float* residual, const float* x, const float* w, const float* scale_by,
                     float* y, uint32_t rows, uint32_t dim, float eps) {
    if (!residual || !w) return fail(ctx, G4A_E_ARG, "null residual/weight");
    return rms_rows_launch(ctx, residual, x, w, scale_by, y, rows, dim, eps);
}

int g4a_add(g4a_ctx* ctx, const float* a, const float* b, float* y, size_t n) {
    return ew_launch(ctx, G4A_EW_ADD, a, b, nullptr, 0.0f, y, n);
}
int g4a_mul(g4a_ctx* ctx, const float* a, const float* b, float* y, size_t n) {
    return ew_launch(ctx, G4A_EW_MUL, a, b, nullptr, 0.0f, y, n);
}
int g4a_scale(g4a_ctx* ctx, const float* a, float s, float* y, size_t n) {
    return ew_launch(ctx, G4A_EW_SCALE, a, nullptr, nullptr, s, y, n);
}
int g4a_scale_by_tensor(g4a_ctx* ctx, const float* a, const float* s, float* y, size_t n) {
    return ew_launch(ctx, G4A_EW_SCALE_BY, a, nullptr, s, 0.0f, y, n);
}
int g4a_gelu_tanh(g4a_ctx* ctx, const float* a, float* y, size_t n) {
    return ew_launch(ctx, G4A_EW_GELU, a, nullptr, nullptr, 0.0f, y, n);
}
int g4a_geglu(g4a_ctx* ctx, const float* gate, const float* up, float* y, size_t n) {
    return ew_launch(ctx, G4A_EW_GEGLU, gate, up, nullptr, 0.0f, y, n);
}
int g4a_softcap(g4a_ctx* ctx, const float* a, float cap, float* y, size_t n) {
    return ew_launch(ctx, G4A_EW_SOFTCAP, a, nullptr, nullptr, cap, y, n);
}

int g4a_slice_cols(g4a_ctx* ctx, const float* x, uint32_t rows, uint32_t stride, uint32_t offset, uint32_t width,
                   float* y) {
    if (!ctx) return fail(ctx, G4A_E_ARG, "null ctx");
    if (uint64_t(offset) + width > stride)
        return fail(ctx, G4A_E_SHAPE, "columns [%u, %u) exceed the row stride %u", offset, offset + width, stride);
    const size_t n = size_t(rows) * width;
    if (n == 0) return G4A_OK;
    if (!x || !y) return fail(ctx, G4A_E_ARG, "null x/y");
    G4aSliceColsParams p{x, y, rows, stride, offset, width};
    return launch(ctx, ctx->slice_cols, ew_grid(ctx, n), dim3(256, 1, 1), p, "slice cols", true);
}

int g4a_embed_rows(g4a_ctx* ctx, const float* table, uint32_t V, uint32_t D, const uint32_t* ids, uint32_t T,
                   float scale, float* out) {
    if (!ctx) return fail(ctx, G4A_E_ARG, "null ctx");
    if (T == 0 || D == 0) return G4A_OK;
    if (!table || !ids || !out) return fail(ctx, G4A_E_ARG, "null table/ids/out");
    for (uint32_t i = 0; i < T; ++i)
        if (ids[i] >= V) return fail(ctx, G4A_E_ARG, "id %u at %u is outside the table's %u rows", ids[i], i, V);
    G4aEmbedF32Params p{table, nullptr, out, T, D, scale};
    if (int rc = upload_positions(ctx, ids, T, nullptr, 0, &p.ids, nullptr)) return rc;
    return launch(ctx, ctx->embed_f32, ew_grid(ctx, size_t(T) * D), dim3(256, 1, 1), p, "embedding", true);
}

int g4a_linear(g4a_ctx* ctx, const float* w, uint32_t N, uint32_t K, const float* x, float* y, uint32_t M) {
    if (!ctx) return fail(ctx, G4A_E_ARG, "null ctx");
    if (N == 0 || K == 0) return fail(ctx, G4A_E_SHAPE, "empty weight [%u, %u]", N, K);
    if (M == 0) return G4A_OK;
    if (!w || !x || !y) return fail(ctx, G4A_E_ARG, "null w/x/y");
    G4aLinearParams p{};
    p.w = reinterpret_cast<const uint32_t*>(w);
    p.x = x;
    p.y = y;
    p.M = M;
    p.N = N;
    p.K = K;
    p.W = K;
    const uint64_t kpad = (uint64_t(K) + 63) / 64 * 64;
    const bool aligned = (reinterpret_cast<uintptr_t>(x) & 15) == 0 && (reinterpret_cast<uintptr_t>(w) & 3) == 0;
    if (!aligned || K % 4 != 0 || kpad * 4 > LINEAR_LDS_BYTES) {
        for (uint32_t m0 = 0; m0 < M; m0 += 65535) {
            G4aLinearParams q = p;
            q.x = x + size_t(m0) * K;
            q.y = y + size_t(m0) * N;
            q.M = std::min<uint32_t>(65535, M - m0);
            if (int rc = launch(ctx, ctx->linear_f32_elem, dim3((N + 63) / 64, q.M, 1), dim3(64, 1, 1), q,
                                "linear (element)", true))
                return rc;
        }
        return G4A_OK;
    }
    const uint64_t cus = uint64_t(std::max(ctx->cu_count, 1));
    int variant, MT, RU;
    if (M >= 2 && 4 * kpad * 4 <= LINEAR_LDS_BYTES) variant = 2, MT = 4, RU = 4;
    else if (N >= cus * 64) variant = 1, MT = 1, RU = 8;
    else variant = 0, MT = 1, RU = 2;
    const uint64_t target = cus * 16;
    uint64_t rpw = (N + target - 1) / target;
    rpw = std::max<uint64_t>(RU, (rpw + RU - 1) / RU * RU);
    p.rows_per_wave = uint32_t(rpw);
    const uint32_t gx = uint32_t((N + 4 * rpw - 1) / (4 * rpw));
    const unsigned lds = unsigned(MT * kpad * 4);
    for (uint32_t m0 = 0; m0 < M; m0 += 65535u * MT) {
        G4aLinearParams q = p;
        q.x = x + size_t(m0) * K;
        q.y = y + size_t(m0) * N;
        q.M = std::min<uint32_t>(65535u * MT, M - m0);
        if (int rc = launch(ctx, ctx->linear_f32_words[variant], dim3(gx, (q.M + MT - 1) / MT, 1), dim3(256, 1, 1), q,
                            "linear", true, lds))
            return rc;
    }
    return G4A_OK;
}

int g4a_rope(g4a_ctx* ctx, const float* x, float* y, uint32_t T, uint32_t heads, uint32_t head_dim,
             uint32_t rotary_dim, const uint32_t* positions, uint32_t pos0, float theta) {
    if (!ctx) return fail(ctx, G4A_E_ARG, "null ctx");
    G4aNormRopeSeg seg{x, nullptr, y, heads, 0u, 1u, 0u, 0u};
    return norm_rope_launch(ctx, &seg, 1, T, head_dim, rotary_dim, positions, pos0, theta, 0.0f, 0, 0);
}

namespace {

int producer_run(g4a_ctx* ctx, const g4a_producer_args* a, const uint32_t* dpos, uint32_t dpos_max) {
    if (!ctx) return fail(ctx, G4A_E_ARG, "null ctx");
    if (!a) return fail(ctx, G4A_E_ARG, "null args");
    if (!a->q || !a->q_out) return fail(ctx, G4A_E_ARG, "null q / q_out");
    if ((a->k == nullptr) != (a->v == nullptr)) return fail(ctx, G4A_E_ARG, "k and v come together");
    if (a->k && (!a->k_cache || !a->v_cache)) return fail(ctx, G4A_E_ARG, "null k_cache / v_cache");
    G4aNormRopeSeg segs[3];
    uint32_t n = 0;
    // q: weighted norm + RoPE, or RoPE only without a q_norm weight (rust/src/model.rs:258-261)
    segs[n++] = G4aNormRopeSeg{a->q, a->q_norm, a->q_out, a->Hq, a->q_norm ? 1u : 0u, 1u, 0u, 0u};
    if (a->k) {
        // a ring keeps only the last kv_ring_cap of the call's rows
        const uint32_t first = a->kv_ring_cap && a->T > a->kv_ring_cap ? a->T - a->kv_ring_cap : 0;
        // k like q (rust/src/model.rs:270-273); v: unweighted norm, no rotation (:275)
        segs[n++] = G4aNormRopeSeg{a->k, a->k_norm, a->k_cache, a->Hkv, a->k_norm ? 1u : 0u, 1u, 1u, first};
        segs[n++] = G4aNormRopeSeg{a->v, nullptr, a->v_cache, a->Hkv, 1u, 0u, 1u, first};
    }
    return norm_rope_launch(ctx, segs, n, a->T, a->Dh, a->rotary_dim, a->positions, a->pos0, a->theta, a->eps,
                            a->cache_row, a->kv_ring_cap, dpos, dpos_max);
}

}  // namespace

int g4a_attn_producer(g4a_ctx* ctx, const g4a_producer_args* a) { return producer_run(ctx, a, nullptr, 0); }

int g4a_attn_producer_devpos(g4a_ctx* ctx, const g4a_producer_args* a, const uint32_t* pos, uint32_t max_pos) {
    if (!ctx) return fail(ctx, G4A_E_ARG, "null ctx");
    if (!a || !pos) return fail(ctx, G4A_E_ARG, "null args / device position");
    if (a->T != 1) return fail(ctx, G4A_E_UNSUPPORTED, "a device-position producer step has one token (T = %u)", a->T);
    if (a->positions) return fail(ctx, G4A_E_ARG, "a device-position producer step takes its position from `pos`");
    return producer_run(ctx, a, pos, max_pos);
}

struct g4a_graph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    std::shared_ptr<g4a_graph_book> book;  // the context it was captured on
};

int g4a_capture_begin(g4a_ctx* ctx) {
    if (!ctx) return fail(ctx, G4A_E_ARG, "null ctx");
    if (ctx->capturing) return fail(ctx, G4A_E_ARG, "a capture is already open on this context");
    if (ctx->timing) return fail(ctx, G4A_E_ARG, "per-kernel timing is on: turn it off before capturing");
    // a graph is where g4a_attention_noalloc is most used, and looking the static
    // scratch array up may load it, which is no stream work: do it before the capture
    if (!ctx->scratch) {
        HIP_TRY(ctx, hipSetDevice(ctx->device));
        if (int rc = scratch_setup(ctx)) return rc;
    }
    HIP_TRY(ctx, hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    ctx->capturing = true;
    ctx->capture_code = 0;
    ctx->capture_msg.clear();
    return G4A_OK;
}

int g4a_capture_end(g4a_ctx* ctx, g4a_graph** graph) {
    if (!ctx || !graph) return fail(ctx, G4A_E_ARG, "null ctx/graph");
    *graph = nullptr;
    if (!ctx->capturing) return fail(ctx, G4A_E_ARG, "no capture is open on this context");
    ctx->capturing = false;
    const int code = ctx->capture_code;
    ctx->capture_code = 0;
    hipGraph_t g = nullptr;
    const hipError_t ee = hipStreamEndCapture(ctx->stream, &g);
    if (code != 0) {
        // a call refused inside the capture is missing from the recording: no graph
        if (g) hipGraphDestroy(g);
        return fail(ctx, code, "a call inside the capture failed, so no graph was made: %s", ctx->capture_msg.c_str());
    }
    if (ee != hipSuccess) return fail(ctx, G4A_E_HIP, "hipStreamEndCapture: %s", hipGetErrorString(ee));
    hipGraphExec_t exec = nullptr;
    const hipError_t e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        hipGraphDestroy(g);
        return fail(ctx, G4A_E_HIP, "hipGraphInstantiate: %s", hipGetErrorString(e));
    }
    *graph = new g4a_graph{g, exec, ctx->book};
    ++ctx->book->live;
    return G4A_OK;
}

int g4a_graph_launch(g4a_ctx* ctx, g4a_graph* graph) {
    if (!ctx || !graph) return fail(ctx, G4A_E_ARG, "null ctx/graph");
    if (graph->book != ctx->book)
        return fail(ctx, G4A_E_ARG, "the graph was captured on another context: launch it on that one");
    if (int rc = refuse_in_capture(ctx, "g4a_graph_launch")) return rc;
    HIP_TRY(ctx, hipGraphLaunch(graph->exec, ctx->stream));
    return G4A_OK;
}

int g4a_graph_destroy(g4a_graph* graph) {
    if (!graph) return G4A_OK;
    g4a_ctx* const ctx = graph->book ? graph->book->ctx : nullptr;
    // a replay may still be running on the context's stream (a stream that is
    // capturing cannot be waited on; its retired workspaces then wait for a later
    // destroy or the context's end)
    const bool can_wait = ctx && !ctx->capturing;
    if (can_wait) hipStreamSynchronize(ctx->stream);
    if (graph->exec) hipGraphExecDestroy(graph->exec);
    if (graph->graph) hipGraphDestroy(graph->graph);
    if (ctx) {
        g4a_graph_book& b = *graph->book;
        if (--b.live == 0 && can_wait) {
            // no graph needs the workspaces the context has outgrown any more
            for (void* p : b.retired) hipFree(p);
            b.retired.clear();
        }
    }
    delete graph;
    return G4A_OK;
}

int g4a_timer_start(g4a_ctx* ctx) {
    if (!ctx) return fail(ctx, G4A_E_ARG, "null ctx");
    if (int rc = refuse_in_capture(ctx, "g4a_timer_start")) return rc;
    HIP_TRY(ctx, hipEventRecord(ctx->ev_start, ctx->stream));
    return G4A_OK;
}

int g4a_timer_stop(g4a_ctx* ctx, float* ms) {
    if (!ctx || !ms) return fail(ctx, G4A_E_ARG, "null ctx/ms");
    if (int rc = refuse_in_capture(ctx, "g4a_timer_stop")) return rc;
    HIP_TRY(ctx, hipEventRecord(ctx->ev_stop, ctx->stream));
    HIP_TRY(ctx, hipEventSynchronize(ctx->ev_stop));
    HIP_TRY(ctx, hipEventElapsedTime(ms, ctx->ev_start, ctx->ev_stop));
    return G4A_OK;
}

int g4a_kernel_timing(g4a_ctx* ctx, int enable) {
    if (!ctx) return fail(ctx, G4A_E_ARG, "null ctx");
    if (int rc = refuse_in_capture(ctx, "g4a_kernel_timing")) return rc;
    if (enable && ctx->kev.empty()) {
        // Timing-only events: without a system-scope fence the timed dispatch ends
        // with the same device-scope release as an untimed one. With the fence, the
        // stop event bound to the kernel makes it write its dirty L2 lines back to
        // memory first (a decode step's 4 MiB of split partials: ~1 us more than the
        // profiler's duration of the same kernel). Results are read only after a
        // stream synchronize, which does not rely on these events.
        ctx->kev.resize(2 * kMaxTimed, nullptr);
        for (auto& ev : ctx->kev) HIP_TRY(ctx, hipEventCreateWithFlags(&ev, hipEventDisableSystemFence));
    }
    if (ctx->kev_used) HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    ctx->timing = enable != 0;
    ctx->kev_used = 0;
    return G4A_OK;
}

int g4a_kernel_timing_read(g4a_ctx* ctx, double* total_ms, uint32_t* count) {
    if (!ctx || !total_ms || !count) return fail(ctx, G4A_E_ARG, "null argument");
    double sum = 0.0;
    for (uint32_t i = 0; i < ctx->kev_used; ++i) {
        float ms = 0.0f;
        HIP_TRY(ctx, hipEventSynchronize(ctx->kev[2 * i + 1]));
        HIP_TRY(ctx, hipEventElapsedTime(&ms, ctx->kev[2 * i], ctx->kev[2 * i + 1]));
        sum += ms;
    }
    *total_ms = sum;
    *count = ctx->kev_used;
    ctx->kev_used = 0;
    return G4A_OK;
}

int g4a_get_device_info(g4a_ctx* ctx, g4a_device_info* info) {
    if (!ctx || !info) return fail(ctx, G4A_E_ARG, "null ctx/info");
    hipDeviceProp_t prop;
    HIP_TRY(ctx, hipGetDeviceProperties(&prop, ctx->device));
    memset(info, 0, sizeof *info);
    info->device = ctx->device;
    info->compute_units = prop.multiProcessorCount;
    info->clock_khz = prop.clockRate;
    info->total_mem = prop.totalGlobalMem;
    snprintf(info->arch, sizeof info->arch, "%s", prop.gcnArchName);
    return G4A_OK;
}

}  // extern "C"
