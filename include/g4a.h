/*
 * g4a — Gemma-4 attention on MI355X (gfx950): the C-ABI of libg4a.so.
 *
 * This is the drop-in boundary for the attention ops of the reference's
 * backend-agnostic op trait (rust/src/backend.rs:88-180). A Rust `HipBackend`
 * implements `Backend::attention` / `Backend::kv_append` over these calls
 * through an FFI crate that declares them as `extern "C"`; the C++ mirror of
 * the trait lives in gemma-4-webgpu-kernels_amd/csrc/hip_backend.hpp.
 *
 * Conventions
 *   - Every call returns G4A_OK (0) or a negative g4a_status; the message of
 *     the last failure is g4a_last_error(ctx). Ops are "infallible" in the
 *     reference (they panic); the Rust binding panics on a nonzero status.
 *   - A context owns one HIP stream; every op is stream-ordered and returns
 *     before the GPU runs it (rust/src/backend_wgpu.rs:1-6). Only g4a_d2h and
 *     g4a_sync block. A context is not thread-safe (the reference backend is
 *     `RefCell`-based and !Sync, rust/src/backend_wgpu.rs:241).
 *   - Tensors are plain device pointers to row-major f32 data with the shapes
 *     the trait uses: q [T,Hq,Dh], k [S,Hkv,Dh], v [S,Hkv,Dv], out [T,Hq*Dv].
 *   - Position slices are HOST pointers borrowed for the duration of the call,
 *     exactly like AttnOpts::q_pos / k_pos (rust/src/backend.rs:61-64).
 */
#ifndef G4A_H
#define G4A_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct g4a_ctx g4a_ctx;

typedef enum g4a_status {
    G4A_OK = 0,
    G4A_E_HIP = -1,         /* a HIP runtime call failed */
    G4A_E_ARG = -2,         /* null pointer / invalid argument */
    G4A_E_SHAPE = -3,       /* inconsistent shapes */
    G4A_E_UNSUPPORTED = -4, /* a combination this build does not handle */
    G4A_E_MODULE = -5,      /* the gfx950 code object could not be loaded */
    G4A_E_NOMEM = -6,       /* device allocation failed */
} g4a_status;

/* ---- context and memory ------------------------------------------------
 * Replaces WgpuBackend::create (rust/src/backend_wgpu.rs:283) and the wgpu
 * device acquisition (rust/src/device.rs:25-66). `hsaco_path` NULL loads
 * g4a_kernels.hsaco from the directory of libg4a.so. */
int g4a_create(int device, const char *hsaco_path, g4a_ctx **out);

/* Kernel-selection options of a context, fixed at creation. g4a_create uses
 * the defaults (g4a_default_options); the others exist to compare kernels and
 * to opt into behaviour that is off by default. No counterpart in the
 * reference (its backend has no such choices). */
typedef struct g4a_options {
    uint32_t size;            /* sizeof(g4a_options), set by g4a_default_options */
    int32_t short_decode;     /* 1 (default): decode splits that fit the CUs with 32 keys run the
                                 short-context kernel; 0: always the streaming kernel */
    uint32_t short_max_wgs;   /* 4 (default), 2 or 1: workgroups sharing one short-kernel split */
    int32_t batch_kernel;     /* g4a_attention_decode_batch: 0 (default) automatic, 1 short, 2 streaming */
    uint32_t batch_keys_per_split; /* streaming batch launches: 0 (default) automatic */
    int32_t linear_i8;        /* -1 (default): the int8 matrix-core projection for M <= 2 weights of
                                 16 MB and more; 1: for every eligible weight; 0: never */
    int32_t fuse_projection;  /* 0 (default); 1: g4a_attention_linear_q merges a decode step's
                                 split partials inside its projection (2..16 splits, short-weight
                                 projections): bit-identical, measured slower on MI355X */
} g4a_options;
void g4a_default_options(g4a_options *opts);
/* g4a_create with options (NULL: the defaults); fails with G4A_E_ARG on an
 * options struct of another size or an option out of range. */
int g4a_create_with(int device, const char *hsaco_path, const g4a_options *opts, g4a_ctx **out);
void g4a_destroy(g4a_ctx *ctx);
/* Message of the last failed call on this context ("" if none). With a NULL
 * ctx: the message of the calling thread's last failure that had no context
 * (a g4a_create, or a call given a NULL context such as a plan query). */
const char *g4a_last_error(const g4a_ctx *ctx);

/* Device buffers. Replace raw_buf / alloc_in (rust/src/backend_wgpu.rs:371-402)
 * and free_tensor (rust/src/backend_wgpu.rs:1126-1130). */
int g4a_malloc(g4a_ctx *ctx, size_t bytes, void **dptr);
int g4a_free(g4a_ctx *ctx, void *dptr);
/* Host -> device copy of `bytes`; the host buffer may be reused on return
 * (Backend::tensor, rust/src/backend_wgpu.rs:428-439). */
int g4a_h2d(g4a_ctx *ctx, void *dst, const void *src, size_t bytes);
/* Device -> host copy; waits for all prior work on the context's stream
 * (Backend::readback, rust/src/backend_wgpu.rs:1057-1085). */
int g4a_d2h(g4a_ctx *ctx, void *dst, const void *src, size_t bytes);
/* Stream-ordered device -> device copy (COPY, rust/src/kernels/copy.wgsl:1-14). */
int g4a_d2d(g4a_ctx *ctx, void *dst, const void *src, size_t bytes);
/* Stream-ordered fill with zero bytes (Backend::zeros, rust/src/backend.rs:95). */
int g4a_zero(g4a_ctx *ctx, void *dst, size_t bytes);
/* Wait for all work on the context's stream (Backend::flush + device poll). */
int g4a_sync(g4a_ctx *ctx);
/* The context's HIP stream (a hipStream_t), for callers that order their own
 * work against the context's by stream order or events instead of g4a_sync
 * (e.g. torch.cuda.ExternalStream). No counterpart in the reference, whose
 * backend hides its queue. The stream stays the context's: do not destroy it,
 * and do not use it after g4a_destroy. */
int g4a_stream(g4a_ctx *ctx, void **stream);

/* ---- attention -----------------------------------------------------------
 * Backend::attention (rust/src/backend.rs:119-120) with AttnOpts
 * (rust/src/backend.rs:59-69); semantics of CpuBackend::attention
 * (rust/src/backend_cpu.rs:270-336): query head h reads kv head h/(Hq/Hkv);
 * key j is visible to query i iff kpos <= qpos && (window == 0 ||
 * qpos - kpos < window); a row with no visible key is 0. Host dispatch replaces
 * WgpuBackend::attention (rust/src/backend_wgpu.rs:895-970).
 *
 * Positions: q_pos (T entries) and k_pos (S entries) are borrowed host arrays
 * as in AttnOpts. A NULL array means the contiguous range q_pos0 + i /
 * k_pos0 + j (what the model always passes, rust/src/engine.rs:155,233), which
 * needs no upload. k_pos must be ascending (the reference's key-range trim,
 * rust/src/backend_wgpu.rs:924-936, relies on it too).
 *
 * KV layout: kv_ring_cap == 0 means logical key row j is physical row j of
 * k/v. kv_ring_cap > 0 means k/v are rings of kv_ring_cap rows and logical row
 * j lives in slot j % kv_ring_cap; every key the queries can see must still be
 * in the ring (G4A_E_SHAPE otherwise).
 *
 * splits: 0 picks the split-K count so a single sequence fills the GPU; > 0
 * forces it (clamped to the number of 64-key tiles).
 * attn_softcap > 0 applies cap*tanh(s/cap) after the scale
 * (rust/src/backend_cpu.rs:303-305). */
typedef struct g4a_attn_args {
    const float *q;
    const float *k;
    const float *v;
    float *out;
    uint32_t T, S, Hq, Hkv, Dh, Dv;
    const uint32_t *q_pos; /* host [T] or NULL */
    const uint32_t *k_pos; /* host [S] or NULL */
    uint32_t q_pos0, k_pos0;
    float scale;
    uint32_t sliding_window;
    float attn_softcap;
    uint32_t kv_ring_cap;
    uint32_t splits;
} g4a_attn_args;

int g4a_attention(g4a_ctx *ctx, const g4a_attn_args *args);

/* g4a_attention without any allocation. No counterpart in the reference: for
 * callers that cannot allocate while they run (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). Same arguments, same
 * kernels and the same results (bit-identical) as g4a_attention, except that a
 * call's split partials and pre-split K/V live in a static scratch array of
 * G4A_NOALLOC_SCRATCH_BYTES compiled into libg4a.so instead of the context's
 * workspace, and that it calls no allocator. Each GPU holds its own copy of the
 * array, looked up (and so loaded onto the GPU) by the first no-alloc call or
 * graph capture on that GPU, and held until the process ends: a process that
 * does neither does not hold it.
 * Fails with G4A_E_UNSUPPORTED, enqueueing nothing, when the call needs more
 * scratch than the array holds (decode: T*Hq*splits*(Dh+2)*4 bytes for more
 * than one split; prefill: about 2*keys*Hkv*Dh*4 bytes plus the partials of
 * split query blocks at head_dim 512; g4a_attention_plan gives the decode
 * figure) or passes non-contiguous explicit positions (they are staged through
 * allocated buffers). Every call on a GPU shares that GPU's array and leaves
 * its contents behind (nothing in it needs clearing: each call writes what it
 * reads first), so calls that overlap on one GPU race: keep them on one stream
 * or order them with events. */
#define G4A_NOALLOC_SCRATCH_BYTES (64u << 20)
int g4a_attention_noalloc(g4a_ctx *ctx, const g4a_attn_args *args);

/* n attention calls enqueued back-to-back on the context's stream, args[i]
 * exactly as for g4a_attention; stops at the first failing call and returns
 * its status (calls before it stay enqueued). No counterpart in the
 * reference: a batched Backend::attention for callers that issue many calls
 * per step (a token's layer schedule, a benchmark loop) and want one FFI
 * crossing for all of them. */
int g4a_attention_batch(g4a_ctx *ctx, const g4a_attn_args *args, uint32_t n);

/* n independent single-query decode steps, e.g. one layer's attention for
 * every sequence of a serving batch, in one decode launch per 64 sequences
 * (plus one LSE-combine launch for the sequences with more than one split)
 * instead of up to two launches per sequence. A launch whose 32-key splits
 * fit one workgroup per CU runs the short-context kernel; a larger one runs
 * the streaming kernel with splits sized for one workgroup per CU over all its
 * keys. args[i] is exactly as for g4a_attention and gives its result within
 * the same tolerance (bit-identical where g4a_attention would run the short
 * kernel with the same splits). A call runs in the batched launches when
 * T = 1, Hq = 8 * Hkv, Dh = Dv in {256, 512}, `splits` is 0, it sees at most
 * 32768 keys and its Hq, Hkv, Dh, sliding_window, kv_ring_cap, scale and
 * attn_softcap equal those of the first such call; every other call runs
 * afterwards as g4a_attention. Calls with explicit, ascending, non-contiguous
 * key positions run in streaming-kernel launches of their own, their visible
 * keys' positions staged from host memory in one upload (while a graph is
 * being captured they run as g4a_attention, which then reports the capture). Every call is
 * validated before any work is enqueued. The calls must be independent: no
 * call's out may overlap another call's q, k, v or out. *n_batched (may be
 * NULL) receives the number of calls that ran batched. No counterpart in the
 * reference, which decodes one sequence (rust/src/engine.rs:202-238): the
 * multi-sequence step a server runs. */
int g4a_attention_decode_batch(g4a_ctx *ctx, const g4a_attn_args *args, uint32_t n, uint32_t *n_batched);

/* The launch plan g4a_attention would use for `args` (no GPU work): the
 * trimmed key range [k_start, k_end) (rust/src/backend_wgpu.rs:929-936), the
 * kernel family and the split-K decomposition. */
typedef enum g4a_kernel_kind {
    G4A_KERNEL_NONE = 0,    /* nothing to launch (T == 0) or zero fill only */
    G4A_KERNEL_DECODE = 1,  /* split-K flash-decode (+ LSE combine if splits > 1) */
    G4A_KERNEL_PREFILL = 2, /* query-tiled prefill */
    G4A_KERNEL_GENERIC = 3, /* per-(query, head) fallback for other shapes */
    G4A_KERNEL_DECODE_SHORT = 4, /* short-context split-K decode, 32-key splits (+ LSE combine if splits > 1) */
} g4a_kernel_kind;

typedef struct g4a_attn_plan {
    uint32_t kernel; /* g4a_kernel_kind */
    uint32_t k_start, k_end;
    uint32_t splits, keys_per_split;
    size_t workspace_bytes;
} g4a_attn_plan;

/* The host dispatch's decisions for a call, without GPU work (a query: a
 * failure here does not discard an open graph capture). */
int g4a_attention_plan(g4a_ctx *ctx, const g4a_attn_args *args, g4a_attn_plan *plan);

/* ---- KV cache writes -----------------------------------------------------
 * Writes n_rows rows of row_elems floats from src (device) into the cache at
 * logical rows dst_row .. dst_row+n_rows-1. ring_cap == 0: linear cache,
 * logical row r is physical row r (the capacity buffer of
 * WgpuBackend::kv_append, rust/src/backend_wgpu.rs:1014-1055, whose growth the
 * caller manages). ring_cap > 0: logical row r lands in slot r % ring_cap; when
 * n_rows > ring_cap only the last ring_cap rows are written (the others would
 * be overwritten anyway). Stream-ordered. */
int g4a_kv_write(g4a_ctx *ctx, float *cache, uint32_t ring_cap, uint32_t row_elems, uint32_t dst_row,
                 const float *src, uint32_t n_rows);

/* ---- the attention producer: per-head RMSNorm, partial RoPE, KV write ----
 * Rows are (token, head) vectors of head_dim f32 values in [T, heads, head_dim]
 * layout. positions: host [T] or NULL (then token i has position pos0 + i).
 * RoPE is the reference's half-split partial rotation of the first rotary_dim
 * dims (rotary_dim even, <= head_dim; rust/src/backend_cpu.rs:248-268):
 * freq_j = theta^(-2j/rotary_dim) (libm powf, as the reference), ang = pos*freq_j,
 * y[j] = a*cos - b*sin, y[j + rotary_dim/2] = b*cos + a*sin. head_dim must be a
 * multiple of 4, at most 1024. Stream-ordered, like every op. */

/* Backend::head_norm_rope (rust/src/backend.rs:146-154; the wgpu backend's
 * RMSNORM_ROPE dispatch, rust/src/backend_wgpu.rs:877-893): y = rope(x * inv * w)
 * per row, inv = 1/sqrt(mean(x^2) + eps) (rust/src/backend_cpu.rs:149-172).
 * w NULL: unweighted norm. y may alias x. */
int g4a_head_norm_rope(g4a_ctx *ctx, const float *x, const float *w, float *y, uint32_t T, uint32_t heads,
                       uint32_t head_dim, uint32_t rotary_dim, const uint32_t *positions, uint32_t pos0,
                       float theta, float eps);
/* Backend::rms_norm (rust/src/backend.rs:103-104; rust/src/backend_cpu.rs:149-172) over
 * `rows` rows of `dim` values: y = x * inv (* w), w NULL for the unweighted
 * variant (the per-head V norm, rust/src/model.rs:274-275). */
int g4a_rms_norm(g4a_ctx *ctx, const float *x, const float *w, float *y, uint32_t rows, uint32_t dim, float eps);
/* Backend::rope (rust/src/backend.rs:117-118; rust/src/backend_cpu.rs:248-268). */
int g4a_rope(g4a_ctx *ctx, const float *x, float *y, uint32_t T, uint32_t heads, uint32_t head_dim,
             uint32_t rotary_dim, const uint32_t *positions, uint32_t pos0, float theta);

/* The attention block's producer in ONE launch (the q/k/v steps of
 * Gemma4Model::attention, rust/src/model.rs:256-281, followed by the KV append
 * of KVCache::append_and_read, rust/src/kvcache.rs:49-62):
 *   q_out = head_norm_rope(q, q_norm)   (rope only when q_norm is NULL);
 *   K rows = head_norm_rope(k, k_norm)  (rope only when k_norm is NULL) and
 *   V rows = unweighted per-head RMSNorm of v, written into k_cache / v_cache at
 *   logical rows cache_row + t: slot (cache_row + t) % kv_ring_cap for a ring,
 *   row cache_row + t for a linear cache (its capacity is the caller's, as for
 *   g4a_kv_write; a ring keeps only the call's last kv_ring_cap rows).
 * k = v = NULL for a layer that reads another layer's cache (rust/src/config.rs:152-159):
 * then only q is produced. */
typedef struct g4a_producer_args {
    const float *q;       /* [T, Hq, Dh] q projection */
    const float *k;       /* [T, Hkv, Dh] k projection, or NULL */
    const float *v;       /* [T, Hkv, Dh] v projection, or NULL */
    const float *q_norm;  /* [Dh] or NULL */
    const float *k_norm;  /* [Dh] or NULL */
    float *q_out;         /* [T, Hq, Dh] */
    float *k_cache;       /* [rows, Hkv, Dh] */
    float *v_cache;       /* [rows, Hkv, Dh] */
    uint32_t T, Hq, Hkv, Dh, rotary_dim;
    const uint32_t *positions; /* host [T] or NULL */
    uint32_t pos0;
    uint32_t cache_row;   /* logical cache row of token 0 */
    uint32_t kv_ring_cap; /* 0: linear cache */
    float theta, eps;
} g4a_producer_args;

int g4a_attn_producer(g4a_ctx *ctx, const g4a_producer_args *args);

/* ---- the rest of the backend trait (rust/src/backend.rs:99-168) -----------
 * Device pointers, n elements (or rows x dim); the same results as the
 * reference CPU backend: add, mul, scale, scale_by_tensor, slice_cols and
 * embed_rows bit-identical; gelu_tanh, geglu and softcap within the device
 * tanhf's last-bit difference; add_rms_norm and wide rms_norm within the
 * reordered sum of squares; g4a_linear as g4a_linear_q.
 * Backend::add / mul / scale / scale_by_tensor / gelu_tanh / geglu / softcap
 * (rust/src/backend.rs:107-116; rust/src/backend_cpu.rs:224-244): */
int g4a_add(g4a_ctx *ctx, const float *a, const float *b, float *y, size_t n);
int g4a_mul(g4a_ctx *ctx, const float *a, const float *b, float *y, size_t n);
int g4a_scale(g4a_ctx *ctx, const float *a, float s, float *y, size_t n);
/* y = a * s[0] with s a device scalar (the learned layer_scalar) */
int g4a_scale_by_tensor(g4a_ctx *ctx, const float *a, const float *s, float *y, size_t n);
int g4a_gelu_tanh(g4a_ctx *ctx, const float *a, float *y, size_t n);
/* y = gelu_tanh(gate) * up */
int g4a_geglu(g4a_ctx *ctx, const float *gate, const float *up, float *y, size_t n);
/* y = cap * tanh(a / cap) */
int g4a_softcap(g4a_ctx *ctx, const float *a, float cap, float *y, size_t n);
/* Backend::slice_cols (rust/src/backend.rs:123-124; rust/src/backend_cpu.rs:343-350):
 * y[r, c] = x[r * stride + offset + c] for c < width. */
int g4a_slice_cols(g4a_ctx *ctx, const float *x, uint32_t rows, uint32_t stride, uint32_t offset, uint32_t width,
                   float *y);
/* Backend::add_rms_norm (rust/src/backend.rs:136-145; the reference GPU's fused
 * RMSNORM, rust/src/kernels/rmsnorm.wgsl): y = (residual + rms_norm(x, w)) *
 * scale_by[0], scale_by (a device scalar) may be NULL. */
int g4a_add_rms_norm(g4a_ctx *ctx, const float *residual, const float *x, const float *w, const float *scale_by,
                     float *y, uint32_t rows, uint32_t dim, float eps);
/* Backend::embed_rows on an f32 table [V, D] (rust/src/backend_cpu.rs:138-144):
 * out[i, d] = table[ids[i] * D + d] * scale, ids a host array of T values < V. */
int g4a_embed_rows(g4a_ctx *ctx, const float *table, uint32_t V, uint32_t D, const uint32_t *ids, uint32_t T,
                   float scale, float *out);
/* Backend::linear with an f32 weight W [N, K] (rust/src/backend_cpu.rs:174-222;
 * the reference GPU's GEMV / MATMUL, rust/src/backend_wgpu.rs:768-806):
 * y[M, N] = x[M, K] . W^T; the word-parallel kernel when K % 4 == 0, x is
 * 16-byte aligned and K <= 16384 (reordered f32 sum), else one thread per
 * output in the CPU's order (bit-identical). */
int g4a_linear(g4a_ctx *ctx, const float *w, uint32_t N, uint32_t K, const float *x, float *y, uint32_t M);

/* ---- quantised projections (the calls on either side of attention) --------
 * A weight as the reference's QuantWeight (rust/src/backend.rs:12-58), in
 * device memory: logical shape [N, K]; row n's packed bytes start at
 * qbytes + n * row_bytes with row_bytes = K (signed_i8) or K / (8 / bits);
 * sub-byte fields are offset binary (value = raw - 2^(bits-1)) packed
 * LSB-first, signed_i8 rows are two's complement bytes (bits = 8, signed_i8
 * = 0 reads 8-bit offset binary); element (n, k) is multiplied by
 * scales[n * ceil(K / group_size) + k / group_size]. K must be a whole number
 * of bytes per row.
 *
 * Rows that are whole 32-bit words (K * bits % 32 == 0) with one scale per row
 * (group_size >= K), a 4-byte aligned qbytes, 16-byte aligned x and at most
 * 16384 activations per row once the row's words are padded to a multiple of
 * 64 run the word-parallel kernel (HBM-bound, f32 sums in another order than the
 * reference's, within f32 reordering error); with M >= 16, K % 64 == 0 and an
 * 8-byte aligned qbytes they run on the matrix cores instead (exact products,
 * f32 accumulation, the same error bound). g4a_linear_q with M <= 2, one scale
 * per row, rows of a multiple of 128 bytes, K <= 4096 (K % 64 == 0), a 16-byte
 * aligned qbytes and at least 16 MB of packed weights (the lm_head) runs on the
 * int8 matrix cores with x cut into exact digits: within a few f32 ulps of the
 * exact sum (an activation row holding an inf or NaN: the reference CPU's
 * order). Every other weight runs one thread per output in the reference CPU's
 * order (bit-identical for g4a_linear_q). */
typedef struct {
    const void *qbytes;
    const float *scales;
    uint32_t N, K;
    uint32_t bits;       /* 2, 4 or 8 */
    uint32_t signed_i8;  /* 1: I8 rows */
    uint32_t group_size; /* K (or more): one scale per row */
} g4a_qweight;

/* Backend::linear on a quantised weight (rust/src/backend.rs:105-106;
 * rust/src/backend_cpu.rs:174-222; the reference GPU's MATMUL_Q mode 0,
 * rust/src/backend_wgpu.rs:768-806): y[M, N] = x[M, K] . W^T (device x, y). */
int g4a_linear_q(g4a_ctx *ctx, const g4a_qweight *w, const float *x, float *y, uint32_t M);
/* Backend::linear_geglu (rust/src/backend.rs:156-161; MATMUL_Q mode 1,
 * rust/src/backend_wgpu.rs:808-821): y = gelu_tanh(x . Wg^T) * (x . Wu^T), both
 * weights of one shape and format. */
int g4a_linear_q_geglu(g4a_ctx *ctx, const g4a_qweight *w_gate, const g4a_qweight *w_up, const float *x, float *y,
                       uint32_t M);
/* Backend::linear_gelu_mul_cols (rust/src/backend.rs:162-168; MATMUL_Q mode 2,
 * rust/src/backend_wgpu.rs:823-832): y[m, n] = gelu_tanh((x . W^T)[m, n]) *
 * b[m * b_stride + b_off + n], b_off + N <= b_stride. */
int g4a_linear_q_gelu_mul_cols(g4a_ctx *ctx, const g4a_qweight *w, const float *x, const float *b, uint32_t b_stride,
                               uint32_t b_off, float *y, uint32_t M);
/* The attention block's output projection after its attention call
 * (Gemma4Model::attention, rust/src/model.rs:287-303: o_proj(attention(q, k, v))):
 * the results of g4a_attention(args) then g4a_linear_q(w, args->out, y, T),
 * with w->K = Hq * Dv; args->out receives the attention rows as usual. On a
 * context created with g4a_options::fuse_projection = 1, a decode
 * step (T = 1) that runs 2 .. 16 splits, with a projection the short-weight
 * word kernel takes (N below 64 per CU, one scale per row, a weight under the
 * int8 kernel's size threshold) and a 16-byte aligned args->out, launches no
 * LSE combine: the projection merges the split partials while it stages its
 * activation row, in the combine kernel's order, so y and args->out are
 * bit-identical to the two separate calls (sliding-window decode steps, 512
 * keys in 16 splits, qualify). Every other call, and every call on a default
 * context, runs the two separately: on MI355X the merged form measured
 * slower (each projection workgroup reads all 16 partials of the row). Replaces a decode step's ATTN_COMBINE dispatch
 * (rust/src/backend_wgpu.rs:958-968) and the o_proj linear after it
 * (rust/src/backend_wgpu.rs:768-806, called at rust/src/model.rs:303). */
int g4a_attention_linear_q(g4a_ctx *ctx, const g4a_attn_args *args, const g4a_qweight *w, float *y);
/* Backend::embed_rows on a quantised table [V, D] = [N, K] (rust/src/backend.rs:101-102;
 * rust/src/backend_cpu.rs:127-137; EMBED_Q, rust/src/backend_wgpu.rs:734-760):
 * out[i, d] = deq(ids[i], d) * scale, ids a host array of T values < N. */
int g4a_embed_rows_q(g4a_ctx *ctx, const g4a_qweight *table, const uint32_t *ids, uint32_t T, float scale,
                     float *out);

/* ---- graph capture ------------------------------------------------------- */
/* No counterpart in the reference (its wgpu backend records a command buffer
 * per pass and submits it on flush, rust/src/backend_wgpu.rs:11-15, :357-366).
 * For launch-bound callers
 * (a decode step's 35 attention calls, each of a few microseconds): every
 * launch the context enqueues between g4a_capture_begin and g4a_capture_end
 * is recorded into a HIP graph instead of running; g4a_graph_launch replays
 * it on the context's stream with the same pointers and arguments.
 * Capturable: attention with contiguous positions (q_pos0 / k_pos0), the
 * producer and norm/RoPE calls with contiguous positions, kv_write, every
 * projection, elementwise and norm op. A call that needs host staging
 * (explicit position arrays, embedding ids), a larger workspace or a new RoPE
 * table, and g4a_h2d / g4a_d2h / g4a_zero / g4a_sync / the timers, fail with
 * G4A_E_ARG while a capture is open: run such calls once before capturing.
 * After any failing call that enqueues work inside a capture, still call
 * g4a_capture_end, which then returns that first failure's code and no graph
 * (the recording would lack the refused call); a failing query
 * (g4a_attention_plan) enqueues nothing and leaves the capture usable. The
 * first g4a_capture_begin on a GPU also sets up g4a_attention_noalloc's
 * static scratch array there, so no-alloc calls record without allocating. Rows without visible keys are cleared by a fill kernel, not a
 * memset, so a replay clears them too. A graph replays with the workspace it
 * was captured with: a later eager call that needs a larger workspace gets a
 * new one and the old one is kept until the context's last graph is
 * destroyed. g4a_graph_launch refuses a graph captured on another context. A
 * graph that outlives its context can only be destroyed. */
typedef struct g4a_graph g4a_graph;
int g4a_capture_begin(g4a_ctx *ctx);
int g4a_capture_end(g4a_ctx *ctx, g4a_graph **graph);
int g4a_graph_launch(g4a_ctx *ctx, g4a_graph *graph);
int g4a_graph_destroy(g4a_graph *graph);

/* ---- decode steps at a device position (a captured decode loop) ----------
 * No counterpart in the reference (it records no graphs). A graph replays the
 * arguments it captured, so a decode step captured with host positions replays
 * the same token. These entry points take the token's position from a u32 in
 * device memory instead, read when the kernels run: a decode step captured
 * once replays token after token when the graph ends with g4a_u32_add on that
 * position.
 *
 * g4a_attention_devpos: g4a_attention for one query (T = 1, contiguous
 * positions: q_pos and k_pos NULL) at position *pos over keys at positions
 * k_pos0, k_pos0 + 1, ... (logical rows 0, 1, ..., of a linear cache or ring):
 * the visible keys are those at or before *pos, the last sliding_window of
 * them when it is set. args->S is the most keys any replay sees (the query at
 * position k_pos0 + S - 1 at most); the split plan and workspace are those of
 * that largest step, q_pos0 is ignored, and a position past it sees only the
 * first S keys. Results match g4a_attention on the same step, bit for bit
 * where both run the same kernels with the same split count (a sliding
 * window's short-kernel step; or g4a_attention with args->splits set to the
 * largest step's count); the splits past the step's keys are empty and merge
 * as zeros. Refused (G4A_E_UNSUPPORTED) for shapes that do not run on the
 * decode kernels.
 *
 * g4a_attn_producer_devpos: g4a_attn_producer for one token (T = 1,
 * positions NULL) at position *pos, written to logical cache row *pos (pos0
 * and cache_row are ignored). max_pos bounds the position: the RoPE tables
 * are built up to it by this call (so a capture of it needs no table growth),
 * and a position past it writes nothing. For a linear cache, max_pos must be
 * a row the cache holds.
 *
 * g4a_u32_add: counters[i] += inc (wrapping) for i < n, by a kernel (so it
 * records into a graph). */
int g4a_attention_devpos(g4a_ctx *ctx, const g4a_attn_args *args, const uint32_t *pos);
int g4a_attn_producer_devpos(g4a_ctx *ctx, const g4a_producer_args *args, const uint32_t *pos, uint32_t max_pos);
int g4a_u32_add(g4a_ctx *ctx, uint32_t *counters, uint32_t n, uint32_t inc);

/* ---- timing (HIP events on the context's stream) ----------------------- */
int g4a_timer_start(g4a_ctx *ctx);
/* Records the stop event, waits for it and returns the elapsed milliseconds. */
int g4a_timer_stop(g4a_ctx *ctx, float *ms);

/* Per-kernel timing: while enabled, every g4a_attention call records a HIP
 * event pair on the context's stream around its main kernel (decode, prefill
 * or generic; not the LSE combine), and so does every norm/RoPE/producer
 * launch, every decode and combine launch of g4a_attention_decode_batch and
 * every quantised projection / embedding launch.
 * g4a_kernel_timing_read waits for the
 * recorded pairs and returns their summed milliseconds and count, then clears
 * them. At most 4096 pairs are kept per read. Enabling clears old pairs. */
int g4a_kernel_timing(g4a_ctx *ctx, int enable);
int g4a_kernel_timing_read(g4a_ctx *ctx, double *total_ms, uint32_t *count);

/* ---- device facts --------------------------------------------------------- */
typedef struct g4a_device_info {
    int device;
    int compute_units;
    int clock_khz;
    size_t total_mem;
    char arch[64];
} g4a_device_info;

int g4a_get_device_info(g4a_ctx *ctx, g4a_device_info *info);

#ifdef __cplusplus
}
#endif
#endif /* G4A_H */
