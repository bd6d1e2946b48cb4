"""Deterministic synthetic inputs for the attention path.

Two generators:

* `normal_f32(seed, stream, n)` — splitmix64 -> Box–Muller N(0,1) -> f32, the
  generator of the benchmark configurations. The reference has only uniform
  RNGs (rust/tests/common/mod.rs:15-42, rust/src/main.rs:306-333), so this one
  is ours; it is fully specified here so any implementation can reproduce it.
* `Lcg` — the LCG of the reference's parity tests
  (rust/tests/common/mod.rs:29-42), bit-exact in f32, so the inputs of
  `grouped_attention_parity` / `kernel_parity` can be regenerated.

Query and key rows are RMS-normalised per head with the reference's unweighted
rms_norm (rust/src/backend_cpu.rs:149-172, eps 1e-6 from
rust/assets/config.json): sequential f32 sum of squares, inv = 1/sqrt(ss/d+eps),
y = x*inv.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
RMS_EPS = np.float32(1e-6)


def _mix(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def splitmix64(seed: int, stream: int, n: int) -> np.ndarray:
    """n outputs of splitmix64 whose state starts at mix(seed*16 + stream)."""
    with np.errstate(over="ignore"):
        base = _mix(np.array([np.uint64(seed * 16 + stream)], dtype=np.uint64))[0]
        idx = np.arange(1, n + 1, dtype=np.uint64)
        return _mix(base + idx * _GOLDEN)


def normal_f32(seed: int, stream: int, n: int) -> np.ndarray:
    """n N(0,1) samples: Box–Muller on pairs of 53-bit uniforms, computed in f64, rounded to f32."""
    m = (n + 1) // 2
    bits = splitmix64(seed, stream, 2 * m) >> np.uint64(11)
    u1 = (bits[0::2].astype(np.float64) + 1.0) * (1.0 / 9007199254740992.0)  # (0, 1]
    u2 = bits[1::2].astype(np.float64) * (1.0 / 9007199254740992.0)  # [0, 1)
    r = np.sqrt(-2.0 * np.log(u1))
    t = 2.0 * np.pi * u2
    out = np.empty(2 * m, dtype=np.float64)
    out[0::2] = r * np.cos(t)
    out[1::2] = r * np.sin(t)
    return out[:n].astype(np.float32)


def rms_norm_rows(x: np.ndarray, eps: np.float32 = RMS_EPS) -> np.ndarray:
    """Unweighted per-row RMSNorm over the last axis with the reference's f32 arithmetic order."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    d = x.shape[-1]
    flat = x.reshape(-1, d)
    ss = np.zeros(flat.shape[0], dtype=np.float32)
    for j in range(d):  # sequential sum, vectorised across rows
        col = flat[:, j]
        ss = ss + col * col
    inv = np.float32(1.0) / np.sqrt(ss / np.float32(d) + eps)
    return (flat * inv[:, None]).reshape(x.shape).astype(np.float32)


@dataclass
class AttnInputs:
    q: np.ndarray  # [T, Hq, Dh]
    k: np.ndarray  # [S, Hkv, Dh]
    v: np.ndarray  # [S, Hkv, Dv]
    q_pos: np.ndarray  # [T] u32
    k_pos: np.ndarray  # [S] u32


def gemma_inputs(T: int, S: int, Dh: int, seed: int, Hq: int = 8, Hkv: int = 1, Dv: int | None = None,
                 q_pos: np.ndarray | None = None) -> AttnInputs:
    """The benchmark distribution: q, k ~ N(0,1) then RMS-normalised per head; v ~ N(0,1).

    Streams: q = 0, k = 1, v = 2. Positions: k_pos = 0..S-1; q_pos defaults to
    the last T positions (decode: S-1; prefill with T == S: 0..S-1).
    """
    Dv = Dh if Dv is None else Dv
    q = rms_norm_rows(normal_f32(seed, 0, T * Hq * Dh).reshape(T, Hq, Dh))
    k = rms_norm_rows(normal_f32(seed, 1, S * Hkv * Dh).reshape(S, Hkv, Dh))
    v = normal_f32(seed, 2, S * Hkv * Dv).reshape(S, Hkv, Dv)
    k_pos = np.arange(S, dtype=np.uint32)
    if q_pos is None:
        q_pos = np.arange(S - T, S, dtype=np.uint32)
    return AttnInputs(q, k, v, np.asarray(q_pos, dtype=np.uint32), k_pos)


class Lcg:
    """rust/tests/common/mod.rs:29-42: s = (s*1103515245 + 12345) & 0x7fffffff;
    f = (s as f32) / (0x7fffffff as f32); rand = (f*2 - 1)*scale, all in f32."""

    _DEN = np.float32(0x7FFFFFFF)  # rounds to 2^31 in f32, as `0x7fffffff as f32` does

    def __init__(self, seed: int):
        self.s = seed & 0xFFFFFFFF

    def states(self, n: int) -> np.ndarray:
        out = np.empty(n, dtype=np.uint32)
        s = self.s
        for i in range(n):
            s = (s * 1103515245 + 12345) & 0x7FFFFFFF
            out[i] = s
        self.s = s
        return out

    def next(self, n: int) -> np.ndarray:
        """n draws of Lcg::next: (s as f32) / (0x7fffffff as f32)."""
        return (self.states(n).astype(np.float32) / self._DEN).astype(np.float32)

    def rand(self, n: int, scale: float) -> np.ndarray:
        f = self.states(n).astype(np.float32) / self._DEN
        return ((f * np.float32(2.0) - np.float32(1.0)) * np.float32(scale)).astype(np.float32)

    def skip(self, n: int) -> None:
        self.states(n)


# The 8 cases of the reference's grouped_attention_parity (rust/tests/gpu.rs:268-277):
# (T, S, Hq, Hkv, Dh, window); Lcg seed 21, q/k/v drawn per case in order with scale 0.5,
# q_pos = last T positions, k_pos = 0..S-1, scale = 1/sqrt(Dh) (rust/tests/gpu.rs:278-291).
GROUPED_CASES = [
    (3, 300, 8, 1, 256, 0),
    (3, 300, 8, 1, 256, 150),
    (1, 700, 8, 1, 512, 0),
    (1, 900, 8, 1, 256, 512),
    (5, 5, 8, 1, 256, 0),
    (6, 70, 8, 1, 256, 3),
    (2, 200, 4, 1, 256, 0),
    (1, 64, 8, 2, 512, 0),
]


def grouped_parity_inputs():
    """Yield (case, q, k, v, q_pos, k_pos, scale, window) for rust/tests/gpu.rs:262-293."""
    r = Lcg(21)
    for (t, s, hq, hkv, dh, window) in GROUPED_CASES:
        q = r.rand(t * hq * dh, 0.5).reshape(t, hq, dh)
        k = r.rand(s * hkv * dh, 0.5).reshape(s, hkv, dh)
        v = r.rand(s * hkv * dh, 0.5).reshape(s, hkv, dh)
        kpos = np.arange(s, dtype=np.uint32)
        qpos = np.arange(s - t, s, dtype=np.uint32)
        scale = np.float32(1.0) / np.sqrt(np.float32(dh))
        yield (t, s, hq, hkv, dh, window), q, k, v, qpos, kpos, float(scale), window


def kernel_parity_attention_inputs():
    """The attention cases of kernel_parity (rust/tests/gpu.rs:122-142), Lcg seed 7.

    The earlier draws of that test are skipped by count: linear 17*40 + 23*40 +
    40, rmsNorm 5*48 + 48, elementwise 100 + 100, embed 30*16, rope 4*2*16,
    slice 4*20 + 2*20 + 3*20, kvAppend 3*200*8 (rust/tests/gpu.rs:43-121).
    """
    r = Lcg(7)
    r.skip(17 * 40 + 23 * 40 + 40 + 5 * 48 + 48 + 100 + 100 + 30 * 16 + 4 * 2 * 16 + 4 * 20 + 2 * 20 + 3 * 20
           + 3 * 200 * 8)
    t, s, hq, hkv, dh = 6, 6, 4, 1, 16
    q = r.rand(t * hq * dh, 1.0).reshape(t, hq, dh)
    k = r.rand(s * hkv * dh, 1.0).reshape(s, hkv, dh)
    v = r.rand(s * hkv * dh, 1.0).reshape(s, hkv, dh)
    pos = np.arange(6, dtype=np.uint32)
    yield "attention(GQA,sliding)", q, k, v, pos, pos, 0.25, 3
    t, s, hq, hkv, dh = 3, 300, 2, 1, 32
    q = r.rand(t * hq * dh, 0.5).reshape(t, hq, dh)
    k = r.rand(s * hkv * dh, 0.5).reshape(s, hkv, dh)
    v = r.rand(s * hkv * dh, 0.5).reshape(s, hkv, dh)
    kpos = np.arange(300, dtype=np.uint32)
    qpos = np.array([297, 298, 299], dtype=np.uint32)
    for window in (0, 150):
        yield f"attention(S=300, window={window})", q, k, v, qpos, kpos, 1.0, window


# ---- quantised weights --------------------------------------------------------

def pack_unsigned(values, bits: int) -> np.ndarray:
    """Raw unsigned fields of `bits` bits packed LSB-first into bytes (the
    reference's test helper rust/src/dequant.rs:53-63)."""
    v = np.asarray(values, np.uint32).ravel()
    per_byte = 8 // bits
    n = -(-v.size // per_byte)
    padded = np.zeros(n * per_byte, np.uint32)
    padded[:v.size] = v & ((1 << bits) - 1)
    fields = padded.reshape(n, per_byte)
    shifts = (np.arange(per_byte, dtype=np.uint32) * bits)[None, :]
    return (fields << shifts).sum(axis=1).astype(np.uint8)


def pack_int(values, bits: int) -> np.ndarray:
    """Signed values as stored by the checkpoint (rust/src/dequant.rs:37-51):
    offset binary (raw = value + 2^(bits-1)) for sub-byte, two's complement I8."""
    v = np.asarray(values, np.int64).ravel()
    if bits == 8:
        return (v & 0xFF).astype(np.uint8)
    return pack_unsigned((v + (1 << (bits - 1))) & ((1 << bits) - 1), bits)


def quant_weight(seed: int, N: int, K: int, bits: int, signed_i8: bool = False, group_size: int | None = None,
                 scale_lo: float = 0.01, scale_span: float = 0.05):
    """A random quantised weight [N, K]: uniform raw fields (or I8 bytes) and
    scales in [scale_lo, scale_lo + scale_span). Returns (qbytes [N, row_bytes],
    scales [N, ceil(K / group)], group_size)."""
    g = group_size or K
    rng = np.random.default_rng(seed)
    if signed_i8:
        qbytes = rng.integers(0, 256, size=(N, K), dtype=np.uint8)
    else:
        raw = rng.integers(0, 1 << bits, size=(N, K), dtype=np.uint32)
        qbytes = pack_unsigned(raw, bits).reshape(N, K * bits // 8)
    stride = -(-K // g)
    scales = (np.float32(scale_lo) + rng.random((N, stride), dtype=np.float32) * np.float32(scale_span))
    return qbytes, scales.astype(np.float32), g


def quant_parity_inputs():
    """The inputs of the reference's quantized_kernel_parity (rust/tests/gpu.rs:146-190),
    regenerated with its Lcg(9) stream in the same draw order. Yields dicts with
    name, qbytes, scales, N, K, bits, signed_i8, group_size and either x (linear)
    or ids + scale (embedding)."""
    r = Lcg(9)

    def scales(n):  # 0.01 + r.next() * 0.05
        return (r.next(n) * np.float32(0.05) + np.float32(0.01)).astype(np.float32)

    def randu(n, bits):  # (r.next() * (1 << bits) as f32).floor() as u32 % (1 << bits)
        return (np.floor(r.next(n) * np.float32(1 << bits)).astype(np.uint32) % (1 << bits)).astype(np.uint32)

    for bits in (4, 2):
        n, k = 40, 64
        vals = randu(n * k, bits)
        qb, sc = pack_unsigned(vals, bits), scales(n)
        for m in (5, 1):
            x = r.rand(m * k, 1.0).reshape(m, k)
            yield dict(name=f"linear_q{bits}_M{m}", qbytes=qb, scales=sc, N=n, K=k, bits=bits, signed_i8=False,
                       group_size=k, x=x)
    bits, n, k, m = 4, 21, 52, 3
    vals = randu(n * k, bits)
    qb, sc = pack_unsigned(vals, bits), scales(n)
    x = r.rand(m * k, 1.0).reshape(m, k)
    yield dict(name="linear_q4_oddK", qbytes=qb, scales=sc, N=n, K=k, bits=bits, signed_i8=False, group_size=k, x=x)
    n, k, m = 30, 48, 4
    qb = np.floor(r.next(n * k) * np.float32(256.0)).astype(np.uint32).astype(np.uint8)
    sc = (r.next(n) * np.float32(0.03) + np.float32(0.01)).astype(np.float32)
    x = r.rand(m * k, 1.0).reshape(m, k)
    yield dict(name="linear_i8", qbytes=qb, scales=sc, N=n, K=k, bits=8, signed_i8=True, group_size=k, x=x)
    v, d, bits, group = 50, 32, 4, 16
    vals = randu(v * d, bits)
    qb = pack_unsigned(vals, bits)
    sc = (r.next(v * (d // group)) * np.float32(0.04) + np.float32(0.02)).astype(np.float32)
    yield dict(name="embed_q4_grouped", qbytes=qb, scales=sc, N=v, K=d, bits=bits, signed_i8=False,
               group_size=group, ids=np.array([3, 7, 49, 0, 21], np.uint32), scale=float(np.sqrt(np.float32(d))))


# ---- the Gemma-4-E2B per-token attention schedule ----------------
# Layer facts of rust/assets/config.json: 35 layers, the last 20 share KV,
# global (full-attention) layers 4, 9, ..., 34 with head_dim 512, the others
# sliding-window-512 with head_dim 256.
E2B_LAYERS = 35
E2B_KV_SHARED = 20
E2B_GLOBAL = frozenset(range(4, E2B_LAYERS, 5))
E2B_WINDOW = 512


def kv_source_layer(i: int, n_layers: int = E2B_LAYERS, n_shared: int = E2B_KV_SHARED,
                    is_global=lambda j: j in E2B_GLOBAL) -> int:
    """The layer whose KV cache layer i reads (rust/src/config.rs:152-159): itself
    below the shared region, else the most recent earlier non-shared layer of the
    same attention type."""
    first_shared = max(n_layers - n_shared, 0)
    if i < first_shared:
        return i
    for j in range(first_shared - 1, -1, -1):
        if is_global(j) == is_global(i):
            return j
    return i


@dataclass
class ScheduleLayer:
    index: int
    is_global: bool
    Dh: int
    src: int           # kv_source_layer(index)
    q: np.ndarray      # [1, 8, Dh], unit-RMS per head


@dataclass
class ScheduleCache:
    k: np.ndarray      # global: [S, 1, 512] rows 0..S-1; local: a [ring, 1, 256] ring
    v: np.ndarray
    ring_cap: int      # 0 for a linear (global) cache
    k_pos: np.ndarray  # absolute position of each logical key the layer can see


def schedule_token(S: int = 32768, seed: int = 4, ring: int = E2B_WINDOW):
    """One decode token of the 35-layer schedule at context S (the query at
    position S-1): (layers, caches). Global caches hold keys 0..S-1; a local
    layer's ring of `ring` slots holds positions S-ring..S-1, position p in slot
    p % ring. Streams per layer li (seed*100 + li): q = 0, k = 1, v = 2, with q
    and k RMS-normalised per head, v N(0,1). Only the 15 source layers own a
    cache (3 global, 12 local)."""
    layers, caches = [], {}
    for i in range(E2B_LAYERS):
        g = i in E2B_GLOBAL
        dh = 512 if g else 256
        q = rms_norm_rows(normal_f32(seed * 100 + i, 0, 8 * dh).reshape(1, 8, dh))
        layers.append(ScheduleLayer(i, g, dh, kv_source_layer(i), q))
    for li in sorted({l.src for l in layers}):
        g = li in E2B_GLOBAL
        rows, dh = (S, 512) if g else (ring, 256)
        k = rms_norm_rows(normal_f32(seed * 100 + li, 1, rows * dh).reshape(rows, 1, dh))
        v = normal_f32(seed * 100 + li, 2, rows * dh).reshape(rows, 1, dh)
        if g:
            caches[li] = ScheduleCache(k, v, 0, np.arange(S, dtype=np.uint32))
        else:
            # ring row r holds the position p in [S-ring, S) with p % ring == r
            caches[li] = ScheduleCache(k, v, ring, np.arange(S - ring, S, dtype=np.uint32))
    return layers, caches


def unroll_ring(c: ScheduleCache):
    """(k, v) of a schedule cache in logical key order (k_pos order), for the oracle."""
    if not c.ring_cap:
        return c.k, c.v
    slots = c.k_pos % np.uint32(c.ring_cap)
    return np.ascontiguousarray(c.k[slots]), np.ascontiguousarray(c.v[slots])


# ---- the reference's kernel benchmark inputs ----------------------------------

def _xs_step(s: int) -> int:
    """One step of rust/src/main.rs:306-316: s ^= s << 13; s ^= s >> 17; s ^= s << 5 (u32)."""
    s ^= (s << 13) & 0xFFFFFFFF
    s ^= s >> 17
    s ^= (s << 5) & 0xFFFFFFFF
    return s


def _gf2_matrix_of(step) -> np.ndarray:
    """The 32x32 GF(2) matrix of a linear map on u32 states, as 32 column images."""
    return np.array([step(1 << b) for b in range(32)], dtype=np.uint64)


def _gf2_apply(cols: np.ndarray, states: np.ndarray) -> np.ndarray:
    """Applies the linear map given by its column images to every state
    (vectorised: one 256-entry table per state byte, four lookups a state)."""
    bits = np.arange(8, dtype=np.uint64)
    idx = np.arange(256, dtype=np.uint64)
    st = states.astype(np.uint64)
    out = np.zeros(st.shape, dtype=np.uint64)
    for byte in range(4):
        col = cols[8 * byte:8 * byte + 8]
        on = ((idx[:, None] >> bits[None, :]) & np.uint64(1)).astype(bool)
        table = np.bitwise_xor.reduce(np.where(on, col[None, :], np.uint64(0)), axis=1)
        out ^= table[((st >> np.uint64(8 * byte)) & np.uint64(255)).astype(np.intp)]
    return out


def _gf2_compose(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Column images of a(b(x))."""
    return _gf2_apply(a, b)


def _gf2_power(cols: np.ndarray, n: int) -> np.ndarray:
    result = np.array([1 << b for b in range(32)], dtype=np.uint64)  # identity
    base = cols.copy()
    while n:
        if n & 1:
            result = _gf2_compose(base, result)
        base = _gf2_compose(base, base)
        n >>= 1
    return result


class Xorshift:
    """The xorshift32 of the reference's benchmark (rust/src/main.rs:306-333):
    next() is the state after one step; f() = next() as f32 / u32::MAX as f32;
    f32s(n, sc, base) = base + (f()*2 - 1)*sc, every op in f32. The map is linear
    over GF(2), so skip(n) jumps ahead by a matrix power, and n draws come out
    in log2(n) vectorised doublings: states 1..m advanced by m steps are states
    m+1..2m."""

    _POW2: list = []  # column images of the step map raised to 2^k

    def __init__(self, seed: int):
        self.s = seed & 0xFFFFFFFF
        if not Xorshift._POW2:
            Xorshift._POW2.append(_gf2_matrix_of(_xs_step))
            for _ in range(40):
                m = Xorshift._POW2[-1]
                Xorshift._POW2.append(_gf2_compose(m, m))

    def skip(self, n: int) -> None:
        st = np.array([self.s], np.uint64)
        k = 0
        while n:
            if n & 1:
                st = _gf2_apply(self._POW2[k], st)
            n >>= 1
            k += 1
        self.s = int(st[0])

    def next(self, n: int) -> np.ndarray:
        """The next n outputs (u32), advancing the state."""
        if n == 0:
            return np.empty(0, dtype=np.uint32)
        states = np.array([_xs_step(self.s)], dtype=np.uint64)
        k = 0
        while states.size < n:
            states = np.concatenate([states, _gf2_apply(self._POW2[k], states)])
            k += 1
        out = states[:n].astype(np.uint32)
        self.s = int(out[-1])
        return out

    def f32s(self, n: int, sc: float, base: float = 0.0) -> np.ndarray:
        f = (self.next(n).astype(np.float32) / np.float32(4294967295.0)).astype(np.float32)
        return (np.float32(base) + (f * np.float32(2.0) - np.float32(1.0)) * np.float32(sc)).astype(np.float32)


# The attention cases of the reference's `bench --kernels` (rust/src/main.rs:544-560):
# (Dh, S, window), batch 1, 8 query heads over 1 kv head, scale 1/16, q_pos = S-1.
REFERENCE_BENCH_CASES = [(256, 512, 512), (256, 2048, 512), (512, 2048, 0), (256, 8192, 512), (512, 8192, 0)]


def reference_bench_draws_before_attention() -> int:
    """Xorshift(987654321) draws the reference's kernel benchmark makes before its
    first attention case (rust/src/main.rs:493-543): each quantised weight draws
    its packed bytes (one draw per 4 bytes; 8/bits fields a byte) then one scale
    per row, each activation one draw per element, the f32 GEMV weight one per
    element, in the order the cases are built."""
    def qt(n, k, bits):
        return (n * k // (8 // bits) + 3) // 4 + n
    return (qt(262144, 1536, 2) + 1536            # lm_head 2b + x
            + qt(6144, 1536, 4) + 1536            # mlp gate 4b + x
            + 2 * qt(6144, 1536, 4) + 1536        # gate + up GeGLU + x
            + qt(12288, 1536, 2) + 64 * 1536      # prefill gate 2b + x (M = 64)
            + qt(1536, 6144, 2) + 6144            # mlp down 2b + x
            + qt(2048, 1536, 4) + 1536            # q_proj 4b + x
            + 8960 * 1536 + 1536)                 # gemv f32 weight + x


def reference_bench_inputs():
    """Yield ((Dh, S, window), q [1,8,Dh], k [S,1,Dh], v [S,1,Dh]) for the five
    attention cases of rust/src/main.rs:544-560, drawn from Xorshift(987654321)
    after the earlier cases' draws: U(-0.1, 0.1) in f32 (rust/src/main.rs:328-330)."""
    r = Xorshift(987654321)
    r.skip(reference_bench_draws_before_attention())
    for dh, s, window in REFERENCE_BENCH_CASES:
        q = r.f32s(8 * dh, 0.1).reshape(1, 8, dh)
        k = r.f32s(s * dh, 0.1).reshape(s, 1, dh)
        v = r.f32s(s * dh, 0.1).reshape(s, 1, dh)
        yield (dh, s, window), q, k, v
