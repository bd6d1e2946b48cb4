"""TEST INFRASTRUCTURE ONLY: ctypes wrapper of the CPU oracle (oracle/attn_oracle.c).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module. It restates rust/src/backend_cpu.rs:270-336 (attention),
:63-91 (par_ranges), :149-172 (rms_norm) and :248-268 (rope); see
attn_oracle.c. head_norm_rope and producer are the compositions the reference
defines on top of them (rust/src/backend.rs:146-154, rust/src/model.rs:256-281,
rust/src/kvcache.rs:49-62). The quantised projections restate
rust/src/backend.rs:44-58 (QuantWeight::deq), rust/src/backend_cpu.rs:174-222
(linear), :55-58 (gelu_tanh) and :127-145 (embed_rows); linear_q_geglu and
linear_q_gelu_mul_cols are the trait's default compositions
(rust/src/backend.rs:156-168); see linear_oracle.c.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "_build" / "liboracle.so"
_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} missing: run __graft_entry__.build()")
        L = ctypes.CDLL(str(LIB_PATH))
        vp, sz = ctypes.c_void_p, ctypes.c_size_t
        L.oracle_attention.restype = ctypes.c_int
        L.oracle_attention.argtypes = [vp, vp, vp, vp, sz, sz, sz, sz, sz, sz, vp, vp, ctypes.c_float,
                                       ctypes.c_uint32, ctypes.c_float, ctypes.c_int]
        L.oracle_attention_f64.restype = None
        L.oracle_attention_f64.argtypes = [vp, vp, vp, vp, sz, sz, sz, sz, sz, sz, vp, vp, ctypes.c_double,
                                           ctypes.c_uint32, ctypes.c_double]
        L.oracle_rms_norm.restype = None
        L.oracle_rms_norm.argtypes = [vp, vp, vp, sz, sz, ctypes.c_float]
        L.oracle_rope.restype = None
        L.oracle_rope.argtypes = [vp, vp, sz, sz, sz, sz, vp, ctypes.c_float]
        L.oracle_deq.restype = ctypes.c_float
        L.oracle_deq.argtypes = [vp, vp, sz, ctypes.c_uint32, ctypes.c_int, sz, sz, sz]
        L.oracle_linear_q.restype = None
        L.oracle_linear_q.argtypes = [vp, vp, sz, sz, ctypes.c_uint32, ctypes.c_int, sz, vp, sz, vp]
        L.oracle_gelu_tanh.restype = ctypes.c_float
        L.oracle_gelu_tanh.argtypes = [ctypes.c_float]
        L.oracle_gelu_tanh_n.restype = None
        L.oracle_gelu_tanh_n.argtypes = [vp, vp, sz]
        L.oracle_embed_rows_q.restype = None
        L.oracle_embed_rows_q.argtypes = [vp, vp, sz, sz, ctypes.c_uint32, ctypes.c_int, sz, vp, sz,
                                          ctypes.c_float, vp]
        L.oracle_linear_f32.restype = None
        L.oracle_linear_f32.argtypes = [vp, sz, sz, vp, sz, vp]
        L.oracle_softcap_n.restype = None
        L.oracle_softcap_n.argtypes = [vp, ctypes.c_float, vp, sz]
        L.oracle_embed_rows_f32.restype = None
        L.oracle_embed_rows_f32.argtypes = [vp, sz, vp, sz, ctypes.c_float, vp]
        L.oracle_thread_count.restype = ctypes.c_size_t
        L.oracle_thread_count.argtypes = [sz, ctypes.c_int]
        _lib = L
    return _lib


def _prep(q, k, v, q_pos, k_pos):
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    T, Hq, Dh = q.shape
    S, Hkv, _ = k.shape
    Dv = v.shape[2]
    if k_pos is None:
        k_pos = np.arange(S, dtype=np.uint32)
    if q_pos is None:
        q_pos = np.arange(S - T, S, dtype=np.uint32)
    q_pos = np.ascontiguousarray(q_pos, np.uint32)
    k_pos = np.ascontiguousarray(k_pos, np.uint32)
    assert q_pos.shape == (T,) and k_pos.shape == (S,)
    return q, k, v, q_pos, k_pos, (T, S, Hq, Hkv, Dh, Dv)


def attention(q, k, v, q_pos=None, k_pos=None, scale=1.0, window=0, softcap=0.0, threads=0):
    """CpuBackend::attention -> [T, Hq*Dv] f32. threads=0 follows GEMMA_CPU_THREADS / nproc."""
    q, k, v, q_pos, k_pos, (T, S, Hq, Hkv, Dh, Dv) = _prep(q, k, v, q_pos, k_pos)
    out = np.empty((T, Hq * Dv), np.float32)
    lib().oracle_attention(q.ctypes.data, k.ctypes.data, v.ctypes.data, out.ctypes.data, T, S, Hq, Hkv, Dh, Dv,
                           q_pos.ctypes.data, k_pos.ctypes.data, scale, window, softcap, threads)
    return out


def attention_f64(q, k, v, q_pos=None, k_pos=None, scale=1.0, window=0, softcap=0.0):
    """f64 brute force of the same masked attention -> [T, Hq*Dv] f64."""
    q, k, v, q_pos, k_pos, (T, S, Hq, Hkv, Dh, Dv) = _prep(q, k, v, q_pos, k_pos)
    out = np.empty((T, Hq * Dv), np.float64)
    lib().oracle_attention_f64(q.ctypes.data, k.ctypes.data, v.ctypes.data, out.ctypes.data, T, S, Hq, Hkv, Dh, Dv,
                               q_pos.ctypes.data, k_pos.ctypes.data, float(scale), window, float(softcap))
    return out


def rms_norm(x, w=None, eps=1e-6):
    x = np.ascontiguousarray(x, np.float32)
    d = x.shape[-1]
    y = np.empty_like(x)
    wp = None
    if w is not None:
        w = np.ascontiguousarray(w, np.float32)
        wp = w.ctypes.data
    lib().oracle_rms_norm(x.ctypes.data, wp, y.ctypes.data, x.size // d, d, eps)
    return y


def thread_count(rows: int, requested: int = 0) -> int:
    return int(lib().oracle_thread_count(rows, requested))


def rope(x, positions, theta, rotary_dim):
    """CpuBackend::rope on x [T, heads, head_dim] -> same shape (rust/src/backend_cpu.rs:248-268)."""
    x = np.ascontiguousarray(x, np.float32)
    T, heads, dh = x.shape
    pos = np.ascontiguousarray(positions, np.uint32)
    assert pos.shape == (T,)
    y = np.empty_like(x)
    lib().oracle_rope(x.ctypes.data, y.ctypes.data, T, heads, dh, rotary_dim, pos.ctypes.data, theta)
    return y


def head_norm_rope(x, w, eps, positions, theta, rotary_dim):
    """Backend::head_norm_rope's default (rust/src/backend.rs:146-154): per-row
    rms_norm over head_dim (weighted when w is given), then rope."""
    x = np.ascontiguousarray(x, np.float32)
    T, heads, dh = x.shape
    normed = rms_norm(x.reshape(T * heads, dh), w, eps).reshape(T, heads, dh)
    return rope(normed, positions, theta, rotary_dim)


def producer(q, k, v, q_norm, k_norm, positions, theta, rotary_dim, eps):
    """The q/k/v steps of Gemma4Model::attention (rust/src/model.rs:256-281):
    q and k through head_norm_rope (rope only without a norm weight), v through
    the unweighted per-head rms_norm. Returns (q_out, k_rows, v_rows)."""
    def qk(x, w):
        return head_norm_rope(x, w, eps, positions, theta, rotary_dim) if w is not None else \
            rope(x, positions, theta, rotary_dim)
    q_out = qk(q, q_norm)
    if k is None:
        return q_out, None, None
    T, hkv, dh = k.shape
    v_rows = rms_norm(np.ascontiguousarray(v, np.float32).reshape(T * hkv, dh), None, eps).reshape(T, hkv, dh)
    return q_out, qk(k, k_norm), v_rows


class QWeight:
    """A quantised weight as the reference's QuantWeight (rust/src/backend.rs:12-25):
    qbytes [N, row_bytes] u8 (sub-byte offset-binary fields packed LSB-first, or
    I8), scales [N, ceil(K / group_size)] f32, logical shape [N, K]."""

    def __init__(self, qbytes, scales, N, K, bits, signed_i8=False, group_size=None):
        self.qbytes = np.ascontiguousarray(qbytes, np.uint8)
        self.scales = np.ascontiguousarray(scales, np.float32)
        self.N, self.K, self.bits, self.signed_i8 = int(N), int(K), int(bits), bool(signed_i8)
        self.group_size = int(group_size or K)


def deq(w: QWeight, n: int, k: int) -> float:
    return float(lib().oracle_deq(w.qbytes.ctypes.data, w.scales.ctypes.data, w.K, w.bits, int(w.signed_i8),
                                  w.group_size, n, k))


def linear_q(x, w: QWeight):
    """CpuBackend::linear on a quantised weight: x [M, K] -> [M, N] f32."""
    x = np.ascontiguousarray(x, np.float32)
    M = x.shape[0]
    assert x.shape == (M, w.K)
    y = np.empty((M, w.N), np.float32)
    lib().oracle_linear_q(w.qbytes.ctypes.data, w.scales.ctypes.data, w.N, w.K, w.bits, int(w.signed_i8),
                          w.group_size, x.ctypes.data, M, y.ctypes.data)
    return y


def gelu_tanh(x):
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    lib().oracle_gelu_tanh_n(x.ctypes.data, y.ctypes.data, x.size)
    return y


def linear_q_geglu(x, w_gate: QWeight, w_up: QWeight):
    """Backend::linear_geglu's default: gelu(x Wg^T) * (x Wu^T)."""
    return gelu_tanh(linear_q(x, w_gate)) * linear_q(x, w_up)


def linear_q_gelu_mul_cols(x, w: QWeight, b, offset):
    """Backend::linear_gelu_mul_cols's default: gelu(x W^T) * b[:, offset:offset+N]."""
    b = np.ascontiguousarray(b, np.float32)
    return gelu_tanh(linear_q(x, w)) * b[:, offset:offset + w.N]


def embed_rows_q(w: QWeight, ids, scale):
    """CpuBackend::embed_rows on a quantised table [V, D]: [T, D] f32."""
    ids = np.ascontiguousarray(ids, np.uint32)
    out = np.empty((ids.size, w.K), np.float32)
    lib().oracle_embed_rows_q(w.qbytes.ctypes.data, w.scales.ctypes.data, w.N, w.K, w.bits, int(w.signed_i8),
                              w.group_size, ids.ctypes.data, ids.size, scale, out.ctypes.data)
    return out


# ---- the rest of the trait's ops (rust/src/backend_cpu.rs:127-145, :224-244, :343-350;
# rust/src/backend.rs:136-145). add / mul / scale are single IEEE f32 operations per
# element, exactly numpy's float32 arithmetic.

def add(a, b):
    return (np.asarray(a, np.float32) + np.asarray(b, np.float32)).astype(np.float32)


def mul(a, b):
    return (np.asarray(a, np.float32) * np.asarray(b, np.float32)).astype(np.float32)


def scale(a, s):
    return (np.asarray(a, np.float32) * np.float32(s)).astype(np.float32)


def geglu(gate, up):
    """CpuBackend::geglu: mul(gelu_tanh(gate), up)."""
    return mul(gelu_tanh(gate), up)


def softcap(a, cap):
    a = np.ascontiguousarray(a, np.float32)
    y = np.empty_like(a)
    lib().oracle_softcap_n(a.ctypes.data, cap, y.ctypes.data, a.size)
    return y


def slice_cols(x, offset, width):
    x = np.asarray(x, np.float32)
    return np.ascontiguousarray(x[:, offset:offset + width])


def add_rms_norm(residual, x, w, eps, scale_by=None):
    """Backend::add_rms_norm's default (rust/src/backend.rs:136-145):
    h = add(residual, rms_norm(x, w)); h * s[0] when scale_by is given."""
    x = np.ascontiguousarray(x, np.float32)
    h = add(residual, rms_norm(x.reshape(-1, x.shape[-1]), w, eps).reshape(x.shape))
    return scale(h, np.float32(scale_by)) if scale_by is not None else h


def linear_f32(x, w):
    """CpuBackend::linear on an f32 weight: x [M, K], w [N, K] -> [M, N]."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    M, K = x.shape
    N = w.shape[0]
    y = np.empty((M, N), np.float32)
    lib().oracle_linear_f32(w.ctypes.data, N, K, x.ctypes.data, M, y.ctypes.data)
    return y


def embed_rows_f32(table, ids, scale_):
    table = np.ascontiguousarray(table, np.float32)
    ids = np.ascontiguousarray(ids, np.uint32)
    out = np.empty((ids.size, table.shape[1]), np.float32)
    lib().oracle_embed_rows_f32(table.ctypes.data, table.shape[1], ids.ctypes.data, ids.size, scale_,
                                out.ctypes.data)
    return out
