"""TEST INFRASTRUCTURE ONLY: ctypes wrapper of the CPU oracle (oracle/attn_oracle.c).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module. It restates rust/src/backend_cpu.rs:270-336 (attention),
:63-91 (par_ranges), :149-172 (rms_norm) and :248-268 (rope); see
attn_oracle.c. head_norm_rope and producer are the compositions the reference
defines on top of them (rust/src/backend.rs:146-154, rust/src/model.rs:256-281,
rust/src/kvcache.rs:49-62).
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
