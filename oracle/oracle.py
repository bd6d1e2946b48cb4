"""TEST INFRASTRUCTURE ONLY: ctypes wrapper of the CPU oracle (oracle/attn_oracle.c).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module. It restates rust/src/backend_cpu.rs:270-336 (attention),
:63-91 (par_ranges) and :149-172 (rms_norm); see attn_oracle.c.
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
