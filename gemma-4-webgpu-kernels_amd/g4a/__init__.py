"""Python binding of libg4a.so (include/g4a.h) over ctypes.

Host-side plumbing for the tests and the benchmark: device buffers, the
attention op with the reference's AttnOpts semantics
(rust/src/backend.rs:59-69), KV writes and stream timers. Every call goes
through the C-ABI; nothing here computes attention. Loading fails loudly when
the library or its gfx950 code object has not been built.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from pathlib import Path
from typing import Optional, Sequence

import numpy as np

PKG_DIR = Path(__file__).resolve().parents[1]
BUILD_DIR = PKG_DIR / "_build"
LIB_PATH = BUILD_DIR / "libg4a.so"
HSACO_PATH = BUILD_DIR / "g4a_kernels.hsaco"
HEADER_PATH = PKG_DIR.parent / "include" / "g4a.h"

G4A_OK = 0
# G4A_NOALLOC_SCRATCH_BYTES of include/g4a.h: the static scratch of g4a_attention_noalloc
NOALLOC_SCRATCH_BYTES = 64 << 20
KERNEL_NAMES = {0: "none", 1: "decode", 2: "prefill", 3: "generic", 4: "decode_short"}

_u32p = ctypes.POINTER(ctypes.c_uint32)
_f32p = ctypes.c_void_p


class Options(ctypes.Structure):
    """g4a_options (include/g4a.h): a context's kernel-selection options."""
    _fields_ = [("size", ctypes.c_uint32), ("short_decode", ctypes.c_int32), ("short_max_wgs", ctypes.c_uint32),
                ("batch_kernel", ctypes.c_int32), ("batch_keys_per_split", ctypes.c_uint32),
                ("linear_i8", ctypes.c_int32), ("fuse_projection", ctypes.c_int32)]


class AttnArgs(ctypes.Structure):
    _fields_ = [
        ("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p), ("out", ctypes.c_void_p),
        ("T", ctypes.c_uint32), ("S", ctypes.c_uint32), ("Hq", ctypes.c_uint32), ("Hkv", ctypes.c_uint32),
        ("Dh", ctypes.c_uint32), ("Dv", ctypes.c_uint32),
        ("q_pos", _u32p), ("k_pos", _u32p), ("q_pos0", ctypes.c_uint32), ("k_pos0", ctypes.c_uint32),
        ("scale", ctypes.c_float), ("sliding_window", ctypes.c_uint32), ("attn_softcap", ctypes.c_float),
        ("kv_ring_cap", ctypes.c_uint32), ("splits", ctypes.c_uint32),
    ]


class AttnPlan(ctypes.Structure):
    _fields_ = [
        ("kernel", ctypes.c_uint32), ("k_start", ctypes.c_uint32), ("k_end", ctypes.c_uint32),
        ("splits", ctypes.c_uint32), ("keys_per_split", ctypes.c_uint32), ("workspace_bytes", ctypes.c_size_t),
    ]


class ProducerArgs(ctypes.Structure):
    _fields_ = [
        ("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p),
        ("q_norm", ctypes.c_void_p), ("k_norm", ctypes.c_void_p), ("q_out", ctypes.c_void_p),
        ("k_cache", ctypes.c_void_p), ("v_cache", ctypes.c_void_p),
        ("T", ctypes.c_uint32), ("Hq", ctypes.c_uint32), ("Hkv", ctypes.c_uint32), ("Dh", ctypes.c_uint32),
        ("rotary_dim", ctypes.c_uint32), ("positions", _u32p), ("pos0", ctypes.c_uint32),
        ("cache_row", ctypes.c_uint32), ("kv_ring_cap", ctypes.c_uint32),
        ("theta", ctypes.c_float), ("eps", ctypes.c_float),
    ]


class QWeightArgs(ctypes.Structure):
    """g4a_qweight: a quantised weight [N, K] in device memory."""
    _fields_ = [
        ("qbytes", ctypes.c_void_p), ("scales", ctypes.c_void_p), ("N", ctypes.c_uint32), ("K", ctypes.c_uint32),
        ("bits", ctypes.c_uint32), ("signed_i8", ctypes.c_uint32), ("group_size", ctypes.c_uint32),
    ]


class DeviceInfo(ctypes.Structure):
    _fields_ = [
        ("device", ctypes.c_int), ("compute_units", ctypes.c_int), ("clock_khz", ctypes.c_int),
        ("total_mem", ctypes.c_size_t), ("arch", ctypes.c_char * 64),
    ]


class G4aError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"g4a error {code}: {msg}")
        self.code = code


_lib: Optional[ctypes.CDLL] = None


def load_library(path: Path = LIB_PATH) -> ctypes.CDLL:
    """Load libg4a.so and declare its C-ABI. Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not Path(path).exists():
        raise RuntimeError(f"{path} is missing: build it first (python -c 'import __graft_entry__ as g; g.build()')")
    lib = ctypes.CDLL(str(path))
    vp, sz, c_int = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int
    ctxp = ctypes.c_void_p
    sig = {
        "g4a_create": (c_int, [c_int, ctypes.c_char_p, ctypes.POINTER(ctxp)]),
        "g4a_create_with": (c_int, [c_int, ctypes.c_char_p, ctypes.POINTER(Options), ctypes.POINTER(ctxp)]),
        "g4a_default_options": (None, [ctypes.POINTER(Options)]),
        "g4a_destroy": (None, [ctxp]),
        "g4a_last_error": (ctypes.c_char_p, [ctxp]),
        "g4a_stream": (c_int, [ctxp, ctypes.POINTER(vp)]),
        "g4a_malloc": (c_int, [ctxp, sz, ctypes.POINTER(vp)]),
        "g4a_free": (c_int, [ctxp, vp]),
        "g4a_h2d": (c_int, [ctxp, vp, vp, sz]),
        "g4a_d2h": (c_int, [ctxp, vp, vp, sz]),
        "g4a_d2d": (c_int, [ctxp, vp, vp, sz]),
        "g4a_zero": (c_int, [ctxp, vp, sz]),
        "g4a_sync": (c_int, [ctxp]),
        "g4a_attention": (c_int, [ctxp, ctypes.POINTER(AttnArgs)]),
        "g4a_attention_noalloc": (c_int, [ctxp, ctypes.POINTER(AttnArgs)]),
        "g4a_attention_devpos": (c_int, [ctxp, ctypes.POINTER(AttnArgs), vp]),
        "g4a_attn_producer_devpos": (c_int, [ctxp, ctypes.POINTER(ProducerArgs), vp, ctypes.c_uint32]),
        "g4a_u32_add": (c_int, [ctxp, vp, ctypes.c_uint32, ctypes.c_uint32]),
        "g4a_attention_batch": (c_int, [ctxp, ctypes.POINTER(AttnArgs), ctypes.c_uint32]),
        "g4a_attention_decode_batch": (c_int, [ctxp, ctypes.POINTER(AttnArgs), ctypes.c_uint32, _u32p]),
        "g4a_attention_plan": (c_int, [ctxp, ctypes.POINTER(AttnArgs), ctypes.POINTER(AttnPlan)]),
        "g4a_kv_write": (c_int, [ctxp, vp, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, vp, ctypes.c_uint32]),
        "g4a_head_norm_rope": (c_int, [ctxp, vp, vp, vp] + [ctypes.c_uint32] * 4 + [_u32p, ctypes.c_uint32,
                                                                                    ctypes.c_float, ctypes.c_float]),
        "g4a_rms_norm": (c_int, [ctxp, vp, vp, vp, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_float]),
        "g4a_rope": (c_int, [ctxp, vp, vp] + [ctypes.c_uint32] * 4 + [_u32p, ctypes.c_uint32, ctypes.c_float]),
        "g4a_attn_producer": (c_int, [ctxp, ctypes.POINTER(ProducerArgs)]),
        "g4a_add": (c_int, [ctxp, vp, vp, vp, sz]),
        "g4a_mul": (c_int, [ctxp, vp, vp, vp, sz]),
        "g4a_scale": (c_int, [ctxp, vp, ctypes.c_float, vp, sz]),
        "g4a_scale_by_tensor": (c_int, [ctxp, vp, vp, vp, sz]),
        "g4a_gelu_tanh": (c_int, [ctxp, vp, vp, sz]),
        "g4a_geglu": (c_int, [ctxp, vp, vp, vp, sz]),
        "g4a_softcap": (c_int, [ctxp, vp, ctypes.c_float, vp, sz]),
        "g4a_slice_cols": (c_int, [ctxp, vp] + [ctypes.c_uint32] * 4 + [vp]),
        "g4a_add_rms_norm": (c_int, [ctxp, vp, vp, vp, vp, vp, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_float]),
        "g4a_embed_rows": (c_int, [ctxp, vp, ctypes.c_uint32, ctypes.c_uint32, _u32p, ctypes.c_uint32, ctypes.c_float,
                                   vp]),
        "g4a_linear": (c_int, [ctxp, vp, ctypes.c_uint32, ctypes.c_uint32, vp, vp, ctypes.c_uint32]),
        "g4a_linear_q": (c_int, [ctxp, ctypes.POINTER(QWeightArgs), vp, vp, ctypes.c_uint32]),
        "g4a_attention_linear_q": (c_int, [ctxp, ctypes.POINTER(AttnArgs), ctypes.POINTER(QWeightArgs), vp]),
        "g4a_linear_q_geglu": (c_int, [ctxp, ctypes.POINTER(QWeightArgs), ctypes.POINTER(QWeightArgs), vp, vp,
                                       ctypes.c_uint32]),
        "g4a_linear_q_gelu_mul_cols": (c_int, [ctxp, ctypes.POINTER(QWeightArgs), vp, vp, ctypes.c_uint32,
                                               ctypes.c_uint32, vp, ctypes.c_uint32]),
        "g4a_embed_rows_q": (c_int, [ctxp, ctypes.POINTER(QWeightArgs), _u32p, ctypes.c_uint32, ctypes.c_float, vp]),
        "g4a_capture_begin": (c_int, [ctxp]),
        "g4a_capture_end": (c_int, [ctxp, ctypes.POINTER(ctypes.c_void_p)]),
        "g4a_graph_launch": (c_int, [ctxp, ctypes.c_void_p]),
        "g4a_graph_destroy": (c_int, [ctypes.c_void_p]),
        "g4a_timer_start": (c_int, [ctxp]),
        "g4a_timer_stop": (c_int, [ctxp, ctypes.POINTER(ctypes.c_float)]),
        "g4a_get_device_info": (c_int, [ctxp, ctypes.POINTER(DeviceInfo)]),
        "g4a_kernel_timing": (c_int, [ctxp, c_int]),
        "g4a_kernel_timing_read": (c_int, [ctxp, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_uint32)]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def header_functions(header: Path = HEADER_PATH) -> list[str]:
    """Names of every function include/g4a.h declares."""
    import re
    text = Path(header).read_text()
    return sorted(set(re.findall(r"^\s*(?:int|void|const char \*)\s*\**\s*(g4a_\w+)\s*\(", text, re.M)))


def _u32_array(xs: Optional[Sequence[int]]):
    if xs is None:
        return None, None
    arr = np.ascontiguousarray(np.asarray(xs, dtype=np.uint32))
    return arr, arr.ctypes.data_as(_u32p)


def make_args(q=0, k=0, v=0, out=0, *, T, S, Hq, Hkv, Dh, Dv, q_pos=None, k_pos=None, q_pos0=0, k_pos0=0,
              scale=1.0, window=0, softcap=0.0, ring_cap=0, splits=0):
    """Build g4a_attn_args. Returns (args, keepalive) — keep the second alive during the call."""
    qa, qp = _u32_array(q_pos)
    ka, kp = _u32_array(k_pos)
    a = AttnArgs(q or None, k or None, v or None, out or None, T, S, Hq, Hkv, Dh, Dv, qp, kp, q_pos0, k_pos0,
                 scale, window, softcap, ring_cap, splits)
    return a, (qa, ka)


def plan(ctx: Optional["Context"] = None, **kw) -> AttnPlan:
    """Launch plan for an attention call (host-only; works without a GPU when ctx is None)."""
    lib = load_library()
    a, keep = make_args(**kw)
    p = AttnPlan()
    rc = lib.g4a_attention_plan(ctx.handle if ctx else None, ctypes.byref(a), ctypes.byref(p))
    if rc != G4A_OK:
        raise G4aError(rc, lib.g4a_last_error(ctx.handle if ctx else None).decode())
    return p


@dataclass
class DeviceArray:
    ctx: "Context"
    ptr: int
    shape: tuple
    dtype: np.dtype

    @property
    def nbytes(self) -> int:
        return int(np.prod(self.shape, dtype=np.int64)) * np.dtype(self.dtype).itemsize

    def to_host(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        self.ctx.d2h(out, self.ptr)
        return out

    def free(self) -> None:
        if self.ptr:
            self.ctx.free(self.ptr)
            self.ptr = 0


@dataclass
class DeviceQWeight:
    """A quantised weight uploaded by Context.upload_qweight (owns its buffers)."""
    args: QWeightArgs
    qbytes: "DeviceArray"
    scales: "DeviceArray"

    def free(self) -> None:
        self.qbytes.free()
        self.scales.free()


class Graph:
    """A captured sequence of a context's launches (g4a_capture_end); replay with launch()."""

    def __init__(self, ctx: "Context", handle: int):
        self.ctx, self.handle = ctx, handle

    def launch(self) -> None:
        self.ctx._check(self.ctx.lib.g4a_graph_launch(self.ctx.handle, self.handle))

    def free(self) -> None:
        if self.handle:
            self.ctx.lib.g4a_graph_destroy(self.handle)
            self.handle = None


class Context:
    """One g4a context: a device, its gfx950 module, one stream. `options`
    (a dict of g4a_options fields, e.g. {"fuse_projection": 1}) overrides the
    library's defaults for this context."""

    def __init__(self, device: int = 0, hsaco: Optional[Path] = None, options: Optional[dict] = None):
        self.lib = load_library()
        h = ctypes.c_void_p()
        path = str(hsaco).encode() if hsaco else None
        opts = Options()
        self.lib.g4a_default_options(ctypes.byref(opts))
        for k, v in (options or {}).items():
            if k not in dict(Options._fields_) or k == "size":
                raise ValueError(f"unknown g4a option {k!r}")
            setattr(opts, k, v)
        rc = self.lib.g4a_create_with(device, path, ctypes.byref(opts), ctypes.byref(h))
        if rc != G4A_OK:
            raise G4aError(rc, self.lib.g4a_last_error(None).decode())
        self.handle = h

    def _check(self, rc: int) -> None:
        if rc != G4A_OK:
            raise G4aError(rc, self.lib.g4a_last_error(self.handle).decode())

    def close(self) -> None:
        if self.handle:
            self.lib.g4a_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # ---- memory ----
    def malloc(self, nbytes: int) -> int:
        p = ctypes.c_void_p()
        self._check(self.lib.g4a_malloc(self.handle, nbytes, ctypes.byref(p)))
        return p.value

    def free(self, ptr: int) -> None:
        self._check(self.lib.g4a_free(self.handle, ptr))

    def h2d(self, dst: int, host: np.ndarray) -> None:
        host = np.ascontiguousarray(host)
        self._check(self.lib.g4a_h2d(self.handle, dst, host.ctypes.data, host.nbytes))

    def d2h(self, host: np.ndarray, src: int) -> None:
        assert host.flags.c_contiguous
        self._check(self.lib.g4a_d2h(self.handle, host.ctypes.data, src, host.nbytes))

    def d2d(self, dst: int, src: int, nbytes: int) -> None:
        self._check(self.lib.g4a_d2d(self.handle, dst, src, nbytes))

    def zero(self, dst: int, nbytes: int) -> None:
        self._check(self.lib.g4a_zero(self.handle, dst, nbytes))

    def stream(self) -> int:
        """The context's HIP stream handle (g4a_stream), e.g. for torch.cuda.ExternalStream."""
        s = ctypes.c_void_p()
        self._check(self.lib.g4a_stream(self.handle, ctypes.byref(s)))
        return s.value

    def sync(self) -> None:
        self._check(self.lib.g4a_sync(self.handle))

    def upload(self, host: np.ndarray) -> DeviceArray:
        host = np.ascontiguousarray(host)
        ptr = self.malloc(max(host.nbytes, 16))
        self.h2d(ptr, host)
        return DeviceArray(self, ptr, tuple(host.shape), host.dtype)

    def empty(self, shape, dtype=np.float32) -> DeviceArray:
        n = int(np.prod(shape, dtype=np.int64)) * np.dtype(dtype).itemsize
        return DeviceArray(self, self.malloc(max(n, 16)), tuple(shape), np.dtype(dtype))

    # ---- ops ----
    def attention(self, q: int, k: int, v: int, out: int, **kw) -> None:
        a, keep = make_args(q, k, v, out, **kw)
        self._check(self.lib.g4a_attention(self.handle, ctypes.byref(a)))

    def attention_noalloc(self, q: int, k: int, v: int, out: int, **kw) -> None:
        """g4a_attention_noalloc: attention() with its scratch in the library's static
        array (no allocation)."""
        a, keep = make_args(q, k, v, out, **kw)
        self._check(self.lib.g4a_attention_noalloc(self.handle, ctypes.byref(a)))

    def attention_devpos(self, q: int, k: int, v: int, out: int, pos: int, **kw) -> None:
        """g4a_attention_devpos: one decode query at the position held by the device u32
        at `pos`; S (in kw) is the most keys any replay sees."""
        a, keep = make_args(q, k, v, out, **kw)
        self._check(self.lib.g4a_attention_devpos(self.handle, ctypes.byref(a), pos))

    def u32_add(self, counters: int, n: int, inc: int) -> None:
        """g4a_u32_add: n device u32 counters += inc, by a kernel (records into a graph)."""
        self._check(self.lib.g4a_u32_add(self.handle, counters, n, inc))

    @staticmethod
    def prepare_batch(calls: list[dict]) -> tuple:
        """Marshal a list of attention() keyword sets into a g4a_attn_args array
        (built once, so a timed region holds only the library call)."""
        built = [make_args(**kw) for kw in calls]
        arr = (AttnArgs * len(built))(*[a for a, _ in built])
        return arr, len(built), [k for _, k in built]

    def attention_batch(self, calls) -> None:
        """One g4a_attention_batch crossing: `calls` is a list of attention() keyword
        sets or the result of prepare_batch()."""
        arr, n, _keep = calls if isinstance(calls, tuple) else self.prepare_batch(calls)
        self._check(self.lib.g4a_attention_batch(self.handle, arr, n))

    def attention_decode_batch(self, calls) -> int:
        """One g4a_attention_decode_batch call over independent decode steps
        (attention() keyword sets, or the result of prepare_batch()); returns how
        many of them ran in the batched launches."""
        arr, n, _keep = calls if isinstance(calls, tuple) else self.prepare_batch(calls)
        done = ctypes.c_uint32(0)
        self._check(self.lib.g4a_attention_decode_batch(self.handle, arr, n, ctypes.byref(done)))
        return done.value

    def plan(self, **kw) -> AttnPlan:
        return plan(self, **kw)

    def kv_write(self, cache: int, ring_cap: int, row_elems: int, dst_row: int, src: int, n_rows: int) -> None:
        self._check(self.lib.g4a_kv_write(self.handle, cache, ring_cap, row_elems, dst_row, src, n_rows))

    # ---- the attention producer (per-head RMSNorm, partial RoPE, KV write) ----
    def head_norm_rope(self, x: int, w: int, y: int, *, T, heads, head_dim, rotary_dim, positions=None, pos0=0,
                       theta, eps) -> None:
        pa, pp = _u32_array(positions)
        self._check(self.lib.g4a_head_norm_rope(self.handle, x, w or None, y, T, heads, head_dim, rotary_dim, pp,
                                                pos0, theta, eps))

    def rope(self, x: int, y: int, *, T, heads, head_dim, rotary_dim, positions=None, pos0=0, theta) -> None:
        pa, pp = _u32_array(positions)
        self._check(self.lib.g4a_rope(self.handle, x, y, T, heads, head_dim, rotary_dim, pp, pos0, theta))

    def rms_norm(self, x: int, w: int, y: int, *, rows, dim, eps) -> None:
        self._check(self.lib.g4a_rms_norm(self.handle, x, w or None, y, rows, dim, eps))

    def attn_producer(self, *, q, k=0, v=0, q_norm=0, k_norm=0, q_out, k_cache=0, v_cache=0, T, Hq, Hkv, Dh,
                      rotary_dim, positions=None, pos0=0, cache_row=0, ring_cap=0, theta, eps) -> None:
        pa, pp = _u32_array(positions)
        a = ProducerArgs(q, k or None, v or None, q_norm or None, k_norm or None, q_out, k_cache or None,
                         v_cache or None, T, Hq, Hkv, Dh, rotary_dim, pp, pos0, cache_row, ring_cap, theta, eps)
        self._check(self.lib.g4a_attn_producer(self.handle, ctypes.byref(a)))

    def attn_producer_devpos(self, *, pos, max_pos, q, k=0, v=0, q_norm=0, k_norm=0, q_out, k_cache=0, v_cache=0,
                             Hq, Hkv, Dh, rotary_dim, ring_cap=0, theta, eps) -> None:
        """g4a_attn_producer_devpos: one token at the position held by the device u32 at
        `pos` (written to cache row *pos); positions past max_pos write nothing."""
        a = ProducerArgs(q, k or None, v or None, q_norm or None, k_norm or None, q_out, k_cache or None,
                         v_cache or None, 1, Hq, Hkv, Dh, rotary_dim, None, 0, 0, ring_cap, theta, eps)
        self._check(self.lib.g4a_attn_producer_devpos(self.handle, ctypes.byref(a), pos, max_pos))

    # ---- the rest of the backend trait (device pointers) ----
    def ew(self, op: str, a: int, y: int, n: int, b: int = 0, s: float = 0.0) -> None:
        """op in add, mul, scale, scale_by_tensor (b = device scalar), gelu_tanh, geglu, softcap (s = cap)."""
        L, h = self.lib, self.handle
        rc = {"add": lambda: L.g4a_add(h, a, b, y, n), "mul": lambda: L.g4a_mul(h, a, b, y, n),
              "scale": lambda: L.g4a_scale(h, a, s, y, n), "scale_by_tensor": lambda: L.g4a_scale_by_tensor(h, a, b, y, n),
              "gelu_tanh": lambda: L.g4a_gelu_tanh(h, a, y, n), "geglu": lambda: L.g4a_geglu(h, a, b, y, n),
              "softcap": lambda: L.g4a_softcap(h, a, s, y, n)}[op]()
        self._check(rc)

    def slice_cols(self, x: int, rows: int, stride: int, offset: int, width: int, y: int) -> None:
        self._check(self.lib.g4a_slice_cols(self.handle, x, rows, stride, offset, width, y))

    def add_rms_norm(self, residual: int, x: int, w: int, scale_by: int, y: int, rows: int, dim: int, eps: float):
        self._check(self.lib.g4a_add_rms_norm(self.handle, residual, x, w, scale_by or None, y, rows, dim, eps))

    def embed_rows(self, table: int, V: int, D: int, ids, scale: float, out: int) -> None:
        arr, ptr = _u32_array(ids)
        self._check(self.lib.g4a_embed_rows(self.handle, table, V, D, ptr, 0 if arr is None else arr.size, scale, out))

    def linear(self, w: int, N: int, K: int, x: int, y: int, M: int) -> None:
        self._check(self.lib.g4a_linear(self.handle, w, N, K, x, y, M))

    # ---- quantised projections ----
    def upload_qweight(self, qbytes: np.ndarray, scales: np.ndarray, N: int, K: int, bits: int,
                       signed_i8: bool = False, group_size: Optional[int] = None) -> "DeviceQWeight":
        qb = self.upload(np.ascontiguousarray(qbytes, np.uint8))
        sc = self.upload(np.ascontiguousarray(scales, np.float32))
        args = QWeightArgs(qb.ptr, sc.ptr, N, K, bits, 1 if signed_i8 else 0, group_size or K)
        return DeviceQWeight(args, qb, sc)

    def attention_linear_q(self, q: int, k: int, v: int, out: int, w: "DeviceQWeight", y: int, **kw) -> None:
        """g4a_attention_linear_q: attention() (same keywords) into out, then its
        output projection w into y; a decode step of 2..16 splits merges its split
        partials inside the projection instead of a combine launch."""
        a, keep = make_args(q, k, v, out, **kw)
        self._check(self.lib.g4a_attention_linear_q(self.handle, ctypes.byref(a), ctypes.byref(w.args), y))

    def linear_q(self, w: "DeviceQWeight", x: int, y: int, M: int) -> None:
        self._check(self.lib.g4a_linear_q(self.handle, ctypes.byref(w.args), x, y, M))

    def linear_q_geglu(self, w_gate: "DeviceQWeight", w_up: "DeviceQWeight", x: int, y: int, M: int) -> None:
        self._check(self.lib.g4a_linear_q_geglu(self.handle, ctypes.byref(w_gate.args), ctypes.byref(w_up.args), x,
                                                y, M))

    def linear_q_gelu_mul_cols(self, w: "DeviceQWeight", x: int, b: int, b_stride: int, b_off: int, y: int,
                               M: int) -> None:
        self._check(self.lib.g4a_linear_q_gelu_mul_cols(self.handle, ctypes.byref(w.args), x, b, b_stride, b_off, y,
                                                        M))

    def embed_rows_q(self, table: "DeviceQWeight", ids, scale: float, out: int) -> None:
        arr, ptr = _u32_array(ids)
        n = 0 if arr is None else arr.size
        self._check(self.lib.g4a_embed_rows_q(self.handle, ctypes.byref(table.args), ptr, n, scale, out))

    # ---- graph capture (launch-bound sequences) ----
    def capture_begin(self) -> None:
        """Record the launches of the following calls into a graph instead of running them."""
        self._check(self.lib.g4a_capture_begin(self.handle))

    def capture_end(self) -> "Graph":
        """Close the capture; returns the replayable graph. Raises, and makes no graph,
        if any call inside the capture failed (the recording would lack it)."""
        g = ctypes.c_void_p()
        self._check(self.lib.g4a_capture_end(self.handle, ctypes.byref(g)))
        return Graph(self, g.value)

    def timer_start(self) -> None:
        self._check(self.lib.g4a_timer_start(self.handle))

    def timer_stop(self) -> float:
        ms = ctypes.c_float()
        self._check(self.lib.g4a_timer_stop(self.handle, ctypes.byref(ms)))
        return float(ms.value)

    def kernel_timing(self, enable: bool) -> None:
        self._check(self.lib.g4a_kernel_timing(self.handle, 1 if enable else 0))

    def kernel_timing_read(self) -> tuple[float, int]:
        """(summed ms, count) of the main-kernel event pairs recorded since the last read."""
        ms, n = ctypes.c_double(), ctypes.c_uint32()
        self._check(self.lib.g4a_kernel_timing_read(self.handle, ctypes.byref(ms), ctypes.byref(n)))
        return float(ms.value), int(n.value)

    def device_info(self) -> DeviceInfo:
        info = DeviceInfo()
        self._check(self.lib.g4a_get_device_info(self.handle, ctypes.byref(info)))
        return info


def attention_host(ctx: Context, q: np.ndarray, k: np.ndarray, v: np.ndarray, *, q_pos=None, k_pos=None,
                   scale: float = 1.0, window: int = 0, softcap: float = 0.0, splits: int = 0,
                   contiguous_positions: bool = True) -> np.ndarray:
    """Backend::attention on host arrays: q [T,Hq,Dh], k [S,Hkv,Dh], v [S,Hkv,Dv] -> [T, Hq*Dv].

    Positions default to the model's convention (k_pos = 0..S-1, q_pos = the
    last T positions). With contiguous_positions the ranges are passed as
    scalars (no upload), otherwise as explicit host arrays.
    """
    T, Hq, Dh = q.shape
    S, Hkv, _ = k.shape
    Dv = v.shape[2]
    if k_pos is None:
        k_pos = np.arange(S, dtype=np.uint32)
    if q_pos is None:
        q_pos = np.arange(S - T, S, dtype=np.uint32) if S >= T else np.arange(T, dtype=np.uint32)
    q_pos = np.asarray(q_pos, np.uint32)
    k_pos = np.asarray(k_pos, np.uint32)
    bufs = [ctx.upload(np.ascontiguousarray(x, np.float32)) for x in (q, k, v)]
    out = ctx.empty((T, Hq * Dv))
    try:
        kw = dict(T=T, S=S, Hq=Hq, Hkv=Hkv, Dh=Dh, Dv=Dv, scale=scale, window=window, softcap=softcap,
                  splits=splits)
        q_contig = T == 0 or bool(np.all(q_pos == q_pos[0] + np.arange(T, dtype=np.uint32)))
        k_contig = S == 0 or bool(np.all(k_pos == k_pos[0] + np.arange(S, dtype=np.uint32)))
        if contiguous_positions and q_contig and k_contig:
            kw.update(q_pos0=int(q_pos[0]) if T else 0, k_pos0=int(k_pos[0]) if S else 0)
        else:
            kw.update(q_pos=q_pos, k_pos=k_pos)
        ctx.attention(bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, out.ptr, **kw)
        return out.to_host()
    finally:
        for b in bufs:
            b.free()
        out.free()
