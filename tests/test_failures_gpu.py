"""Failures the host can force on a GPU box, through the C-ABI: a missing or
unreadable code object at g4a_create, and calls the library must refuse. The
reference's backend has only one fallible step, its construction
(WgpuBackend::create -> Result<Self, String>, rust/src/backend_wgpu.rs:283);
the C-ABI returns a status from every call, leaves no context behind a failed
create, and enqueues nothing for a refused call. No kernel is made to fail:
every refusal here happens on the host before a launch."""
import ctypes

import numpy as np
import pytest

import g4a

pytestmark = pytest.mark.gpu

# g4a_status (include/g4a.h)
E_ARG, E_SHAPE, E_UNSUPPORTED, E_MODULE = -2, -3, -4, -5


def _create(path):
    lib = g4a.load_library()
    h = ctypes.c_void_p()
    rc = lib.g4a_create(0, str(path).encode(), ctypes.byref(h))
    return rc, h.value, lib.g4a_last_error(None).decode()


def test_create_with_a_missing_code_object(tmp_path):
    rc, h, msg = _create(tmp_path / "missing.hsaco")
    print(f"[gpu] missing code object: status {rc}: {msg}", flush=True)
    assert rc == E_MODULE and not h
    assert "hipModuleLoad" in msg and "missing.hsaco" in msg


def test_create_with_a_file_that_is_no_code_object(tmp_path):
    bad = tmp_path / "not_a_code_object.hsaco"
    bad.write_bytes(b"this is not an ELF code object\n" * 64)
    rc, h, msg = _create(bad)
    print(f"[gpu] invalid code object: status {rc}: {msg}", flush=True)
    assert rc == E_MODULE and not h
    assert "not_a_code_object" in msg


def test_a_good_context_after_failed_creates(ctx, tmp_path):
    """A failed create leaves nothing that breaks the next one."""
    _create(tmp_path / "missing.hsaco")
    c = g4a.Context(0)
    try:
        x = np.arange(4096, dtype=np.float32)
        d = c.upload(x)
        assert np.array_equal(d.to_host(), x)
        d.free()
    finally:
        c.close()


def test_refused_calls_enqueue_nothing(ctx):
    """Head dims past the generic kernel's limit, a soft-cap below zero and a
    window that cannot fit the ring are refused before any launch: the output
    keeps its sentinel and the context keeps working."""
    q = ctx.upload(np.ones((1, 8, 256), np.float32))
    kv = ctx.upload(np.ones((64, 1, 256), np.float32))
    out = ctx.empty((1, 8 * 256))
    try:
        ctx.h2d(out.ptr, np.full((1, 8 * 256), 7.0, np.float32))
        base = dict(T=1, S=64, Hq=8, Hkv=1, Dh=256, Dv=256, q_pos0=63, k_pos0=0)
        for label, kw, code in [("head_dim 2048", dict(Dh=2048, Dv=2048), E_UNSUPPORTED),
                                ("soft-cap below zero", dict(softcap=-1.0), E_ARG),
                                ("8 query heads over 3 kv heads", dict(Hkv=3), E_SHAPE),
                                ("64 visible keys in a 16-row ring", dict(window=0, ring_cap=16), E_SHAPE)]:
            with pytest.raises(g4a.G4aError) as e:
                ctx.attention(q.ptr, kv.ptr, kv.ptr, out.ptr, **dict(base, **kw))
            print(f"[gpu] {label}: status {e.value.code}: {e.value}", flush=True)
            assert e.value.code == code, label
        ctx.sync()
        assert np.all(out.to_host() == 7.0), "a refused call wrote its output"
        ctx.attention(q.ptr, kv.ptr, kv.ptr, out.ptr, **base)  # the context still works
        got = out.to_host()
        assert np.allclose(got, 1.0), "all-ones attention is the mean of the all-ones values"
    finally:
        for b in (q, kv, out):
            b.free()
