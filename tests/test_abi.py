"""The C-ABI library without a GPU: it loads, exports every function
include/g4a.h declares, and its host-side planning follows the reference's
dispatch rules (key-range trim rust/src/backend_wgpu.rs:924-936, split-K
decomposition, argument errors). No compute calls. CPU only."""
import ctypes

import numpy as np
import pytest

import g4a


def test_library_loads_and_exports_every_header_function():
    lib = g4a.load_library()
    names = g4a.header_functions()
    assert len(names) >= 15, names
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"declared in include/g4a.h but not exported: {missing}"


def test_code_object_was_built_for_gfx950():
    data = g4a.HSACO_PATH.read_bytes()
    assert data[:4] == b"\x7fELF" or data.startswith(b"__CLANG_OFFLOAD_BUNDLE__")
    for name in (b"g4a_decode_d512_g8", b"g4a_decode_d256_g8", b"g4a_combine_d512", b"g4a_generic_attention"):
        assert name in data, name
    assert b"gfx950" in data


def _plan(**kw):
    base = dict(T=1, S=512, Hq=8, Hkv=1, Dh=256, Dv=256)
    base.update(kw)
    return g4a.plan(None, **base)


def test_decode_trim_for_sliding_window_keeps_last_window_keys():
    # decode at position 8191 with window 512: keys 7680..8191 only
    p = _plan(S=8192, q_pos0=8191, window=512)
    assert (p.k_start, p.k_end) == (8192 - 512, 8192)
    assert g4a.KERNEL_NAMES[p.kernel] in ("decode", "decode_short")


def test_trim_matches_reference_partition_points_on_explicit_positions():
    rng = np.random.default_rng(0)
    kp = np.sort(rng.choice(10000, size=700, replace=False)).astype(np.uint32)
    for qpos, w in [(5000, 0), (5000, 300), (9999, 100), (3, 0), (kp[0], 1)]:
        p = _plan(S=700, q_pos=[qpos], k_pos=kp, window=w)
        k_end = int(np.searchsorted(kp, qpos, side="right"))
        k_start = int(np.searchsorted(kp, qpos - w, side="right")) if (w and qpos >= w) else 0
        assert (p.k_start, p.k_end) == (min(k_start, k_end), k_end)


def test_multi_query_trim_uses_min_and_max_query():
    p = _plan(T=3, S=300, q_pos=[297, 298, 299], window=150)
    assert (p.k_start, p.k_end) == (297 - 150 + 1, 300)


def test_no_visible_key_plans_a_zero_fill():
    p = _plan(S=100, k_pos0=50, q_pos0=10)
    assert g4a.KERNEL_NAMES[p.kernel] == "none" and p.k_end == 0


@pytest.mark.parametrize("S,Dh", [(512, 256), (8192, 512), (32768, 512), (131072, 512)])
def test_auto_splits_cover_the_range(S, Dh):
    p = _plan(S=S, Dh=Dh, Dv=Dh, q_pos0=S - 1)
    if g4a.KERNEL_NAMES[p.kernel] == "decode_short":
        # 32-key splits (two 16-key tiles per 4-wave workgroup), at most one workgroup per CU
        assert p.keys_per_split == 32 and S <= 256 * 32
    else:
        assert S > 256 * 32
        assert p.keys_per_split % 64 == 0
    assert p.splits * p.keys_per_split >= S > (p.splits - 1) * p.keys_per_split
    assert p.splits <= 256  # one 8-wave workgroup per CU at most
    if p.splits > 1:
        assert p.workspace_bytes == 8 * p.splits * (Dh + 2) * 4


def test_forced_split_counts_for_the_long_context_sweep():
    for want in (8, 16, 32, 64, 128, 256, 512):
        p = _plan(S=131072, Dh=512, Dv=512, q_pos0=131071, splits=want)
        assert p.splits == want and p.keys_per_split == 131072 // want


def test_shapes_outside_the_fast_path_use_the_generic_kernel():
    assert g4a.KERNEL_NAMES[_plan(T=6, S=6, Hq=4, Dh=16, Dv=16).kernel] == "generic"
    assert g4a.KERNEL_NAMES[_plan(Hq=2, Dh=32, Dv=32).kernel] == "generic"
    assert g4a.KERNEL_NAMES[_plan(Hq=8, Hkv=2, Dh=512, Dv=512).kernel] == "decode"  # group 4
    assert g4a.KERNEL_NAMES[_plan(Dh=256, Dv=128).kernel] == "generic"


def test_argument_errors_are_reported_not_crashed():
    with pytest.raises(g4a.G4aError) as e:
        _plan(Hq=6, Hkv=4)
    assert e.value.code == -3
    with pytest.raises(g4a.G4aError) as e:
        _plan(softcap=-1.0)
    assert e.value.code == -2
    with pytest.raises(g4a.G4aError) as e:
        _plan(S=2048, q_pos0=2047, window=0, ring_cap=512)  # 2048 visible keys cannot live in a 512-row ring
    assert e.value.code == -3
    assert "ring" in g4a.load_library().g4a_last_error(None).decode()


def test_context_free_errors_are_per_thread():
    """g4a_last_error(NULL) is the calling thread's own last context-free failure:
    two threads failing plan queries at once, each with its own error, each read
    their own message (rust/src/backend_wgpu.rs:283 reports construction errors
    as a String per call; the C-ABI keeps one per thread)."""
    import threading
    lib = g4a.load_library()
    bad = {"heads": dict(Hq=6, Hkv=4), "ring": dict(S=2048, q_pos0=2047, window=0, ring_cap=512)}
    seen = {k: [] for k in bad}
    start = threading.Barrier(2)

    def worker(kind):
        start.wait()
        for _ in range(300):
            kw = dict(T=1, S=300, Hq=8, Hkv=1, Dh=256, Dv=256, q_pos0=299)
            kw.update(bad[kind])
            a, keep = g4a.make_args(0, 0, 0, 0, **kw)
            p = g4a.AttnPlan()
            rc = lib.g4a_attention_plan(None, ctypes.byref(a), ctypes.byref(p))
            seen[kind].append((rc, lib.g4a_last_error(None).decode()))

    threads = [threading.Thread(target=worker, args=(k,)) for k in bad]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert all(rc == -3 and "multiple of Hkv" in msg for rc, msg in seen["heads"]), seen["heads"][:3]
    assert all(rc == -3 and "ring" in msg for rc, msg in seen["ring"]), seen["ring"][:3]


def test_ring_plan_accepts_window_inside_ring():
    p = _plan(S=40000, q_pos0=39999, window=512, ring_cap=512)
    assert (p.k_start, p.k_end) == (40000 - 512, 40000)


def test_create_without_gpu_fails_cleanly():
    import os
    lib = g4a.load_library()
    h = ctypes.c_void_p()
    if os.path.exists("/dev/kfd"):
        pytest.skip("a GPU may be present")
    rc = lib.g4a_create(0, None, ctypes.byref(h))
    assert rc != 0 and not h.value
    assert lib.g4a_last_error(None)


def test_backend_mirror_driver_links_and_reports_a_missing_device():
    """The C++ Backend mirror and its parity driver link and start; without a
    device, construction fails with an error (like WgpuBackend::create's Err)."""
    import subprocess
    from g4a import build
    if not build.TEST_BACKEND.exists():
        pytest.skip("C++ backend driver not built")
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present: the gpu test runs the driver")
    r = subprocess.run([str(build.TEST_BACKEND)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 2, (r.returncode, r.stdout, r.stderr)
    assert "g4a_create failed" in r.stderr


def test_short_decode_rule():
    """Contiguous-position decode of an 8-head group whose 32-key splits fit one
    workgroup per CU takes the short kernel; explicit positions, 4-head groups
    and forced split counts keep the streaming kernel."""
    p = _plan(S=512, q_pos0=511, window=512)
    assert g4a.KERNEL_NAMES[p.kernel] == "decode_short"
    assert (p.splits, p.keys_per_split) == (16, 32)
    assert p.workspace_bytes == 8 * 16 * (256 + 2) * 4
    p = _plan(S=30, Dh=512, Dv=512, q_pos0=29)
    assert g4a.KERNEL_NAMES[p.kernel] == "decode_short" and p.splits == 1 and p.workspace_bytes == 0
    p = _plan(T=4, S=2048, Dh=512, Dv=512, q_pos0=2044)
    assert g4a.KERNEL_NAMES[p.kernel] == "decode_short" and p.splits == 64
    p = _plan(T=5, S=2048, Dh=512, Dv=512, q_pos0=2043)
    assert g4a.KERNEL_NAMES[p.kernel] == "decode"  # 5 x 64 workgroups exceed one per CU
    assert g4a.KERNEL_NAMES[_plan(S=8193, Dh=512, Dv=512, q_pos0=8192).kernel] == "decode"
    assert g4a.KERNEL_NAMES[_plan(S=512, q_pos=[511], k_pos=np.arange(512) * 2).kernel] == "decode"
    assert g4a.KERNEL_NAMES[_plan(S=512, Hq=4, q_pos0=511).kernel] == "decode"
    assert g4a.KERNEL_NAMES[_plan(S=512, q_pos0=511, splits=8).kernel] == "decode"


def test_kv_source_map_is_the_reference_one():
    import g4a.synth as synth
    # rust/src/config.rs:152-159 on the E2B layer types: 15 caches, shared layers read 13 / 14
    src = [synth.kv_source_layer(i) for i in range(35)]
    assert src[:15] == list(range(15))
    assert all(src[i] == (14 if i in synth.E2B_GLOBAL else 13) for i in range(15, 35))
    assert len(set(src)) == 15 and sum(1 for s in set(src) if s in synth.E2B_GLOBAL) == 3
