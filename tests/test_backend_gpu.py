"""The C++ mirror of the reference's Backend trait (hip_backend.hpp) on the GPU:
runs its parity driver (tests/cpp/test_backend.cpp), which repeats the
reference's grouped_attention_parity and kv_append tests
(rust/tests/gpu.rs:96-120, 262-293) through the mirror and adds a KV-cache
decode over a sliding-window ring and a growing global cache, every checked
step compared with the CPU oracle at max-abs 1e-5 / mean-abs 1e-6."""
import subprocess

import pytest

from g4a import build

pytestmark = pytest.mark.gpu


def test_backend_mirror_parity_driver():
    exe = build.TEST_BACKEND
    assert exe.exists(), f"{exe} is not built (run __graft_entry__.build())"
    print(f"[gpu] running {exe.name}", flush=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=100)
    print(r.stdout[-6000:], flush=True)
    print(r.stderr[-2000:], flush=True)
    assert r.returncode == 0, f"test_backend exited {r.returncode}"
    assert "PASSED: 0 failure(s)" in r.stdout
