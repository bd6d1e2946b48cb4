"""The reference's whole-model tests on its tiny config (rust/tests/gpu.rs:190-227
full_model_parity; rust/tests/model.rs:24-90), run by the C++ driver
tests/cpp/test_model.cpp: Gemma4Model's forward (rust/src/model.rs:142-313)
composed once over the C++ HipBackend (the GPU, with its KV cache growing through
kv_append) and once over the CPU oracle's ops, 6 layers with 2 KV-shared, window 3,
the reference's SyntheticWeights. GPU: a 5-token prefill, 5 incremental steps
(also against the GPU's own full pass) and 300 decode steps past the 256-row
first capacity, at the reference's 5e-3 bar with the achieved difference printed.
CPU (no GPU needed): the reference's model tests on the oracle composition."""
import subprocess

import pytest

from g4a import build


def _run(args, timeout):
    exe = build.TEST_MODEL
    assert exe.exists(), f"{exe} is not built (run __graft_entry__.build())"
    print(f"[model] running {exe.name} {' '.join(args)}", flush=True)
    r = subprocess.run([str(exe), *args], capture_output=True, text=True, timeout=timeout)
    print(r.stdout[-6000:], flush=True)
    print(r.stderr[-2000:], flush=True)
    assert r.returncode == 0, f"test_model exited {r.returncode}"
    assert "PASSED: 0 failure(s)" in r.stdout


def test_tiny_model_on_the_oracle_composition():
    """incremental == full sequence, a 20-token sequence stays finite, reset reproduces (CPU only)."""
    _run(["--cpu-only"], 60)


@pytest.mark.gpu
def test_tiny_model_full_parity_on_the_gpu():
    _run([], 110)
