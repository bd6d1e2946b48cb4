"""The C-ABI over device memory that PyTorch owns: its entry points take plain
device pointers, so tensors from torch's caching allocator (`data_ptr()`) go
in directly. A g4a context runs on its own stream; work is ordered against
torch's stream by synchronizing on each side (torch.cuda.synchronize() before,
Context.sync() after). The results must equal the same calls on buffers the
library allocated, bit for bit, and the oracle's within the north star's bar.
A caller may also share the context's stream (g4a_stream, wrapped as
torch.cuda.ExternalStream) and interleave its own kernels with the library's
calls in stream order, with no synchronization between them.

The check runs in a child process. The PyTorch wheel carries its own HIP
runtime under the same soname as /opt/rocm's (libamdhip64.so.7), and the one
loaded first serves both: importing torch into the test session would move
every later test onto torch's copy. The child imports torch first, as a torch
program would."""
import importlib.util
import subprocess
import sys
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

REPO = Path(__file__).resolve().parents[1]

_SCRIPT = r"""
import sys
sys.path[:0] = [sys.argv[1], sys.argv[2]]
import torch  # first: as in a torch program, its HIP runtime serves the process
import numpy as np
import g4a, g4a.synth as synth, oracle

assert torch.cuda.is_available()
dev = torch.device("cuda:0")
ctx = g4a.Context(0)
ins = synth.gemma_inputs(T=1, S=5000, Dh=512, seed=31)
q, k, v = (torch.from_numpy(np.ascontiguousarray(x)).to(dev) for x in (ins.q, ins.k, ins.v))
out = torch.full((1, 8 * 512), float("nan"), device=dev)
torch.cuda.synchronize()
ctx.attention(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), T=1, S=5000, Hq=8, Hkv=1, Dh=512, Dv=512,
              q_pos0=4999, k_pos0=0)
ctx.sync()
got = out.cpu().numpy()
ref = g4a.attention_host(ctx, ins.q, ins.k, ins.v)
assert np.array_equal(got, ref), "torch-owned buffers give other bits than library-owned ones"
d = np.abs(got.astype(np.float64) - oracle.attention(ins.q, ins.k, ins.v, ins.q_pos, ins.k_pos))
print(f"ATTENTION max-abs {d.max():.3e} mean-abs {d.mean():.3e}", flush=True)
assert d.max() <= 1e-5 and d.mean() <= 1e-6

# a 4-bit projection whose packed weight and scales live in torch tensors
N, K = 2048, 1536
qb, sc, _ = synth.quant_weight(32, N, K, 4)
tq = torch.from_numpy(np.ascontiguousarray(qb, np.uint8)).to(dev)
ts = torch.from_numpy(np.ascontiguousarray(sc, np.float32)).to(dev)
x_h = synth.normal_f32(33, 0, K).reshape(1, K)
tx = torch.from_numpy(x_h).to(dev)
ty = torch.empty((1, N), device=dev)
w = g4a.DeviceQWeight(g4a.QWeightArgs(tq.data_ptr(), ts.data_ptr(), N, K, 4, 0, K), None, None)
torch.cuda.synchronize()
ctx.linear_q(w, tx.data_ptr(), ty.data_ptr(), 1)
ctx.sync()
own = ctx.upload_qweight(qb, sc, N, K, 4)
x_d, y_d = ctx.upload(x_h), ctx.empty((1, N))
ctx.linear_q(own, x_d.ptr, y_d.ptr, 1)
assert np.array_equal(ty.cpu().numpy(), y_d.to_host()), "projection on torch tensors differs"
own.free(); x_d.free(); y_d.free()

# the context's stream shared with torch (g4a_stream): torch kernels and library
# calls in one stream order, with no synchronization between them
s = torch.cuda.ExternalStream(ctx.stream())
with torch.cuda.stream(s):
    q3 = (q * 2.0) * 0.5  # torch kernels on the context's stream: q again, bit for bit
    out3 = torch.full_like(out, float("nan"))
    ctx.attention(q3.data_ptr(), k.data_ptr(), v.data_ptr(), out3.data_ptr(), T=1, S=5000, Hq=8, Hkv=1, Dh=512,
                  Dv=512, q_pos0=4999, k_pos0=0)
    res3 = out3 + 0.0  # a torch kernel reading the library's output in stream order
s.synchronize()
assert np.array_equal(res3.cpu().numpy(), got), "the shared-stream sequence differs"
print("SHARED STREAM torch -> g4a -> torch in stream order: bit-identical", flush=True)
ctx.close()
print("PROJECTION bit-identical to library-owned buffers", flush=True)
print("INTEROP OK", flush=True)
"""


def test_attention_and_projection_on_torch_tensors():
    # looked up, not imported: this process keeps the runtime it loaded
    if importlib.util.find_spec("torch") is None:
        pytest.skip("torch is not installed")
    args = [sys.executable, "-c", _SCRIPT, str(REPO / "gemma-4-webgpu-kernels_amd"), str(REPO / "oracle")]
    print("[gpu] torch interop in a child process", flush=True)
    r = subprocess.run(args, capture_output=True, text=True, timeout=300)
    print(r.stdout[-3000:], r.stderr[-3000:], flush=True)
    assert r.returncode == 0, "the child process failed"
    assert "INTEROP OK" in r.stdout
