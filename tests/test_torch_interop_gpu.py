"""The C-ABI over device memory that PyTorch owns: its entry points take plain
device pointers, so tensors from torch's caching allocator (`data_ptr()`) go
in directly. A g4a context runs on its own stream; work is ordered against
torch's stream by synchronizing on each side (torch.cuda.synchronize() before,
Context.sync() after). The results must equal the same calls on buffers the
library allocated, bit for bit, and the oracle's within the north star's bar."""
import numpy as np
import pytest

import g4a
import g4a.synth as synth
import oracle

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def test_attention_and_projection_on_torch_tensors(ctx):
    assert torch.cuda.is_available()
    dev = torch.device("cuda:0")
    ins = synth.gemma_inputs(T=1, S=5000, Dh=512, seed=31)
    q, k, v = (torch.from_numpy(np.ascontiguousarray(x)).to(dev) for x in (ins.q, ins.k, ins.v))
    out = torch.full((1, 8 * 512), float("nan"), device=dev)
    torch.cuda.synchronize()
    ctx.attention(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), T=1, S=5000, Hq=8, Hkv=1, Dh=512,
                  Dv=512, q_pos0=4999, k_pos0=0)
    ctx.sync()
    got = out.cpu().numpy()
    ref = g4a.attention_host(ctx, ins.q, ins.k, ins.v)
    assert np.array_equal(got, ref), "torch-owned buffers give other bits than library-owned ones"
    d = np.abs(got.astype(np.float64) - oracle.attention(ins.q, ins.k, ins.v, ins.q_pos, ins.k_pos))
    print(f"[gpu] attention on torch tensors: max-abs {d.max():.3e} mean-abs {d.mean():.3e}", flush=True)
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
    try:
        ctx.linear_q(own, x_d.ptr, y_d.ptr, 1)
        assert np.array_equal(ty.cpu().numpy(), y_d.to_host()), "projection on torch tensors differs"
    finally:
        own.free()
        x_d.free()
        y_d.free()
    print("[gpu] projection on torch tensors: bit-identical to library-owned buffers", flush=True)
