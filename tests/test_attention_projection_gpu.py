"""GPU parity of g4a_attention_linear_q (an attention call followed by its
quantised output projection, Gemma4Model::attention's `o_proj(attention(..))`,
rust/src/model.rs:302-303). A decode step with 2..16 splits skips the combine
launch: the projection merges the split partials while staging x, in the
combine kernel's order. Bars:
  - y and the attention rows bit-identical to g4a_attention + g4a_linear_q;
  - y against the CPU oracle chain (rust/src/backend_cpu.rs:270-336 then
    :174-222): |d| <= 2e-6 sum|x w| + 1e-5 sum|w| + 1e-7 (the attention rows'
    1e-5 bar carried through the projection, plus the reordered sum).
Covers fused steps (sliding window on a ring, global, two kv heads, 2/4/8-bit)
and calls that must not fuse (one split, more than 16 splits, several queries)."""
import numpy as np
import pytest

import g4a
import g4a.synth as synth
import oracle
from test_linear_gpu import _bound, _deq_abs

pytestmark = pytest.mark.gpu


def step(msg):
    print(f"[gpu] {msg}", flush=True)


CASES = [
    # label, T, S, Dh, window, ring, Hkv, bits, fused
    ("sliding step, 512-slot ring", 1, 5000, 256, 512, 512, 1, 4, True),
    ("sliding step, short context", 1, 300, 256, 512, 0, 1, 4, True),
    ("global step, 10 splits", 1, 300, 512, 0, 0, 1, 4, True),
    ("two kv heads", 1, 400, 256, 512, 0, 2, 4, True),
    ("2-bit projection", 1, 600, 256, 512, 0, 1, 2, True),
    ("I8 projection", 1, 600, 256, 512, 0, 1, 8, True),
    ("one split (no combine)", 1, 20, 256, 512, 0, 1, 4, False),
    ("94 splits (combine launch)", 1, 3000, 512, 0, 0, 1, 4, False),
    ("three queries", 3, 700, 256, 512, 0, 1, 4, False),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_attention_then_projection(ctx, case):
    label, T, S, Dh, W, cap, Hkv, bits, fused = case
    c = ctx
    Hq = 8 * Hkv
    ins = synth.gemma_inputs(T=T, S=S, Dh=Dh, seed=S + T + bits, Hq=Hq, Hkv=Hkv)
    k, v = ins.k, ins.v
    if cap:
        k, v = np.zeros((cap, Hkv, Dh), np.float32), np.zeros((cap, Hkv, Dh), np.float32)
        for pos in range(S - cap, S):
            k[pos % cap], v[pos % cap] = ins.k[pos], ins.v[pos]
    N, K = 1536, Hq * Dh
    qb, sc, _ = synth.quant_weight(S + 1, N, K, bits, signed_i8=bits == 8)
    w = oracle.QWeight(qb, sc, N, K, bits, bits == 8)
    kw = dict(T=T, S=S, Hq=Hq, Hkv=Hkv, Dh=Dh, Dv=Dh, q_pos0=S - T, k_pos0=0, window=W, ring_cap=cap)
    pl = c.plan(**kw)
    short_or_decode = g4a.KERNEL_NAMES[pl.kernel] in ("decode", "decode_short")
    assert (T == 1 and short_or_decode and 2 <= pl.splits <= 16) == fused, (label, pl.splits)
    step(f"{label}: kernel {g4a.KERNEL_NAMES[pl.kernel]}, {pl.splits} splits")
    bufs = [c.upload(x) for x in (ins.q, k, v)]
    dw = c.upload_qweight(qb, sc, N, K, bits, bits == 8)
    out_f, out_s = c.empty((T, K)), c.empty((T, K))
    y_f, y_s = c.empty((T, N)), c.empty((T, N))
    try:
        c.attention_linear_q(bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, out_f.ptr, dw, y_f.ptr, **kw)
        c.attention(bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, out_s.ptr, **kw)
        c.linear_q(dw, out_s.ptr, y_s.ptr, T)
        yf, ys = y_f.to_host(), y_s.to_host()
        assert np.array_equal(out_f.to_host(), out_s.to_host()), f"{label}: attention rows differ"
        assert np.array_equal(yf, ys), f"{label}: fused projection differs from the separate calls"
        x_ref = oracle.attention(ins.q, ins.k, ins.v, ins.q_pos, ins.k_pos, window=W)
        y_ref = oracle.linear_q(x_ref, w).astype(np.float64)
        tol = 2e-6 * _bound(x_ref, w) + 1e-5 * _deq_abs(w).sum(axis=1)[None, :] + 1e-7
        err = np.abs(yf.astype(np.float64) - y_ref)
        print(f"  {label}: max-abs vs oracle {err.max():.3e}, worst err/tol {(err / tol).max():.3f}", flush=True)
        assert np.all(err <= tol), f"{label}: max-abs {err.max():.3e}"
    finally:
        for b in bufs + [out_f, out_s, y_f, y_s]:
            b.free()
        dw.free()


def test_shape_mismatch_is_an_error(ctx):
    c = ctx
    qb, sc, _ = synth.quant_weight(1, 64, 1024, 4)
    dw = c.upload_qweight(qb, sc, 64, 1024, 4)
    try:
        with pytest.raises(g4a.G4aError, match="projection K"):
            c.attention_linear_q(0, 0, 0, 0, dw, 0, T=1, S=10, Hq=8, Hkv=1, Dh=256, Dv=256, q_pos0=9)
    finally:
        dw.free()
