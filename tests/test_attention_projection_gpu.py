"""GPU parity of g4a_attention_linear_q: an attention call followed by its
quantised output projection (Gemma4Model::attention's `o_proj(attention(..))`,
rust/src/model.rs:287-303). On a context created with the fuse_projection option, a
decode step with 2..16 splits and a projection on the short-weight word kernel
launches no LSE combine: the projection merges the split partials while it
stages its activation row, in the combine kernel's order. A default context
runs the combine and the projection separately. Bars:
  - y and the attention rows of both contexts bit-identical to g4a_attention +
    g4a_linear_q;
  - y against the CPU oracle chain (rust/src/backend_cpu.rs:270-336 then
    :174-222): |d| <= 2e-6 sum|x w| + 1e-5 sum|w| + 1e-7 (the attention rows'
    1e-5 bar carried through the projection, plus the reordered sum);
  - a captured graph of the fused call replays bit-identically to the eager call.
Covers fused steps (sliding window on a ring, global at a short context, two kv
heads, 2/4/8-bit and I8 weights, 2..16 splits) and calls that must not fuse
(one split, more than 16 splits, several queries, an unaligned output)."""

import numpy as np
import pytest

import g4a
import g4a.synth as synth
import oracle
from test_linear_gpu import _bound, _deq_abs

pytestmark = pytest.mark.gpu


def step(msg):
    print(f"[gpu] {msg}", flush=True)


@pytest.fixture(scope="module")
def fctx():
    """A context whose g4a_attention_linear_q merges eligible decode steps in the projection."""
    c = g4a.Context(0, options={"fuse_projection": 1})
    yield c
    c.close()


CASES = [
    # label, T, S, Dh, window, ring, Hkv, bits, signed, forced splits, fused
    ("sliding step, 512-slot ring", 1, 5000, 256, 512, 512, 1, 4, False, 0, True),
    ("sliding step, short context", 1, 300, 256, 512, 0, 1, 4, False, 0, True),
    ("global step, short context", 1, 300, 512, 0, 0, 1, 4, False, 0, True),
    ("global step, 16 splits forced", 1, 4096, 512, 0, 0, 1, 4, False, 16, True),
    ("two kv heads", 1, 400, 256, 512, 0, 2, 4, False, 0, True),
    ("2-bit projection", 1, 600, 256, 512, 0, 1, 2, False, 0, True),
    ("I8 projection", 1, 600, 256, 512, 0, 1, 8, True, 0, True),
    ("8-bit projection, 12 splits forced", 1, 600, 512, 0, 0, 1, 8, False, 12, True),
    ("two splits forced", 1, 700, 256, 0, 0, 1, 4, False, 2, True),
    ("one split (no combine)", 1, 20, 256, 512, 0, 1, 4, False, 0, False),
    ("94 splits (combine launch)", 1, 3000, 512, 0, 0, 1, 4, False, 0, False),
    ("three queries", 3, 700, 256, 512, 0, 1, 4, False, 0, False),
]


def _inputs(S, Dh, W, cap, Hkv, T, seed):
    Hq = 8 * Hkv
    ins = synth.gemma_inputs(T=T, S=S, Dh=Dh, seed=seed, Hq=Hq, Hkv=Hkv)
    k, v = ins.k, ins.v
    if cap:
        k, v = np.zeros((cap, Hkv, Dh), np.float32), np.zeros((cap, Hkv, Dh), np.float32)
        for pos in range(S - cap, S):
            k[pos % cap], v[pos % cap] = ins.k[pos], ins.v[pos]
    return ins, k, v


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_attention_then_projection(ctx, fctx, case):
    label, T, S, Dh, W, cap, Hkv, bits, signed, splits, fused = case
    c = ctx
    Hq = 8 * Hkv
    ins, k, v = _inputs(S, Dh, W, cap, Hkv, T, S + T + bits)
    N, K = 1536, Hq * Dh
    qb, sc, _ = synth.quant_weight(S + 1, N, K, bits, signed_i8=signed)
    w = oracle.QWeight(qb, sc, N, K, bits, signed)
    kw = dict(T=T, S=S, Hq=Hq, Hkv=Hkv, Dh=Dh, Dv=Dh, q_pos0=S - T, k_pos0=0, window=W, ring_cap=cap, splits=splits)
    pl = c.plan(**kw)
    short_or_decode = g4a.KERNEL_NAMES[pl.kernel] in ("decode", "decode_short")
    assert (T == 1 and short_or_decode and 2 <= pl.splits <= 16) == fused, (label, pl.splits)
    step(f"{label}: kernel {g4a.KERNEL_NAMES[pl.kernel]}, {pl.splits} splits, {bits}-bit [{N}, {K}]")
    bufs = [c.upload(x) for x in (ins.q, k, v)]
    dw = c.upload_qweight(qb, sc, N, K, bits, signed)
    out_f, out_s, out_d = c.empty((T, K)), c.empty((T, K)), c.empty((T, K))
    y_f, y_s, y_d = c.empty((T, N)), c.empty((T, N)), c.empty((T, N))
    try:
        fctx.attention_linear_q(bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, out_f.ptr, dw, y_f.ptr, **kw)
        fctx.sync()
        c.attention_linear_q(bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, out_d.ptr, dw, y_d.ptr, **kw)
        c.attention(bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, out_s.ptr, **kw)
        c.linear_q(dw, out_s.ptr, y_s.ptr, T)
        yf, ys = y_f.to_host(), y_s.to_host()
        for o, y, form in ((out_f, yf, "fused"), (out_d, y_d.to_host(), "default")):
            assert np.array_equal(o.to_host(), out_s.to_host()), f"{label}: {form} attention rows differ"
            assert np.array_equal(y, ys), f"{label}: {form} projection differs from the separate calls"
        x_ref = oracle.attention(ins.q, ins.k, ins.v, ins.q_pos, ins.k_pos, window=W)
        y_ref = oracle.linear_q(x_ref, w).astype(np.float64)
        tol = 2e-6 * _bound(x_ref, w) + 1e-5 * _deq_abs(w).sum(axis=1)[None, :] + 1e-7
        err = np.abs(yf.astype(np.float64) - y_ref)
        print(f"  {label}: max-abs vs oracle {err.max():.3e}, worst err/tol {(err / tol).max():.3f}", flush=True)
        assert np.all(err <= tol), f"{label}: max-abs {err.max():.3e}"
    finally:
        for b in bufs + [out_f, out_s, out_d, y_f, y_s, y_d]:
            b.free()
        dw.free()


def test_unaligned_output_runs_separately(ctx, fctx):
    """An attention output 4 bytes past a 16-byte boundary: the call runs the
    combine and the projection separately (the merged row is stored in float4s),
    with the results of the two separate calls on that same unaligned row (whose
    projection runs on the element kernel: the word kernel reads x in float4s)."""
    c = ctx
    S, Dh, N = 300, 256, 1536
    K = 8 * Dh
    ins, k, v = _inputs(S, Dh, 512, 0, 1, 1, 31)
    qb, sc, _ = synth.quant_weight(31, N, K, 4)
    kw = dict(T=1, S=S, Hq=8, Hkv=1, Dh=Dh, Dv=Dh, q_pos0=S - 1, window=512)
    bufs = [c.upload(x) for x in (ins.q, k, v)]
    dw = c.upload_qweight(qb, sc, N, K, 4)
    big = c.empty((1, K + 4))
    out_s, y_f, y_s = c.empty((1, K)), c.empty((1, N)), c.empty((1, N))
    try:
        step("unaligned attention output")
        fctx.attention_linear_q(bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, big.ptr + 4, dw, y_f.ptr, **kw)
        fctx.sync()
        c.attention(bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, out_s.ptr, **kw)
        assert np.array_equal(big.to_host()[0, 1:K + 1], out_s.to_host()[0])
        c.linear_q(dw, big.ptr + 4, y_s.ptr, 1)
        assert np.array_equal(y_f.to_host(), y_s.to_host())
    finally:
        for b in bufs + [big, out_s, y_f, y_s]:
            b.free()
        dw.free()


def test_fused_call_replays_from_a_graph(fctx):
    """The fused sliding step captured and replayed: bit-identical to the eager call,
    with the outputs overwritten and unrelated eager work before every replay."""
    c = fctx
    S, Dh, cap, N = 5000, 256, 512, 1536
    K = 8 * Dh
    ins, k, v = _inputs(S, Dh, 512, cap, 1, 1, 77)
    qb, sc, _ = synth.quant_weight(77, N, K, 4)
    kw = dict(T=1, S=S, Hq=8, Hkv=1, Dh=Dh, Dv=Dh, q_pos0=S - 1, window=512, ring_cap=cap)
    bufs = [c.upload(x) for x in (ins.q, k, v)]
    dw = c.upload_qweight(qb, sc, N, K, 4)
    out, y = c.empty((1, K)), c.empty((1, N))
    o2, y2 = c.empty((1, K)), c.empty((1, N))
    graph = None
    try:
        step("eager fused sliding step")
        c.attention_linear_q(bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, out.ptr, dw, y.ptr, **kw)
        want_o, want_y = out.to_host(), y.to_host()
        step("capture")
        c.capture_begin()
        try:
            c.attention_linear_q(bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, out.ptr, dw, y.ptr, **kw)
            graph = c.capture_end()
        except Exception:
            try:
                c.capture_end().free()
            except g4a.G4aError:
                pass
            raise
        rng = np.random.default_rng(1)
        for rep in range(3):
            step(f"replay {rep}")
            c.h2d(out.ptr, rng.standard_normal((1, K)).astype(np.float32))
            c.h2d(y.ptr, rng.standard_normal((1, N)).astype(np.float32))
            # unrelated eager work on the same workspace: a global step with other partials
            c.attention_linear_q(bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, o2.ptr, dw, y2.ptr,
                                 **dict(kw, S=cap, ring_cap=0, window=0, q_pos0=cap - 1))
            c.sync()
            graph.launch()
            c.sync()
            assert np.array_equal(out.to_host(), want_o), f"replay {rep}: attention rows"
            assert np.array_equal(y.to_host(), want_y), f"replay {rep}: projection"
    finally:
        if graph is not None:
            graph.free()
        for b in bufs + [out, y, o2, y2]:
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
