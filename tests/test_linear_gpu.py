"""GPU parity of the quantised projections (g4a_linear_q, g4a_linear_q_geglu,
g4a_linear_q_gelu_mul_cols, g4a_embed_rows_q) against the CPU oracle
(rust/src/backend_cpu.rs:127-145, :174-222, :55-58 and the trait's
compositions rust/src/backend.rs:156-168, restated in oracle/linear_oracle.c),
through the C-ABI.

Bars, written per test:
  - element kernel (any K, grouped scales) and the embedding: bit-identical to
    the oracle (the CPU's exact order);
  - word-parallel kernel: another f32 summation order, so per output
    |gpu - oracle| <= 2e-6 * sum_k |x_k w_nk| + 1e-7 (a reordered f32 sum of K
    terms stays well inside K * 2^-24 of sum |terms|); the reference's own test
    allows 2e-3 absolute (rust/tests/gpu.rs:156-190);
  - GeGLU / gelu-times-columns: the same bound carried through gelu
    (|gelu'| < 1.13) plus 2e-6 relative for tanhf.
"""
import numpy as np
import pytest

import g4a
import g4a.synth as synth
import oracle
from golden_io import load_linear_golden

pytestmark = pytest.mark.gpu


def step(msg):
    print(f"[gpu] {msg}", flush=True)


def _deq_abs(w):
    """|dequantised W| in f64 [N, K], for the error bound."""
    N, K, bits = w.N, w.K, w.bits
    qb = w.qbytes.reshape(N, -1)
    if w.signed_i8:
        q = qb.view(np.int8).astype(np.float64)
    else:
        per = 8 // bits
        f = np.stack([(qb >> (j * bits)) & ((1 << bits) - 1) for j in range(per)], axis=-1).reshape(N, K)
        q = f.astype(np.float64) - (1 << (bits - 1))
    g = w.group_size
    s = np.repeat(w.scales.reshape(N, -1).astype(np.float64), g, axis=1)[:, :K]
    return np.abs(q * s)


def _bound(x, w):
    return np.abs(x.astype(np.float64)) @ _deq_abs(w).T


def _check_sum(got, want, bound, label):
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    tol = 2e-6 * bound + 1e-7
    worst = float((err / tol).max())
    print(f"  {label}: max-abs {err.max():.3e}, worst err/tol {worst:.3f}", flush=True)
    assert np.all(err <= tol), f"{label}: max-abs {err.max():.3e}, err/tol {worst:.2f}"


class Dev:
    """Device copies of a weight (or two) and activations, freed on exit."""

    def __init__(self, c):
        self.c, self.bufs = c, []

    def w(self, w):
        d = self.c.upload_qweight(w.qbytes, w.scales, w.N, w.K, w.bits, w.signed_i8, w.group_size)
        self.bufs.append(d)
        return d

    def arr(self, a):
        d = self.c.upload(np.ascontiguousarray(a, np.float32))
        self.bufs.append(d)
        return d

    def empty(self, shape):
        d = self.c.empty(shape)
        self.bufs.append(d)
        return d

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        for b in self.bufs:
            b.free()


def _qw(seed, N, K, bits, signed=False, group=None):
    qb, sc, g = synth.quant_weight(seed, N, K, bits, signed_i8=signed, group_size=group)
    return oracle.QWeight(qb, sc, N, K, bits, signed, g)


def _linear_gpu(c, w, x):
    with Dev(c) as d:
        dw, dx = d.w(w), d.arr(x)
        y = d.empty((x.shape[0], w.N))
        c.linear_q(dw, dx.ptr, y.ptr, x.shape[0])
        return y.to_host()


def _words_path(w):
    words = w.K * w.bits // 32
    kpad = -(-words // 64) * 64 * (32 // w.bits)  # the row padded to whole 64-word strides
    return (w.K * w.bits) % 32 == 0 and w.group_size >= w.K and kpad * 4 <= 65536


def test_golden_fixtures(ctx):
    c = ctx
    for name, case in load_linear_golden().items():
        step(name)
        w = oracle.QWeight(case.w["qbytes"], case.w["scales"], case.w["N"], case.w["K"], case.w["bits"],
                           case.w["signed_i8"], case.w["group_size"])
        with Dev(c) as d:
            dw = d.w(w)
            if case.op == "embed":
                out = d.empty((case.ids.size, w.K))
                c.embed_rows_q(dw, case.ids, case.scale, out.ptr)
                assert np.array_equal(out.to_host(), case.out), name
                continue
            M = case.x.shape[0]
            dx = d.arr(case.x)
            y = d.empty((M, w.N))
            if case.op == "linear":
                c.linear_q(dw, dx.ptr, y.ptr, M)
                if _words_path(w):
                    _check_sum(y.to_host(), case.out, _bound(case.x, w), name)
                else:
                    assert np.array_equal(y.to_host(), case.out), f"{name}: element kernel not bit-exact"
            elif case.op == "geglu":
                w2 = oracle.QWeight(case.w2["qbytes"], case.w2["scales"], case.w2["N"], case.w2["K"],
                                    case.w2["bits"], case.w2["signed_i8"], case.w2["group_size"])
                c.linear_q_geglu(dw, d.w(w2), dx.ptr, y.ptr, M)
                _check_fused(y.to_host(), case.x, w, w2, None, 0, name)
            else:
                db = d.arr(case.b)
                c.linear_q_gelu_mul_cols(dw, dx.ptr, db.ptr, case.b.shape[1], case.b_off, y.ptr, M)
                _check_fused(y.to_host(), case.x, w, None, case.b, case.b_off, name)


def _check_fused(got, x, w, w2, b, b_off, label):
    g = oracle.linear_q(x, w).astype(np.float64)
    bg = _bound(x, w)
    gel = oracle.gelu_tanh(g.astype(np.float32)).astype(np.float64)
    if w2 is not None:
        u = oracle.linear_q(x, w2).astype(np.float64)
        want = oracle.linear_q_geglu(x, w, w2).astype(np.float64)
        tol = 1.13 * (2e-6 * bg + 1e-7) * np.abs(u) + np.abs(gel) * (2e-6 * _bound(x, w2) + 1e-7)
    else:
        cols = b[:, b_off:b_off + w.N].astype(np.float64)
        want = oracle.linear_q_gelu_mul_cols(x, w, b, b_off).astype(np.float64)
        tol = 1.13 * (2e-6 * bg + 1e-7) * np.abs(cols)
    tol = tol + 2e-6 * np.abs(want) + 1e-7
    err = np.abs(got.astype(np.float64) - want)
    print(f"  {label}: max-abs {err.max():.3e}, worst err/tol {(err / tol).max():.3f}", flush=True)
    assert np.all(err <= tol), f"{label}: max-abs {err.max():.3e}"


@pytest.mark.parametrize("bits,signed", [(2, False), (4, False), (8, True), (8, False)])
def test_word_kernel_shapes(ctx, bits, signed):
    """Every (activation rows, weight rows) variant: M = 1 with short and tall
    weights (2 or 8 rows in flight), M >= 2 in 4-row tiles with ragged M, N not a
    multiple of the rows per wave, K from one word per lane to the LDS limit.
    2-bit rows of an odd multiple of 32 words (K = 512, 1536, 3584, 4608) take
    the half-wave kernels (two rows per wave step), also at M = 2 when four
    activation rows do not fit the LDS share."""
    c = ctx
    cus = c.device_info().compute_units
    for N, K, M in [(1, 64, 1), (7, 128, 1), (255, 1536, 1), (2048, 1536, 1), (cus * 64 + 5, 1536, 1),
                    (1536, 2048, 1), (1536, 6144, 1), (1536, 16384, 1), (300, 1536, 2), (300, 1536, 3),
                    (257, 2048, 5), (96, 4096, 8), (64, 6144, 3), (40, 64, 17), (5, 512, 1),
                    (cus * 64 + 3, 3584, 1), (41, 4608, 2)]:
        label = f"b{bits}{'s' if signed else ''} N={N} K={K} M={M}"
        step(label)
        w = _qw(N * 7 + K + M, N, K, bits, signed)
        x = synth.normal_f32(N + K, M, M * K).reshape(M, K)
        _check_sum(_linear_gpu(c, w, x), oracle.linear_q(x, w), _bound(x, w), label)


def test_element_kernel_is_bit_exact(ctx):
    """Rows that are not whole words, grouped scales, and K past the word
    kernel's LDS limit run in the CPU's order: bit-identical."""
    c = ctx
    for N, K, M, bits, signed, group in [(21, 52, 3, 4, False, None), (33, 92, 2, 2, False, None),
                                         (17, 99, 4, 8, True, None), (96, 256, 2, 4, False, 64),
                                         (40, 1536, 1, 2, False, 256), (8, 16448, 2, 4, False, None)]:
        label = f"b{bits} N={N} K={K} M={M} group={group}"
        step(label)
        w = _qw(N + K, N, K, bits, signed, group)
        x = synth.normal_f32(K, M, M * K).reshape(M, K)
        assert np.array_equal(_linear_gpu(c, w, x), oracle.linear_q(x, w)), label


def test_geglu_and_gelu_mul_cols_at_gemma_shapes(ctx):
    c = ctx
    for N, K, M, bits in [(6144, 1536, 1, 4), (6144, 1536, 4, 4), (12288, 1536, 1, 2), (256, 1536, 7, 2)]:
        label = f"geglu b{bits} [{N}, {K}] M={M}"
        step(label)
        wg, wu = _qw(N + 1, N, K, bits), _qw(N + 2, N, K, bits)
        x = synth.normal_f32(N, M, M * K).reshape(M, K)
        with Dev(c) as d:
            y = d.empty((M, N))
            c.linear_q_geglu(d.w(wg), d.w(wu), d.arr(x).ptr, y.ptr, M)
            _check_fused(y.to_host(), x, wg, wu, None, 0, label)
    for M, off, bits in [(1, 0, 4), (1, 34 * 256, 4), (3, 11 * 256, 4), (1, 5 * 256, 2)]:
        label = f"per-layer gate b{bits} [256, 1536] M={M} cols {off}"
        step(label)
        w = _qw(77, 256, 1536, bits)
        x = synth.normal_f32(78, M, M * 1536).reshape(M, 1536)
        b = synth.normal_f32(79, M, M * 35 * 256).reshape(M, 35 * 256)
        with Dev(c) as d:
            y = d.empty((M, 256))
            c.linear_q_gelu_mul_cols(d.w(w), d.arr(x).ptr, d.arr(b).ptr, 35 * 256, off, y.ptr, M)
            _check_fused(y.to_host(), x, w, None, b, off, label)
    # the element kernel's fused epilogues (K not whole words)
    wg, wu = _qw(5, 30, 52, 4), _qw(6, 30, 52, 4)
    x = synth.normal_f32(7, 3, 3 * 52).reshape(3, 52)
    step("geglu element kernel")
    with Dev(c) as d:
        y = d.empty((3, 30))
        c.linear_q_geglu(d.w(wg), d.w(wu), d.arr(x).ptr, y.ptr, 3)
        _check_fused(y.to_host(), x, wg, wu, None, 0, "geglu element kernel")


def test_embedding_rows(ctx):
    """The per-layer embedding layout: [V, 35 * 256] 4-bit with one scale per
    (row, 256-wide layer block), and a per-row 2-bit table."""
    c = ctx
    for V, D, bits, group, ids in [(1000, 35 * 256, 4, 256, [0, 999, 17, 17, 500]),
                                   (4096, 1536, 2, None, list(range(0, 4096, 97)))]:
        step(f"embed [{V}, {D}] b{bits}")
        w = _qw(V + D, V, D, bits, False, group)
        ids = np.array(ids, np.uint32)
        with Dev(c) as d:
            out = d.empty((ids.size, D))
            c.embed_rows_q(d.w(w), ids, float(np.sqrt(np.float32(D))), out.ptr)
            assert np.array_equal(out.to_host(), oracle.embed_rows_q(w, ids, float(np.sqrt(np.float32(D)))))


def test_argument_errors(ctx):
    c = ctx
    w = _qw(1, 16, 64, 4)
    with Dev(c) as d:
        dw = d.w(w)
        x, y = d.arr(np.zeros((1, 64), np.float32)), d.empty((1, 16))
        with pytest.raises(g4a.G4aError, match="outside the table"):
            c.embed_rows_q(dw, [3, 16], 1.0, d.empty((2, 64)).ptr)
        w2 = d.w(_qw(2, 16, 64, 2))
        with pytest.raises(g4a.G4aError, match="differ"):
            c.linear_q_geglu(dw, w2, x.ptr, y.ptr, 1)
        with pytest.raises(g4a.G4aError, match="exceed the row stride"):
            c.linear_q_gelu_mul_cols(dw, x.ptr, x.ptr, 20, 8, y.ptr, 1)
        bad = c.upload_qweight(np.zeros(64, np.uint8), np.ones(16, np.float32), 16, 7, 2)
        try:
            with pytest.raises(g4a.G4aError, match="whole number of bytes"):
                c.linear_q(bad, x.ptr, y.ptr, 1)
        finally:
            bad.free()
        c.linear_q(dw, x.ptr, y.ptr, 0)  # M = 0: nothing to do


@pytest.mark.parametrize("bits,signed", [(2, False), (4, False), (8, True)])
def test_matrix_core_shapes(ctx, bits, signed):
    """M >= 16 with K % 64 == 0 runs on the matrix cores (x split into three exact
    bf16 parts, exact products, f32 accumulation): ragged token and weight-row
    tiles, K past the word kernel's LDS limit, Gemma-4 prefill shapes."""
    c = ctx
    for N, K, M in [(40, 64, 17), (64, 1536, 16), (1536, 2048, 100), (256, 6144, 300), (12288, 1536, 64),
                    (64, 20480, 16), (100, 4096, 65)]:
        label = f"mfma b{bits}{'s' if signed else ''} N={N} K={K} M={M}"
        step(label)
        w = _qw(N * 3 + K + M, N, K, bits, signed)
        x = synth.normal_f32(N + 2 * K, M, M * K).reshape(M, K)
        _check_sum(_linear_gpu(c, w, x), oracle.linear_q(x, w), _bound(x, w), label)


def test_matrix_core_fused_epilogues(ctx):
    c = ctx
    N, K, M = 2048, 1536, 64
    wg, wu = _qw(91, N, K, 4), _qw(92, N, K, 4)
    x = synth.normal_f32(93, M, M * K).reshape(M, K)
    step("mfma geglu [2048, 1536] M=64")
    with Dev(c) as d:
        y = d.empty((M, N))
        c.linear_q_geglu(d.w(wg), d.w(wu), d.arr(x).ptr, y.ptr, M)
        _check_fused(y.to_host(), x, wg, wu, None, 0, "mfma geglu")
    w = _qw(94, 256, 1536, 4)
    x = synth.normal_f32(95, 33, 33 * 1536).reshape(33, 1536)
    b = synth.normal_f32(96, 33, 33 * 35 * 256).reshape(33, 35 * 256)
    step("mfma per-layer gate [256, 1536] M=33")
    with Dev(c) as d:
        y = d.empty((33, 256))
        c.linear_q_gelu_mul_cols(d.w(w), d.arr(x).ptr, d.arr(b).ptr, 35 * 256, 20 * 256, y.ptr, 33)
        _check_fused(y.to_host(), x, w, None, b, 20 * 256, "mfma per-layer gate")
