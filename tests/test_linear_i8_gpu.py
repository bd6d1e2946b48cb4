"""GPU parity of the int8 matrix-core projection (g4a_linear_q with M <= 2, one
scale per row: the decode path of large weights such as the 2-bit lm_head)
against the CPU oracle (rust/src/backend_cpu.rs:174-222, rust/src/backend.rs:44-58
restated in oracle/linear_oracle.c), through the C-ABI.

The kernel cuts each activation row into 8 signed digits against one power of
two, so every digit column's dot product with the weight fields is an exact
int32 sum; only the f32 sum of the 8 column totals and the final scaling round.
Bars, written per test:
  - the word kernel's bar against the oracle: |gpu - oracle| <= 2e-6 * sum_k
    |x_k w_nk| + 1e-7 (the oracle sums in f32, in k order);
  - closeness to the exact sum (numpy f64 over the dequantised weight):
    |gpu - exact| <= 4e-7 * sum_k |x_k w_nk| + 2 ulp(exact) + 1e-30, with no
    absolute floor beyond the last term: five times tighter than the word
    kernel's bar, which an f32 summation in another order does not meet in
    general;
  - an activation row holding an inf or NaN: bit-identical to the oracle (that
    row is computed in the CPU's order), NaN where the oracle has NaN.
Contexts here set the linear_i8 option to 1, which sends every eligible projection to
this kernel; the default context sends weights of 16 MB and more.
"""

import numpy as np
import pytest

import g4a
import g4a.synth as synth
import oracle
from test_linear_gpu import Dev, _qw, _deq_abs

pytestmark = pytest.mark.gpu


def step(msg):
    print(f"[gpu] {msg}", flush=True)


@pytest.fixture(scope="module")
def ictx():
    """A context that runs every eligible M <= 2 projection on the int8 kernel."""
    c = g4a.Context(0, options={"linear_i8": 1})
    yield c
    c.close()


def _deq(w):
    """The dequantised weight in f64 [N, K] (QuantWeight::deq)."""
    N, K, bits = w.N, w.K, w.bits
    qb = w.qbytes.reshape(N, -1)
    if w.signed_i8:
        q = qb.view(np.int8).astype(np.float64)
    else:
        per = 8 // bits
        f = np.stack([(qb >> (j * bits)) & ((1 << bits) - 1) for j in range(per)], axis=-1).reshape(N, K)
        q = f.astype(np.float64) - (1 << (bits - 1))
    return q * w.scales.reshape(N, -1).astype(np.float64)[:, :1]


def _run(c, w, x):
    with Dev(c) as d:
        dw, dx = d.w(w), d.arr(x)
        y = d.empty((x.shape[0], w.N))
        c.linear_q(dw, dx.ptr, y.ptr, x.shape[0])
        return y.to_host()


def _check(got, x, w, label, rows=None):
    """Both bars, over the activation rows `rows` (all by default)."""
    rows = list(range(x.shape[0])) if rows is None else rows
    want = oracle.linear_q(x, w)
    dq = _deq(w)
    x64 = x[rows].astype(np.float64)  # only the checked rows: another may hold an inf or NaN
    exact = x64 @ dq.T
    bound = np.abs(x64) @ np.abs(dq).T
    for i, m in enumerate(rows):
        e_or = np.abs(got[m].astype(np.float64) - want[m].astype(np.float64))
        tol_or = 2e-6 * bound[i] + 1e-7
        ulp = np.spacing(np.abs(exact[i]).astype(np.float32)).astype(np.float64)
        e_ex = np.abs(got[m].astype(np.float64) - exact[i])
        tol_ex = 4e-7 * bound[i] + 2 * ulp + 1e-30
        print(f"  {label} row {m}: vs oracle {e_or.max():.3e} (err/tol {(e_or / tol_or).max():.3f}), "
              f"vs exact {e_ex.max():.3e} (err/tol {(e_ex / tol_ex).max():.3f})", flush=True)
        assert np.all(e_or <= tol_or), f"{label} row {m}: oracle bar"
        assert np.all(e_ex <= tol_ex), f"{label} row {m}: exact-sum bar"


# K: the smallest whole unit per bit width (rows of one 128-byte unit), Gemma's
# 1536, and the 4096 LDS limit; N: one row, partial 32-row chunks, many chunks.
SHAPES = [(1, None, 1), (15, 512, 2), (33, 1536, 1), (1000, 1536, 2), (4099, 1536, 1), (257, 4096, 2),
          (20000, 1536, 1)]


@pytest.mark.parametrize("bits,signed", [(2, False), (4, False), (8, True), (8, False)])
def test_int8_kernel_shapes(ictx, bits, signed):
    for N, K, M in SHAPES:
        K = K or 1024 // bits
        label = f"b{bits}{'s' if signed else ''} N={N} K={K} M={M}"
        step(label)
        w = _qw(N * 5 + K + M + bits, N, K, bits, signed)
        x = synth.normal_f32(N + 3 * K, M, M * K).reshape(M, K)
        _check(_run(ictx, w, x), x, w, label)


def test_int8_kernel_dynamic_range(ictx):
    """Elements spread over 2^-60 .. 2^60 of one another: the digits hold every
    element within 2^-32 of the row maximum exactly and lose at most 2^-56 of
    the maximum on the others. Also a row of zeros and a row with a single
    nonzero element."""
    K, N = 1536, 777
    w = _qw(91, N, K, 2)
    rng = np.random.default_rng(5)
    g = synth.normal_f32(17, 2, 2 * K).reshape(2, K)
    x = (g * np.exp2(rng.integers(-60, 61, size=(2, K)))).astype(np.float32)
    step("dynamic range 2^+-60")
    _check(_run(ictx, w, x), x, w, "range")
    x = np.zeros((2, K), np.float32)
    x[1, 700] = -3.5e-20
    step("zeros, one nonzero element")
    got = _run(ictx, w, x)
    assert np.all(got[0] == 0.0)
    _check(got, x, w, "single", rows=[1])
    x = np.full((1, K), 1.0e37, np.float32)  # large but finite: digits scale by 2^(6-E)
    x[0, ::3] *= -1.0
    step("large finite values")
    _check(_run(ictx, w, x), x, w, "large")


def test_int8_kernel_nonfinite_rows(ictx):
    """A row holding an inf or NaN runs in the CPU's order: bit-identical to the
    oracle, NaN where it is NaN; the other row of the call keeps the digit path."""
    K, N = 1536, 300
    w = _qw(7, N, K, 4)
    for bad in (np.inf, -np.inf, np.nan):
        x = synth.normal_f32(3, 4, 2 * K).reshape(2, K)
        x[1, 123] = bad
        step(f"row 1 holds {bad}")
        got = _run(ictx, w, x)
        want = oracle.linear_q(x, w)
        assert np.array_equal(got[1], want[1], equal_nan=True)
        _check(got, x, w, f"finite row beside {bad}", rows=[0])


def test_default_context_takes_large_weights(ctx):
    """The default context (linear_i8 -1) sends a 2-bit weight of 16 MB or
    more at M = 1 to the int8 kernel: [49152, 1536] is 18.9 MB."""
    N, K = 49152, 1536
    w = _qw(12, N, K, 2)
    x = synth.normal_f32(12, 1, K).reshape(1, K)
    step("auto: 2-bit [49152, 1536] M=1")
    _check(_run(ctx, w, x), x, w, "auto 2-bit lm_head slice")


def test_int8_and_word_kernels_agree(ictx, ctx):
    """The same eligible projection on both kernels (forced here, a 4-bit
    [2048, 1536] weight that the default context keeps on the word kernel):
    both within the oracle bar, so within twice it of each other."""
    N, K = 2048, 1536
    w = _qw(33, N, K, 4)
    x = synth.normal_f32(33, 2, 2 * K).reshape(2, K)
    a, b = _run(ictx, w, x), _run(ctx, w, x)
    bound = np.abs(x.astype(np.float64)) @ _deq_abs(w).T
    assert np.all(np.abs(a.astype(np.float64) - b) <= 4e-6 * bound + 2e-7)
