"""Pinning the oracle's restatement of the attention producer's ops (CPU only):
rms_norm (rust/src/backend_cpu.rs:149-172), rope (:248-268) and their
composition head_norm_rope (rust/src/backend.rs:146-154), with checks that do
not retype the oracle's formula: closed forms, invariants of a rotation, an
f64 brute force through complex multiplication, the libm frequencies against
f64 powers, and the committed fixtures regenerated from the reference's own
parity-test inputs (kernel_parity, fused_op_parity)."""
import numpy as np
import pytest

import g4a.synth as synth
import oracle
from golden_io import load_norm_rope_golden, norm_rope_eval


def _x(seed, *shape, s=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * s).astype(np.float32)


def test_golden_fixtures_match_the_oracle_bit_exactly():
    for name, c in load_norm_rope_golden().items():
        got = norm_rope_eval(c, oracle)
        assert np.array_equal(got, c.out), name


def test_rope_at_position_zero_is_the_identity():
    x = _x(1, 3, 4, 64)
    y = oracle.rope(x, np.zeros(3, np.uint32), 1e4, 64)
    assert np.array_equal(x, y)  # cos 0 = 1, sin 0 = 0: a*1 - b*0 == a exactly


@pytest.mark.parametrize("rot", [0, 8, 128])
def test_rope_passes_the_tail_through_bit_exactly(rot):
    x = _x(2, 2, 3, 256)
    y = oracle.rope(x, np.array([5, 32767], np.uint32), 1e6, rot)
    assert np.array_equal(x[..., rot:], y[..., rot:])
    if rot == 0:
        assert np.array_equal(x, y)


def test_rope_is_a_rotation_of_each_pair():
    x = _x(3, 4, 2, 512)
    pos = np.array([0, 17, 4096, 131071], np.uint32)
    y = oracle.rope(x, pos, 1e6, 128).astype(np.float64)
    x = x.astype(np.float64)
    n_in = x[..., :64] ** 2 + x[..., 64:128] ** 2
    n_out = y[..., :64] ** 2 + y[..., 64:128] ** 2
    np.testing.assert_allclose(n_out, n_in, rtol=2e-6, atol=1e-6)


def test_rope_frequencies_are_the_correctly_rounded_powers():
    # recover each freq from a unit vector at position 1 (ang = freq exactly): the
    # libm powf value must be within one ulp of the f64 power rounded to f32
    for theta, rot in [(1e4, 256), (1e6, 128), (1e4, 8)]:
        half = rot // 2
        x = np.zeros((1, 1, rot), np.float32)
        x[0, 0, :half] = 1.0
        y = oracle.rope(x, np.array([1], np.uint32), theta, rot).astype(np.float64)
        ang = np.arctan2(y[0, 0, half:], y[0, 0, :half])
        exp32 = (-(np.float32(2.0) * np.arange(half, dtype=np.float32)) / np.float32(rot)).astype(np.float32)
        want = np.float32(np.float64(theta) ** exp32.astype(np.float64))
        ulp = np.spacing(want).astype(np.float64)
        assert np.all(np.abs(ang - want.astype(np.float64)) <= ulp + 2e-7 * np.abs(ang))


def test_rope_matches_complex_multiplication_in_f64():
    # small positions keep the f32 angle within 1e-6 rad of the f64 one
    x = _x(4, 5, 3, 256)
    pos = np.array([0, 1, 7, 33, 100], np.uint32)
    y = oracle.rope(x, pos, 1e4, 256).astype(np.float64)
    j = np.arange(128)
    freq = 1e4 ** (-(2.0 * j) / 256.0)
    z = (x[..., :128].astype(np.float64) + 1j * x[..., 128:].astype(np.float64)) * \
        np.exp(1j * pos[:, None, None].astype(np.float64) * freq)
    np.testing.assert_allclose(y[..., :128], z.real, atol=5e-5)
    np.testing.assert_allclose(y[..., 128:], z.imag, atol=5e-5)


def test_rope_composes_positions():
    x = _x(5, 1, 2, 64)
    a = oracle.rope(oracle.rope(x, np.array([20], np.uint32), 1e4, 64), np.array([13], np.uint32), 1e4, 64)
    b = oracle.rope(x, np.array([33], np.uint32), 1e4, 64)
    np.testing.assert_allclose(a, b, atol=2e-5)


def test_rms_norm_gives_unit_rms_and_scales_by_the_weight():
    x = _x(6, 7, 256, s=3.0)
    y = oracle.rms_norm(x, None, 1e-6).astype(np.float64)
    np.testing.assert_allclose(np.sqrt((y ** 2).mean(axis=1)), 1.0, rtol=1e-5)
    w = _x(7, 256)
    yw = oracle.rms_norm(x, w, 1e-6).astype(np.float64)
    np.testing.assert_allclose(yw, y * w, rtol=1e-6, atol=1e-7)
    # f64 brute force
    ref = x / np.sqrt((x.astype(np.float64) ** 2).mean(axis=1, keepdims=True) + 1e-6)
    np.testing.assert_allclose(y, ref, rtol=2e-6, atol=1e-7)


def test_rms_norm_of_zero_rows_is_zero():
    y = oracle.rms_norm(np.zeros((2, 64), np.float32), None, 1e-6)
    assert np.all(y == 0.0)


def test_head_norm_rope_is_norm_then_rope_and_producer_composes_it():
    x = _x(8, 2, 8, 512)
    w = (1.0 + 0.1 * _x(9, 512)).astype(np.float32)
    pos = np.array([40000, 40001], np.uint32)
    want = oracle.rope(oracle.rms_norm(x.reshape(16, 512), w, 1e-6).reshape(2, 8, 512), pos, 1e6, 128)
    assert np.array_equal(oracle.head_norm_rope(x, w, 1e-6, pos, 1e6, 128), want)
    k, v = _x(10, 2, 1, 512), _x(11, 2, 1, 512)
    qo, ko, vo = oracle.producer(x, k, v, w, w, pos, 1e6, 128, 1e-6)
    assert np.array_equal(qo, want)
    assert np.array_equal(ko, oracle.head_norm_rope(k, w, 1e-6, pos, 1e6, 128))
    assert np.array_equal(vo, oracle.rms_norm(v.reshape(2, 512), None, 1e-6).reshape(2, 1, 512))
    qo2, ko2, _ = oracle.producer(x, k, v, None, None, pos, 1e6, 128, 1e-6)
    assert np.array_equal(qo2, oracle.rope(x, pos, 1e6, 128))  # no norm weight: rope only
    assert np.array_equal(ko2, oracle.rope(k, pos, 1e6, 128))


def test_synthetic_gemma_inputs_use_the_same_rms_norm():
    # the benchmark generator's unit-RMS rows are the oracle's unweighted rms_norm
    x = synth.normal_f32(3, 0, 4 * 256).reshape(4, 256)
    assert np.array_equal(synth.rms_norm_rows(x), oracle.rms_norm(x, None, 1e-6))
