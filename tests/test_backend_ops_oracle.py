"""Pinning the oracle's restatement of the trait's remaining ops (CPU only):
add / mul / scale / scale_by_tensor / gelu_tanh / geglu / softcap
(rust/src/backend_cpu.rs:224-244), slice_cols (:343-350), embed_rows on an f32
table (:138-144), linear on an f32 weight (:174-222) and the trait's
add_rms_norm composition (rust/src/backend.rs:136-145). Closed forms, f64
brute force and the committed fixtures regenerated from the reference's own
kernel_parity / fused_op_parity inputs."""
import numpy as np

import g4a.synth as synth
import oracle
from golden_io import load_ops_golden, ops_eval


def test_golden_fixtures_match_the_oracle_bit_exactly():
    for name, c in load_ops_golden().items():
        assert np.array_equal(ops_eval(c, oracle), c.out), name


def test_softcap_closed_forms():
    x = np.array([0.0, 1e-4, -1e-4, 15.0, -15.0, 300.0, -300.0, 1e30], np.float32)
    y = oracle.softcap(x, 30.0).astype(np.float64)
    ref = 30.0 * np.tanh(x.astype(np.float64) / 30.0)
    np.testing.assert_allclose(y, ref, rtol=3e-7, atol=0)
    assert y[0] == 0.0 and y[5] == 30.0 and y[7] == 30.0   # saturation, no overflow
    assert np.all(np.abs(y) <= 30.0)
    xs = synth.normal_f32(1, 0, 256) * np.float32(40.0)
    assert np.array_equal(oracle.softcap(-xs, 30.0), -oracle.softcap(xs, 30.0))  # odd


def test_add_rms_norm_is_residual_plus_norm_times_scalar():
    x = synth.normal_f32(2, 0, 4 * 96).reshape(4, 96) * np.float32(3.0)
    res = synth.normal_f32(2, 1, 4 * 96).reshape(4, 96)
    w = (np.float32(1.0) + np.float32(0.1) * synth.normal_f32(2, 2, 96)).astype(np.float32)
    y = oracle.add_rms_norm(res, x, w, 1e-6).astype(np.float64)
    xd = x.astype(np.float64)
    ref = res + xd / np.sqrt((xd ** 2).mean(axis=1, keepdims=True) + 1e-6) * w
    np.testing.assert_allclose(y, ref, rtol=1e-5, atol=1e-6)
    ys = oracle.add_rms_norm(res, x, w, 1e-6, np.float32(0.5))
    assert np.array_equal(ys, (oracle.add_rms_norm(res, x, w, 1e-6) * np.float32(0.5)).astype(np.float32))
    # zero rows leave the residual
    z = oracle.add_rms_norm(res, np.zeros_like(x), w, 1e-6)
    assert np.array_equal(z, res)


def test_linear_f32_against_an_f64_matmul():
    x = synth.normal_f32(3, 0, 5 * 1536).reshape(5, 1536)
    w = (synth.normal_f32(3, 1, 64 * 1536) * np.float32(0.05)).reshape(64, 1536)
    y = oracle.linear_f32(x, w).astype(np.float64)
    ref = x.astype(np.float64) @ w.astype(np.float64).T
    bound = np.abs(x.astype(np.float64)) @ np.abs(w.astype(np.float64)).T
    assert np.all(np.abs(y - ref) <= 2e-6 * bound + 1e-12)
    # one-hot rows read single weights exactly
    e = np.eye(1536, dtype=np.float32)[[0, 700, 1535]]
    assert np.array_equal(oracle.linear_f32(e, w), w[:, [0, 700, 1535]].T)


def test_embed_and_slice_are_exact_gathers():
    table = synth.normal_f32(4, 0, 50 * 24).reshape(50, 24)
    ids = np.array([49, 0, 7, 7], np.uint32)
    assert np.array_equal(oracle.embed_rows_f32(table, ids, 2.0), table[ids] * np.float32(2.0))
    x = synth.normal_f32(4, 1, 6 * 40).reshape(6, 40)
    assert np.array_equal(oracle.slice_cols(x, 13, 9), x[:, 13:22])


def test_geglu_and_elementwise_compositions():
    a, b = synth.normal_f32(5, 0, 64), synth.normal_f32(5, 1, 64)
    assert np.array_equal(oracle.geglu(a, b), oracle.gelu_tanh(a) * b)
    assert np.array_equal(oracle.scale(a, 3.5), (a * np.float32(3.5)).astype(np.float32))
