"""Pinning the oracle's restatement of the quantised projections (CPU only):
QuantWeight::deq (rust/src/backend.rs:44-58), CpuBackend::linear on a
quantised weight (rust/src/backend_cpu.rs:174-222), gelu_tanh (:55-58),
embed_rows (:127-145) and the trait's fused compositions
(rust/src/backend.rs:156-168). The checks do not retype the oracle: bytes
packed by hand with known field values, one-hot activations that read a single
dequantised weight, a vectorised numpy unpack with an f64 matmul, grouped
against per-row scales, closed forms of gelu, and the committed fixtures
regenerated from the reference's own test inputs (quantized_kernel_parity)."""
import numpy as np
import pytest

import g4a.synth as synth
import oracle
from golden_io import load_linear_golden, linear_eval


def _w(qbytes, scales, N, K, bits, signed_i8=False, group_size=None):
    return oracle.QWeight(np.asarray(qbytes, np.uint8), np.asarray(scales, np.float32), N, K, bits, signed_i8,
                          group_size)


def test_golden_fixtures_match_the_oracle_bit_exactly():
    for name, c in load_linear_golden().items():
        assert np.array_equal(linear_eval(c, oracle), c.out), name


def test_hand_packed_fields():
    # 4-bit, LSB first: byte 0x0F holds raw 15 (k = 0) then raw 0 (k = 1); offset 8
    w = _w([[0x0F, 0x87]], [[1.0]], 1, 4, 4)
    assert [oracle.deq(w, 0, k) for k in range(4)] == [7.0, -8.0, -1.0, 0.0]
    # 2-bit: byte 0b11_10_01_00 holds raw 0, 1, 2, 3 (offset 2)
    w = _w([[0b11100100]], [[0.5]], 1, 4, 2)
    assert [oracle.deq(w, 0, k) for k in range(4)] == [-1.0, -0.5, 0.0, 0.5]
    # I8: two's complement
    w = _w([[0x80, 0x7F, 0xFF, 0x00]], [[2.0]], 1, 4, 8, signed_i8=True)
    assert [oracle.deq(w, 0, k) for k in range(4)] == [-256.0, 254.0, -2.0, 0.0]
    # 8-bit offset binary (U8 at 8 bits): raw - 128
    w = _w([[0x80, 0x7F, 0xFF, 0x00]], [[1.0]], 1, 4, 8)
    assert [oracle.deq(w, 0, k) for k in range(4)] == [0.0, -1.0, 127.0, -128.0]


def test_pack_helpers_round_trip_through_deq():
    rng = np.random.default_rng(1)
    for bits in (2, 4, 8):
        lo, hi = -(1 << (bits - 1)), (1 << (bits - 1))
        vals = rng.integers(lo, hi, size=(3, 16))
        w = _w(synth.pack_int(vals, bits).reshape(3, -1), np.ones((3, 1), np.float32), 3, 16, bits,
               signed_i8=bits == 8)
        got = np.array([[oracle.deq(w, n, k) for k in range(16)] for n in range(3)])
        assert np.array_equal(got, vals.astype(np.float64)), bits


@pytest.mark.parametrize("bits,signed", [(2, False), (4, False), (8, True), (8, False)])
def test_one_hot_rows_read_single_weights_exactly(bits, signed):
    N, K = 5, 32
    qb, sc, _ = synth.quant_weight(7, N, K, bits, signed_i8=signed)
    w = _w(qb, sc, N, K, bits, signed)
    x = np.eye(K, dtype=np.float32)[[0, 3, 17, 31]]
    y = oracle.linear_q(x, w)
    for i, k in enumerate([0, 3, 17, 31]):
        assert np.array_equal(y[i], np.array([oracle.deq(w, n, k) for n in range(N)], np.float32))


def _unpack_f64(qb, N, K, bits, signed):
    """Independent vectorised decode of the packed rows."""
    qb = np.asarray(qb, np.uint8).reshape(N, -1)
    if signed:
        return qb.view(np.int8).astype(np.float64)
    per = 8 // bits
    fields = np.stack([(qb >> (j * bits)) & ((1 << bits) - 1) for j in range(per)], axis=-1).reshape(N, K)
    return fields.astype(np.float64) - (1 << (bits - 1))


@pytest.mark.parametrize("bits,signed,group", [(2, False, None), (4, False, None), (8, True, None), (4, False, 64)])
def test_linear_against_an_f64_matmul(bits, signed, group):
    N, K, M = 64, 1536 if group is None else 256, 3
    qb, sc, g = synth.quant_weight(11, N, K, bits, signed_i8=signed, group_size=group)
    w = _w(qb, sc, N, K, bits, signed, g)
    x = synth.normal_f32(11, 5, M * K).reshape(M, K)
    y = oracle.linear_q(x, w).astype(np.float64)
    deq = _unpack_f64(qb, N, K, bits, signed) * np.repeat(sc.astype(np.float64), g, axis=1)[:, :K]
    ref = x.astype(np.float64) @ deq.T
    bound = np.abs(x.astype(np.float64)) @ np.abs(deq).T  # sum |x w|: the scale of the rounding error
    assert np.all(np.abs(y - ref) <= 2e-6 * bound + 1e-12)


def test_grouped_scales_with_equal_groups_equal_per_row_scales():
    N, K = 8, 128
    qb, sc, _ = synth.quant_weight(12, N, K, 4)
    x = synth.normal_f32(12, 5, 2 * K).reshape(2, K)
    per_row = oracle.linear_q(x, _w(qb, sc, N, K, 4))
    grouped = oracle.linear_q(x, _w(qb, np.repeat(sc, 4, axis=1), N, K, 4, group_size=32))
    assert np.array_equal(per_row, grouped)
    # and a group's scale reaches only its own columns
    sc2 = np.repeat(sc, 4, axis=1)
    sc2[:, 1] *= 2.0
    w2 = _w(qb, sc2, N, K, 4, group_size=32)
    assert oracle.deq(w2, 3, 40) == 2.0 * oracle.deq(_w(qb, sc, N, K, 4), 3, 40)
    assert oracle.deq(w2, 3, 70) == oracle.deq(_w(qb, sc, N, K, 4), 3, 70)


def test_gelu_tanh_closed_forms():
    x = np.array([0.0, 1e-3, 0.5, 1.0, 2.5, 6.0, 12.0, -12.0, 40.0, -40.0], np.float32)
    y = oracle.gelu_tanh(x).astype(np.float64)
    xd = x.astype(np.float64)
    ref = 0.5 * xd * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (xd + 0.044715 * xd ** 3)))
    np.testing.assert_allclose(y, ref, rtol=1e-6, atol=1e-30)
    assert y[0] == 0.0
    assert y[8] == 40.0 and y[9] == 0.0  # tanh saturates to +-1 in f32
    # gelu(x) - gelu(-x) = x
    xs = synth.normal_f32(3, 0, 64) * np.float32(3.0)
    d = oracle.gelu_tanh(xs).astype(np.float64) - oracle.gelu_tanh(-xs).astype(np.float64)
    np.testing.assert_allclose(d, xs.astype(np.float64), rtol=2e-6, atol=1e-6)


def test_fused_compositions_select_the_right_columns():
    N, K, M = 16, 64, 2
    qb, sc, _ = synth.quant_weight(13, N, K, 4)
    w = _w(qb, sc, N, K, 4)
    x = synth.normal_f32(13, 5, M * K).reshape(M, K)
    b = np.arange(M * 80, dtype=np.float32).reshape(M, 80)
    y = oracle.linear_q_gelu_mul_cols(x, w, b, 30)
    g = oracle.gelu_tanh(oracle.linear_q(x, w))
    assert np.array_equal(y, g * b[:, 30:46])
    assert np.array_equal(oracle.linear_q_geglu(x, w, w), g * oracle.linear_q(x, w))


def test_embed_rows_reads_the_selected_rows_with_grouped_scales():
    V, D = 10, 32
    qb, sc, g = synth.quant_weight(14, V, D, 4, group_size=16)
    w = _w(qb, sc, V, D, 4, group_size=g)
    ids = np.array([9, 0, 4, 4], np.uint32)
    out = oracle.embed_rows_q(w, ids, 2.0)
    deq = (_unpack_f64(qb, V, D, 4, False) * np.repeat(sc.astype(np.float64), 16, axis=1)).astype(np.float32)
    assert np.array_equal(out, (deq[ids] * np.float32(2.0)).astype(np.float32))
