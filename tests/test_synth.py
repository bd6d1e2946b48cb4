"""The reference's benchmark RNG as synth.Xorshift restates it (rust/src/main.rs:306-333):
the vectorised generator (jump-ahead by GF(2) matrix powers, doubling blocks) must give
exactly the states of the plain recurrence, and f32s the f32 arithmetic of the formula."""
import numpy as np

import g4a.synth as synth


def scalar_states(seed, n):
    s, out = seed, []
    for _ in range(n):
        s ^= (s << 13) & 0xFFFFFFFF
        s ^= s >> 17
        s ^= (s << 5) & 0xFFFFFFFF
        out.append(s)
    return np.array(out, dtype=np.uint32)


def test_xorshift_matches_the_recurrence():
    for seed in (987654321, 12345, 0x9E3779B9, 1):
        got = synth.Xorshift(seed).next(70000)
        assert np.array_equal(got, scalar_states(seed, 70000)), seed


def test_xorshift_skip_and_continuation():
    r = synth.Xorshift(987654321)
    r.skip(12345)
    want = scalar_states(987654321, 12345 + 10)[-10:]
    assert np.array_equal(r.next(10), want)
    # consecutive calls continue the stream
    a = synth.Xorshift(7)
    first, second = a.next(1000), a.next(333)
    assert np.array_equal(np.concatenate([first, second]), scalar_states(7, 1333))


def test_xorshift_f32s_formula():
    """base + (f*2 - 1)*sc with f = next as f32 / u32::MAX as f32, each op rounded in f32."""
    states = scalar_states(987654321, 64)
    got = synth.Xorshift(987654321).f32s(64, 0.1, 0.0)
    for s, g in zip(states, got):
        f = np.float32(np.float32(int(s)) / np.float32(4294967296.0))  # u32::MAX as f32 rounds to 2^32
        want = np.float32(np.float32(0.0) + np.float32(np.float32(f * np.float32(2.0)) - np.float32(1.0))
                          * np.float32(0.1))
        assert g == want
    assert np.all(np.abs(got) <= np.float32(0.1))


def test_reference_bench_draw_count():
    """Draws before the first attention case, counted from rust/src/main.rs:493-543 by hand
    (one draw per 4 packed bytes, per row scale, per activation and per f32 weight):
    packed words 25165824 (2-bit lm_head) + 4 x 1179648 (4-bit gate, GeGLU gate and up,
    2-bit prefill gate) + 589824 (2-bit down) + 393216 (4-bit q_proj); scales 262144 +
    3 x 6144 + 12288 + 1536 + 2048; activations 1536 x 5 + 64 x 1536 + 6144; GEMV weight
    8960 x 1536."""
    words = 25165824 + 4 * 1179648 + 589824 + 393216
    scales = 262144 + 3 * 6144 + 12288 + 1536 + 2048
    acts = 5 * 1536 + 64 * 1536 + 6144
    assert synth.reference_bench_draws_before_attention() == words + scales + acts + 8960 * 1536 == 45038592


def test_reference_bench_inputs_shapes():
    cases = list(synth.reference_bench_inputs())
    assert [c[0] for c in cases] == synth.REFERENCE_BENCH_CASES
    for (dh, S, _), q, k, v in cases:
        assert q.shape == (1, 8, dh) and k.shape == (S, 1, dh) and v.shape == (S, 1, dh)
        assert q.dtype == k.dtype == v.dtype == np.float32
        assert np.abs(k).max() <= np.float32(0.1)
