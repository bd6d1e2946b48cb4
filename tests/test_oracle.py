"""Pinning the CPU oracle (oracle/attn_oracle.c, a restatement of
rust/src/backend_cpu.rs:270-336) with checks that do not retype its formula:
closed forms, invariants the mathematics fixes, an f64 brute force, thread
invariance of par_ranges (rust/src/backend_cpu.rs:63-91), and the committed
golden vectors regenerated from the reference's own parity-test inputs.

CPU only."""
import numpy as np
import pytest

import oracle
import g4a.synth as synth
from golden_io import load_golden


def _rand(rng, *shape, s=1.0):
    return (rng.uniform(-s, s, size=shape)).astype(np.float32)


def test_single_visible_key_returns_its_value_row():
    # with one visible key e = exp(0) = 1, inv = 1, w = 1: out == v row exactly
    rng = np.random.default_rng(1)
    q, k, v = _rand(rng, 1, 8, 256), _rand(rng, 40, 1, 256), _rand(rng, 40, 1, 256)
    for j in (0, 17, 39):
        out = oracle.attention(q, k, v, q_pos=[j], k_pos=np.arange(40), window=1)
        assert np.array_equal(out.reshape(8, 256), np.broadcast_to(v[j, 0], (8, 256)))


def test_zero_query_gives_mean_of_visible_values():
    rng = np.random.default_rng(2)
    S = 300
    q = np.zeros((2, 4, 64), np.float32)
    k, v = _rand(rng, S, 2, 64), _rand(rng, S, 2, 64)
    out = oracle.attention(q, k, v, q_pos=[100, 299], k_pos=np.arange(S), window=50).reshape(2, 4, 64)
    for i, qp in enumerate((100, 299)):
        vis = np.arange(qp - 49, qp + 1)
        for h in range(4):
            want = v[vis, h // 2].astype(np.float64).mean(axis=0)
            np.testing.assert_allclose(out[i, h], want, atol=2e-6, rtol=0)


def test_all_future_keys_give_zero():
    rng = np.random.default_rng(3)
    q, k, v = _rand(rng, 3, 8, 32), _rand(rng, 10, 1, 32), _rand(rng, 10, 1, 32)
    out = oracle.attention(q, k, v, q_pos=[0, 1, 2], k_pos=np.arange(10, 20))
    assert np.all(out == 0.0)


def test_window_isolation_is_bit_exact():
    # values outside [qpos - window + 1, qpos] must not influence the output at all
    rng = np.random.default_rng(4)
    S, W = 700, 64
    q, k, v = _rand(rng, 2, 8, 256), _rand(rng, S, 1, 256), _rand(rng, S, 1, 256)
    qp = [500, 699]
    base = oracle.attention(q, k, v, q_pos=qp, k_pos=np.arange(S), window=W)
    v2 = v.copy()
    v2[:500 - W + 1] = 1e3
    v2[436] = -7.0  # outside row 500's window (500 - 436 >= 64) and row 699's
    k2 = k.copy()
    k2[:437] *= -3.0  # keys 0..436 are outside both windows
    out = oracle.attention(q, k2, v2, q_pos=qp, k_pos=np.arange(S), window=W)
    assert np.array_equal(base, out)


def test_key_range_trim_equals_full_masking_bit_exact():
    # the wgpu host trims [k_start, k_end) (rust/src/backend_wgpu.rs:924-936); masked keys add
    # nothing to the max, the sum or the output, so slicing the cache must be bit-identical
    rng = np.random.default_rng(5)
    S, W = 900, 512
    q, k, v = _rand(rng, 1, 8, 256), _rand(rng, S, 1, 256), _rand(rng, S, 1, 256)
    full = oracle.attention(q, k, v, q_pos=[899], k_pos=np.arange(S), window=W)
    lo = 899 - W + 1
    trimmed = oracle.attention(q, k[lo:], v[lo:], q_pos=[899], k_pos=np.arange(lo, S), window=W)
    assert np.array_equal(full, trimmed)


def test_key_permutation_changes_only_rounding():
    rng = np.random.default_rng(6)
    S = 257
    q, k, v = _rand(rng, 2, 8, 128), _rand(rng, S, 1, 128), _rand(rng, S, 1, 128)
    kp = np.arange(S, dtype=np.uint32)
    base = oracle.attention(q, k, v, q_pos=[200, 256], k_pos=kp, window=100)
    perm = rng.permutation(S)
    out = oracle.attention(q, k[perm], v[perm], q_pos=[200, 256], k_pos=kp[perm], window=100)
    np.testing.assert_allclose(out, base, atol=1e-6, rtol=0)


@pytest.mark.parametrize("case", [(4, 50, 8, 1, 64, 0, 0.125), (3, 33, 4, 2, 48, 7, 1.0), (1, 512, 8, 1, 256, 512, 1.0)])
def test_against_f64_brute_force(case):
    # structural mistakes (wrong head mapping, transposed operands, bad masks) give O(1) errors;
    # the f32 restatement must sit within f32 rounding of the exact result
    T, S, Hq, Hkv, D, W, scale = case
    rng = np.random.default_rng(7)
    q, k, v = _rand(rng, T, Hq, D), _rand(rng, S, Hkv, D), _rand(rng, S, Hkv, D)
    got = oracle.attention(q, k, v, scale=scale, window=W)
    want = oracle.attention_f64(q, k, v, scale=scale, window=W)
    # measured f32-vs-f64 gaps: 9e-8, 2.3e-7, 4.3e-6 (the 256-term dots at scale 1)
    assert np.abs(got - want).max() < 1e-5


def test_gqa_head_mapping_against_numpy_f64():
    # independent numpy restatement of the mapping h -> kv head h // (Hq/Hkv) and the masks
    rng = np.random.default_rng(8)
    T, S, Hq, Hkv, D, W = 3, 20, 6, 3, 16, 5
    q, k, v = _rand(rng, T, Hq, D), _rand(rng, S, Hkv, D), _rand(rng, S, Hkv, D)
    qpos = np.array([4, 12, 19])
    got = oracle.attention(q, k, v, q_pos=qpos, k_pos=np.arange(S), scale=0.5, window=W).reshape(T, Hq, D)
    for i in range(T):
        for h in range(Hq):
            kv = h // (Hq // Hkv)
            js = [j for j in range(S) if j <= qpos[i] and qpos[i] - j < W]
            s = np.array([0.5 * np.dot(q[i, h].astype(np.float64), k[j, kv]) for j in js])
            p = np.exp(s - s.max())
            p /= p.sum()
            want = (p[:, None] * v[js, kv].astype(np.float64)).sum(0)
            np.testing.assert_allclose(got[i, h], want, atol=2e-6, rtol=0)


def _numpy_attention_f64(q, k, v, q_pos, k_pos, scale, window, softcap):
    """Masked softmax attention in float64, vectorised with numpy, written from the
    definition (not from the C oracle's loops): scores = scale * q . k, optional
    cap * tanh(s / cap), key j visible to query i iff kpos <= qpos and (no window
    or qpos - kpos < window), softmax over the visible keys, weights times v; a
    row with no visible key is 0."""
    T, Hq, _ = q.shape
    S, Hkv, Dv = v.shape
    g = Hq // Hkv
    kk = np.repeat(k.astype(np.float64), g, axis=1)  # [S, Hq, Dh]: query head h reads kv head h // g
    vv = np.repeat(v.astype(np.float64), g, axis=1)  # [S, Hq, Dv]
    s = scale * np.einsum("thd,shd->ths", q.astype(np.float64), kk)
    if softcap > 0:
        s = softcap * np.tanh(s / softcap)
    qp, kp = q_pos.astype(np.int64)[:, None], k_pos.astype(np.int64)[None, :]
    vis = (kp <= qp) & ((window == 0) | (qp - kp < window))  # [T, S]
    s = np.where(vis[:, None, :], s, -np.inf)
    m = s.max(axis=2, keepdims=True)
    e = np.where(vis[:, None, :], np.exp(s - np.where(np.isfinite(m), m, 0.0)), 0.0)
    l = e.sum(axis=2, keepdims=True)
    p = np.divide(e, l, out=np.zeros_like(e), where=l > 0)
    return np.einsum("ths,shd->thd", p, vv).reshape(T, Hq * Dv)


def _draw_oracle_case(rng):
    Hkv = int(rng.choice([1, 2, 3]))
    Hq = Hkv * int(rng.choice([1, 2, 4, 8]))
    Dh = int(rng.choice([8, 16, 40, 64, 128]))
    Dv = int(rng.choice([Dh, Dh, 24, 96]))
    T, S = int(rng.integers(1, 9)), int(rng.integers(1, 300))
    window = int(rng.choice([0, 0, 1, 5, 64, int(rng.integers(1, 400))]))
    softcap = float(rng.choice([0.0, 0.0, 3.0, 30.0]))
    scale = float(rng.choice([1.0, 1.0 / np.sqrt(Dh), 0.0625]))
    if rng.random() < 0.4:  # explicit positions: gaps, any order, repeats
        k_pos = rng.integers(0, 2 * S + 5, size=S).astype(np.uint32)
        q_pos = rng.integers(0, 2 * S + 10, size=T).astype(np.uint32)
    else:
        k0 = int(rng.integers(0, 100))
        k_pos = np.arange(k0, k0 + S, dtype=np.uint32)
        q_pos = np.arange(k0 + S - T, k0 + S, dtype=np.uint32) if S >= T else np.arange(k0, k0 + T, dtype=np.uint32)
    return T, S, Hq, Hkv, Dh, Dv, window, softcap, scale, q_pos, k_pos


@pytest.mark.parametrize("seed", range(40))
def test_random_shapes_against_an_independent_numpy_f64_restatement(seed):
    """The oracle against a float64 numpy restatement written from the definition,
    over seeded random shapes: head groups (including 3 kv heads), value dims other
    than the key dims, windows down to 1, soft-cap, scales, and explicit positions
    with gaps, repeats and any order. A wrong head mapping, a swapped operand, an
    off-by-one mask or a dropped soft-cap gives an O(1) error; f32 rounding stays
    far below 1e-5 at these sizes."""
    rng = np.random.default_rng(4000 + seed)
    T, S, Hq, Hkv, Dh, Dv, window, softcap, scale, q_pos, k_pos = _draw_oracle_case(rng)
    q, k, v = _rand(rng, T, Hq, Dh), _rand(rng, S, Hkv, Dh), _rand(rng, S, Hkv, Dv)
    got = oracle.attention(q, k, v, q_pos=q_pos, k_pos=k_pos, scale=scale, window=window, softcap=softcap)
    want = _numpy_attention_f64(q, k, v, q_pos, k_pos, scale, window, softcap)
    d = np.abs(got.astype(np.float64) - want)
    assert d.max() < 1e-5, (f"T={T} S={S} Hq={Hq} Hkv={Hkv} Dh={Dh} Dv={Dv} window={window} softcap={softcap} "
                            f"scale={scale}: max-abs {d.max():.3e}")


def test_softcap_applies_tanh():
    rng = np.random.default_rng(9)
    q, k, v = _rand(rng, 1, 2, 32, s=3.0), _rand(rng, 30, 1, 32, s=3.0), _rand(rng, 30, 1, 32)
    got = oracle.attention(q, k, v, softcap=5.0)
    want = oracle.attention_f64(q, k, v, softcap=5.0)
    assert np.abs(got - want).max() < 2e-6
    plain = oracle.attention(q, k, v)
    assert np.abs(plain - got).max() > 1e-3  # the cap changes the answer at these magnitudes


def test_thread_count_does_not_change_results():
    # par_ranges gives each chunk disjoint rows; per-row arithmetic is thread-independent
    ins = synth.gemma_inputs(T=7, S=600, Dh=256, seed=11)
    a = oracle.attention(ins.q, ins.k, ins.v, ins.q_pos, ins.k_pos, window=512, threads=1)
    b = oracle.attention(ins.q, ins.k, ins.v, ins.q_pos, ins.k_pos, window=512, threads=5)
    c = oracle.attention(ins.q, ins.k, ins.v, ins.q_pos, ins.k_pos, window=512, threads=56)
    assert np.array_equal(a, b) and np.array_equal(a, c)


def test_thread_count_rule(monkeypatch):
    # rust/src/backend_cpu.rs:72-78: env override if >= 1, else cores; capped at rows; at least 1
    monkeypatch.setenv("GEMMA_CPU_THREADS", "3")
    assert oracle.thread_count(8) == 3
    assert oracle.thread_count(2) == 2
    monkeypatch.setenv("GEMMA_CPU_THREADS", "0")
    assert oracle.thread_count(1000) >= 1
    monkeypatch.setenv("GEMMA_CPU_THREADS", "x")
    assert oracle.thread_count(1) == 1
    assert oracle.thread_count(8, requested=4) == 4


def test_rms_norm_matches_synth_restatement_and_f64():
    rng = np.random.default_rng(10)
    x = rng.standard_normal((33, 512)).astype(np.float32)
    a = oracle.rms_norm(x)
    b = synth.rms_norm_rows(x)
    assert np.array_equal(a, b)
    want = x / np.sqrt((x.astype(np.float64) ** 2).mean(-1, keepdims=True) + 1e-6)
    np.testing.assert_allclose(a, want, atol=2e-6, rtol=0)


def test_incremental_decode_equals_full_prefill():
    # rust/tests/model.rs:38-51 at the attention level: row i of a causal prefill equals the
    # decode of query i against keys 0..i (bit-exact: masked keys contribute nothing)
    ins = synth.gemma_inputs(T=9, S=9, Dh=256, seed=12, q_pos=np.arange(9))
    full = oracle.attention(ins.q, ins.k, ins.v, ins.q_pos, ins.k_pos, window=4)
    for i in range(9):
        one = oracle.attention(ins.q[i:i + 1], ins.k[: i + 1], ins.v[: i + 1], [i], np.arange(i + 1), window=4)
        assert np.array_equal(one[0], full[i])


def test_golden_vectors_reproduce():
    """The committed fixtures (tests/golden/make_golden.py) — oracle outputs on the
    reference's own parity inputs (Lcg) and on small seeded Gaussian cases — are
    reproduced bit-exactly, and their inputs regenerate to the stored hashes."""
    for name, case in load_golden().items():
        out = oracle.attention(case.q, case.k, case.v, case.q_pos, case.k_pos, scale=case.scale,
                               window=case.window, softcap=case.softcap)
        assert np.array_equal(out, case.out), name
