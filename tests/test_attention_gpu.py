"""GPU parity of the HIP attention path against the CPU oracle
(rust/src/backend_cpu.rs:270-336 restated in oracle/attn_oracle.c), through
the C-ABI of libg4a.so. The bar is the north star's: max-abs <= 1e-5 and
mean-abs <= 1e-6 in f32, on identical seeded inputs.

Mirrors the reference's own GPU tests (grouped_attention_parity,
rust/tests/gpu.rs:262-293; the attention part of kernel_parity,
rust/tests/gpu.rs:122-142) and adds the benchmark configurations at full size,
the split-K sweep, the KV ring layout, explicit positions, the soft-cap and
the empty cases."""
import numpy as np
import pytest

import g4a
import g4a.synth as synth
import oracle
from golden_io import load_golden

pytestmark = pytest.mark.gpu

MAX_ABS = 1e-5
MEAN_ABS = 1e-6


def assert_parity(got, want, label):
    d = np.abs(got.astype(np.float64) - np.asarray(want, np.float64))
    mx, mean = float(d.max()) if d.size else 0.0, float(d.mean()) if d.size else 0.0
    print(f"  {label}: max-abs {mx:.3e} mean-abs {mean:.3e}", flush=True)
    assert mx <= MAX_ABS and mean <= MEAN_ABS, f"{label}: max-abs {mx:.3e} mean-abs {mean:.3e}"


def step(msg):
    print(f"[gpu] {msg}", flush=True)


def test_golden_vectors(ctx):
    """Every committed golden case (the reference's Lcg parity inputs and seeded Gaussian cases)."""
    for name, c in load_golden().items():
        step(f"golden {name}")
        got = g4a.attention_host(ctx, c.q, c.k, c.v, q_pos=c.q_pos, k_pos=c.k_pos, scale=c.scale,
                                 window=c.window, softcap=c.softcap)
        assert_parity(got, c.out, name)


def test_reference_grouped_cases_with_explicit_positions(ctx):
    """grouped_attention_parity cases with positions passed as uploaded arrays (the general path)."""
    for case, q, k, v, qp, kp, scale, window in synth.grouped_parity_inputs():
        step(f"grouped explicit positions {case}")
        want = oracle.attention(q, k, v, qp, kp, scale=scale, window=window)
        got = g4a.attention_host(ctx, q, k, v, q_pos=qp, k_pos=kp, scale=scale, window=window,
                                 contiguous_positions=False)
        assert_parity(got, want, str(case))


@pytest.mark.parametrize("name,T,S,Dh,window,seed", [
    ("configs[0] sliding decode hd256 S512", 1, 512, 256, 512, 0),
    ("configs[1] global decode hd512 S8192", 1, 8192, 512, 0, 0),
    ("headline global decode hd512 S32768", 1, 32768, 512, 0, 4),
])
def test_benchmark_decode_configs(ctx, name, T, S, Dh, window, seed):
    step(name)
    ins = synth.gemma_inputs(T=T, S=S, Dh=Dh, seed=seed)
    want = oracle.attention(ins.q, ins.k, ins.v, ins.q_pos, ins.k_pos, scale=1.0, window=window)
    got = g4a.attention_host(ctx, ins.q, ins.k, ins.v, window=window)
    assert_parity(got, want, name)


def test_config2_long_context_split_sweep(ctx):
    """hd512 global decode over 131072 keys, split count swept 8..512,
    plus counts that leave ragged 16-split groups in the merge (100, 300, and
    1000, which the 192-key splits make 683)."""
    ins = synth.gemma_inputs(T=1, S=131072, Dh=512, seed=2)
    step("configs[2] oracle")
    want = oracle.attention(ins.q, ins.k, ins.v, ins.q_pos, ins.k_pos)
    dev = [ctx.upload(x) for x in (ins.q, ins.k, ins.v)]
    out = ctx.empty((1, 8 * 512))
    try:
        results = {}
        for splits in (8, 16, 32, 64, 100, 128, 256, 300, 512, 1000, 0):
            step(f"configs[2] splits={splits}")
            ctx.attention(dev[0].ptr, dev[1].ptr, dev[2].ptr, out.ptr, T=1, S=131072, Hq=8, Hkv=1, Dh=512,
                          Dv=512, q_pos0=131071, k_pos0=0, splits=splits)
            results[splits] = out.to_host()
            assert_parity(results[splits], want, f"configs[2] splits={splits}")
        for s, r in results.items():  # split-K + LSE combine only reassociates the softmax sums (a few ulps)
            np.testing.assert_allclose(r, results[8], atol=5e-6, rtol=0)
    finally:
        for d in dev:
            d.free()
        out.free()


def test_multi_query_decode_and_window_edges(ctx):
    """T > 1 through the decode kernel (one workgroup row per query), with the
    window edge falling inside tiles and a 3-key window."""
    for T, S, Dh, W in [(5, 777, 256, 512), (7, 300, 512, 0), (6, 70, 256, 3), (16, 1000, 256, 100)]:
        step(f"multi-query T={T} S={S} Dh={Dh} window={W}")
        ins = synth.gemma_inputs(T=T, S=S, Dh=Dh, seed=T + S)
        want = oracle.attention(ins.q, ins.k, ins.v, ins.q_pos, ins.k_pos, window=W)
        got = g4a.attention_host(ctx, ins.q, ins.k, ins.v, window=W)
        assert_parity(got, want, f"T={T} S={S} Dh={Dh} window={W}")


def test_ring_layout_matches_linear_bit_exactly(ctx):
    """A sliding-window cache stored as a ring (slot = pos % cap) gives the same bits
    as the linear cache, and matches the oracle on the full history."""
    L, Dh, W = 5000, 256, 512
    ins = synth.gemma_inputs(T=1, S=L, Dh=Dh, seed=21)
    want = oracle.attention(ins.q, ins.k, ins.v, ins.q_pos, ins.k_pos, window=W)
    lin = g4a.attention_host(ctx, ins.q, ins.k, ins.v, window=W)
    assert_parity(lin, want, "linear")
    for cap in (512, 576, 1000):
        step(f"ring cap={cap}")
        ring_k = np.zeros((cap, 1, Dh), np.float32)
        ring_v = np.zeros((cap, 1, Dh), np.float32)
        for p in range(max(0, L - cap), L):
            ring_k[p % cap] = ins.k[p]
            ring_v[p % cap] = ins.v[p]
        dev = [ctx.upload(x) for x in (ins.q, ring_k, ring_v)]
        out = ctx.empty((1, 8 * Dh))
        try:
            ctx.attention(dev[0].ptr, dev[1].ptr, dev[2].ptr, out.ptr, T=1, S=L, Hq=8, Hkv=1, Dh=Dh, Dv=Dh,
                          q_pos0=L - 1, k_pos0=0, window=W, ring_cap=cap)
            got = out.to_host()
        finally:
            for d in dev:
                d.free()
            out.free()
        assert_parity(got, want, f"ring cap={cap}")
        assert np.array_equal(got, lin), f"ring cap={cap} differs from the linear cache"


def test_kv_write_linear_and_ring(ctx):
    rng = np.random.default_rng(0)
    row = 256
    for cap, dst, n in [(0, 0, 5), (0, 37, 3), (512, 510, 5), (512, 1000, 700), (64, 3, 64)]:
        step(f"kv_write ring_cap={cap} dst={dst} n={n}")
        rows = cap if cap else dst + n
        init = rng.standard_normal((rows, row)).astype(np.float32)
        src = rng.standard_normal((n, row)).astype(np.float32)
        cache, s = ctx.upload(init), ctx.upload(src)
        try:
            ctx.kv_write(cache.ptr, cap, row, dst, s.ptr, n)
            got = cache.to_host()
        finally:
            cache.free()
            s.free()
        want = init.copy()
        for r in range(n):
            slot = (dst + r) % cap if cap else dst + r
            want[slot] = src[r]
        assert np.array_equal(got, want)


def test_explicit_non_contiguous_positions(ctx):
    rng = np.random.default_rng(3)
    S, Dh = 2000, 512
    kp = np.sort(rng.choice(50000, size=S, replace=False)).astype(np.uint32)
    ins = synth.gemma_inputs(T=3, S=S, Dh=Dh, seed=33)
    qp = np.array([kp[1500] + 1, kp[-1], kp[10]], np.uint32)
    for W in (0, 4000):
        step(f"explicit positions window={W}")
        want = oracle.attention(ins.q, ins.k, ins.v, qp, kp, window=W)
        got = g4a.attention_host(ctx, ins.q, ins.k, ins.v, q_pos=qp, k_pos=kp, window=W)
        assert_parity(got, want, f"explicit positions window={W}")


def test_softcap_on_fast_and_generic_paths(ctx):
    for Dh, Hq in [(256, 8), (64, 2)]:
        step(f"softcap Dh={Dh} Hq={Hq}")
        ins = synth.gemma_inputs(T=2, S=700, Dh=Dh, Hq=Hq, seed=Dh)
        want = oracle.attention(ins.q, ins.k, ins.v, ins.q_pos, ins.k_pos, softcap=30.0)
        got = g4a.attention_host(ctx, ins.q, ins.k, ins.v, softcap=30.0)
        assert_parity(got, want, f"softcap Dh={Dh}")


def test_rows_without_visible_keys_are_zero(ctx):
    step("all keys in the future")
    ins = synth.gemma_inputs(T=2, S=300, Dh=512, seed=5)
    got = g4a.attention_host(ctx, ins.q, ins.k, ins.v, q_pos=[3, 4], k_pos=np.arange(100, 400))
    assert np.all(got == 0.0)
    step("mixed: first query sees nothing, second sees keys")
    kp = np.arange(100, 400, dtype=np.uint32)
    qp = np.array([50, 250], np.uint32)
    want = oracle.attention(ins.q, ins.k, ins.v, qp, kp)
    got = g4a.attention_host(ctx, ins.q, ins.k, ins.v, q_pos=qp, k_pos=kp)
    assert np.all(got[0] == 0.0)
    assert_parity(got, want, "mixed visibility")


def test_zero_queries_is_a_no_op(ctx):
    step("T=0")
    k = np.zeros((10, 1, 256), np.float32)
    ctx.attention(0, 0, 0, 0, T=0, S=10, Hq=8, Hkv=1, Dh=256, Dv=256)
    ctx.sync()


def test_reference_kernel_bench_cases(ctx):
    """The five attention cases of the reference's `bench --kernels` (rust/src/main.rs:544-560)
    on their own inputs (Xorshift(987654321) after the earlier cases' draws, U(-0.1, 0.1),
    scale 1/16, q at position S-1): the inputs bench.py times them on."""
    for (dh, S, window), q, k, v in synth.reference_bench_inputs():
        label = f"reference bench Dh{dh} S{S} window{window}"
        step(label)
        qp, kp = np.array([S - 1], np.uint32), np.arange(S, dtype=np.uint32)
        want = oracle.attention(q, k, v, qp, kp, scale=1.0 / 16.0, window=window)
        got = g4a.attention_host(ctx, q, k, v, q_pos=qp, k_pos=kp, scale=1.0 / 16.0, window=window)
        assert_parity(got, want, label)
