"""GPU parity of the short-context decode kernel (g4a_decode_short_d256/d512:
32-key splits of two 16-key tiles, every load issued up front, one exact dot
per lane) against the CPU oracle (rust/src/backend_cpu.rs:270-336 restated in
oracle/attn_oracle.c), through the C-ABI. Bar: max-abs <= 1e-5, mean-abs <=
1e-6 (f32). Covers ragged key counts, windows whose edge falls inside a tile,
several queries, a wrapping 512-slot ring, scale and soft-cap, two kv heads,
idle tiles, and calls queued back to back with different split counts."""
import numpy as np
import pytest

import g4a
import g4a.synth as synth
import oracle

pytestmark = pytest.mark.gpu

MAX_ABS = 1e-5
MEAN_ABS = 1e-6


def assert_parity(got, want, label):
    d = np.abs(got.astype(np.float64) - np.asarray(want, np.float64))
    mx, mean = float(d.max()), float(d.mean())
    print(f"  {label}: max-abs {mx:.3e} mean-abs {mean:.3e}", flush=True)
    assert mx <= MAX_ABS and mean <= MEAN_ABS, f"{label}: max-abs {mx:.3e} mean-abs {mean:.3e}"


def step(msg):
    print(f"[gpu] {msg}", flush=True)


def _check_plan(c, **kw):
    p = c.plan(**kw)
    assert g4a.KERNEL_NAMES[p.kernel] == "decode_short", kw
    assert p.keys_per_split == 32
    return p


CASES = [
    # (T, S, Dh, window, seed): the benchmark decode configs, ragged key counts,
    # windows whose edge falls inside a wave tile, several queries
    (1, 512, 256, 512, 0),       # configs[0]
    (1, 8192, 512, 0, 0),        # configs[1]
    (1, 1, 256, 0, 1),
    (1, 7, 512, 0, 2),
    (1, 9, 256, 0, 3),
    (1, 100, 512, 0, 4),
    (1, 513, 256, 512, 5),
    (1, 1000, 256, 512, 6),
    (1, 2047, 512, 0, 7),
    (1, 4099, 512, 0, 8),
    (3, 700, 256, 512, 9),
    (5, 333, 512, 0, 10),
    (4, 90, 256, 3, 11),
]


def test_short_decode_cases(ctx):
    c = ctx
    for T, S, Dh, W, seed in CASES:
        label = f"T={T} S={S} Dh={Dh} window={W}"
        kw = dict(T=T, S=S, Hq=8, Hkv=1, Dh=Dh, Dv=Dh, q_pos0=S - T, k_pos0=0, window=W)
        p = c.plan(**kw)
        if p.splits * T > c.device_info().compute_units:
            continue  # beyond one workgroup per CU: the streaming kernel's range
        _check_plan(c, **kw)
        step(label)
        ins = synth.gemma_inputs(T=T, S=S, Dh=Dh, seed=seed)
        want = oracle.attention(ins.q, ins.k, ins.v, ins.q_pos, ins.k_pos, window=W)
        got = g4a.attention_host(c, ins.q, ins.k, ins.v, window=W)
        assert_parity(got, want, label)


def test_every_split_count_of_the_small_combine(ctx):
    """Split counts 2..16 merge on the one-block-per-head combine (combine_rows),
    in which every wave takes the split weights from lanes 0..ns-1 and loads each
    split's partial at an index clamped into the split range. Every count, both
    head dims, one and two queries (the combine's second grid row), a ragged
    last split; the counts that are multiples of 8 also run the decode kernels
    that place a split's workgroups on one XCD."""
    c = ctx
    for Dh in (256, 512):
        for ns in range(2, 17):
            for T in (1, 2):
                S = 32 * (ns - 1) + 1 + (7 * ns + 3 * T) % 32  # in (32 (ns - 1), 32 ns]: ns splits
                label = f"{ns} splits: T={T} S={S} Dh={Dh}"
                kw = dict(T=T, S=S, Hq=8, Hkv=1, Dh=Dh, Dv=Dh, q_pos0=S - T, k_pos0=0)
                _check_plan(c, **kw)
                assert c.plan(**kw).splits == ns, label
                step(label)
                ins = synth.gemma_inputs(T=T, S=S, Dh=Dh, seed=1000 + 40 * ns + 2 * T + Dh // 256)
                want = oracle.attention(ins.q, ins.k, ins.v, ins.q_pos, ins.k_pos)
                got = g4a.attention_host(c, ins.q, ins.k, ins.v)
                assert_parity(got, want, label)


def test_back_to_back_calls(ctx):
    """Calls with different split counts, query counts and head dims queued in
    one stream without a sync between them (they share the context's partial
    workspace in stream order)."""
    c = ctx
    shapes = [(1, 512, 256, 512), (2, 3000, 512, 0), (1, 64, 256, 0), (1, 512, 256, 512), (3, 1500, 256, 512),
              (1, 5000, 512, 0), (1, 512, 256, 512)]
    pending = []
    for n, (T, S, Dh, W) in enumerate(shapes):
        ins = synth.gemma_inputs(T=T, S=S, Dh=Dh, seed=100 + n)
        dev = [c.upload(x) for x in (ins.q, ins.k, ins.v)]
        out = c.empty((T, 8 * Dh))
        c.attention(dev[0].ptr, dev[1].ptr, dev[2].ptr, out.ptr, T=T, S=S, Hq=8, Hkv=1, Dh=Dh, Dv=Dh,
                    q_pos0=S - T, k_pos0=0, window=W)
        pending.append((ins, W, dev, out, f"call {n}: T={T} S={S} Dh={Dh}"))
    for ins, W, dev, out, label in pending:
        step(label)
        want = oracle.attention(ins.q, ins.k, ins.v, ins.q_pos, ins.k_pos, window=W)
        assert_parity(out.to_host(), want, label)
        for d in dev:
            d.free()
        out.free()


def test_sliding_ring_and_options(ctx):
    """A 512-slot ring whose window wraps the buffer end, scale != 1, a soft-cap
    and two kv heads (groups of 8 query heads each)."""
    c = ctx
    L, Dh, W, cap = 3000, 256, 512, 512
    ins = synth.gemma_inputs(T=1, S=L, Dh=Dh, seed=31)
    want = oracle.attention(ins.q, ins.k, ins.v, ins.q_pos, ins.k_pos, window=W)
    ring_k = np.zeros((cap, 1, Dh), np.float32)
    ring_v = np.zeros((cap, 1, Dh), np.float32)
    for pos in range(L - cap, L):
        ring_k[pos % cap] = ins.k[pos]
        ring_v[pos % cap] = ins.v[pos]
    dev = [c.upload(x) for x in (ins.q, ring_k, ring_v)]
    out = c.empty((1, 8 * Dh))
    try:
        kw = dict(T=1, S=L, Hq=8, Hkv=1, Dh=Dh, Dv=Dh, q_pos0=L - 1, k_pos0=0, window=W, ring_cap=cap)
        _check_plan(c, **kw)
        step("ring 512 wrapping")
        c.attention(dev[0].ptr, dev[1].ptr, dev[2].ptr, out.ptr, **kw)
        assert_parity(out.to_host(), want, "ring 512")
    finally:
        for d in dev:
            d.free()
        out.free()

    ins = synth.gemma_inputs(T=1, S=600, Dh=512, seed=32)
    for scale, cap_ in [(0.0625, 0.0), (1.0, 30.0)]:
        step(f"scale={scale} softcap={cap_}")
        want = oracle.attention(ins.q, ins.k, ins.v, ins.q_pos, ins.k_pos, scale=scale, softcap=cap_)
        got = g4a.attention_host(c, ins.q, ins.k, ins.v, scale=scale, softcap=cap_)
        assert_parity(got, want, f"scale={scale} softcap={cap_}")

    rng = np.random.default_rng(33)
    q = rng.standard_normal((2, 16, 256)).astype(np.float32)
    k = rng.standard_normal((400, 2, 256)).astype(np.float32) * 0.25
    v = rng.standard_normal((400, 2, 256)).astype(np.float32)
    qp = np.array([398, 399], np.uint32)
    kp = np.arange(400, dtype=np.uint32)
    step("two kv heads")
    want = oracle.attention(q, k, v, qp, kp)
    got = g4a.attention_host(c, q, k, v, q_pos=qp)
    assert_parity(got, want, "two kv heads")


def test_future_and_empty_tiles(ctx):
    """Keys past the query (the trim keeps them for the largest query of a
    multi-query call) and a window that leaves whole wave tiles empty."""
    c = ctx
    for T, S, Dh, W in [(6, 200, 256, 0), (9, 257, 512, 5), (2, 1024, 256, 17)]:
        ins = synth.gemma_inputs(T=T, S=S, Dh=Dh, seed=T * S)
        qp = np.arange(S - 5 * T, S - 4 * T, dtype=np.uint32)  # well before the last keys
        step(f"T={T} S={S} Dh={Dh} window={W} queries {qp[0]}..{qp[-1]}")
        want = oracle.attention(ins.q, ins.k, ins.v, qp, ins.k_pos, window=W)
        got = g4a.attention_host(c, ins.q, ins.k, ins.v, q_pos=qp, window=W)
        assert_parity(got, want, f"T={T} S={S} Dh={Dh} window={W}")
