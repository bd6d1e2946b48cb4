"""g4a_attention_noalloc (the entry point that allocates nothing: its split
partials and pre-split K/V live in the library's static scratch array) gives
bit-identical results to g4a_attention on the same inputs, through the C-ABI:
two calls in a row per kernel family, the second smaller than the first (so it
runs over what the first left in the shared array), and it refuses, enqueueing
nothing, what would need an allocation."""
import numpy as np
import pytest

import g4a
import g4a.synth as synth
import oracle

pytestmark = pytest.mark.gpu


def step(msg):
    print(f"[gpu] {msg}", flush=True)


def _run_both(ctx, ins, label, **kw):
    """Run one call through g4a_attention and g4a_attention_noalloc into separate outputs."""
    T, Hq, Dh = ins.q.shape
    S, Hkv, _ = ins.k.shape
    Dv = ins.v.shape[2]
    dev = [ctx.upload(x) for x in (ins.q, ins.k, ins.v)]
    o1, o2 = ctx.empty((T, Hq * Dv)), ctx.empty((T, Hq * Dv))
    args = dict(T=T, S=kw.pop("S", S), Hq=Hq, Hkv=Hkv, Dh=Dh, Dv=Dv, q_pos0=int(ins.q_pos[0]),
                k_pos0=int(ins.k_pos[0]), **kw)
    try:
        plan = ctx.plan(**args)
        step(f"{label}: kernel {g4a.KERNEL_NAMES[plan.kernel]}, {plan.splits} splits")
        ctx.h2d(o2.ptr, np.full((T, Hq * Dv), np.nan, np.float32))
        ctx.attention_noalloc(dev[0].ptr, dev[1].ptr, dev[2].ptr, o2.ptr, **args)
        ctx.attention(dev[0].ptr, dev[1].ptr, dev[2].ptr, o1.ptr, **args)
        return o1.to_host(), o2.to_host(), plan
    finally:
        for d in dev + [o1, o2]:
            d.free()


CASES = [
    # label, (T, S, Dh, seed), extra kwargs; each pair: a larger call, then a smaller one
    ("decode hd512 @32768 (256 splits)", (1, 32768, 512, 1), {}),
    ("decode hd512 @9000 (streaming, fewer splits)", (1, 9000, 512, 2), {}),
    ("sliding decode hd256 on a ring (short kernel)", (1, 5000, 256, 3), dict(window=512, ring=512)),
    ("sliding decode hd256 @700 (short kernel)", (1, 700, 256, 4), dict(window=512)),
    ("prefill hd512 T2048 causal (split blocks)", (2048, 2048, 512, 5), {}),
    ("prefill hd256 T300 window 512", (300, 300, 256, 6), dict(window=512)),
    ("generic head_dim 64, 3 queries", (3, 400, 64, 7), {}),
    ("generic head_dim 64, 1 query", (1, 90, 64, 8), {}),
]


@pytest.mark.parametrize("first,second", [(0, 1), (2, 3), (4, 5), (6, 7)])
def test_noalloc_matches_attention_twice(ctx, first, second):
    for idx in (first, second):
        label, (T, S, Dh, seed), kw = CASES[idx]
        kw = dict(kw)
        ring = kw.pop("ring", 0)
        ins = synth.gemma_inputs(T=T, S=S, Dh=Dh, seed=seed, q_pos=np.arange(S - T, S) if T > 1 else None)
        if ring:
            # keep only a ring of the last `ring` positions (slot p % ring)
            rk = np.zeros((ring, 1, Dh), np.float32)
            rv = np.zeros((ring, 1, Dh), np.float32)
            for p_ in range(S - ring, S):
                rk[p_ % ring], rv[p_ % ring] = ins.k[p_], ins.v[p_]
            full = ins
            ins = synth.AttnInputs(full.q, rk, rv, full.q_pos, full.k_pos)
            got, got_na, _ = _run_both(ctx, ins, label, S=S, ring_cap=ring, **kw)
            want = oracle.attention(full.q, full.k, full.v, full.q_pos, full.k_pos, **kw)
        else:
            got, got_na, _ = _run_both(ctx, ins, label, **kw)
            want = None if T * S * Dh > 2e8 else oracle.attention(ins.q, ins.k, ins.v, ins.q_pos, ins.k_pos, **kw)
        assert np.array_equal(got_na, got), f"{label}: noalloc differs from g4a_attention"
        if want is not None:
            d = np.abs(got_na.astype(np.float64) - want)
            print(f"  {label}: bit-identical; vs oracle max-abs {d.max():.3e} mean-abs {d.mean():.3e}", flush=True)
            assert d.max() <= 1e-5 and d.mean() <= 1e-6, label
        else:
            print(f"  {label}: bit-identical", flush=True)


def _draw_noalloc_case(rng, i):
    Hkv = int(rng.choice([1, 1, 2]))
    Hq = Hkv * int(rng.choice([8, 8, 8, 4, 2]))
    Dh = int(rng.choice([256, 256, 512, 512, 64]))
    T = int(rng.choice([1, 1, 2, 5, 16, 40, 300]))
    S = int(rng.integers(T, 8000))
    window = int(rng.choice([0, 0, 512, int(rng.integers(1, 2000))]))
    softcap = float(rng.choice([0.0, 0.0, 30.0]))
    scale = float(rng.choice([1.0, 0.0625]))
    k0 = int(rng.choice([0, int(rng.integers(1, 1000))]))
    return dict(i=i, T=T, S=S, Hq=Hq, Hkv=Hkv, Dh=Dh, window=window, softcap=softcap, scale=scale, k0=k0)


RANDOM_CASES = [_draw_noalloc_case(np.random.default_rng(9100 + i), i) for i in range(16)]


@pytest.mark.parametrize("c", RANDOM_CASES, ids=[f"case{c['i']}" for c in RANDOM_CASES])
def test_noalloc_random_shapes_match_attention(ctx, c):
    """Seeded random shapes (head groups, head dims, windows, soft-cap, scale, query
    counts, caches from a non-zero position), one after another on the shared
    array: g4a_attention_noalloc gives g4a_attention's bits, or, where the call's
    scratch would pass the array, refuses it and writes nothing."""
    T, S, k0 = c["T"], c["S"], c["k0"]
    ins = synth.gemma_inputs(T=T, S=S, Dh=c["Dh"], seed=9200 + c["i"], Hq=c["Hq"], Hkv=c["Hkv"],
                             q_pos=np.arange(k0 + S - T, k0 + S))
    ins = synth.AttnInputs(ins.q, ins.k, ins.v, np.arange(k0 + S - T, k0 + S, dtype=np.uint32),
                           np.arange(k0, k0 + S, dtype=np.uint32))
    kw = dict(window=c["window"], softcap=c["softcap"], scale=c["scale"])
    label = (f"random case {c['i']}: T={T} S={S} Hq={c['Hq']} Hkv={c['Hkv']} Dh={c['Dh']} window={c['window']} "
             f"softcap={c['softcap']} scale={c['scale']} k_pos0={k0}")
    plan = ctx.plan(T=T, S=S, Hq=c["Hq"], Hkv=c["Hkv"], Dh=c["Dh"], Dv=c["Dh"], q_pos0=k0 + S - T, k_pos0=k0, **kw)
    if plan.workspace_bytes > g4a.NOALLOC_SCRATCH_BYTES:
        step(f"{label}: {plan.workspace_bytes} bytes of scratch, past the array: refused")
        with pytest.raises(g4a.G4aError, match="bytes of scratch"):
            _run_both(ctx, ins, label, **kw)
        return
    got, got_na, _ = _run_both(ctx, ins, label, **kw)
    assert np.array_equal(got_na, got), f"{label}: noalloc differs from g4a_attention"
    print(f"  {label}: bit-identical", flush=True)


def test_noalloc_refuses_what_needs_an_allocation(ctx):
    ins = synth.gemma_inputs(T=1, S=300, Dh=256, seed=9)
    k_pos = np.arange(300, dtype=np.uint32)
    k_pos[150:] += 7  # a gap: explicit positions would have to be staged through allocated buffers
    dev = [ctx.upload(x) for x in (ins.q, ins.k, ins.v)]
    out = ctx.empty((1, 8 * 256))
    try:
        ctx.h2d(out.ptr, np.full((1, 8 * 256), 7.0, np.float32))
        with pytest.raises(g4a.G4aError, match="contiguous positions only"):
            ctx.attention_noalloc(dev[0].ptr, dev[1].ptr, dev[2].ptr, out.ptr, T=1, S=300, Hq=8, Hkv=1, Dh=256,
                                  Dv=256, q_pos=np.array([310], np.uint32), k_pos=k_pos)
        # 15 queries (decode path) over 65536 keys with 1024 forced splits: 15*8*1024*514*4 bytes
        # of partials, beyond the array; refused before anything is enqueued
        args = dict(T=15, S=65536, Hq=8, Hkv=1, Dh=512, Dv=512, q_pos0=65521, splits=1024)
        plan = ctx.plan(**args)
        assert plan.workspace_bytes > g4a.NOALLOC_SCRATCH_BYTES
        big = ctx.malloc(65536 * 512 * 4)
        qb, ob = ctx.malloc(15 * 8 * 512 * 4), ctx.malloc(15 * 8 * 512 * 4)
        try:
            with pytest.raises(g4a.G4aError, match="bytes of scratch"):
                ctx.attention_noalloc(qb, big, big, ob, **args)
        finally:
            for x in (big, qb, ob):
                ctx.free(x)
        ctx.sync()
        assert np.all(out.to_host() == 7.0), "a refused call wrote its output"
    finally:
        for d in dev + [out]:
            d.free()


def test_noalloc_records_into_a_graph_on_a_fresh_context():
    """The no-allocation property itself: on a fresh context (no workspace yet), a HIP graph
    capture refuses any workspace growth, so g4a_attention cannot record a 256-split decode
    or a head_dim 512 prefill there, while g4a_attention_noalloc records both. The graph's
    replays (outputs overwritten in between, other eager work between them) match eager
    g4a_attention runs of the same calls bit for bit."""
    fresh = g4a.Context(0)
    decode = synth.gemma_inputs(T=1, S=32768, Dh=512, seed=11)
    prefill = synth.gemma_inputs(T=1024, S=1024, Dh=512, seed=12, q_pos=np.arange(1024))
    bufs, graph = [], None
    try:
        calls = []
        for ins, label in ((decode, "decode hd512 @32768"), (prefill, "prefill hd512 T1024")):
            T, Hq, Dh = ins.q.shape
            dq, dk, dv = (fresh.upload(x) for x in (ins.q, ins.k, ins.v))
            out = fresh.empty((T, Hq * Dh))
            bufs += [dq, dk, dv, out]
            kw = dict(T=T, S=ins.k.shape[0], Hq=Hq, Hkv=1, Dh=Dh, Dv=Dh, q_pos0=int(ins.q_pos[0]), k_pos0=0)
            calls.append((label, dq, dk, dv, out, kw))
        for label, dq, dk, dv, out, kw in calls:
            step(f"g4a_attention under a capture on a fresh context, {label}: refused (its workspace would grow)")
            fresh.capture_begin()
            try:
                with pytest.raises(g4a.G4aError, match="workspace must grow"):
                    fresh.attention(dq.ptr, dk.ptr, dv.ptr, out.ptr, **kw)
            finally:
                with pytest.raises(g4a.G4aError):
                    fresh.capture_end()
        step("g4a_attention_noalloc under a capture on the same fresh context: recorded")
        fresh.capture_begin()
        try:
            for label, dq, dk, dv, out, kw in calls:
                fresh.attention_noalloc(dq.ptr, dk.ptr, dv.ptr, out.ptr, **kw)
        except Exception:
            try:
                fresh.capture_end().free()
            except g4a.G4aError:
                pass
            raise
        graph = fresh.capture_end()
        # eager reference results through g4a_attention (which may now grow its workspace)
        want = []
        for label, dq, dk, dv, out, kw in calls:
            fresh.attention(dq.ptr, dk.ptr, dv.ptr, out.ptr, **kw)
            want.append(out.to_host())
        rng = np.random.default_rng(5)
        for rep in range(3):
            step(f"graph replay {rep}")
            for label, dq, dk, dv, out, kw in calls:
                fresh.h2d(out.ptr, rng.standard_normal(out.shape).astype(np.float32))
            graph.launch()
            fresh.sync()
            for (label, *_rest), w in zip(calls, want):
                got = _rest[3].to_host()
                assert np.array_equal(got, w), f"replay {rep}, {label}: differs from eager g4a_attention"
            # eager work between replays
            label, dq, dk, dv, out, kw = calls[0]
            fresh.attention(dq.ptr, dk.ptr, dv.ptr, out.ptr, **kw)
            fresh.sync()
        print("  both calls recorded without an allocation; replays bit-identical to eager runs", flush=True)
    finally:
        if graph is not None:
            graph.free()
        for d in bufs:
            d.free()
        fresh.close()


_LAZY_SCRIPT = r"""
import ctypes, sys
sys.path.insert(0, sys.argv[1])
import numpy as np
import g4a
hip = ctypes.CDLL("libamdhip64.so")
def free_bytes():
    f, t = ctypes.c_size_t(), ctypes.c_size_t()
    assert hip.hipMemGetInfo(ctypes.byref(f), ctypes.byref(t)) == 0
    return f.value
ctx = g4a.Context(0)
q, k, v, out = ctx.empty((1, 8, 256)), ctx.empty((512, 1, 256)), ctx.empty((512, 1, 256)), ctx.empty((1, 2048))
for b in (q, k, v):
    ctx.zero(b.ptr, b.nbytes)
ctx.sync()
before = free_bytes()
ctx.attention_noalloc(q.ptr, k.ptr, v.ptr, out.ptr, T=1, S=512, Hq=8, Hkv=1, Dh=256, Dv=256, q_pos0=511, k_pos0=0,
                      window=512)
ctx.sync()
after = free_bytes()
print(f"FREE_BEFORE {before} FREE_AFTER {after}", flush=True)
ctx.close()
"""


def test_noalloc_scratch_is_taken_at_first_use():
    """A process that creates a context holds no scratch array until its first no-alloc call
    (the array is looked up, and so loaded onto the GPU, there): the device's free memory
    drops by the array's size at that call, not at g4a_create."""
    import subprocess
    import sys
    from pathlib import Path
    pkg = str(Path(g4a.__file__).resolve().parents[1])
    r = subprocess.run([sys.executable, "-c", _LAZY_SCRIPT, pkg], capture_output=True, text=True, timeout=100)
    print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0
    line = [x for x in r.stdout.splitlines() if x.startswith("FREE_BEFORE")][-1].split()
    before, after = int(line[1]), int(line[3])
    taken = before - after
    print(f"  free device memory dropped by {taken / 2**20:.1f} MiB at the first no-alloc call "
          f"(array {g4a.NOALLOC_SCRATCH_BYTES / 2**20:.0f} MiB)", flush=True)
    assert taken >= g4a.NOALLOC_SCRATCH_BYTES, "the scratch array was not taken at the first no-alloc call"
