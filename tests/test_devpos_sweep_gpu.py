"""A seeded random sweep of decode steps whose query position lives in device
memory (g4a_attention_devpos: the plan is made once for the largest key range
S, the kernel reads the position and trims the range) through the C-ABI
against the CPU oracle (rust/src/backend_cpu.rs:270-336 restated in
oracle/attn_oracle.c) on the keys that position sees, at the north star's bar
(1e-5 max-abs, 1e-6 mean-abs).

The fixed cases take Gemma's two layer shapes; the draws here take rings of any
size at least the window, windows over linear caches, full attention, groups
of 8 and of 4 query heads, one or two kv heads, both head dims, caches that
start at a non-zero position, and positions anywhere from the first key to
the last one the plan covers. The draws come from one seed."""
import numpy as np
import pytest

import g4a.synth as synth
import oracle

pytestmark = pytest.mark.gpu

MAX_ABS = 1e-5
MEAN_ABS = 1e-6
N_LAYERS = 12
N_POS = 4


def draw_layer(rng, i):
    Dh = int(rng.choice([256, 512]))
    Hkv = int(rng.choice([1, 1, 2]))
    group = int(rng.choice([8, 8, 4]))
    kind = str(rng.choice(["ring", "linear_window", "global"]))
    S = int(rng.choice([int(rng.integers(1, 200)), int(rng.integers(200, 20000))]))
    window = int(rng.choice([512, int(rng.integers(1, 1500))])) if kind != "global" else 0
    cap = int(rng.choice([window, window + int(rng.integers(0, 300))])) if kind == "ring" else 0
    k0 = 0 if kind == "ring" else int(rng.choice([0, int(rng.integers(1, 100000))]))
    positions = sorted({k0, k0 + S - 1} | {k0 + int(x) for x in rng.integers(0, S, N_POS - 2)})
    return dict(i=i, Dh=Dh, Hkv=Hkv, Hq=group * Hkv, kind=kind, S=S, window=window, cap=cap, k0=k0,
                positions=positions)


LAYERS = [draw_layer(np.random.default_rng(7000 + i), i) for i in range(N_LAYERS)]


def label(c):
    return (f"layer {c['i']}: {c['kind']} Dh={c['Dh']} Hq={c['Hq']} Hkv={c['Hkv']} S={c['S']} "
            f"window={c['window']} ring_cap={c['cap']} k_pos0={c['k0']}")


@pytest.mark.parametrize("c", LAYERS, ids=[f"layer{c['i']}" for c in LAYERS])
def test_random_devpos_layer(ctx, c):
    name = label(c)
    print(f"[gpu] {name}", flush=True)
    Dh, Hkv, Hq, S, W, cap, k0 = c["Dh"], c["Hkv"], c["Hq"], c["S"], c["window"], c["cap"], c["k0"]
    ins = synth.gemma_inputs(T=1, S=S, Dh=Dh, seed=8000 + c["i"], Hq=Hq, Hkv=Hkv)
    q = ctx.upload(ins.q)
    pos = ctx.empty((1,), np.uint32)
    out = ctx.empty((1, Hq * Dh))
    bufs = [q, pos, out]
    try:
        if not cap:
            k, v = ctx.upload(ins.k), ctx.upload(ins.v)
            bufs += [k, v]
        for p in c["positions"]:
            n = p - k0 + 1  # keys the query at p can see before the window cuts them
            lo = max(0, n - W) if W else 0
            if cap:
                # the ring holds the window ending at the query (key j in slot j % cap)
                ring_k = np.zeros((cap, Hkv, Dh), np.float32)
                ring_v = np.zeros((cap, Hkv, Dh), np.float32)
                for j in range(lo, n):
                    ring_k[j % cap], ring_v[j % cap] = ins.k[j], ins.v[j]
                k, v = ctx.upload(ring_k), ctx.upload(ring_v)
            try:
                print(f"  position {p} (keys {lo}..{n - 1})", flush=True)
                ctx.h2d(pos.ptr, np.array([p], np.uint32))
                ctx.attention_devpos(q.ptr, k.ptr, v.ptr, out.ptr, pos.ptr, T=1, S=S, Hq=Hq, Hkv=Hkv, Dh=Dh, Dv=Dh,
                                     k_pos0=k0, window=W, ring_cap=cap)
                got = out.to_host()
            finally:
                if cap:
                    k.free()
                    v.free()
            want = oracle.attention(ins.q, ins.k[lo:n], ins.v[lo:n], np.array([p], np.uint32),
                                    np.arange(k0 + lo, k0 + n, dtype=np.uint32), window=W)
            d = np.abs(got.astype(np.float64) - want.astype(np.float64))
            mx, mean = float(d.max()), float(d.mean())
            print(f"    max-abs {mx:.3e} mean-abs {mean:.3e}", flush=True)
            assert mx <= MAX_ABS and mean <= MEAN_ABS, f"{name} at position {p}: max-abs {mx:.3e} mean-abs {mean:.3e}"
    finally:
        for b in bufs:
            b.free()
