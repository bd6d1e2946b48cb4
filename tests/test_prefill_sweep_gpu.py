"""A seeded random sweep of prefill-shaped attention calls (16 or more queries,
groups of 8 query heads per kv head, contiguous positions: the query-tiled
prefill kernels with their fp16-split score estimate and exact rescoring band)
through the C-ABI against the CPU oracle (rust/src/backend_cpu.rs:270-336
restated in oracle/attn_oracle.c), at the north star's bar (1e-5 max-abs,
1e-6 mean-abs).

The draws mix prompt lengths that are not multiples of the 8-query blocks or
16-key tiles, chunks that start after a cached prefix, one or two kv heads,
both head dims, full causal attention and windows shorter or longer than the
chunk, scale 1 and 1/16, and queries whose window reaches before the cache's
first key. The draws come from one seed."""
import numpy as np
import pytest

import g4a
import g4a.synth as synth
import oracle

pytestmark = pytest.mark.gpu

MAX_ABS = 1e-5
MEAN_ABS = 1e-6
N_CASES = 30


def draw_case(rng, i):
    Dh = int(rng.choice([256, 512]))
    Hkv = int(rng.choice([1, 1, 1, 2]))
    T = int(rng.choice([16, 17, 24, 63, 100, 257, int(rng.integers(16, 700))]))
    prefix = int(rng.choice([0, 0, int(rng.integers(1, 40)), int(rng.integers(1, 3000))]))
    S = T + prefix
    window = int(rng.choice([0, 0, 512, 3, 64, int(rng.integers(1, 1500))]))
    scale = float(rng.choice([1.0, 1.0, 0.0625]))
    k0 = int(rng.choice([0, 0, int(rng.integers(1, 5000))]))
    # keep the 8-thread oracle to a few seconds
    while T * S * 8 * Hkv * Dh > 2.5e9 and S > T:
        S = T + (S - T) // 2
    return dict(i=i, Dh=Dh, Hkv=Hkv, T=T, S=S, window=window, scale=scale, k0=k0)


CASES = [draw_case(np.random.default_rng(4000 + i), i) for i in range(N_CASES)]


def label(c):
    return (f"case {c['i']}: T={c['T']} S={c['S']} Hq={8 * c['Hkv']} Hkv={c['Hkv']} Dh={c['Dh']} "
            f"window={c['window']} scale={c['scale']} k_pos0={c['k0']}")


@pytest.mark.parametrize("c", CASES, ids=[f"case{c['i']}" for c in CASES])
def test_random_prefill_shape(ctx, c):
    name = label(c)
    print(f"[gpu] {name}", flush=True)
    T, S, Hkv, Dh, k0 = c["T"], c["S"], c["Hkv"], c["Dh"], c["k0"]
    q_pos = np.arange(k0 + S - T, k0 + S, dtype=np.uint32)  # the chunk's queries are the last T positions
    k_pos = np.arange(k0, k0 + S, dtype=np.uint32)
    ins = synth.gemma_inputs(T=T, S=S, Dh=Dh, seed=6000 + c["i"], Hq=8 * Hkv, Hkv=Hkv, q_pos=q_pos)
    plan = ctx.plan(T=T, S=S, Hq=8 * Hkv, Hkv=Hkv, Dh=Dh, Dv=Dh, q_pos0=int(q_pos[0]), k_pos0=k0,
                    window=c["window"], scale=c["scale"])
    assert g4a.KERNEL_NAMES[plan.kernel] == "prefill", f"{name}: planned {g4a.KERNEL_NAMES[plan.kernel]}"
    want = oracle.attention(ins.q, ins.k, ins.v, q_pos, k_pos, scale=c["scale"], window=c["window"])
    got = g4a.attention_host(ctx, ins.q, ins.k, ins.v, q_pos=q_pos, k_pos=k_pos, scale=c["scale"],
                             window=c["window"])
    d = np.abs(got.astype(np.float64) - want.astype(np.float64))
    mx, mean = float(d.max()), float(d.mean())
    print(f"  max-abs {mx:.3e} mean-abs {mean:.3e}", flush=True)
    assert mx <= MAX_ABS and mean <= MEAN_ABS, f"{name}: max-abs {mx:.3e} mean-abs {mean:.3e}"
