"""A seeded random sweep of Backend::attention shapes through the C-ABI against
the CPU oracle (rust/src/backend_cpu.rs:270-336 restated in
oracle/attn_oracle.c), at the north star's bar (1e-5 max-abs, 1e-6 mean-abs).

The fixed cases elsewhere pin each kernel on the shapes it was written for; this
sweep draws the arguments the trait allows together (query count, key count,
head groups, head dims, window, soft-cap, scale, contiguous or explicit
positions with holes, queries before or between the keys), so that every
choice the host dispatch makes (range trim, split count, short / streaming /
prefill / generic kernel, the combine form) meets inputs it was not tuned on.
The draws come from one seed: the cases are the same on every run."""
import numpy as np
import pytest

import g4a
import g4a.synth as synth
import oracle

pytestmark = pytest.mark.gpu

MAX_ABS = 1e-5
MEAN_ABS = 1e-6
N_CASES = 60

# (Hq, Hkv): groups of 8 and 4 take the fast kernels at head_dim 256 / 512, the rest the generic one
HEADS = [(8, 1), (8, 1), (8, 1), (16, 2), (8, 2), (4, 1), (4, 2), (2, 2)]
DIMS = [256, 256, 512, 512, 128, 64]


def draw_case(rng, i):
    Hq, Hkv = HEADS[rng.integers(len(HEADS))]
    Dh = int(DIMS[rng.integers(len(DIMS))])
    T = int(rng.choice([1, 1, 1, 2, 3, 7, 15, 16, 17, 33, 48]))
    S = int(rng.integers(1, 6001)) if rng.random() < 0.8 else int(rng.integers(1, 40))
    window = int(rng.choice([0, 0, 3, 64, 512, int(rng.integers(1, 2000))]))
    softcap = float(rng.choice([0.0, 0.0, 0.0, 30.0]))
    scale = float(rng.choice([1.0, 1.0, 0.0625]))
    explicit = rng.random() < 0.3
    if explicit:
        # strictly increasing key positions with holes (evicted or padded slots)
        k_pos = np.cumsum(rng.integers(1, 4, size=S)).astype(np.uint32) + np.uint32(rng.integers(0, 100))
        top = int(k_pos[-1])
        if rng.random() < 0.5:
            q_pos = np.arange(top + 1, top + 1 + T, dtype=np.uint32)  # decode after the cache
        else:
            q_pos = np.sort(rng.integers(0, top + 2, size=T)).astype(np.uint32)  # queries among the keys
    else:
        k0 = int(rng.integers(0, 50))
        k_pos = np.arange(k0, k0 + S, dtype=np.uint32)
        # the model's convention (the last T positions), or a chunk that starts before the cache ends
        q0 = k0 + S - T if (rng.random() < 0.7 and S >= T) else k0 + int(rng.integers(0, S + 1))
        q_pos = np.arange(q0, q0 + T, dtype=np.uint32)
    return dict(i=i, Hq=Hq, Hkv=Hkv, Dh=Dh, T=T, S=S, window=window, softcap=softcap, scale=scale,
                explicit=explicit, q_pos=q_pos, k_pos=k_pos)


CASES = [draw_case(np.random.default_rng(1000 + i), i) for i in range(N_CASES)]


def label(c):
    kind = "explicit" if c["explicit"] else "contiguous"
    return (f"case {c['i']}: T={c['T']} S={c['S']} Hq={c['Hq']} Hkv={c['Hkv']} Dh={c['Dh']} "
            f"window={c['window']} softcap={c['softcap']} scale={c['scale']} {kind} "
            f"q_pos {int(c['q_pos'][0])}..{int(c['q_pos'][-1])} k_pos {int(c['k_pos'][0])}..{int(c['k_pos'][-1])}")


@pytest.mark.parametrize("c", CASES, ids=[f"case{c['i']}" for c in CASES])
def test_random_attention_shape(ctx, c):
    name = label(c)
    print(f"[gpu] {name}", flush=True)
    ins = synth.gemma_inputs(T=c["T"], S=c["S"], Dh=c["Dh"], seed=5000 + c["i"], Hq=c["Hq"], Hkv=c["Hkv"],
                             q_pos=c["q_pos"])
    want = oracle.attention(ins.q, ins.k, ins.v, c["q_pos"], c["k_pos"], scale=c["scale"], window=c["window"],
                            softcap=c["softcap"])
    got = g4a.attention_host(ctx, ins.q, ins.k, ins.v, q_pos=c["q_pos"], k_pos=c["k_pos"], scale=c["scale"],
                             window=c["window"], softcap=c["softcap"], contiguous_positions=not c["explicit"])
    d = np.abs(got.astype(np.float64) - want.astype(np.float64))
    mx, mean = float(d.max()), float(d.mean())
    print(f"  max-abs {mx:.3e} mean-abs {mean:.3e}", flush=True)
    assert mx <= MAX_ABS and mean <= MEAN_ABS, f"{name}: max-abs {mx:.3e} mean-abs {mean:.3e}"
