"""A seeded random sweep of the attention producer (g4a_attn_producer: per-head
q/k RMSNorm + partial RoPE, the unweighted v norm, K/V rows into a linear or
ring cache; rust/src/model.rs:256-285, rust/src/kvcache.rs:49-62) through the
C-ABI against the CPU oracle's composition (rust/src/backend_cpu.rs:149-172,
:248-268). Bar: bit-identical rows (the kernel sums the squares in the
reference's order and takes sin/cos from tables of libm values), and cache rows
outside the append untouched.

The draws put together what the fixed cases take one at a time: token counts
across a ring's end and past its capacity, head counts and groups, head dims
down to 8 and rotary dims that are not multiples of 4, both RoPE bases,
positions far into the context (contiguous or explicit), layers without norm
weights and layers that read a shared cache. The draws come from one seed."""
import numpy as np
import pytest

import oracle
import g4a.synth as synth

pytestmark = pytest.mark.gpu

N_CASES = 40
# positions the host's (sinf, cosf) tables cover: past them the device's sincosf
# (a few ulps from libm) takes over, and the rows are no longer bit-identical
TABLE_ROWS = 1 << 20


def draw_case(rng, i):
    Hkv = int(rng.choice([1, 1, 2]))
    Hq = Hkv * int(rng.choice([1, 2, 4, 8]))
    Dh = int(rng.choice([8, 40, 64, 128, 256, 256, 512, 512]))
    rot = int(rng.choice([Dh, Dh, Dh // 4 * 2, 2 * int(rng.integers(1, Dh // 2 + 1))]))
    T = int(rng.choice([1, 1, 2, 5, 37, 130, 600]))
    ring_cap = int(rng.choice([0, 0, 512, 64, int(rng.integers(T, T + 300))]))
    pos0 = int(rng.choice([0, int(rng.integers(0, 40000)), int(rng.integers(0, TABLE_ROWS - T))]))
    explicit = rng.random() < 0.25
    if explicit:
        positions = np.sort(rng.choice(TABLE_ROWS - 1, size=T, replace=False)).astype(np.uint32)
    else:
        positions = np.arange(pos0, pos0 + T, dtype=np.uint32)
    cache_row = int(rng.integers(0, ring_cap)) if ring_cap else int(rng.integers(0, 300))
    return dict(i=i, Hq=Hq, Hkv=Hkv, Dh=Dh, rot=rot, T=T, ring_cap=ring_cap, theta=float(rng.choice([1e4, 1e6])),
                explicit=explicit, positions=positions, cache_row=cache_row,
                norms=bool(rng.random() < 0.85), shared=bool(rng.random() < 0.15))


CASES = [draw_case(np.random.default_rng(2000 + i), i) for i in range(N_CASES)]


def label(c):
    kind = "explicit" if c["explicit"] else "contiguous"
    return (f"case {c['i']}: T={c['T']} Hq={c['Hq']} Hkv={c['Hkv']} Dh={c['Dh']} rot={c['rot']} "
            f"theta={c['theta']:g} ring_cap={c['ring_cap']} cache_row={c['cache_row']} {kind} positions "
            f"{int(c['positions'][0])}..{int(c['positions'][-1])} norms={c['norms']} shared={c['shared']}")


def _gauss(seed, stream, shape, s=2.0):
    return (synth.normal_f32(seed, stream, int(np.prod(shape))) * np.float32(s)).reshape(shape)


@pytest.mark.parametrize("c", CASES, ids=[f"case{c['i']}" for c in CASES])
def test_random_producer_shape(ctx, c):
    name = label(c)
    print(f"[gpu] {name}", flush=True)
    T, Hq, Hkv, Dh, seed = c["T"], c["Hq"], c["Hkv"], c["Dh"], 7000 + c["i"]
    q_h, k_h, v_h = _gauss(seed, 0, (T, Hq, Dh)), _gauss(seed, 1, (T, Hkv, Dh)), _gauss(seed, 2, (T, Hkv, Dh))
    qn_h = (np.float32(1.0) + np.float32(0.1) * synth.normal_f32(seed, 3, Dh)).astype(np.float32)
    kn_h = (np.float32(1.0) + np.float32(0.1) * synth.normal_f32(seed, 4, Dh)).astype(np.float32)
    shared, norms = c["shared"], c["norms"]
    qo, ko, vo = oracle.producer(q_h, None if shared else k_h, None if shared else v_h, qn_h if norms else None,
                                 kn_h if norms else None, c["positions"], c["theta"], c["rot"], 1e-6)
    cap = c["ring_cap"]
    rows = cap if cap else c["cache_row"] + T
    # sentinels: rows outside the append must keep them
    kc_h = np.full((rows, Hkv, Dh), 7.0, np.float32)
    vc_h = np.full((rows, Hkv, Dh), -7.0, np.float32)
    bufs = dict(q=ctx.upload(q_h), k=ctx.upload(k_h), v=ctx.upload(v_h), qn=ctx.upload(qn_h), kn=ctx.upload(kn_h),
                qo=ctx.empty(q_h.shape), kc=ctx.upload(kc_h), vc=ctx.upload(vc_h))
    try:
        pos_kw = dict(positions=c["positions"]) if c["explicit"] else dict(pos0=int(c["positions"][0]))
        ctx.attn_producer(q=bufs["q"].ptr, k=0 if shared else bufs["k"].ptr, v=0 if shared else bufs["v"].ptr,
                          q_norm=bufs["qn"].ptr if norms else 0, k_norm=bufs["kn"].ptr if norms else 0,
                          q_out=bufs["qo"].ptr, k_cache=bufs["kc"].ptr, v_cache=bufs["vc"].ptr, T=T, Hq=Hq, Hkv=Hkv,
                          Dh=Dh, rotary_dim=c["rot"], cache_row=c["cache_row"], ring_cap=cap, theta=c["theta"],
                          eps=1e-6, **pos_kw)
        got = {n: bufs[n].to_host() for n in ("qo", "kc", "vc")}
    finally:
        for b in bufs.values():
            b.free()
    want_kc, want_vc = kc_h.copy(), vc_h.copy()
    if not shared:
        # a chunk longer than the ring leaves only its last `cap` rows
        for t in range(T - cap if cap and T > cap else 0, T):
            row = (c["cache_row"] + t) % cap if cap else c["cache_row"] + t
            want_kc[row], want_vc[row] = ko[t], vo[t]
    for part, g, w in (("q", got["qo"], qo), ("K cache", got["kc"], want_kc), ("V cache", got["vc"], want_vc)):
        ndiff = int((g != w).sum())
        d = float(np.abs(g.astype(np.float64) - w.astype(np.float64)).max())
        print(f"  {part}: {ndiff} of {g.size} values differ, max-abs {d:.3e}", flush=True)
        assert ndiff == 0, f"{name}: {part}: {ndiff} values differ from the oracle's (max-abs {d:.3e})"
