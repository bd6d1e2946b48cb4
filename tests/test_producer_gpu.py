"""GPU parity of the attention producer (g4a_norm_rope kernel) through the
C-ABI against the CPU oracle: Backend::rms_norm / rope / head_norm_rope
(rust/src/backend_cpu.rs:149-172, :248-268; rust/src/backend.rs:146-154) and
the fused per-layer producer g4a_attn_producer (rust/src/model.rs:256-281 with
the KV append of rust/src/kvcache.rs:49-62) writing into linear and ring
caches. Bar: bit-identical to the oracle (and so within max-abs 1e-5,
mean-abs 1e-6): the kernel sums the squares in the reference's order and takes
sin/cos from libm tables built on the host."""
import numpy as np
import pytest

import g4a
import g4a.synth as synth
import oracle
from golden_io import load_norm_rope_golden

pytestmark = pytest.mark.gpu

MAX_ABS = 1e-5
MEAN_ABS = 1e-6


def assert_parity(got, want, label, exact=True):
    """max-abs / mean-abs bar, and with `exact` (every producer output) bit-identity."""
    got, want = np.asarray(got, np.float32), np.asarray(want, np.float32)
    d = np.abs(got.astype(np.float64) - want.astype(np.float64))
    mx, mean = float(d.max()), float(d.mean())
    ndiff = int((got != want).sum())
    print(f"  {label}: max-abs {mx:.3e} mean-abs {mean:.3e}, {ndiff} of {got.size} values not bit-identical",
          flush=True)
    assert mx <= MAX_ABS and mean <= MEAN_ABS, f"{label}: max-abs {mx:.3e} mean-abs {mean:.3e}"
    # the producer does every op in the reference's order (sequential sum of squares, libm sin/cos
    # tables), so its rows are the CPU backend's bit for bit
    if exact:
        assert ndiff == 0, f"{label}: {ndiff} values differ from the oracle's"


def step(msg):
    print(f"[gpu] {msg}", flush=True)


def _gauss(seed, *shape, s=2.0):
    return (synth.normal_f32(seed, 0, int(np.prod(shape))) * np.float32(s)).reshape(shape)


def _weight(seed, d):
    return (np.float32(1.0) + np.float32(0.1) * synth.normal_f32(seed, 1, d)).astype(np.float32)


def test_golden_fixtures(ctx):
    """The reference's rmsNorm / rope(partial) / head_norm_rope parity inputs and Gemma shapes."""
    for name, c in load_norm_rope_golden().items():
        step(f"golden {name}")
        T, heads, dh = c.x.shape
        x = ctx.upload(c.x)
        w = ctx.upload(c.w) if c.w is not None else None
        y = ctx.empty(c.x.shape)
        try:
            if c.op == "rms_norm":
                ctx.rms_norm(x.ptr, w.ptr if w else 0, y.ptr, rows=T * heads, dim=dh, eps=c.eps)
            elif c.op == "rope":
                ctx.rope(x.ptr, y.ptr, T=T, heads=heads, head_dim=dh, rotary_dim=c.rotary_dim, positions=c.positions,
                         theta=c.theta)
            else:
                ctx.head_norm_rope(x.ptr, w.ptr, y.ptr, T=T, heads=heads, head_dim=dh, rotary_dim=c.rotary_dim,
                                   positions=c.positions, theta=c.theta, eps=c.eps)
            assert_parity(y.to_host(), c.out, name)
        finally:
            for a in (x, w, y):
                if a is not None:
                    a.free()


@pytest.mark.parametrize("T,heads,dh,theta,rot,pos0", [
    (1, 8, 256, 1e4, 256, 32767),      # sliding-layer q at the configs[4] context
    (1, 8, 512, 1e6, 128, 32767),      # global-layer q (partial_rotary_factor 0.25)
    (7, 1, 512, 1e6, 128, 131065),     # global k at the configs[2] context
    (64, 8, 256, 1e4, 256, 0),         # a prefill chunk from position 0
    (3, 4, 16, 1e4, 8, 3),             # the reference's tiny head
    (2, 2, 40, 1e4, 10, 12),           # rotary_dim not a multiple of 4
])
def test_head_norm_rope_shapes(ctx, T, heads, dh, theta, rot, pos0):
    x_h = _gauss(T * heads + dh, T, heads, dh)
    w_h = _weight(dh, dh)
    pos = np.arange(pos0, pos0 + T, dtype=np.uint32)
    want = oracle.head_norm_rope(x_h, w_h, 1e-6, pos, theta, rot)
    x, w, y = ctx.upload(x_h), ctx.upload(w_h), ctx.empty(x_h.shape)
    try:
        label = f"head_norm_rope T={T} heads={heads} Dh={dh} rot={rot} pos0={pos0}"
        step(label)
        ctx.head_norm_rope(x.ptr, w.ptr, y.ptr, T=T, heads=heads, head_dim=dh, rotary_dim=rot, pos0=pos0,
                           theta=theta, eps=1e-6)
        assert_parity(y.to_host(), want, label)
        # explicit, non-contiguous positions (uploaded), written in place
        rng = np.random.default_rng(T + dh)
        pos2 = rng.integers(0, 200000, size=T).astype(np.uint32)
        want2 = oracle.head_norm_rope(x_h, w_h, 1e-6, pos2, theta, rot)
        ctx.head_norm_rope(x.ptr, w.ptr, x.ptr, T=T, heads=heads, head_dim=dh, rotary_dim=rot, positions=pos2,
                           theta=theta, eps=1e-6)
        assert_parity(x.to_host(), want2, label + " (explicit positions, in place)")
    finally:
        for a in (x, w, y):
            a.free()


def test_rope_only_and_unweighted_norm(ctx):
    x_h = _gauss(5, 4, 8, 512)
    pos = np.array([9, 90, 900, 9000], np.uint32)
    x, y = ctx.upload(x_h), ctx.empty(x_h.shape)
    try:
        step("rope only")
        ctx.rope(x.ptr, y.ptr, T=4, heads=8, head_dim=512, rotary_dim=128, positions=pos, theta=1e6)
        assert_parity(y.to_host(), oracle.rope(x_h, pos, 1e6, 128), "rope hd512 rot128")
        step("unweighted rms_norm")
        ctx.rms_norm(x.ptr, 0, y.ptr, rows=32, dim=512, eps=1e-6)
        assert_parity(y.to_host(), oracle.rms_norm(x_h.reshape(32, 512), None, 1e-6).reshape(4, 8, 512),
                      "rms_norm unweighted")
    finally:
        x.free()
        y.free()


def _producer_case(ctx, *, T, Dh, theta, rot, pos0, cache_row, ring_cap, cache_rows, shared=False, norms=True,
                   seed=0):
    Hq, Hkv = 8, 1
    q_h, k_h, v_h = _gauss(seed, T, Hq, Dh), _gauss(seed + 1, T, Hkv, Dh), _gauss(seed + 2, T, Hkv, Dh)
    qn_h, kn_h = _weight(seed + 3, Dh), _weight(seed + 4, Dh)
    pos = np.arange(pos0, pos0 + T, dtype=np.uint32)
    qo, ko, vo = oracle.producer(q_h, None if shared else k_h, None if shared else v_h,
                                 qn_h if norms else None, kn_h if norms else None, pos, theta, rot, 1e-6)
    # caches start with a sentinel so untouched rows can be checked
    kc_h = np.full((cache_rows, Hkv, Dh), 7.0, np.float32)
    vc_h = np.full((cache_rows, Hkv, Dh), -7.0, np.float32)
    bufs = dict(q=ctx.upload(q_h), k=ctx.upload(k_h), v=ctx.upload(v_h), qn=ctx.upload(qn_h), kn=ctx.upload(kn_h),
                qo=ctx.empty(q_h.shape), kc=ctx.upload(kc_h), vc=ctx.upload(vc_h))
    try:
        ctx.attn_producer(q=bufs["q"].ptr, k=0 if shared else bufs["k"].ptr, v=0 if shared else bufs["v"].ptr,
                          q_norm=bufs["qn"].ptr if norms else 0, k_norm=bufs["kn"].ptr if norms else 0,
                          q_out=bufs["qo"].ptr, k_cache=bufs["kc"].ptr, v_cache=bufs["vc"].ptr, T=T, Hq=Hq, Hkv=Hkv,
                          Dh=Dh, rotary_dim=rot, pos0=pos0, cache_row=cache_row, ring_cap=ring_cap, theta=theta,
                          eps=1e-6)
        got = {n: bufs[n].to_host() for n in ("qo", "kc", "vc")}
    finally:
        for b in bufs.values():
            b.free()
    want_kc, want_vc = kc_h.copy(), vc_h.copy()
    if not shared:
        first = T - ring_cap if ring_cap and T > ring_cap else 0
        for t in range(first, T):
            row = (cache_row + t) % ring_cap if ring_cap else cache_row + t
            want_kc[row], want_vc[row] = ko[t], vo[t]
    return got, qo, want_kc, want_vc


@pytest.mark.parametrize("name,kw", [
    ("sliding decode into a ring (wraps)", dict(T=1, Dh=256, theta=1e4, rot=256, pos0=33279, cache_row=33279,
                                                 ring_cap=512, cache_rows=512)),
    ("global decode into a linear cache", dict(T=1, Dh=512, theta=1e6, rot=128, pos0=32767, cache_row=32767,
                                                ring_cap=0, cache_rows=32768)),
    ("sliding prefill chunk across the ring end", dict(T=37, Dh=256, theta=1e4, rot=256, pos0=490, cache_row=490,
                                                        ring_cap=512, cache_rows=512)),
    ("sliding prefill longer than the ring", dict(T=600, Dh=256, theta=1e4, rot=256, pos0=0, cache_row=0,
                                                   ring_cap=512, cache_rows=512)),
    ("global prefill chunk into a linear cache", dict(T=40, Dh=512, theta=1e6, rot=128, pos0=100, cache_row=100,
                                                       ring_cap=0, cache_rows=200)),
    ("layer without q/k norm weights", dict(T=3, Dh=512, theta=1e6, rot=128, pos0=5, cache_row=5, ring_cap=0,
                                            cache_rows=16, norms=False)),
    ("layer reading a shared cache", dict(T=2, Dh=256, theta=1e4, rot=256, pos0=70, cache_row=70, ring_cap=512,
                                          cache_rows=512, shared=True)),
])
def test_attn_producer(ctx, name, kw):
    step(name)
    got, qo, want_kc, want_vc = _producer_case(ctx, seed=len(name), **kw)
    assert_parity(got["qo"], qo, name + ": q")
    assert_parity(got["kc"], want_kc, name + ": K cache")
    assert_parity(got["vc"], want_vc, name + ": V cache")
    assert np.array_equal(got["kc"] == 7.0, want_kc == 7.0), "rows outside the append must stay untouched"


def test_producer_feeds_the_decode_kernel(ctx):
    """One sliding-layer decode step end to end on the GPU: the producer writes the
    new K/V row into a 512-slot ring holding the previous 511 positions, then the
    attention call reads the ring. The producer's outputs are checked against the
    oracle's producer, and the attention output against the oracle's attention on
    exactly the q and ring the GPU produced (so the check does not compound the
    two ops' tolerances through scores of ~90)."""
    Dh, cap, P = 256, 512, 40000
    hist = synth.gemma_inputs(T=1, S=P, Dh=Dh, seed=50)
    ring_k = np.zeros((cap, 1, Dh), np.float32)
    ring_v = np.zeros((cap, 1, Dh), np.float32)
    for p in range(P - cap + 1, P):
        ring_k[p % cap] = hist.k[p]
        ring_v[p % cap] = hist.v[p]
    q_h, k_h, v_h = _gauss(60, 1, 8, Dh), _gauss(61, 1, 1, Dh), _gauss(62, 1, 1, Dh)
    qn_h, kn_h = _weight(63, Dh), _weight(64, Dh)
    pos = np.array([P], np.uint32)
    qo, ko, vo = oracle.producer(q_h, k_h, v_h, qn_h, kn_h, pos, 1e4, 256, 1e-6)
    bufs = [ctx.upload(a) for a in (q_h, k_h, v_h, qn_h, kn_h, ring_k, ring_v)]
    qo_d, out = ctx.empty((1, 8, Dh)), ctx.empty((1, 8 * Dh))
    try:
        step("producer + decode on a ring")
        ctx.attn_producer(q=bufs[0].ptr, k=bufs[1].ptr, v=bufs[2].ptr, q_norm=bufs[3].ptr, k_norm=bufs[4].ptr,
                          q_out=qo_d.ptr, k_cache=bufs[5].ptr, v_cache=bufs[6].ptr, T=1, Hq=8, Hkv=1, Dh=Dh,
                          rotary_dim=256, pos0=P, cache_row=P, ring_cap=cap, theta=1e4, eps=1e-6)
        ctx.attention(qo_d.ptr, bufs[5].ptr, bufs[6].ptr, out.ptr, T=1, S=P + 1, Hq=8, Hkv=1, Dh=Dh, Dv=Dh,
                      q_pos0=P, k_pos0=0, window=512, ring_cap=cap)
        q_gpu, rk, rv = qo_d.to_host(), bufs[5].to_host(), bufs[6].to_host()
        assert_parity(q_gpu, qo, "producer q")
        assert_parity(rk[P % cap], ko[0], "producer K row")
        assert_parity(rv[P % cap], vo[0], "producer V row")
        order = [(p % cap) for p in range(P - cap + 1, P + 1)]
        want = oracle.attention(q_gpu, rk[order], rv[order], pos, np.arange(P - cap + 1, P + 1, dtype=np.uint32),
                                window=512)
        # the attention itself sums its splits in another order than the CPU: the tolerance only
        assert_parity(out.to_host(), want, "producer -> attention", exact=False)
    finally:
        for b in bufs + [qo_d, out]:
            b.free()
