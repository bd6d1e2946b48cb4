"""Decode steps at a device position (g4a_attention_devpos, g4a_attn_producer_devpos,
g4a_u32_add) through the C-ABI: the position of the token lives in device memory,
so one captured decode step replays token after token.

- Eager: a device-position attention step equals g4a_attention on the same step
  (bit for bit where both run the same kernels: the sliding window's short
  kernel past its first split, the streaming kernel once the eager step plans
  the same split count) and meets the oracle's bar
  (rust/src/backend_cpu.rs:270-336) at every position.
- Captured: the producer and attention of a sliding layer (512-slot ring) and of
  a global layer (linear cache), then the position's increment, captured once and
  replayed for 24 tokens with new projections uploaded between replays. Every
  replay's outputs and caches equal an eager mirror of the same steps with host
  positions, bit for bit, and the attention meets the oracle's bar.
- A position past max_pos makes the producer write nothing."""
import numpy as np
import pytest

import g4a
import g4a.synth as synth
import oracle

pytestmark = pytest.mark.gpu

MAX_ABS, MEAN_ABS = 1e-5, 1e-6


def step(msg):
    print(f"[gpu] {msg}", flush=True)


def within_bar(got, want, label):
    d = np.abs(np.asarray(got, np.float64) - np.asarray(want, np.float64))
    print(f"  {label}: max-abs {d.max():.3e} mean-abs {d.mean():.3e}", flush=True)
    assert d.max() <= MAX_ABS and d.mean() <= MEAN_ABS, label


def set_pos(ctx, buf, p):
    ctx.h2d(buf.ptr, np.array([p], np.uint32))


def test_devpos_attention_matches_host_positions(ctx):
    """Sliding hd256 on a 512-slot ring (short kernel) and global hd512 at 32K (streaming
    kernel, the same split count forced on the eager call) at several positions."""
    Dh, cap, W, S_MAX = 256, 512, 512, 4096
    ins = synth.gemma_inputs(T=1, S=S_MAX, Dh=Dh, seed=81)
    pos = ctx.empty((1,), np.uint32)
    out_d, out_e = ctx.empty((1, 8 * Dh)), ctx.empty((1, 8 * Dh))
    q = ctx.upload(ins.q)
    bufs = [pos, out_d, out_e, q]
    try:
        for p in (0, 5, 31, 32, 200, 511, 512, 1000, 4095):
            ring_k = np.zeros((cap, 1, Dh), np.float32)
            ring_v = np.zeros((cap, 1, Dh), np.float32)
            for j in range(max(0, p - cap + 1), p + 1):
                ring_k[j % cap], ring_v[j % cap] = ins.k[j], ins.v[j]
            rk, rv = ctx.upload(ring_k), ctx.upload(ring_v)
            try:
                set_pos(ctx, pos, p)
                step(f"sliding hd256 ring {cap} at position {p}")
                ctx.attention_devpos(q.ptr, rk.ptr, rv.ptr, out_d.ptr, pos.ptr, T=1, S=S_MAX, Hq=8, Hkv=1, Dh=Dh,
                                     Dv=Dh, k_pos0=0, window=W, ring_cap=cap)
                ctx.attention(q.ptr, rk.ptr, rv.ptr, out_e.ptr, T=1, S=p + 1, Hq=8, Hkv=1, Dh=Dh, Dv=Dh,
                              q_pos0=p, k_pos0=0, window=W, ring_cap=cap)
                got, eager = out_d.to_host(), out_e.to_host()
            finally:
                rk.free()
                rv.free()
            lo = max(0, p - W + 1)
            want = oracle.attention(ins.q, ins.k[lo:p + 1], ins.v[lo:p + 1], np.array([p], np.uint32),
                                    np.arange(lo, p + 1, dtype=np.uint32), window=W)
            within_bar(got, want, f"devpos sliding at {p}")
            if p >= 32:  # both merge their splits in the combine (one split writes the output directly)
                assert np.array_equal(got, eager), f"sliding at {p}: differs from g4a_attention"
    finally:
        for b in bufs:
            b.free()

    Dh, S_MAX = 512, 32768
    ins = synth.gemma_inputs(T=1, S=S_MAX, Dh=Dh, seed=82)
    dev = [ctx.upload(x) for x in (ins.q, ins.k, ins.v)]
    pos = ctx.empty((1,), np.uint32)
    out_d, out_e = ctx.empty((1, 8 * Dh)), ctx.empty((1, 8 * Dh))
    try:
        splits = ctx.plan(T=1, S=S_MAX, Hq=8, Hkv=1, Dh=Dh, Dv=Dh, q_pos0=S_MAX - 1, k_pos0=0).splits
        for p in (0, 100, 9000, 20000, S_MAX - 1):
            set_pos(ctx, pos, p)
            step(f"global hd512 linear cache at position {p} ({splits} splits)")
            ctx.attention_devpos(dev[0].ptr, dev[1].ptr, dev[2].ptr, out_d.ptr, pos.ptr, T=1, S=S_MAX, Hq=8, Hkv=1,
                                 Dh=Dh, Dv=Dh, k_pos0=0)
            ctx.attention(dev[0].ptr, dev[1].ptr, dev[2].ptr, out_e.ptr, T=1, S=p + 1, Hq=8, Hkv=1, Dh=Dh, Dv=Dh,
                          q_pos0=p, k_pos0=0, splits=splits)
            got, eager = out_d.to_host(), out_e.to_host()
            # bit for bit once the eager step has as many splits (at few keys its forced count is
            # clamped to the key tiles, and its merge then takes the small-split combine)
            eager_splits = ctx.plan(T=1, S=p + 1, Hq=8, Hkv=1, Dh=Dh, Dv=Dh, q_pos0=p, k_pos0=0,
                                    splits=splits).splits
            if eager_splits == splits:
                assert np.array_equal(got, eager), f"global at {p}: differs from g4a_attention at {splits} splits"
            if p < 10000:
                want = oracle.attention(ins.q, ins.k[:p + 1], ins.v[:p + 1], np.array([p], np.uint32),
                                        np.arange(p + 1, dtype=np.uint32))
                within_bar(got, want, f"devpos global at {p}")
    finally:
        for b in dev + [pos, out_d, out_e]:
            b.free()


def _layer_inputs(rng, Dh):
    q = rng.standard_normal((1, 8, Dh)).astype(np.float32)
    k = rng.standard_normal((1, 1, Dh)).astype(np.float32)
    v = rng.standard_normal((1, 1, Dh)).astype(np.float32)
    return q, k, v


def test_captured_decode_step_replays_token_after_token(ctx):
    P0, STEPS = 1000, 24
    CAP = P0 + STEPS + 8  # rows of the global layer's linear cache; the plan's S
    RING, W = 512, 512
    rng = np.random.default_rng(17)
    # history: positions 0 .. P0-1 of both layers (a sliding ring holds the last RING)
    hist_s = synth.gemma_inputs(T=1, S=P0, Dh=256, seed=91)
    hist_g = synth.gemma_inputs(T=1, S=P0, Dh=512, seed=92)
    ring_k0 = np.zeros((RING, 1, 256), np.float32)
    ring_v0 = np.zeros((RING, 1, 256), np.float32)
    for j in range(P0 - RING, P0):
        ring_k0[j % RING], ring_v0[j % RING] = hist_s.k[j], hist_s.v[j]
    lin_k0 = np.zeros((CAP, 1, 512), np.float32)
    lin_v0 = np.zeros((CAP, 1, 512), np.float32)
    lin_k0[:P0], lin_v0[:P0] = hist_g.k, hist_g.v
    wq_s, wk_s = (1.0 + 0.1 * rng.standard_normal(256)).astype(np.float32), (1.0 + 0.1 * rng.standard_normal(256)).astype(np.float32)
    wq_g, wk_g = (1.0 + 0.1 * rng.standard_normal(512)).astype(np.float32), (1.0 + 0.1 * rng.standard_normal(512)).astype(np.float32)

    owned = []

    def up(a):
        d = ctx.upload(a)
        owned.append(d)
        return d

    def em(shape, dtype=np.float32):
        d = ctx.empty(shape, dtype)
        owned.append(d)
        return d

    graph = None
    try:
        # two copies of every cache: the graph's (device positions) and the eager mirror's (host positions)
        rk, rv, lk, lv = up(ring_k0), up(ring_v0), up(lin_k0), up(lin_v0)
        mrk, mrv, mlk, mlv = up(ring_k0), up(ring_v0), up(lin_k0), up(lin_v0)
        ws = [up(x) for x in (wq_s, wk_s, wq_g, wk_g)]
        qs_in, ks_in, vs_in = em((1, 8, 256)), em((1, 1, 256)), em((1, 1, 256))
        qg_in, kg_in, vg_in = em((1, 8, 512)), em((1, 1, 512)), em((1, 1, 512))
        qs_out, qg_out = em((1, 8, 256)), em((1, 8, 512))
        out_s, out_g = em((1, 8 * 256)), em((1, 8 * 512))
        mqs_out, mqg_out, mout_s, mout_g = em((1, 8, 256)), em((1, 8, 512)), em((1, 8 * 256)), em((1, 8 * 512))
        pos = em((1,), np.uint32)

        def token_devpos():
            ctx.attn_producer_devpos(pos=pos.ptr, max_pos=CAP - 1, q=qs_in.ptr, k=ks_in.ptr, v=vs_in.ptr,
                                     q_norm=ws[0].ptr, k_norm=ws[1].ptr, q_out=qs_out.ptr, k_cache=rk.ptr,
                                     v_cache=rv.ptr, Hq=8, Hkv=1, Dh=256, rotary_dim=256, ring_cap=RING, theta=1e4,
                                     eps=1e-6)
            ctx.attention_devpos(qs_out.ptr, rk.ptr, rv.ptr, out_s.ptr, pos.ptr, T=1, S=CAP, Hq=8, Hkv=1, Dh=256,
                                 Dv=256, k_pos0=0, window=W, ring_cap=RING)
            ctx.attn_producer_devpos(pos=pos.ptr, max_pos=CAP - 1, q=qg_in.ptr, k=kg_in.ptr, v=vg_in.ptr,
                                     q_norm=ws[2].ptr, k_norm=ws[3].ptr, q_out=qg_out.ptr, k_cache=lk.ptr,
                                     v_cache=lv.ptr, Hq=8, Hkv=1, Dh=512, rotary_dim=128, ring_cap=0, theta=1e6,
                                     eps=1e-6)
            ctx.attention_devpos(qg_out.ptr, lk.ptr, lv.ptr, out_g.ptr, pos.ptr, T=1, S=CAP, Hq=8, Hkv=1, Dh=512,
                                 Dv=512, k_pos0=0)
            ctx.u32_add(pos.ptr, 1, 1)

        def token_eager(p):
            ctx.attn_producer(q=qs_in.ptr, k=ks_in.ptr, v=vs_in.ptr, q_norm=ws[0].ptr, k_norm=ws[1].ptr,
                              q_out=mqs_out.ptr, k_cache=mrk.ptr, v_cache=mrv.ptr, T=1, Hq=8, Hkv=1, Dh=256,
                              rotary_dim=256, pos0=p, cache_row=p, ring_cap=RING, theta=1e4, eps=1e-6)
            ctx.attention(mqs_out.ptr, mrk.ptr, mrv.ptr, mout_s.ptr, T=1, S=p + 1, Hq=8, Hkv=1, Dh=256, Dv=256,
                          q_pos0=p, k_pos0=0, window=W, ring_cap=RING)
            ctx.attn_producer(q=qg_in.ptr, k=kg_in.ptr, v=vg_in.ptr, q_norm=ws[2].ptr, k_norm=ws[3].ptr,
                              q_out=mqg_out.ptr, k_cache=mlk.ptr, v_cache=mlv.ptr, T=1, Hq=8, Hkv=1, Dh=512,
                              rotary_dim=128, pos0=p, cache_row=p, ring_cap=0, theta=1e6, eps=1e-6)
            ctx.attention(mqg_out.ptr, mlk.ptr, mlv.ptr, mout_g.ptr, T=1, S=p + 1, Hq=8, Hkv=1, Dh=512, Dv=512,
                          q_pos0=p, k_pos0=0)

        def upload_inputs():
            for buf, (q, k, v) in ((0, _layer_inputs(rng, 256)), (1, _layer_inputs(rng, 512))):
                ins = (qs_in, ks_in, vs_in) if buf == 0 else (qg_in, kg_in, vg_in)
                for d, x in zip(ins, (q, k, v)):
                    ctx.h2d(d.ptr, x)

        # one eager run of each device-position call at the largest position builds the RoPE
        # tables and the workspace (a capture can do neither), on scratch copies of the caches
        step("warm-up of the device-position calls at the last position (tables, workspace)")
        scratch = [up(x) for x in (ring_k0, ring_v0, lin_k0, lin_v0)]
        set_pos(ctx, pos, CAP - 1)
        saved = (rk, rv, lk, lv)
        rk, rv, lk, lv = scratch
        token_devpos()
        rk, rv, lk, lv = saved
        ctx.sync()

        step("capture one decode step (2 producers, 2 attentions, the position increment)")
        set_pos(ctx, pos, P0)
        ctx.sync()
        ctx.capture_begin()
        try:
            token_devpos()
        except Exception:
            try:
                ctx.capture_end().free()
            except g4a.G4aError:
                pass
            raise
        graph = ctx.capture_end()

        for t in range(STEPS):
            p = P0 + t
            upload_inputs()
            graph.launch()
            token_eager(p)
            ctx.sync()
            got = [out_s.to_host(), out_g.to_host(), qs_out.to_host(), qg_out.to_host()]
            want = [mout_s.to_host(), mout_g.to_host(), mqs_out.to_host(), mqg_out.to_host()]
            for name, a, b in zip(("sliding out", "global out", "sliding q", "global q"), got, want):
                assert np.array_equal(a, b), f"replay {t} (position {p}): {name} differs from the eager step"
            assert int(pos.to_host()[0]) == p + 1
            if t in (0, STEPS - 1):
                step(f"replay {t} at position {p}: against the oracle")
                kk, vv = mlk.to_host()[:p + 1], mlv.to_host()[:p + 1]
                want_g = oracle.attention(mqg_out.to_host(), kk, vv, np.array([p], np.uint32),
                                          np.arange(p + 1, dtype=np.uint32))
                within_bar(got[1], want_g, f"global layer at {p}")
                ring_k, ring_v = mrk.to_host(), mrv.to_host()
                lo = p - W + 1
                order = [j % RING for j in range(lo, p + 1)]
                want_s = oracle.attention(mqs_out.to_host(), ring_k[order], ring_v[order], np.array([p], np.uint32),
                                          np.arange(lo, p + 1, dtype=np.uint32), window=W)
                within_bar(got[0], want_s, f"sliding layer at {p}")
        step("caches after the replays")
        for name, a, b in (("ring K", rk, mrk), ("ring V", rv, mrv), ("linear K", lk, mlk), ("linear V", lv, mlv)):
            assert np.array_equal(a.to_host(), b.to_host()), f"{name} differs from the eager mirror"
        print(f"  {STEPS} replays of one captured step, positions {P0} .. {P0 + STEPS - 1}: bit-identical to the "
              f"eager steps", flush=True)
    finally:
        if graph is not None:
            graph.free()
        for d in owned:
            d.free()


def test_producer_position_past_max_pos_writes_nothing(ctx):
    rng = np.random.default_rng(3)
    q, k, v = _layer_inputs(rng, 256)
    dq, dk, dv = ctx.upload(q), ctx.upload(k), ctx.upload(v)
    cache_k, cache_v = ctx.upload(np.full((64, 1, 256), 7.0, np.float32)), ctx.upload(np.full((64, 1, 256), 7.0, np.float32))
    q_out = ctx.upload(np.full((1, 8, 256), 5.0, np.float32))
    pos = ctx.empty((1,), np.uint32)
    try:
        set_pos(ctx, pos, 64)
        step("producer at position 64 with max_pos 63: nothing written")
        ctx.attn_producer_devpos(pos=pos.ptr, max_pos=63, q=dq.ptr, k=dk.ptr, v=dv.ptr, q_out=q_out.ptr,
                                 k_cache=cache_k.ptr, v_cache=cache_v.ptr, Hq=8, Hkv=1, Dh=256, rotary_dim=256,
                                 theta=1e4, eps=1e-6)
        assert np.all(cache_k.to_host() == 7.0) and np.all(cache_v.to_host() == 7.0)
        assert np.all(q_out.to_host() == 5.0)
        set_pos(ctx, pos, 63)
        ctx.attn_producer_devpos(pos=pos.ptr, max_pos=63, q=dq.ptr, k=dk.ptr, v=dv.ptr, q_out=q_out.ptr,
                                 k_cache=cache_k.ptr, v_cache=cache_v.ptr, Hq=8, Hkv=1, Dh=256, rotary_dim=256,
                                 theta=1e4, eps=1e-6)
        qo, ko, vo = oracle.producer(q, k, v, None, None, np.array([63], np.uint32), 1e4, 256, 1e-6)
        assert np.array_equal(q_out.to_host(), qo)
        assert np.array_equal(cache_k.to_host()[63], ko[0]) and np.array_equal(cache_v.to_host()[63], vo[0])
        assert np.all(cache_k.to_host()[:63] == 7.0)
    finally:
        for b in (dq, dk, dv, cache_k, cache_v, q_out, pos):
            b.free()
