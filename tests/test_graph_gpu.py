"""Graph capture (g4a_capture_begin / g4a_capture_end / g4a_graph_launch): a
captured sequence of attention calls (and one of projections) replays
bit-identically to the same calls run eagerly. Each replay runs after the output buffers are overwritten and
after unrelated eager work and a synchronisation, and every replay is checked.
Calls that need host staging are refused while a capture is open, and the
context stays usable after such a refusal."""
import numpy as np
import pytest

import g4a
import g4a.synth as synth

pytestmark = pytest.mark.gpu


def step(msg):
    print(f"[gpu] {msg}", flush=True)


def _calls(ctx, keep):
    """(attention() keyword sets, output buffers): sliding decode on a ring, a
    multi-split global decode (partials + combine), multi-query decode, a
    prefill, and a call whose keys all lie in the future (its rows are zero)."""
    specs = [dict(T=1, S=5000, Dh=256, window=512, ring_cap=512, q_pos0=4999, seed=1),
             dict(T=1, S=32768, Dh=512, seed=2, q_pos0=32767),
             dict(T=5, S=777, Dh=256, window=512, seed=3, q_pos0=772),
             dict(T=64, S=64, Dh=256, window=512, seed=4, q_pos0=0),
             dict(T=2, S=100, Dh=512, seed=5, q_pos0=0, k_pos0=50)]
    calls, outs = [], []
    for sp in specs:
        T, S, Dh = sp["T"], sp["S"], sp["Dh"]
        rows = sp.get("ring_cap") or S
        ins = synth.gemma_inputs(T=T, S=rows, Dh=Dh, seed=sp["seed"])
        q, k, v = (keep(ctx.upload(x)) for x in (ins.q, ins.k, ins.v))
        out = keep(ctx.empty((T, 8 * Dh)))
        calls.append(dict(q=q.ptr, k=k.ptr, v=v.ptr, out=out.ptr, T=T, S=S, Hq=8, Hkv=1, Dh=Dh, Dv=Dh,
                          q_pos0=sp["q_pos0"], k_pos0=sp.get("k_pos0", 0), window=sp.get("window", 0),
                          ring_cap=sp.get("ring_cap", 0)))
        outs.append(out)
    return calls, outs


def test_captured_sequence_replays_bit_exactly(ctx):
    bufs = []
    keep = lambda d: bufs.append(d) or d  # noqa: E731
    try:
        calls, outs = _calls(ctx, keep)
        step("eager run")
        ctx.attention_batch(calls)
        want = [o.to_host() for o in outs]
        assert not np.any(want[4]), "rows with only future keys are zero"
        step("capture")
        ctx.capture_begin()
        try:
            ctx.attention_batch(calls)
            graph = ctx.capture_end()
        except Exception:
            _end_open_capture(ctx)
            raise
        # the capture ran nothing: the outputs still hold the eager results
        for o, w in zip(outs, want):
            assert np.array_equal(o.to_host(), w)
        other = _calls(ctx, keep)[0][1]  # unrelated eager work between replays
        rng = np.random.default_rng(0)
        try:
            for rep in range(4):
                step(f"replay {rep}")
                for o in outs:  # overwrite every output (the zero rows included)
                    ctx.h2d(o.ptr, rng.standard_normal(o.shape).astype(np.float32))
                ctx.attention(**other)
                ctx.sync()
                graph.launch()
                ctx.sync()
                for i, (o, w) in enumerate(zip(outs, want)):
                    assert np.array_equal(o.to_host(), w), f"replay {rep}, call {i}"
        finally:
            graph.free()
    finally:
        for d in bufs:
            d.free()


def _end_open_capture(ctx):
    """Close a capture a failed assertion left open (the context is shared by the session)."""
    try:
        ctx.capture_end().free()
    except g4a.G4aError:
        pass


def test_capture_refuses_host_staging_and_recovers(ctx):
    ins = synth.gemma_inputs(T=1, S=300, Dh=256, seed=9)
    k_pos = np.arange(300, dtype=np.uint32)
    k_pos[150:] += 7  # a gap: the positions must be staged to the device
    q_pos = np.array([320], np.uint32)
    q, k, v = (ctx.upload(x) for x in (ins.q, ins.k, ins.v))
    out = ctx.empty((1, 8 * 256))
    kw = dict(T=1, S=300, Hq=8, Hkv=1, Dh=256, Dv=256, q_pos=q_pos, k_pos=k_pos)
    try:
        ctx.capture_begin()
        try:
            with pytest.raises(g4a.G4aError, match="cannot hold"):
                ctx.attention(q.ptr, k.ptr, v.ptr, out.ptr, **kw)
            with pytest.raises(g4a.G4aError, match="cannot be captured"):
                ctx.sync()
            with pytest.raises(g4a.G4aError, match="already open"):
                ctx.capture_begin()
            # the refused calls are missing from the recording: no graph, the first failure reported
            with pytest.raises(g4a.G4aError, match="failed, so no graph was made.*cannot hold"):
                ctx.capture_end()
        finally:
            _end_open_capture(ctx)
        with pytest.raises(g4a.G4aError, match="no capture is open"):
            ctx.capture_end()
        # the context works as before: the refused call runs eagerly, twice alike
        ctx.attention(q.ptr, k.ptr, v.ptr, out.ptr, **kw)
        a = out.to_host()
        assert np.all(np.isfinite(a)) and np.any(a)
        ctx.attention(q.ptr, k.ptr, v.ptr, out.ptr, **kw)
        assert np.array_equal(out.to_host(), a)
    finally:
        for d in (q, k, v, out):
            d.free()


def test_replay_after_the_workspace_grows_and_graph_ownership(ctx):
    # A graph keeps the workspace it was captured with: an eager call that needs a larger one
    # afterwards (a 2048-token hd512 prefill) must not free it under the graph, whose replays stay
    # bit-identical. A generic-path call (head_dim 64) with contiguous positions is capturable too.
    # A graph replays only on the context it was captured on.
    own = g4a.Context(0)  # a fresh context: its workspace starts small
    bufs = []
    keep = lambda d: bufs.append(d) or d  # noqa: E731
    graph = None
    try:
        ins = synth.gemma_inputs(T=1, S=32768, Dh=512, seed=12)
        q, k, v = (keep(own.upload(x)) for x in (ins.q, ins.k, ins.v))
        out = keep(own.empty((1, 8 * 512)))
        gen = synth.gemma_inputs(T=3, S=200, Dh=64, seed=13)
        gq, gk, gv = (keep(own.upload(x)) for x in (gen.q, gen.k, gen.v))
        gout = keep(own.empty((3, 8 * 64)))
        calls = [dict(q=q.ptr, k=k.ptr, v=v.ptr, out=out.ptr, T=1, S=32768, Hq=8, Hkv=1, Dh=512, Dv=512,
                      q_pos0=32767),
                 dict(q=gq.ptr, k=gk.ptr, v=gv.ptr, out=gout.ptr, T=3, S=200, Hq=8, Hkv=1, Dh=64, Dv=64,
                      q_pos0=197)]
        assert g4a.KERNEL_NAMES[own.plan(**{k_: v_ for k_, v_ in calls[1].items() if k_ not in
                                            ("q", "k", "v", "out")}).kernel] == "generic"
        step("eager run (fresh context)")
        own.attention_batch(calls)
        want = [out.to_host(), gout.to_host()]
        step("capture")
        own.capture_begin()
        try:
            own.attention_batch(calls)
        except Exception:
            _end_open_capture(own)
            raise
        graph = own.capture_end()
        step("eager 2048-token hd512 prefill (grows the workspace)")
        pf = synth.gemma_inputs(T=2048, S=2048, Dh=512, seed=3, q_pos=np.arange(2048))
        pq, pk, pv = (keep(own.upload(x)) for x in (pf.q, pf.k, pf.v))
        pout = keep(own.empty((2048, 8 * 512)))
        plan = own.plan(T=2048, S=2048, Hq=8, Hkv=1, Dh=512, Dv=512, q_pos0=0)
        assert g4a.KERNEL_NAMES[plan.kernel] == "prefill"
        own.attention(pq.ptr, pk.ptr, pv.ptr, pout.ptr, T=2048, S=2048, Hq=8, Hkv=1, Dh=512, Dv=512, q_pos0=0)
        own.sync()
        rng = np.random.default_rng(1)
        for rep in range(3):
            step(f"replay {rep} after the growth")
            for o in (out, gout):
                own.h2d(o.ptr, rng.standard_normal(o.shape).astype(np.float32))
            graph.launch()
            own.sync()
            assert np.array_equal(out.to_host(), want[0]), f"replay {rep}: decode"
            assert np.array_equal(gout.to_host(), want[1]), f"replay {rep}: generic"
            # eager work in between, through the grown workspace
            own.attention(pq.ptr, pk.ptr, pv.ptr, pout.ptr, T=2048, S=2048, Hq=8, Hkv=1, Dh=512, Dv=512, q_pos0=0)
        step("a graph launched on another context is refused")
        with pytest.raises(g4a.G4aError, match="another context"):
            ctx._check(ctx.lib.g4a_graph_launch(ctx.handle, graph.handle))
    finally:
        if graph is not None:
            graph.free()
        for d in bufs:
            d.free()
        own.close()


def test_captured_projections_replay_bit_exactly(ctx):
    """The projection kernels under capture: a 2-bit [49152, 1536] weight at M = 1
    (the int8 matrix-core kernel, with its dynamic LDS), a 4-bit [2048, 1536] at
    M = 1 (the word kernel) and a 2-bit [12288, 1536] at M = 64 (the bf16 matrix
    cores), captured as one graph and replayed three times, each replay checked
    bit-exactly against the eager run."""
    cases = [(49152, 1536, 2, 1), (2048, 1536, 4, 1), (12288, 1536, 2, 64)]
    bufs = []
    try:
        calls = []
        for i, (N, K, bits, M) in enumerate(cases):
            qb, sc, _ = synth.quant_weight(60 + i, N, K, bits)
            w = ctx.upload_qweight(qb, sc, N, K, bits)
            x = ctx.upload(synth.normal_f32(70 + i, 0, M * K).reshape(M, K))
            y = ctx.empty((M, N))
            bufs += [w, x, y]
            calls.append((w, x, y, M))
        step("eager projections")
        for w, x, y, M in calls:
            ctx.linear_q(w, x.ptr, y.ptr, M)
        want = [y.to_host() for _, _, y, _ in calls]
        step("capture")
        ctx.capture_begin()
        try:
            for w, x, y, M in calls:
                ctx.linear_q(w, x.ptr, y.ptr, M)
            graph = ctx.capture_end()
        except Exception:
            _end_open_capture(ctx)
            raise
        rng = np.random.default_rng(1)
        try:
            for rep in range(3):
                step(f"replay {rep}")
                for _, _, y, _ in calls:
                    ctx.h2d(y.ptr, rng.standard_normal(y.shape).astype(np.float32))
                w0, x0, _, _ = calls[1]
                scratch = ctx.empty((1, 2048))
                ctx.linear_q(w0, x0.ptr, scratch.ptr, 1)  # unrelated eager work
                ctx.sync()
                scratch.free()
                graph.launch()
                ctx.sync()
                for i, ((_, _, y, _), wv) in enumerate(zip(calls, want)):
                    assert np.array_equal(y.to_host(), wv), f"replay {rep}, projection {i}"
        finally:
            graph.free()
    finally:
        for d in bufs:
            d.free()
