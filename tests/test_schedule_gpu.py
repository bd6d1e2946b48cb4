"""GPU parity of configs[4]: one decode token of the 35-layer Gemma-4-E2B
attention schedule at 32768 context, against the CPU oracle
(rust/src/backend_cpu.rs:270-336) on every one of its 35 outputs.

The token is the bench's (synth.schedule_token): 7 global calls (hd512, full
context) over 3 caches and 28 sliding calls (hd256, window 512) over 12
512-slot rings, layers 15..34 reading the cache of layer 13 or 14 as
kv_source_layer maps them (rust/src/config.rs:152-159, the shared-layer read of
rust/src/model.rs:282-285). The 35 calls run back to back through
g4a_attention_batch, so one workspace is reused in stream order across the
hd256 and hd512 calls, and again as replays of a captured HIP graph. A shared
layer is also run the way the model runs it: the producer with no k/v
(g4a_attn_producer with k = v = NULL: only the q norm and RoPE) followed by
attention over the source layer's cache, each op checked on its own inputs.
Bar: max-abs <= 1e-5, mean-abs <= 1e-6."""
import numpy as np
import pytest

import g4a
import g4a.synth as synth
import oracle

pytestmark = pytest.mark.gpu

MAX_ABS, MEAN_ABS = 1e-5, 1e-6
S = 32768


def step(msg):
    print(f"[gpu] {msg}", flush=True)


def assert_parity(got, want, label):
    d = np.abs(np.asarray(got, np.float64) - np.asarray(want, np.float64))
    mx, mean = float(d.max()), float(d.mean())
    assert mx <= MAX_ABS and mean <= MEAN_ABS, f"{label}: max-abs {mx:.3e} mean-abs {mean:.3e}"
    return mx, mean


@pytest.fixture(scope="module")
def schedule():
    layers, caches = synth.schedule_token(S, seed=4)
    want = []
    for L in layers:
        k, v = synth.unroll_ring(caches[L.src])
        c = caches[L.src]
        want.append(oracle.attention(L.q, k, v, np.array([S - 1], np.uint32), c.k_pos,
                                     window=0 if L.is_global else synth.E2B_WINDOW).reshape(1, -1))
    return layers, caches, want


def test_35_layer_token_batch_and_graph_replay(ctx, schedule):
    layers, caches, want = schedule
    bufs = []
    keep = lambda d: bufs.append(d) or d  # noqa: E731
    graph = None
    try:
        dev = {li: (keep(ctx.upload(c.k)), keep(ctx.upload(c.v))) for li, c in caches.items()}
        outs, token = [], []
        for L in layers:
            q = keep(ctx.upload(L.q))
            out = keep(ctx.empty((1, 8 * L.Dh)))
            k, v = dev[L.src]
            token.append(dict(q=q.ptr, k=k.ptr, v=v.ptr, out=out.ptr, T=1, S=S, Hq=8, Hkv=1, Dh=L.Dh, Dv=L.Dh,
                              q_pos0=S - 1, k_pos0=0, window=0 if L.is_global else synth.E2B_WINDOW,
                              ring_cap=caches[L.src].ring_cap))
            outs.append(out)
        step("35-call token through g4a_attention_batch")
        ctx.attention_batch(token)
        eager = [o.to_host() for o in outs]
        worst = (0.0, 0.0)
        for L, got, w in zip(layers, eager, want):
            mx, mean = assert_parity(got, w, f"layer {L.index} (reads {L.src})")
            worst = (max(worst[0], mx), max(worst[1], mean))
        print(f"  35 outputs vs oracle: worst max-abs {worst[0]:.3e}, worst mean-abs {worst[1]:.3e}", flush=True)

        step("capture the token")
        ctx.capture_begin()
        try:
            ctx.attention_batch(token)
        except Exception:
            try:
                ctx.capture_end().free()
            except g4a.G4aError:
                pass
            raise
        graph = ctx.capture_end()
        rng = np.random.default_rng(4)
        for rep in range(3):
            step(f"graph replay {rep}")
            for o in outs:
                ctx.h2d(o.ptr, rng.standard_normal(o.shape).astype(np.float32))
            graph.launch()
            ctx.sync()
            for L, o, e, w in zip(layers, outs, eager, want):
                got = o.to_host()
                assert np.array_equal(got, e), f"replay {rep}, layer {L.index}: differs from the eager run"
                assert_parity(got, w, f"replay {rep}, layer {L.index}")
    finally:
        if graph is not None:
            graph.free()
        for d in bufs:
            d.free()


@pytest.mark.parametrize("layer", [19, 15])
def test_shared_layer_producer_then_attention(ctx, schedule, layer):
    # a layer of the shared region (19: global, reads 14; 15: sliding, reads 13): the producer
    # normalises and rotates q only (k = v = NULL, rust/src/model.rs:256-261 then :282-285), and
    # attention reads the source layer's cache, which the producer leaves untouched. The chain is
    # held to the bar against the CPU chain: attention over the device's q against the oracle's
    # attention over the oracle's head_norm_rope q. Scores of ~90 turn an ulp of q into ~1e-5 of
    # output, so this needs q bit-identical: the sum of squares in the reference's order and
    # libm's sin/cos (the device's tree sum alone moved layer 19 by 5e-5).
    layers, caches, _ = schedule
    L = layers[layer]
    assert L.src != layer
    c = caches[L.src]
    theta, rot = (1e6, L.Dh // 4) if L.is_global else (1e4, L.Dh)  # rope_parameters of the config
    q_raw = synth.normal_f32(977 + layer, 0, 8 * L.Dh).reshape(1, 8, L.Dh)
    w = (np.float32(1.0) + np.float32(0.1) * synth.normal_f32(977 + layer, 1, L.Dh)).astype(np.float32)
    pos = np.array([S - 1], np.uint32)
    q_ref = oracle.head_norm_rope(q_raw, w, 1e-6, pos, theta, rot)
    k_lin, v_lin = synth.unroll_ring(c)
    dq, dw = ctx.upload(q_raw), ctx.upload(w)
    dk, dv = ctx.upload(c.k), ctx.upload(c.v)
    qo, out = ctx.empty((1, 8, L.Dh)), ctx.empty((1, 8 * L.Dh))
    try:
        step(f"shared layer {layer}: producer (q only) + attention over layer {L.src}'s cache")
        ctx.attn_producer(q=dq.ptr, q_norm=dw.ptr, q_out=qo.ptr, T=1, Hq=8, Hkv=1, Dh=L.Dh, rotary_dim=rot,
                          pos0=S - 1, theta=theta, eps=1e-6)
        ctx.attention(qo.ptr, dk.ptr, dv.ptr, out.ptr, T=1, S=S, Hq=8, Hkv=1, Dh=L.Dh, Dv=L.Dh, q_pos0=S - 1,
                      k_pos0=0, window=0 if L.is_global else synth.E2B_WINDOW, ring_cap=c.ring_cap)
        got_q, got = qo.to_host(), out.to_host()
        assert np.array_equal(dk.to_host(), c.k) and np.array_equal(dv.to_host(), c.v), "the cache was written"
    finally:
        for d in (dq, dw, dk, dv, qo, out):
            d.free()
    nq = int((got_q != q_ref).sum())
    print(f"  layer {layer} q: {nq} of {q_ref.size} values differ from the oracle's head_norm_rope", flush=True)
    assert nq == 0, f"layer {layer}: q differs from the oracle's in {nq} values"
    want = oracle.attention(q_ref, k_lin, v_lin, pos, c.k_pos,
                            window=0 if L.is_global else synth.E2B_WINDOW).reshape(1, -1)
    mx, mean = assert_parity(got, want, f"layer {layer} attention vs the oracle chain")
    print(f"  layer {layer}: max-abs {mx:.3e} mean-abs {mean:.3e}", flush=True)
