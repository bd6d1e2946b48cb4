"""GPU parity of the query-tiled MFMA prefill kernel (approximate matrix-core
scores + exact rescoring of every key near its row maximum) against the CPU
oracle (rust/src/backend_cpu.rs:270-336), through the C-ABI. Same bar as
decode: max-abs <= 1e-5, mean-abs <= 1e-6 in f32.

Covers configs[3] at full size (2048-token prompts, sliding window 512 at
head_dim 256 and full causal at 512), ragged query counts, chunked prefill
continuing from a cache, KV rings, and degenerate near-tie inputs that
overflow the per-wave candidate list (compaction and early correction)."""
import numpy as np
import pytest

import g4a
import g4a.synth as synth
import oracle

pytestmark = pytest.mark.gpu

MAX_ABS, MEAN_ABS = 1e-5, 1e-6


def assert_parity(got, want, label):
    d = np.abs(got.astype(np.float64) - np.asarray(want, np.float64))
    mx, mean = float(d.max()), float(d.mean())
    print(f"  {label}: max-abs {mx:.3e} mean-abs {mean:.3e}", flush=True)
    assert mx <= MAX_ABS and mean <= MEAN_ABS, f"{label}: max-abs {mx:.3e} mean-abs {mean:.3e}"


def run(ctx, ins, window, label, **kw):
    print(f"[gpu] {label}", flush=True)
    T, S = ins.q.shape[0], ins.k.shape[0]
    plan = ctx.plan(T=T, S=S, Hq=ins.q.shape[1], Hkv=ins.k.shape[1], Dh=ins.q.shape[2], Dv=ins.v.shape[2],
                    q_pos0=int(ins.q_pos[0]), k_pos0=int(ins.k_pos[0]), window=window)
    assert g4a.KERNEL_NAMES[plan.kernel] == "prefill", label
    want = oracle.attention(ins.q, ins.k, ins.v, ins.q_pos, ins.k_pos, window=window, **kw)
    got = g4a.attention_host(ctx, ins.q, ins.k, ins.v, q_pos=ins.q_pos, k_pos=ins.k_pos, window=window, **kw)
    assert_parity(got, want, label)
    return got


@pytest.mark.parametrize("name,T,Dh,W", [
    ("configs[3a] local prefill hd256 T2048 window512", 2048, 256, 512),
    ("configs[3b] global prefill hd512 T2048 causal", 2048, 512, 0),
])
def test_configs3_full_size(ctx, name, T, Dh, W):
    ins = synth.gemma_inputs(T=T, S=T, Dh=Dh, seed=3, q_pos=np.arange(T))
    run(ctx, ins, W, name)


@pytest.mark.parametrize("T,S,Dh,W", [(16, 16, 256, 0), (37, 37, 256, 5), (29, 29, 512, 0), (100, 100, 512, 17),
                                      (24, 900, 256, 512), (40, 3000, 512, 0), (64, 700, 256, 64)])
def test_ragged_and_chunked(ctx, T, S, Dh, W):
    # T queries are the last T positions of S keys (a prompt chunk after S - T cached tokens)
    ins = synth.gemma_inputs(T=T, S=S, Dh=Dh, seed=T * 7 + S)
    run(ctx, ins, W, f"T={T} S={S} Dh={Dh} window={W}")


def test_scale_not_one(ctx):
    ins = synth.gemma_inputs(T=48, S=48, Dh=256, seed=9, q_pos=np.arange(48))
    run(ctx, ins, 0, "scale 1/16", scale=0.0625)


def test_all_tied_scores_overflow_the_candidate_list(ctx):
    # q = 0: every visible key ties at score 0, so every key is a candidate and the
    # per-wave list overflows repeatedly; the answer is the mean of the visible values
    for T, S, Dh, W in [(64, 2048, 256, 0), (32, 1500, 512, 0), (48, 2000, 256, 700)]:
        ins = synth.gemma_inputs(T=T, S=S, Dh=Dh, seed=5)
        ins.q[:] = 0.0
        got = run(ctx, ins, W, f"q=0 T={T} S={S} Dh={Dh} window={W}")
        i = T - 1
        lo = max(0, S - 1 - W + 1) if W else 0
        np.testing.assert_allclose(got[i].reshape(8, Dh)[0], ins.v[lo:S, 0].astype(np.float64).mean(0), atol=2e-6)


def test_near_ties_from_repeated_keys(ctx):
    # every key repeated 8 times: exact ties in the sequential order, tiny differences on the matrix cores
    base = synth.gemma_inputs(T=64, S=256, Dh=256, seed=13, q_pos=np.arange(64))
    k = np.repeat(base.k[:32], 8, axis=0)
    ins = synth.AttnInputs(base.q, k, base.v, np.arange(192, 256, dtype=np.uint32), base.k_pos)
    run(ctx, ins, 0, "repeated keys")


def test_prefill_from_a_ring(ctx):
    # a 1024-slot ring holding positions 976..1999; 24 new queries at 1976..1999 with window 512
    L, cap, T, Dh, W = 2000, 1024, 24, 256, 512
    ins = synth.gemma_inputs(T=T, S=L, Dh=Dh, seed=77)
    want = oracle.attention(ins.q, ins.k, ins.v, ins.q_pos, ins.k_pos, window=W)
    ring_k = np.zeros((cap, 1, Dh), np.float32)
    ring_v = np.zeros((cap, 1, Dh), np.float32)
    for p_ in range(L - cap, L):
        ring_k[p_ % cap] = ins.k[p_]
        ring_v[p_ % cap] = ins.v[p_]
    dev = [ctx.upload(x) for x in (ins.q, ring_k, ring_v)]
    out = ctx.empty((T, 8 * Dh))
    try:
        print("[gpu] prefill from ring", flush=True)
        ctx.attention(dev[0].ptr, dev[1].ptr, dev[2].ptr, out.ptr, T=T, S=L, Hq=8, Hkv=1, Dh=Dh, Dv=Dh,
                      q_pos0=L - T, k_pos0=0, window=W, ring_cap=cap)
        got = out.to_host()
    finally:
        for d in dev:
            d.free()
        out.free()
    assert_parity(got, want, "prefill from ring")


def test_prefill_matches_decode_kernel_rows(ctx):
    # the last query of a prefill equals a decode of that query (independent kernels)
    ins = synth.gemma_inputs(T=32, S=32, Dh=512, seed=21, q_pos=np.arange(32))
    full = run(ctx, ins, 0, "prefill T=32")
    last = g4a.attention_host(ctx, ins.q[-1:], ins.k, ins.v, q_pos=[31], k_pos=ins.k_pos)
    assert np.abs(full[-1] - last[0]).max() < 2e-6


def test_two_kv_heads(ctx):
    # Hq 16 over Hkv 2 (groups of 8): the pre-split K rows and V key quads interleave the kv heads
    for Dh, W in [(256, 40), (512, 0)]:
        ins = synth.gemma_inputs(T=72, S=100, Dh=Dh, seed=31 + Dh, Hq=16, Hkv=2)
        run(ctx, ins, W, f"Hq 16 / Hkv 2, Dh {Dh}, window {W}")


@pytest.mark.parametrize("where", ["all", "one"])
def test_v_beyond_the_fp16_split_range(ctx, where):
    # V values past +-32768 cannot be split into fp16 parts: the kernel must take its f32 P.V
    # path and stay exact; absolute errors scale with |v|, so compare in units of the scale
    ins = synth.gemma_inputs(T=48, S=300, Dh=256, seed=5)
    scale = 1e5 if where == "all" else 1.0
    v = (ins.v * np.float32(scale)).astype(np.float32)
    if where == "one":
        v[123, 0, 77] = np.float32(5e4)  # a single out-of-range value, in a visible key
    big = synth.AttnInputs(ins.q, ins.k, v, ins.q_pos, ins.k_pos)
    print(f"[gpu] V beyond the fp16 range ({where})", flush=True)
    want = oracle.attention(big.q, big.k, big.v, big.q_pos, big.k_pos, window=512)
    got = g4a.attention_host(ctx, big.q, big.k, big.v, q_pos=big.q_pos, k_pos=big.k_pos, window=512)
    unit = float(np.abs(v).max())
    assert_parity(got / unit, np.asarray(want) / unit, f"V beyond the fp16 range ({where}), in units of max|v|")


@pytest.mark.parametrize("Dh,vscale", [(256, 1.0), (512, 1.0), (256, 1e5), (512, 1e5)])
def test_ring_prefill_ignores_nan_in_dead_slots(ctx, Dh, vscale):
    # A 37-token chunk at positions 600..636 (S = 637, not a multiple of 16) with window 512 reads
    # keys 89..636 from a 560-slot ring. The slots of keys 77..88 are dead (outside every query's
    # window) and hold NaN, as unwritten memory may: the tiles that round the key range out to
    # multiples of 16 touch them (keys 80..88 before it, 637..639 past it wrap onto slots 77..79),
    # with P = 0. The output must stay finite and equal the oracle's, on the fp16 P.V path and, with
    # V scaled past the fp16 range, on the f32 one.
    S, T, cap, W = 637, 37, 560, 512
    ins = synth.gemma_inputs(T=T, S=S, Dh=Dh, seed=101 + Dh)
    v = (ins.v * np.float32(vscale)).astype(np.float32)
    ring_k = np.full((cap, 1, Dh), np.nan, np.float32)
    ring_v = np.full((cap, 1, Dh), np.nan, np.float32)
    lo = S - T - W + 1  # first key any query sees
    for p_ in range(lo, S):
        ring_k[p_ % cap] = ins.k[p_]
        ring_v[p_ % cap] = v[p_]
    assert np.isnan(ring_k[77:89]).all() and not np.isnan(ring_k[89:]).any() and not np.isnan(ring_k[:77]).any()
    plan = ctx.plan(T=T, S=S, Hq=8, Hkv=1, Dh=Dh, Dv=Dh, q_pos0=S - T, k_pos0=0, window=W, ring_cap=cap)
    assert g4a.KERNEL_NAMES[plan.kernel] == "prefill" and (plan.k_start, plan.k_end) == (lo, S)
    want = oracle.attention(ins.q, ins.k, v, ins.q_pos, ins.k_pos, window=W)
    dev = [ctx.upload(x) for x in (ins.q, ring_k, ring_v)]
    out = ctx.empty((T, 8 * Dh))
    try:
        print(f"[gpu] ring prefill with NaN dead slots, Dh {Dh}, V x {vscale:g}", flush=True)
        ctx.attention(dev[0].ptr, dev[1].ptr, dev[2].ptr, out.ptr, T=T, S=S, Hq=8, Hkv=1, Dh=Dh, Dv=Dh,
                      q_pos0=S - T, k_pos0=0, window=W, ring_cap=cap)
        got = out.to_host()
    finally:
        for d in dev:
            d.free()
        out.free()
    assert np.isfinite(got).all(), "NaN from a dead ring slot reached the output"
    unit = float(np.abs(v[lo:]).max()) if vscale != 1.0 else 1.0
    assert_parity(got / unit, np.asarray(want) / unit, f"ring prefill, NaN dead slots, Dh {Dh}, V x {vscale:g}")


def rescoring_band(n_keys):
    """The band the host passes the prefill kernels (G4aPrefillParams::tau) for rows
    of n_keys keys: keys whose estimated score is more than this below their row's
    maximum keep the estimate."""
    return max(7.0, float(np.log(np.float32(n_keys))) + 2.0)


def _fp16_split(x):
    """The kernels' split of rows x: per row a power of two 2^a putting max|x 2^-a| in
    [2^14, 2^15), then fp16 hi / lo of x 2^-a. Returns (hi, lo, 2^a) as f64."""
    x = np.atleast_2d(np.asarray(x, np.float32))
    a = np.frexp(np.abs(x).max(axis=1, keepdims=True))[1] - 15
    y = np.ldexp(x, -a).astype(np.float32)
    hi = y.astype(np.float16).astype(np.float32)
    lo = (y - hi).astype(np.float16).astype(np.float32)
    return hi.astype(np.float64), lo.astype(np.float64), np.ldexp(1.0, a)


def _split_scores(q, k):
    """The kernels' score estimate of q [Dh] against keys k [S, Dh]: Khi.Qhi + Klo.Qhi +
    Khi.Qlo of the scaled fp16 splits, summed in f64, times the rows' powers of two."""
    qh, ql, qs = _fp16_split(q)
    kh, kl, ks = _fp16_split(k)
    return (kh @ qh[0] + kl @ qh[0] + kh @ ql[0]) * qs[0, 0] * ks[:, 0]


@pytest.mark.parametrize("Dh", [256, 512])
@pytest.mark.parametrize("below", [0.5, 2.0])
def test_many_keys_just_outside_the_rescoring_band(ctx, Dh, below):
    # Adversarial case for the approximate scores: one key scores 30, the other 2047 all score
    # 30 - tau - `below` (just outside the exact-rescoring band, so each keeps its estimate,
    # whose error delta is ~1e-5), and each such key's V row is sign(delta) in every dim, so all
    # their errors push every output the same way. 16 queries x 8 heads share one q row.
    # Aggregate bound: |d out| <= max|delta| * (W_out / l) * max|v - out|, W_out / l the weight
    # share of the keys that keep their estimate.
    S, T = 2048, 16
    tau = rescoring_band(S)
    q0 = synth.rms_norm_rows(synth.normal_f32(71, 0, Dh).reshape(1, Dh))[0].astype(np.float64)
    r = synth.normal_f32(71, 1, S * Dh).reshape(S, Dh).astype(np.float64)
    r -= np.outer(r @ q0, q0) / (q0 @ q0)  # orthogonal to q0
    target = np.full(S, 30.0 - tau - below)
    target[0] = 30.0
    k = (np.outer(target / (q0 @ q0), q0) + r).astype(np.float32).reshape(S, 1, Dh)
    q = np.broadcast_to(q0.astype(np.float32), (T, 8, Dh)).copy()
    # the oracle's exact f32 scores, and the estimate's error per key
    seq = np.zeros(S, np.float32)
    for d in range(Dh):
        seq = (seq + (np.float32(q0[d]) * k[:, 0, d]).astype(np.float32)).astype(np.float32)
    delta = _split_scores(q0.astype(np.float32), k[:, 0, :]) - seq.astype(np.float64)
    assert np.abs(seq[1:] - target[1:]).max() < 1e-3 and abs(seq[0] - 30.0) < 1e-3
    v = np.repeat(np.sign(delta)[:, None], Dh, axis=1).astype(np.float32).reshape(S, 1, Dh)
    v[0] = 0.0
    ins = synth.AttnInputs(q, k, v, np.arange(S - T, S, dtype=np.uint32), np.arange(S, dtype=np.uint32))
    w_out = (S - T) * np.exp(-(tau + below))
    share = w_out / (1.0 + w_out)
    print(f"  outside-band weight share {share:.3e}, |delta| mean {np.abs(delta[1:]).mean():.2e} "
          f"max {np.abs(delta[1:]).max():.2e}; bound {np.abs(delta).max() * share * 2:.2e}", flush=True)
    run(ctx, ins, 0, f"2047 keys at max - tau - {below}, V = sign(score error), Dh {Dh}")
