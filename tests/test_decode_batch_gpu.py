"""GPU parity of the batched decode entry point (g4a_attention_decode_batch:
many independent single-query steps per launch of the short-context or the
streaming decode kernel, 64 sequences per launch, descriptors in the kernel
arguments) through the C-ABI. Each batched step must equal the CPU oracle
(rust/src/backend_cpu.rs:270-336 restated in oracle/attn_oracle.c) to max-abs
<= 1e-5, mean-abs <= 1e-6 (f32), and where the batch runs the short kernel,
the single g4a_attention call bit for bit. Covers both kernels, batches across
the 64-sequence launch boundary, ragged lengths, windows, wrapping rings, the
32768-key limit, explicit non-contiguous key positions, calls that must not
batch, scale and soft-cap, two kv heads and argument errors."""
import numpy as np
import pytest

import g4a
import g4a.synth as synth
import oracle

pytestmark = pytest.mark.gpu

MAX_ABS = 1e-5
MEAN_ABS = 1e-6


def assert_parity(got, want, label):
    d = np.abs(got.astype(np.float64) - np.asarray(want, np.float64))
    mx, mean = float(d.max()), float(d.mean())
    assert mx <= MAX_ABS and mean <= MEAN_ABS, f"{label}: max-abs {mx:.3e} mean-abs {mean:.3e}"
    return mx


def step(msg):
    print(f"[gpu] {msg}", flush=True)


class Seq:
    """One decode step: a query at position L-1 over keys 0..L-1, held linearly or
    in a ring of `cap` rows (row = position % cap). Only the keys the step can
    see are generated (the last `window` positions, or all); the rest of the
    cache stays zero."""

    def __init__(self, c, L, Dh, seed, window=0, cap=0, Hkv=1, scale=1.0, softcap=0.0):
        self.c, self.L, self.Dh, self.window, self.cap, self.Hkv = c, L, Dh, window, cap, Hkv
        self.scale, self.softcap = scale, softcap
        nv = min(L, window) if window else L
        ins = synth.gemma_inputs(T=1, S=nv, Dh=Dh, seed=seed, Hq=8 * Hkv, Hkv=Hkv)
        self.q = ins.q
        self.k_vis, self.v_vis = ins.k, ins.v
        self.k_pos = np.arange(L - nv, L, dtype=np.uint32)
        rows = cap if cap else L
        k = np.zeros((rows, Hkv, Dh), np.float32)
        v = np.zeros((rows, Hkv, Dh), np.float32)
        idx = self.k_pos % cap if cap else self.k_pos
        k[idx] = self.k_vis
        v[idx] = self.v_vis
        self.dev = [c.upload(x) for x in (self.q, k, v)]
        self.out = c.empty((1, 8 * Hkv * Dh))
        c.zero(self.out.ptr, self.out.nbytes)

    def kw(self):
        return dict(q=self.dev[0].ptr, k=self.dev[1].ptr, v=self.dev[2].ptr, out=self.out.ptr, T=1, S=self.L,
                    Hq=8 * self.Hkv, Hkv=self.Hkv, Dh=self.Dh, Dv=self.Dh, q_pos0=self.L - 1, k_pos0=0,
                    window=self.window, ring_cap=self.cap, scale=self.scale, softcap=self.softcap)

    def want(self):
        return oracle.attention(self.q, self.k_vis, self.v_vis, np.array([self.L - 1], np.uint32), self.k_pos,
                                window=self.window, scale=self.scale, softcap=self.softcap)

    def single(self):
        """The same step through g4a_attention, into a fresh output."""
        out = self.c.empty((1, 8 * self.Hkv * self.Dh))
        try:
            kw = self.kw()
            q, k, v = kw.pop("q"), kw.pop("k"), kw.pop("v")
            kw.pop("out")
            self.c.attention(q, k, v, out.ptr, **kw)
            return out.to_host()
        finally:
            out.free()

    def free(self):
        for d in self.dev:
            d.free()
        self.out.free()


def _run(c, seqs, expect_batched, label):
    step(f"{label}: {len(seqs)} calls")
    n = c.attention_decode_batch([s.kw() for s in seqs])
    assert n == expect_batched, f"{label}: {n} batched, expected {expect_batched}"
    worst = 0.0
    for i, s in enumerate(seqs):
        worst = max(worst, assert_parity(s.out.to_host(), s.want(), f"{label} call {i} L={s.L} Dh={s.Dh}"))
    print(f"  {label}: max-abs {worst:.3e} over {len(seqs)} calls", flush=True)


def _same_as_single_calls(c, seqs, label):
    """Each batched result equals the single call's bit for bit (the short
    kernel with the same 32-key splits in both)."""
    step(f"{label}: single-call comparison")
    for i, s in enumerate(seqs):
        kw = s.kw()
        for key in ("q", "k", "v", "out"):
            kw.pop(key)
        assert g4a.KERNEL_NAMES[c.plan(**kw).kernel] == "decode_short"
        assert np.array_equal(s.single(), s.out.to_host()), f"{label} call {i} L={s.L}: batched != single call"


def _free(seqs):
    for s in seqs:
        s.free()


def test_short_kernel_batches_match_single_calls(ctx):
    """Batches whose 32-key splits fit one workgroup per CU run the short
    kernel: ragged sliding-window steps in wrapping 512-slot rings, hd512 full
    attention, and 70 tiny steps over two launches (64 + 6)."""
    c = ctx
    lens = [1, 2, 15, 16, 17, 31, 32, 33, 511, 512, 513, 1000]
    seqs = [Seq(c, L, 256, seed=200 + i, window=512, cap=512) for i, L in enumerate(lens)]
    try:
        _run(c, seqs, len(seqs), "local rings")
        _same_as_single_calls(c, seqs, "local rings")
    finally:
        _free(seqs)
    seqs = [Seq(c, L, 512, seed=230 + i) for i, L in enumerate([7, 100, 2047, 4099])]
    try:
        _run(c, seqs, len(seqs), "global")
        _same_as_single_calls(c, seqs, "global")
    finally:
        _free(seqs)
    rng = np.random.default_rng(5)
    seqs = [Seq(c, int(L), 256, seed=240 + i, window=512, cap=512) for i, L in enumerate(rng.integers(1, 33, 70))]
    try:
        _run(c, seqs, len(seqs), "two launches")
        _same_as_single_calls(c, seqs, "two launches")
    finally:
        _free(seqs)


def test_streaming_kernel_batches(ctx):
    """Batches too large for one short-kernel round run the streaming kernel:
    100 sliding-window steps of contexts up to 40000 in 512-slot rings (two
    launches: 64 + 36), and hd512 full attention up to the 32768-key limit
    (1024 short splits); a 32769-key step runs as a single call."""
    c = ctx
    rng = np.random.default_rng(8)
    lens = [1, 32, 511, 512, 513, 40000] + [int(x) for x in rng.integers(1, 40000, 94)]
    seqs = [Seq(c, L, 256, seed=300 + i, window=512, cap=512) for i, L in enumerate(lens)]
    try:
        _run(c, seqs, len(seqs), "local rings, two launches")
    finally:
        _free(seqs)
    seqs = [Seq(c, L, 512, seed=400 + i) for i, L in enumerate([7, 100, 4099, 8192, 12345, 32768])]
    try:
        _run(c, seqs, len(seqs), "global long")
    finally:
        _free(seqs)
    seqs = [Seq(c, 32769, 512, seed=410), Seq(c, 3000, 512, seed=411)]
    try:
        _run(c, seqs, 1, "past the key limit")
    finally:
        _free(seqs)


def test_calls_that_do_not_batch_run_as_single_calls(ctx):
    """Multi-query steps, another head dim than the first batched call, a fixed
    split count and group 4 are run by g4a_attention; the batched ones keep
    their results, among them a step with explicit non-contiguous key positions
    (a launch of its own beside the contiguous ones)."""
    c = ctx
    a = Seq(c, 700, 256, seed=400, window=512)
    b = Seq(c, 900, 512, seed=401)          # other Dh than the first batched call
    d = Seq(c, 1200, 256, seed=402, window=512)
    ins_t = synth.gemma_inputs(T=3, S=800, Dh=256, seed=403)
    ins_g4 = synth.gemma_inputs(T=1, S=300, Dh=256, seed=404, Hq=4, Hkv=1)
    ins_kp = synth.gemma_inputs(T=1, S=500, Dh=256, seed=405)
    kp = np.arange(500, dtype=np.uint32) * 2  # every other position
    qp = np.array([998], np.uint32)
    extra = []
    try:
        dev_t = [c.upload(x) for x in (ins_t.q, ins_t.k, ins_t.v)] + [c.empty((3, 8 * 256))]
        dev_g4 = [c.upload(x) for x in (ins_g4.q, ins_g4.k, ins_g4.v)] + [c.empty((1, 4 * 256))]
        dev_kp = [c.upload(x) for x in (ins_kp.q, ins_kp.k, ins_kp.v)] + [c.empty((1, 8 * 256))]
        dev_fs = a.dev + [c.empty((1, 8 * 256))]
        extra = dev_t + dev_g4 + dev_kp + dev_fs[3:]
        calls = [
            a.kw(),
            dict(q=dev_t[0].ptr, k=dev_t[1].ptr, v=dev_t[2].ptr, out=dev_t[3].ptr, T=3, S=800, Hq=8, Hkv=1, Dh=256,
                 Dv=256, q_pos0=797, k_pos0=0, window=512),
            b.kw(),
            dict(q=dev_g4[0].ptr, k=dev_g4[1].ptr, v=dev_g4[2].ptr, out=dev_g4[3].ptr, T=1, S=300, Hq=4, Hkv=1,
                 Dh=256, Dv=256, q_pos0=299, k_pos0=0),
            dict(q=dev_kp[0].ptr, k=dev_kp[1].ptr, v=dev_kp[2].ptr, out=dev_kp[3].ptr, T=1, S=500, Hq=8, Hkv=1,
                 Dh=256, Dv=256, q_pos=qp, k_pos=kp, window=512),
            dict(q=dev_fs[0].ptr, k=dev_fs[1].ptr, v=dev_fs[2].ptr, out=dev_fs[3].ptr, T=1, S=700, Hq=8, Hkv=1,
                 Dh=256, Dv=256, q_pos0=699, k_pos0=0, window=512, splits=3),
            d.kw(),
        ]
        step("mixed batch")
        assert c.attention_decode_batch(calls) == 3  # a, the explicit positions and d
        assert_parity(a.out.to_host(), a.want(), "batched a")
        assert_parity(d.out.to_host(), d.want(), "batched d")
        assert_parity(b.out.to_host(), b.want(), "other head dim")
        assert_parity(dev_t[3].to_host(), oracle.attention(ins_t.q, ins_t.k, ins_t.v, ins_t.q_pos, ins_t.k_pos,
                                                           window=512), "three queries")
        assert_parity(dev_g4[3].to_host(), oracle.attention(ins_g4.q, ins_g4.k, ins_g4.v, ins_g4.q_pos,
                                                            ins_g4.k_pos), "group 4")
        assert_parity(dev_kp[3].to_host(), oracle.attention(ins_kp.q, ins_kp.k, ins_kp.v, qp, kp, window=512),
                      "explicit key positions")
        assert_parity(dev_fs[3].to_host(), a.want(), "fixed splits")
    finally:
        for s in (a, b, d):
            s.free()
        for x in extra:
            x.free()


def test_scale_softcap_and_two_kv_heads(ctx):
    c = ctx
    for scale, cap in [(0.0625, 0.0), (1.0, 30.0)]:
        seqs = [Seq(c, L, 512, seed=500 + L, scale=scale, softcap=cap) for L in (5, 600, 2100)]
        try:
            _run(c, seqs, 3, f"scale={scale} softcap={cap}")
        finally:
            for s in seqs:
                s.free()
    seqs = [Seq(c, L, 256, seed=600 + L, window=512, Hkv=2, cap=512) for L in (3, 400, 1500, 700)]
    try:
        _run(c, seqs, 4, "two kv heads")
        _same_as_single_calls(c, seqs, "two kv heads")
    finally:
        _free(seqs)
    seqs = [Seq(c, L, 512, seed=650 + L, Hkv=2) for L in (3000, 5000, 9000, 100)]
    try:
        _run(c, seqs, 4, "two kv heads, streaming")
    finally:
        _free(seqs)


def test_argument_errors_enqueue_nothing(ctx):
    c = ctx
    seqs = [Seq(c, L, 256, seed=700 + L, window=512) for L in (100, 200)]
    try:
        for s in seqs:
            c.h2d(s.out.ptr, np.full((1, 8 * 256), np.nan, np.float32))
        bad = dict(seqs[1].kw(), Hkv=3)  # 8 query heads over 3 kv heads
        with pytest.raises(g4a.G4aError) as e:
            c.attention_decode_batch([seqs[0].kw(), bad])
        assert "call 1" in str(e.value)
        c.sync()
        assert np.all(np.isnan(seqs[0].out.to_host()))  # the valid call did not run either
        assert c.attention_decode_batch([]) == 0
    finally:
        for s in seqs:
            s.free()


def test_positions_offset_from_the_cache_start(ctx):
    """Key j at position k_pos0 + j with k_pos0 > 0 (a cache that starts
    mid-sequence): only position differences enter, so the steps give the
    results of the same steps at k_pos0 = 0."""
    c = ctx
    for label, Dh, window, lens in [("short", 256, 512, (5, 300, 900)), ("streaming", 512, 0, (3000, 9000, 20000))]:
        seqs = [Seq(c, L, Dh, seed=800 + L, window=window) for L in lens]
        try:
            calls = [dict(s.kw(), k_pos0=7000, q_pos0=7000 + s.L - 1) for s in seqs]
            step(f"offset positions, {label}")
            assert c.attention_decode_batch(calls) == len(seqs)
            for s in seqs:
                assert_parity(s.out.to_host(), s.want(), f"offset {label} L={s.L}")
        finally:
            _free(seqs)


class KposSeq:
    """A decode step over a linear cache whose S keys sit at explicit ascending
    positions with holes (gaps of 1-3: evicted or padded slots); the query sits
    at `q_at` (an index into the positions, plus 0-2), so the keys after it are
    cut off, and a window cuts the cache's start."""

    def __init__(self, c, S, Dh, seed, window, q_at, rng):
        self.c, self.window = c, window
        ins = synth.gemma_inputs(T=1, S=S, Dh=Dh, seed=seed)
        self.q, self.k, self.v = ins.q, ins.k, ins.v
        self.k_pos = np.cumsum(rng.integers(1, 4, S)).astype(np.uint32)
        self.q_pos = np.array([int(self.k_pos[q_at]) + int(rng.integers(0, 3))], np.uint32)
        self.S, self.Dh = S, Dh
        self.dev = [c.upload(x) for x in (self.q, self.k, self.v)]
        self.out = c.empty((1, 8 * Dh))
        c.zero(self.out.ptr, self.out.nbytes)

    def kw(self):
        return dict(q=self.dev[0].ptr, k=self.dev[1].ptr, v=self.dev[2].ptr, out=self.out.ptr, T=1, S=self.S,
                    Hq=8, Hkv=1, Dh=self.Dh, Dv=self.Dh, q_pos=self.q_pos, k_pos=self.k_pos, window=self.window)

    def want(self):
        return oracle.attention(self.q, self.k, self.v, self.q_pos, self.k_pos, window=self.window)

    def free(self):
        for d in self.dev:
            d.free()
        self.out.free()


def test_explicit_key_positions_batch(ctx):
    """Steps whose keys sit at explicit, ascending, non-contiguous positions
    batch in streaming-kernel launches of their own, beside contiguous steps of
    the same shape in the same call: 70 hd256 sliding-window steps (two
    launches, 64 + 6) whose windows start far into their caches and whose
    queries sit before their last keys, then hd512 full attention up to the
    32768-key limit, where a step over 32769 visible keys runs as a single
    call."""
    c = ctx
    rng = np.random.default_rng(12)
    sizes = [1, 2, 17, 300, 1000, 5000] + [int(x) for x in rng.integers(1, 6000, 64)]
    seqs = [KposSeq(c, S, 256, 900 + i, 512, int(rng.integers(S // 2, S)), rng) for i, S in enumerate(sizes)]
    contig = [Seq(c, L, 256, seed=980 + i, window=512) for i, L in enumerate((40, 700, 3000))]
    try:
        step("explicit positions, hd256 window 512: 70 + 3 contiguous calls")
        assert c.attention_decode_batch([contig[0].kw()] + [s.kw() for s in seqs] +
                                        [x.kw() for x in contig[1:]]) == len(seqs) + len(contig)
        worst = 0.0
        for i, s in enumerate(seqs):
            worst = max(worst, assert_parity(s.out.to_host(), s.want(), f"explicit call {i} S={s.S}"))
        for s in contig:
            assert_parity(s.out.to_host(), s.want(), f"contiguous L={s.L}")
        print(f"  explicit positions hd256: max-abs {worst:.3e}", flush=True)
    finally:
        _free(seqs)
        _free(contig)
    seqs = [KposSeq(c, S, 512, 990 + i, 0, qa, rng)
            for i, (S, qa) in enumerate([(64, 63), (4099, 4000), (20000, 12345), (32768, 32767), (32769, 32768)])]
    try:
        step("explicit positions, hd512 global")
        assert c.attention_decode_batch([s.kw() for s in seqs]) == 4
        for s in seqs:
            assert_parity(s.out.to_host(), s.want(), f"explicit hd512 S={s.S}")
    finally:
        _free(seqs)
