"""Two contexts driven from two host threads at once, through the C-ABI. A
context is not thread-safe (like the reference backend, whose state sits in a
RefCell: rust/src/backend_wgpu.rs:241), but separate contexts share nothing a
call writes: each has its own stream, module, workspace, staging buffers and
tables. Each thread here runs its own mix of calls (short and streaming decode,
prefill, the producer, a projection) many times over while the other does the
same, and every result must equal the one the same calls give on one thread,
bit for bit."""
import threading

import numpy as np
import pytest

import g4a
import g4a.synth as synth
import oracle

pytestmark = pytest.mark.gpu

ROUNDS = 30


class Work:
    """One thread's calls on its own context: device inputs, outputs, and a run()
    that enqueues them all; results() reads the outputs back."""

    def __init__(self, ctx, seed):
        self.ctx, self.bufs = ctx, []
        dec = synth.gemma_inputs(T=1, S=8192, Dh=512, seed=seed)            # short decode, 256 splits
        glob = synth.gemma_inputs(T=1, S=40000, Dh=512, seed=seed + 1)      # streaming decode
        pre = synth.gemma_inputs(T=300, S=300, Dh=256, seed=seed + 2, q_pos=np.arange(300))  # prefill
        self.calls = []
        for ins, window in ((dec, 0), (glob, 0), (pre, 512)):
            q, k, v = (self.up(x) for x in (ins.q, ins.k, ins.v))
            T, Hq, Dh = ins.q.shape
            out = self.empty((T, Hq * Dh))
            self.calls.append(dict(q=q.ptr, k=k.ptr, v=v.ptr, out=out.ptr, T=T, S=ins.k.shape[0], Hq=Hq, Hkv=1,
                                   Dh=Dh, Dv=Dh, q_pos0=int(ins.q_pos[0]), k_pos0=0, window=window))
        self.outs = [c["out"] for c in self.calls]
        self.out_shapes = [(c["T"], c["Hq"] * c["Dh"]) for c in self.calls]
        qb, sc, _ = synth.quant_weight(seed + 3, 2048, 1536, 4)
        self.w = ctx.upload_qweight(qb, sc, 2048, 1536, 4)
        self.x = self.up(synth.normal_f32(seed + 4, 0, 1536).reshape(1, 1536))
        self.y = self.empty((1, 2048))
        w_h = (np.float32(1.0) + np.float32(0.1) * synth.normal_f32(seed + 5, 0, 256)).astype(np.float32)
        self.pq = self.up(synth.normal_f32(seed + 6, 0, 8 * 256).reshape(1, 8, 256))
        self.pk = self.up(synth.normal_f32(seed + 7, 0, 256).reshape(1, 1, 256))
        self.pv = self.up(synth.normal_f32(seed + 8, 0, 256).reshape(1, 1, 256))
        self.pw = self.up(w_h)
        self.pqo = self.empty((1, 8, 256))
        self.kc, self.vc = self.empty((512, 1, 256)), self.empty((512, 1, 256))
        for cache in (self.kc, self.vc):  # rows the producer does not write are compared too
            ctx.zero(cache.ptr, cache.nbytes)

    def up(self, x):
        d = self.ctx.upload(np.ascontiguousarray(x, np.float32))
        self.bufs.append(d)
        return d

    def empty(self, shape):
        d = self.ctx.empty(shape)
        self.bufs.append(d)
        return d

    def run(self):
        c = self.ctx
        for kw in self.calls:
            kw = dict(kw)
            c.attention(kw.pop("q"), kw.pop("k"), kw.pop("v"), kw.pop("out"), **kw)
        c.linear_q(self.w, self.x.ptr, self.y.ptr, 1)
        c.attn_producer(q=self.pq.ptr, k=self.pk.ptr, v=self.pv.ptr, q_norm=self.pw.ptr, k_norm=self.pw.ptr,
                        q_out=self.pqo.ptr, k_cache=self.kc.ptr, v_cache=self.vc.ptr, T=1, Hq=8, Hkv=1, Dh=256,
                        rotary_dim=256, pos0=33000, cache_row=33000, ring_cap=512, theta=1e4, eps=1e-6)

    def results(self):
        self.ctx.sync()
        outs = [self._host(p, s) for p, s in zip(self.outs, self.out_shapes)]
        return outs + [self.y.to_host(), self.pqo.to_host(), self.kc.to_host(), self.vc.to_host()]

    def _host(self, ptr, shape):
        h = np.empty(shape, np.float32)
        self.ctx.d2h(h, ptr)
        return h

    def free(self):
        self.w.free()
        for b in self.bufs:
            b.free()


def test_two_contexts_on_two_threads():
    ctxs = [g4a.Context(0), g4a.Context(0)]
    works = [Work(ctxs[0], 100), Work(ctxs[1], 200)]
    try:
        # each context's results on its own, one thread
        want = []
        for wk in works:
            wk.run()
            want.append(wk.results())
        print("[gpu] single-thread results taken; two threads now", flush=True)
        errors = []
        start = threading.Barrier(2)

        def thread(i):
            try:
                start.wait()
                for r in range(ROUNDS):
                    works[i].run()
                    got = works[i].results()
                    for j, (g, w) in enumerate(zip(got, want[i])):
                        if not np.array_equal(g, w):
                            errors.append(f"context {i} round {r} output {j} differs")
                            return
            except Exception as e:  # reported by the main thread
                errors.append(f"context {i}: {e!r}")

        ts = [threading.Thread(target=thread, args=(i,)) for i in range(2)]
        for t in ts:
            t.start()
        for t in ts:
            t.join(timeout=120)
        assert not any(t.is_alive() for t in ts), "a thread did not finish"
        assert not errors, errors[:4]
        # and the single-thread results are right
        ins = synth.gemma_inputs(T=1, S=8192, Dh=512, seed=100)
        d = np.abs(want[0][0].astype(np.float64) - oracle.attention(ins.q, ins.k, ins.v, ins.q_pos, ins.k_pos))
        assert d.max() <= 1e-5 and d.mean() <= 1e-6
        print(f"  {ROUNDS} rounds per thread, every output bit-identical to its single-thread result", flush=True)
    finally:
        for wk in works:
            wk.free()
        for c in ctxs:
            c.close()
