"""Two Gemma-4 decoder layers composed from the trait's ops on the GPU through
the C-ABI, as Gemma4Model composes them (rust/src/model.rs:142-206 forward,
:207-245 decoder_layer, :247-304 attention), against the same composition
through the CPU oracle. Layer 0 slides (Dh 256, window 512, full RoPE, a
520-slot ring cache: a T-token chunk needs window + T - 1 rows, which the
library checks); layer 1 is global (Dh 512, partial RoPE 0.25, a linear
cache). Gemma-4-E2B widths (hidden 1536, 8 query heads over 1 kv head, GeGLU
6144, per-layer inputs 256), 4-bit projections and embeddings, a 2-bit lm_head,
random weights.

As the reference's full_model_parity (rust/tests/gpu.rs:190-227): a 5-token
prefill, then decode steps that append to the caches, the logits of each pass
compared. A second run starts the caches with 516 rows of history (the same
random K/V on both sides), so the decode steps wrap the sliding layer's ring
and its oldest keys leave the window.
Bar: the reference's own, max |d| < 5e-3 (rust/tests/gpu.rs:200).
The composition reorders no sum beyond the individual ops' (each pinned
elsewhere), so the test also holds the logits to 1e-4 relative to their
largest magnitude and prints the achieved difference."""
import numpy as np
import pytest

import g4a.synth as synth
import oracle

pytestmark = pytest.mark.gpu

H, HQ, HKV, I, DPLE, L, V, EPS = 1536, 8, 1, 6144, 256, 2, 300, 1e-6
LAYERS = [dict(dh=256, window=512, theta=10000.0, rot=256, ring=520),
          dict(dh=512, window=0, theta=1000000.0, rot=128, ring=0)]


def step(msg):
    print(f"[gpu] {msg}", flush=True)


def _norm_w(seed, n):
    return (np.float32(1.0) + np.float32(0.1) * synth.normal_f32(seed, 0, n)).astype(np.float32)


def make_weights():
    seed = iter(range(1000, 2000))
    q = lambda N, K, bits=4: (synth.quant_weight(next(seed), N, K, bits)[:2], N, K, bits)  # noqa: E731
    w = {"embed": q(V, H), "embed_pl": q(V, L * DPLE), "ple_proj": q(L * DPLE, H),
         "ple_proj_norm": _norm_w(next(seed), DPLE), "final_norm": _norm_w(next(seed), H), "lm_head": q(V, H, 2),
         "layers": []}
    for lc in LAYERS:
        dh = lc["dh"]
        w["layers"].append({
            "input_ln": _norm_w(next(seed), H), "post_attn_ln": _norm_w(next(seed), H),
            "pre_ffn_ln": _norm_w(next(seed), H), "post_ffn_ln": _norm_w(next(seed), H),
            "q_norm": _norm_w(next(seed), dh), "k_norm": _norm_w(next(seed), dh), "ple_norm": _norm_w(next(seed), H),
            "layer_scalar": np.array([0.75], np.float32),
            "q_proj": q(HQ * dh, H), "k_proj": q(HKV * dh, H), "v_proj": q(HKV * dh, H), "o_proj": q(H, HQ * dh),
            "gate": q(I, H), "up": q(I, H), "down": q(H, I), "ple_gate": q(DPLE, H), "ple_proj": q(H, DPLE),
        })
    return w


class CpuModel:
    """The composition through the oracle (host arrays)."""

    def __init__(self, w, hist):
        qw = lambda t: oracle.QWeight(t[0][0], t[0][1], t[1], t[2], t[3])  # noqa: E731
        self.w = {k: (qw(v) if isinstance(v, tuple) else v) for k, v in w.items() if k != "layers"}
        self.layers = [{k: (qw(v) if isinstance(v, tuple) else v) for k, v in lw.items()} for lw in w["layers"]]
        self.k = [h[0] for h in hist]
        self.v = [h[1] for h in hist]

    def attention(self, i, x, pos):
        lc, lw, T = LAYERS[i], self.layers[i], x.shape[0]
        dh = lc["dh"]
        q = oracle.linear_q(x, lw["q_proj"]).reshape(T, HQ, dh)
        k = oracle.linear_q(x, lw["k_proj"]).reshape(T, HKV, dh)
        v = oracle.linear_q(x, lw["v_proj"]).reshape(T, HKV, dh)
        q, k, v = oracle.producer(q, k, v, lw["q_norm"], lw["k_norm"], pos, lc["theta"], lc["rot"], EPS)
        self.k[i] = np.concatenate([self.k[i], k])
        self.v[i] = np.concatenate([self.v[i], v])
        S = self.k[i].shape[0]
        out = oracle.attention(q, self.k[i], self.v[i], pos, np.arange(S, dtype=np.uint32), scale=1.0,
                               window=lc["window"])
        return oracle.linear_q(out, lw["o_proj"])

    def forward(self, ids, pos):
        w, T = self.w, len(ids)
        h = oracle.embed_rows_q(w["embed"], ids, float(np.sqrt(np.float32(H))))
        emb = oracle.embed_rows_q(w["embed_pl"], ids, float(np.sqrt(np.float32(DPLE))))
        proj = oracle.linear_q(h, w["ple_proj"]).reshape(T * L, DPLE)
        proj = oracle.rms_norm(proj, w["ple_proj_norm"], EPS).reshape(T, L * DPLE)
        ple = oracle.scale(oracle.add(proj, emb), float(np.float32(np.sqrt(0.5))))
        for i, lw in enumerate(self.layers):
            attn = self.attention(i, oracle.rms_norm(h, lw["input_ln"], EPS), pos)
            h = oracle.add_rms_norm(h, attn, lw["post_attn_ln"], EPS)
            ff = oracle.linear_q_geglu(oracle.rms_norm(h, lw["pre_ffn_ln"], EPS), lw["gate"], lw["up"])
            h = oracle.add_rms_norm(h, oracle.linear_q(ff, lw["down"]), lw["post_ffn_ln"], EPS)
            inj = oracle.linear_q(oracle.linear_q_gelu_mul_cols(h, lw["ple_gate"], ple, i * DPLE), lw["ple_proj"])
            h = oracle.add_rms_norm(h, inj, lw["ple_norm"], EPS, lw["layer_scalar"][0])
        h = oracle.rms_norm(h, w["final_norm"], EPS)
        return oracle.linear_q(h[T - 1:], w["lm_head"])


class GpuModel:
    """The same composition on the GPU: every op a C-ABI call on device buffers."""

    def __init__(self, c, w, hist):
        self.c, self.keep = c, []
        up = lambda t: self._keep(c.upload_qweight(t[0][0], t[0][1], t[1], t[2], t[3]))  # noqa: E731
        dev = lambda a: self._keep(c.upload(a))  # noqa: E731
        self.w = {k: (up(v) if isinstance(v, tuple) else dev(v)) for k, v in w.items() if k != "layers"}
        self.layers = [{k: (up(v) if isinstance(v, tuple) else dev(v)) for k, v in lw.items()} for lw in w["layers"]]
        n = hist[0][0].shape[0]
        rows = [lc["ring"] or n + 16 for lc in LAYERS]
        self.kc = [self._keep(c.empty((r, HKV, lc["dh"]))) for r, lc in zip(rows, LAYERS)]
        self.vc = [self._keep(c.empty((r, HKV, lc["dh"]))) for r, lc in zip(rows, LAYERS)]
        self.tmp = []
        for i, lc in enumerate(LAYERS):  # the history rows, through the cache write (ring slots wrap)
            if n:
                for cache, src in ((self.kc[i], hist[i][0]), (self.vc[i], hist[i][1])):
                    d = self.buf(*src.shape)
                    c.h2d(d.ptr, np.ascontiguousarray(src))
                    c.kv_write(cache.ptr, lc["ring"], HKV * lc["dh"], 0, d.ptr, n)
        self.len = n

    def _keep(self, d):
        self.keep.append(d)
        return d

    def buf(self, *shape):
        d = self.c.empty(shape)
        self.tmp.append(d)
        return d

    def lin(self, wq, x, M, N):
        y = self.buf(M, N)
        self.c.linear_q(wq, x.ptr, y.ptr, M)
        return y

    def rms(self, x, w, rows, dim):
        y = self.buf(rows, dim)
        self.c.rms_norm(x.ptr, w.ptr, y.ptr, rows=rows, dim=dim, eps=EPS)
        return y

    def add_rms(self, res, x, w, rows, scale_by=None):
        y = self.buf(rows, H)
        self.c.add_rms_norm(res.ptr, x.ptr, w.ptr, scale_by.ptr if scale_by else 0, y.ptr, rows, H, EPS)
        return y

    def attention(self, i, x, T, pos0):
        c, lc, lw = self.c, LAYERS[i], self.layers[i]
        dh = lc["dh"]
        q = self.lin(lw["q_proj"], x, T, HQ * dh)
        k = self.lin(lw["k_proj"], x, T, HKV * dh)
        v = self.lin(lw["v_proj"], x, T, HKV * dh)
        qo = self.buf(T, HQ, dh)
        c.attn_producer(q=q.ptr, k=k.ptr, v=v.ptr, q_norm=lw["q_norm"].ptr, k_norm=lw["k_norm"].ptr, q_out=qo.ptr,
                        k_cache=self.kc[i].ptr, v_cache=self.vc[i].ptr, T=T, Hq=HQ, Hkv=HKV, Dh=dh,
                        rotary_dim=lc["rot"], pos0=pos0, cache_row=self.len, ring_cap=lc["ring"],
                        theta=lc["theta"], eps=EPS)
        out = self.buf(T, HQ * dh)
        c.attention(qo.ptr, self.kc[i].ptr, self.vc[i].ptr, out.ptr, T=T, S=self.len + T, Hq=HQ, Hkv=HKV, Dh=dh,
                    Dv=dh, q_pos0=pos0, k_pos0=0, window=lc["window"], ring_cap=lc["ring"])
        return self.lin(lw["o_proj"], out, T, H)

    def forward(self, ids, pos0):
        c, w, T = self.c, self.w, len(ids)
        h = self.buf(T, H)
        c.embed_rows_q(w["embed"], ids, float(np.sqrt(np.float32(H))), h.ptr)
        emb = self.buf(T, L * DPLE)
        c.embed_rows_q(w["embed_pl"], ids, float(np.sqrt(np.float32(DPLE))), emb.ptr)
        proj = self.lin(w["ple_proj"], h, T, L * DPLE)
        proj = self.rms(proj, w["ple_proj_norm"], T * L, DPLE)
        ple = self.buf(T, L * DPLE)
        c.ew("add", proj.ptr, ple.ptr, T * L * DPLE, b=emb.ptr)
        c.ew("scale", ple.ptr, ple.ptr, T * L * DPLE, s=float(np.float32(np.sqrt(0.5))))
        for i, lw in enumerate(self.layers):
            attn = self.attention(i, self.rms(h, lw["input_ln"], T, H), T, pos0)
            h = self.add_rms(h, attn, lw["post_attn_ln"], T)
            ff = self.buf(T, I)
            c.linear_q_geglu(lw["gate"], lw["up"], self.rms(h, lw["pre_ffn_ln"], T, H).ptr, ff.ptr, T)
            h = self.add_rms(h, self.lin(lw["down"], ff, T, H), lw["post_ffn_ln"], T)
            g = self.buf(T, DPLE)
            c.linear_q_gelu_mul_cols(lw["ple_gate"], h.ptr, ple.ptr, L * DPLE, i * DPLE, g.ptr, T)
            h = self.add_rms(h, self.lin(lw["ple_proj"], g, T, H), lw["ple_norm"], T, scale_by=lw["layer_scalar"])
        self.len += T
        last = self.rms(h, w["final_norm"], T, H)
        logits = self.buf(1, V)
        last_row = last.ptr + (T - 1) * H * 4
        c.linear_q(w["lm_head"], last_row, logits.ptr, 1)
        out = logits.to_host()
        for d in self.tmp:
            d.free()
        self.tmp = []
        return out

    def free(self):
        for d in self.keep:
            d.free()


def _check(got, want, label):
    d = float(np.abs(got.astype(np.float64) - want.astype(np.float64)).max())
    top = float(np.abs(want).max())
    print(f"  {label}: max |d| {d:.3e} (logits up to {top:.3e})", flush=True)
    assert d < 5e-3, f"{label}: max diff {d:e} (reference bar 5e-3)"
    assert d <= 1e-4 * max(top, 1.0), f"{label}: max diff {d:e} above 1e-4 of the largest logit"


@pytest.mark.parametrize("history", [0, 516])
def test_two_layer_prefill_then_incremental_decode(ctx, history):
    w = make_weights()
    hist = []
    for i, lc in enumerate(LAYERS):
        n, dh = history * HKV * lc["dh"], lc["dh"]
        hist.append((synth.normal_f32(3000 + i, 0, n).reshape(history, HKV, dh),
                     synth.normal_f32(3000 + i, 1, n).reshape(history, HKV, dh)))
    cpu, gpu = CpuModel(w, hist), GpuModel(ctx, w, hist)
    try:
        ids = [2, 5, 11, 19, 30]
        step(f"history {history}: prefill T=5")
        _check(gpu.forward(ids, history), cpu.forward(ids, np.arange(history, history + 5, dtype=np.uint32)),
               f"history {history} prefill logits")
        for n, tok in enumerate([44, 7, 299]):
            p = history + 5 + n
            step(f"history {history}: decode step at position {p}")
            _check(gpu.forward([tok], p), cpu.forward([tok], np.array([p], np.uint32)), f"decode pos {p}")
    finally:
        gpu.free()
