"""GPU parity of the trait's remaining ops through the C-ABI (g4a_add, g4a_mul,
g4a_scale, g4a_scale_by_tensor, g4a_gelu_tanh, g4a_geglu, g4a_softcap,
g4a_slice_cols, g4a_rms_norm on wide rows, g4a_add_rms_norm, g4a_embed_rows,
g4a_linear) against the CPU oracle (rust/src/backend_cpu.rs:127-350 and
rust/src/backend.rs:136-168 restated in oracle/), on the reference's own
kernel_parity / fused_op_parity inputs and Gemma-4 widths.

Bars, per op:
  - add, mul, scale, scale_by_tensor, slice_cols, embed_rows: bit-identical;
  - gelu_tanh, geglu, softcap: the device tanhf may differ from libm's in the
    last bits: |d| <= 2.5e-7 |x| (* |b|) + 5e-7 |want| (gelu's 1 + tanh cancels
    for negative x, so the bound scales with x, not with the result);
  - rms_norm / add_rms_norm: the sum of squares is reduced in another order:
    |d| <= 2e-6 |norm part| + 2e-7 |want| + 1e-7;
  - linear (f32 and quantised): |d| <= 2e-6 sum_k |x_k w_nk| + 1e-7 (reordered
    sum), the element kernels bit-identical.
"""
import numpy as np
import pytest

import g4a
import g4a.synth as synth
import oracle
from golden_io import load_ops_golden
from test_linear_gpu import _bound, _check_fused, _check_sum

pytestmark = pytest.mark.gpu


def step(msg):
    print(f"[gpu] {msg}", flush=True)


class Dev:
    def __init__(self, c):
        self.c, self.bufs = c, []

    def arr(self, a):
        d = self.c.upload(np.ascontiguousarray(a))
        self.bufs.append(d)
        return d

    def empty(self, shape):
        d = self.c.empty(shape)
        self.bufs.append(d)
        return d

    def qw(self, a, p, prefix):
        d = self.c.upload_qweight(a[prefix + "qbytes"], a[prefix + "scales"], p[prefix + "N"], p[prefix + "K"],
                                  p[prefix + "bits"], p[prefix + "signed_i8"])
        self.bufs.append(d)
        return d

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        for b in self.bufs:
            b.free()


def _ow(a, p, prefix):
    return oracle.QWeight(a[prefix + "qbytes"], a[prefix + "scales"], p[prefix + "N"], p[prefix + "K"],
                          p[prefix + "bits"], p[prefix + "signed_i8"])


def run_op(c, case):
    """The op on the GPU; returns the host result."""
    a, p, op = case.arrays, case.params, case.op
    with Dev(c) as d:
        if op in ("add", "mul", "gelu_tanh", "geglu", "softcap", "scale", "scale_by_tensor"):
            x = a["a"]
            y = d.empty(x.shape)
            b = d.arr(a["b"]).ptr if "b" in a else (d.arr(a["s"]).ptr if "s" in a else 0)
            c.ew(op, d.arr(x).ptr, y.ptr, x.size, b=b, s=p.get("s", p.get("cap", 0.0)))
            return y.to_host()
        if op == "slice_cols":
            x = a["x"]
            y = d.empty((x.shape[0], p["width"]))
            c.slice_cols(d.arr(x).ptr, x.shape[0], x.shape[1], p["offset"], p["width"], y.ptr)
            return y.to_host()
        if op == "rms_norm":
            x = a["x"]
            y = d.empty(x.shape)
            c._check(c.lib.g4a_rms_norm(c.handle, d.arr(x).ptr, d.arr(a["w"]).ptr, y.ptr, x.shape[0], x.shape[1],
                                        p["eps"]))
            return y.to_host()
        if op == "add_rms_norm":
            x = a["x"]
            y = d.empty(x.shape)
            s = d.arr(a["s"]).ptr if "s" in a else 0
            c.add_rms_norm(d.arr(a["res"]).ptr, d.arr(x).ptr, d.arr(a["w"]).ptr, s, y.ptr, x.shape[0], x.shape[1],
                           p["eps"])
            return y.to_host()
        if op == "embed_rows":
            t = a["table"]
            y = d.empty((a["ids"].size, t.shape[1]))
            c.embed_rows(d.arr(t).ptr, t.shape[0], t.shape[1], a["ids"], p["scale"], y.ptr)
            return y.to_host()
        if op == "linear_f32":
            x, w = a["x"], a["w"]
            y = d.empty((x.shape[0], w.shape[0]))
            c.linear(d.arr(w).ptr, w.shape[0], w.shape[1], d.arr(x).ptr, y.ptr, x.shape[0])
            return y.to_host()
        x = a["x"]
        n = p["w_N"]
        y = d.empty((x.shape[0], n))
        if op == "linear_q":
            c.linear_q(d.qw(a, p, "w_"), d.arr(x).ptr, y.ptr, x.shape[0])
        elif op == "geglu_q":
            c.linear_q_geglu(d.qw(a, p, "w_"), d.qw(a, p, "u_"), d.arr(x).ptr, y.ptr, x.shape[0])
        else:
            c.linear_q_gelu_mul_cols(d.qw(a, p, "w_"), d.arr(x).ptr, d.arr(a["b"]).ptr, a["b"].shape[1], p["offset"],
                                     y.ptr, x.shape[0])
        return y.to_host()


def check(case, got, want, label):
    a, p, op = case.arrays, case.params, case.op
    g64, w64 = got.astype(np.float64), np.asarray(want, np.float64)
    if op in ("add", "mul", "scale", "scale_by_tensor", "slice_cols", "embed_rows"):
        assert np.array_equal(got, want), label
        return
    if op in ("gelu_tanh", "geglu", "softcap"):
        x = np.abs(a["a"].astype(np.float64))
        tol = (2.5e-7 * x * (np.abs(a["b"]) if op == "geglu" else 1.0) if op != "softcap" else 0.0) + \
            5e-7 * np.abs(w64) + 1e-38
        err = np.abs(g64 - w64)
        assert np.all(err <= tol), f"{label}: max-abs {err.max():.3e}"
        return
    if op in ("rms_norm", "add_rms_norm"):
        norm = w64 - (a["res"].astype(np.float64) if "res" in a else 0.0)
        if "s" in a:
            norm = w64 / float(a["s"][0]) - a["res"].astype(np.float64)
        tol = 2e-6 * np.abs(norm) * (float(a["s"][0]) if "s" in a else 1.0) + 2e-7 * np.abs(w64) + 1e-7
        err = np.abs(g64 - w64)
        assert np.all(err <= tol), f"{label}: max-abs {err.max():.3e}"
        return
    if op == "linear_f32":
        K = a["x"].shape[1]
        if K % 4 == 0 and -(-K // 64) * 64 <= 16384:
            bound = np.abs(a["x"].astype(np.float64)) @ np.abs(a["w"].astype(np.float64)).T
            err = np.abs(g64 - w64)
            assert np.all(err <= 2e-6 * bound + 1e-7), f"{label}: max-abs {err.max():.3e}"
        else:
            assert np.array_equal(got, want), f"{label}: element kernel not bit-exact"
        return
    w = _ow(a, p, "w_")
    if op == "linear_q":
        _check_sum(got, want, _bound(a["x"], w), label)
    elif op == "geglu_q":
        _check_fused(got, a["x"], w, _ow(a, p, "u_"), None, 0, label)
    else:
        _check_fused(got, a["x"], w, None, a["b"], p["offset"], label)


def test_golden_fixtures(ctx):
    for name, case in load_ops_golden().items():
        step(name)
        check(case, run_op(ctx, case), case.out, name)


def test_large_and_ragged_sizes(ctx):
    """Element counts that are not multiples of the grid, grid-stride loops over
    millions of elements, rows wider than one wave's 1024, odd widths, K past the
    word kernel's limit (element kernel, bit-exact)."""
    c = ctx
    from golden_io import OpCase
    n = 3 * 1024 * 1024 + 7
    a, b = synth.normal_f32(70, 0, n) * np.float32(3.0), synth.normal_f32(70, 1, n)
    for op in ("add", "mul", "geglu", "softcap"):
        case = OpCase(op, {"a": a, "b": b} if op != "softcap" else {"a": a}, {"cap": 2.0} if op == "softcap" else {})
        step(f"{op} n={n}")
        want = {"add": oracle.add, "mul": oracle.mul, "geglu": oracle.geglu}[op](a, b) if op != "softcap" \
            else oracle.softcap(a, 2.0)
        check(case, run_op(c, case), want, f"{op} n={n}")
    for rows, dim in [(7, 1536), (3, 1537), (2, 4096), (1, 9000)]:
        x = synth.normal_f32(71, rows, rows * dim).reshape(rows, dim) * np.float32(2.0)
        res = synth.normal_f32(72, rows, rows * dim).reshape(rows, dim)
        w = (np.float32(1.0) + np.float32(0.1) * synth.normal_f32(73, 0, dim)).astype(np.float32)
        for case in (OpCase("rms_norm", {"x": x, "w": w}, {"eps": 1e-6}),
                     OpCase("add_rms_norm", {"res": res, "x": x, "w": w, "s": np.array([1.25], np.float32)},
                            {"eps": 1e-6})):
            step(f"{case.op} [{rows}, {dim}]")
            check(case, run_op(c, case), oracle.add_rms_norm(res, x, w, 1e-6, np.float32(1.25))
                  if case.op == "add_rms_norm" else oracle.rms_norm(x, w, 1e-6), f"{case.op} [{rows}, {dim}]")
    for M, N, K in [(1, 2048, 1536), (3, 300, 2048), (17, 64, 4096), (2, 40, 16448), (2, 33, 1538)]:
        x = synth.normal_f32(74, M, M * K).reshape(M, K)
        w = (synth.normal_f32(75, N, N * K) * np.float32(0.05)).reshape(N, K)
        case = OpCase("linear_f32", {"x": x, "w": w}, {})
        step(f"linear f32 M={M} N={N} K={K}")
        check(case, run_op(c, case), oracle.linear_f32(x, w), f"linear f32 M={M} N={N} K={K}")
    table = synth.normal_f32(76, 0, 5000 * 1536).reshape(5000, 1536)
    ids = np.array([0, 4999, 2500, 2500, 17], np.uint32)
    case = OpCase("embed_rows", {"table": table, "ids": ids}, {"scale": float(np.sqrt(np.float32(1536)))})
    step("embed [5000, 1536]")
    check(case, run_op(c, case), oracle.embed_rows_f32(table, ids, float(np.sqrt(np.float32(1536)))), "embed")


def test_argument_errors(ctx):
    c = ctx
    with Dev(c) as d:
        x = d.arr(np.zeros((2, 10), np.float32))
        y = d.empty((2, 10))
        with pytest.raises(g4a.G4aError, match="exceed the row stride"):
            c.slice_cols(x.ptr, 2, 10, 5, 6, y.ptr)
        with pytest.raises(g4a.G4aError, match="outside the table"):
            c.embed_rows(x.ptr, 2, 10, [2], 1.0, y.ptr)
        with pytest.raises(g4a.G4aError, match="null"):
            c.ew("add", x.ptr, y.ptr, 20)  # no second operand
        c.ew("add", x.ptr, y.ptr, 0, b=x.ptr)  # n = 0: nothing to do
