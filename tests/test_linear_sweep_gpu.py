"""A seeded random sweep of the quantised projections (g4a_linear_q,
g4a_linear_q_geglu, g4a_linear_q_gelu_mul_cols) through the C-ABI against the
CPU oracle (rust/src/backend_cpu.rs:174-222 and the trait's compositions
rust/src/backend.rs:156-168, restated in oracle/linear_oracle.c).

The draws mix what the fixed cases take one at a time: 2-, 4- and 8-bit
weights (offset binary or I8), row counts that are not multiples of any tile,
row lengths from one word per lane to several LDS strides and ones that are not
whole words, grouped scales, 1 to 100 activation rows (the word kernel's 1- and
4-row forms, the half-wave 2-bit form, the int8 and bf16 matrix-core kernels)
and the three epilogues. Bars as in tests/test_linear_gpu.py: per output
|gpu - oracle| <= 2e-6 * sum_k |x_k w_nk| + 1e-7 (another f32 summation
order), carried through gelu for the fused forms; bit-identity where the
element kernel (the CPU's order) must run. The draws come from one seed."""
import numpy as np
import pytest

import g4a.synth as synth
import oracle
from test_linear_gpu import Dev, _bound, _check_fused, _check_sum, _qw

pytestmark = pytest.mark.gpu

N_CASES = 40
KS = [32, 64, 256, 512, 1536, 1536, 2048, 3584, 4096, 6144, 52, 99, 1000]


def draw_case(rng, i):
    bits, signed = [(2, False), (4, False), (4, False), (8, True), (8, False)][rng.integers(5)]
    K = int(rng.choice(KS))
    while (K * bits) % 8:  # rows are whole bytes
        K = int(rng.choice(KS))
    M = int(rng.choice([1, 1, 1, 2, 3, 5, 16, 17, 33, 64, 100]))
    N = int(rng.choice([1, 7, 255, 256, 1000, 1536, 2048, 4099, int(rng.integers(1, 5000))]))
    while M * N * K > 3e8:  # keep the single-threaded oracle to about a second
        N = max(1, N // 2)
    group = int(rng.choice([64, 128])) if rng.random() < 0.2 and K % 64 == 0 else None
    op = str(rng.choice(["linear", "linear", "geglu", "gelu_cols"]))
    return dict(i=i, bits=bits, signed=signed, K=K, M=M, N=N, group=group, op=op)


CASES = [draw_case(np.random.default_rng(3000 + i), i) for i in range(N_CASES)]


def label(c):
    return (f"case {c['i']}: {c['op']} b{c['bits']}{'s' if c['signed'] else ''} N={c['N']} K={c['K']} M={c['M']} "
            f"group={c['group']}")


def _element_only(c):
    """Shapes only the element kernel (the CPU's order) takes: rows that are not
    whole 32-bit words, or more than one scale group per row."""
    return (c["K"] * c["bits"]) % 32 != 0 or (c["group"] is not None and c["group"] < c["K"])


@pytest.mark.parametrize("c", CASES, ids=[f"case{c['i']}" for c in CASES])
def test_random_projection_shape(ctx, c):
    name = label(c)
    print(f"[gpu] {name}", flush=True)
    N, K, M, bits, seed = c["N"], c["K"], c["M"], c["bits"], 9000 + c["i"]
    w = _qw(seed, N, K, bits, c["signed"], c["group"])
    x = synth.normal_f32(seed, 1, M * K).reshape(M, K)
    with Dev(ctx) as d:
        dw, dx, y = d.w(w), d.arr(x), d.empty((M, N))
        if c["op"] == "linear":
            ctx.linear_q(dw, dx.ptr, y.ptr, M)
            got, want = y.to_host(), oracle.linear_q(x, w)
            _check_sum(got, want, _bound(x, w), name)
            if _element_only(c):
                assert np.array_equal(got, want), f"{name}: the element kernel is not bit-identical"
        elif c["op"] == "geglu":
            w2 = _qw(seed + 1, N, K, bits, c["signed"], c["group"])
            ctx.linear_q_geglu(dw, d.w(w2), dx.ptr, y.ptr, M)
            _check_fused(y.to_host(), x, w, w2, None, 0, name)
        else:
            width = N + 3 * 64
            off = int(np.random.default_rng(seed).integers(0, width - N + 1))
            b = synth.normal_f32(seed, 2, M * width).reshape(M, width)
            ctx.linear_q_gelu_mul_cols(dw, dx.ptr, d.arr(b).ptr, width, off, y.ptr, M)
            _check_fused(y.to_host(), x, w, None, b, off, name)
