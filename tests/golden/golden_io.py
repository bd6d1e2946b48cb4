"""Golden attention vectors: recipes that regenerate the inputs, plus the
committed oracle outputs (attention_golden.npz, written by make_golden.py).

The reference stores no golden vectors (its parity tests compare GPU and CPU
on seeded inputs, rust/tests/gpu.rs:262-293), so the fixtures here are:
  - the inputs of the reference's own attention parity cases, regenerated
    bit-exactly from its Lcg (rust/tests/common/mod.rs:29-42), with the CPU
    oracle's outputs;
  - small seeded Gaussian cases of the benchmark distribution (unit-RMS q/k,
    scale 1.0) at the real head shapes, decode and prefill, global and sliding.
They pin regressions of the oracle and of the GPU path against the same data.
"""
from __future__ import annotations

import hashlib
from dataclasses import dataclass
from pathlib import Path

import numpy as np

import g4a.synth as synth

GOLDEN_PATH = Path(__file__).resolve().parent / "attention_golden.npz"
NORM_ROPE_GOLDEN_PATH = Path(__file__).resolve().parent / "norm_rope_golden.npz"


@dataclass
class Case:
    q: np.ndarray
    k: np.ndarray
    v: np.ndarray
    q_pos: np.ndarray
    k_pos: np.ndarray
    scale: float
    window: int
    softcap: float = 0.0
    out: np.ndarray | None = None


def input_hash(c: Case) -> str:
    h = hashlib.sha256()
    for a in (c.q, c.k, c.v, c.q_pos, c.k_pos):
        h.update(np.ascontiguousarray(a).tobytes())
    h.update(np.array([c.scale, c.window, c.softcap], np.float64).tobytes())
    return h.hexdigest()


def recipes() -> dict[str, Case]:
    cases: dict[str, Case] = {}
    for (t, s, hq, hkv, dh, w), q, k, v, qp, kp, scale, window in synth.grouped_parity_inputs():
        cases[f"grouped_T{t}_S{s}_Hq{hq}_Hkv{hkv}_Dh{dh}_w{w}"] = Case(q, k, v, qp, kp, scale, window)
    for name, q, k, v, qp, kp, scale, window in synth.kernel_parity_attention_inputs():
        key = "kernel_parity_" + name.replace("(", "_").replace(")", "").replace(",", "_").replace("=", "").replace(" ", "")
        cases[key] = Case(q, k, v, qp, kp, scale, window)
    # benchmark distribution at the real head shapes (small S so the oracle is instant)
    g = synth.gemma_inputs(T=1, S=512, Dh=256, seed=0)
    cases["gauss_decode_sliding_Dh256_S512"] = Case(g.q, g.k, g.v, g.q_pos, g.k_pos, 1.0, 512)
    g = synth.gemma_inputs(T=1, S=1000, Dh=512, seed=1)
    cases["gauss_decode_global_Dh512_S1000"] = Case(g.q, g.k, g.v, g.q_pos, g.k_pos, 1.0, 0)
    g = synth.gemma_inputs(T=20, S=20, Dh=256, seed=3, q_pos=np.arange(20))
    cases["gauss_prefill_sliding_Dh256_T20_w8"] = Case(g.q, g.k, g.v, g.q_pos, g.k_pos, 1.0, 8)
    g = synth.gemma_inputs(T=8, S=8, Dh=512, seed=3, q_pos=np.arange(8))
    cases["gauss_prefill_global_Dh512_T8"] = Case(g.q, g.k, g.v, g.q_pos, g.k_pos, 1.0, 0)
    return cases


def load_golden() -> dict[str, Case]:
    data = np.load(GOLDEN_PATH, allow_pickle=False)
    cases = recipes()
    for name, c in cases.items():
        assert str(data[name + "__hash"]) == input_hash(c), f"{name}: regenerated inputs differ from the fixture's"
        c.out = data[name + "__out"]
    return cases


# ---- the attention producer: rms_norm, rope, head_norm_rope ----------------

@dataclass
class NormRopeCase:
    """op in {"rms_norm", "rope", "head_norm_rope"}; x [T, heads, Dh] (rms_norm: [rows, 1, d])."""
    op: str
    x: np.ndarray
    w: np.ndarray | None
    positions: np.ndarray
    theta: float
    rotary_dim: int
    eps: float
    out: np.ndarray | None = None


def norm_rope_hash(c: NormRopeCase) -> str:
    h = hashlib.sha256(c.op.encode())
    for a in (c.x, c.w if c.w is not None else np.zeros(0, np.float32), c.positions):
        h.update(np.ascontiguousarray(a).tobytes())
    h.update(np.array([c.theta, c.rotary_dim, c.eps], np.float64).tobytes())
    return h.hexdigest()


def norm_rope_recipes() -> dict[str, NormRopeCase]:
    """The reference's own cases, regenerated from its Lcg (rust/tests/common/mod.rs:29-42):
      - kernel_parity's rmsNorm and rope(partial) (rust/tests/gpu.rs:53-59, :84-90; seed 7,
        earlier draws skipped by count: linear 17*40 + 23*40 + 40, then rmsNorm 5*48 + 48,
        elementwise 100 + 100, embed 30*16);
      - fused_op_parity's head_norm_rope cases (rust/tests/gpu.rs:322-334; seed 33 after
        add_rms_norm's 5*48 + 5*48 + 48 draws), positions i*7 + 3, theta 1e4, eps 1e-6;
    and seeded Gaussian Gemma-4 shapes: the sliding layer (Dh 256, theta 1e4, full
    rotation) and the global layer (Dh 512, theta 1e6, partial_rotary_factor 0.25 -> 128
    dims, rust/assets/config.json) at positions up to 131071, where the angle is large."""
    cases: dict[str, NormRopeCase] = {}
    r = synth.Lcg(7)
    r.skip(17 * 40 + 23 * 40 + 40)
    x = r.rand(5 * 48, 1.0).reshape(5, 1, 48)
    w = r.rand(48, 0.1)
    cases["kernel_parity_rmsNorm"] = NormRopeCase("rms_norm", x, w, np.zeros(0, np.uint32), 0.0, 0, 1e-6)
    cases["kernel_parity_rmsNorm_unweighted"] = NormRopeCase("rms_norm", x, None, np.zeros(0, np.uint32), 0.0, 0,
                                                             1e-6)
    r.skip(100 + 100 + 30 * 16)
    x = r.rand(4 * 2 * 16, 1.0).reshape(4, 2, 16)
    cases["kernel_parity_rope_partial"] = NormRopeCase("rope", x, None, np.array([0, 1, 5, 9], np.uint32), 1e4, 8,
                                                       0.0)
    r = synth.Lcg(33)
    r.skip(5 * 48 + 5 * 48 + 48)
    for t, heads, dh, rot in [(3, 4, 16, 8), (2, 8, 256, 256), (2, 1, 512, 128)]:
        x = r.rand(t * heads * dh, 1.0).reshape(t, heads, dh)
        w = r.rand(dh, 0.1)
        pos = (np.arange(t, dtype=np.uint32) * 7 + 3).astype(np.uint32)
        cases[f"fused_op_head_norm_rope_h{heads}_d{dh}_r{rot}"] = NormRopeCase("head_norm_rope", x, w, pos, 1e4, rot,
                                                                               1e-6)
    for name, t, heads, dh, theta, rot, p0, seed in [
        ("gemma_sliding_q_T1_pos32767", 1, 8, 256, 1e4, 256, 32767, 40),
        ("gemma_global_q_T1_pos32767", 1, 8, 512, 1e6, 128, 32767, 41),
        ("gemma_global_k_T3_pos131069", 3, 1, 512, 1e6, 128, 131069, 42),
        ("gemma_sliding_k_T6_pos1000", 6, 1, 256, 1e4, 256, 1000, 43),
    ]:
        x = (synth.normal_f32(seed, 0, t * heads * dh) * np.float32(2.0)).reshape(t, heads, dh)
        w = (np.float32(1.0) + np.float32(0.1) * synth.normal_f32(seed, 1, dh)).astype(np.float32)
        pos = np.arange(p0, p0 + t, dtype=np.uint32)
        cases[name] = NormRopeCase("head_norm_rope", x, w, pos, theta, rot, 1e-6)
    return cases


def norm_rope_eval(c: NormRopeCase, oracle) -> np.ndarray:
    """The oracle's output for a recipe."""
    if c.op == "rms_norm":
        return oracle.rms_norm(c.x.reshape(c.x.shape[0], -1), c.w, c.eps).reshape(c.x.shape)
    if c.op == "rope":
        return oracle.rope(c.x, c.positions, c.theta, c.rotary_dim)
    return oracle.head_norm_rope(c.x, c.w, c.eps, c.positions, c.theta, c.rotary_dim)


def load_norm_rope_golden() -> dict[str, NormRopeCase]:
    data = np.load(NORM_ROPE_GOLDEN_PATH, allow_pickle=False)
    cases = norm_rope_recipes()
    for name, c in cases.items():
        assert str(data[name + "__hash"]) == norm_rope_hash(c), f"{name}: regenerated inputs differ from the fixture's"
        c.out = data[name + "__out"]
    return cases


# ---- quantised projections ----------------------------------------------------

LINEAR_GOLDEN_PATH = Path(__file__).resolve().parent / "linear_golden.npz"


@dataclass
class LinearCase:
    op: str                  # linear | geglu | gelu_mul_cols | embed
    w: dict                  # qbytes, scales, N, K, bits, signed_i8, group_size
    x: np.ndarray | None     # [M, K] (linear ops)
    w2: dict | None = None   # geglu: the up weight
    b: np.ndarray | None = None
    b_off: int = 0
    ids: np.ndarray | None = None
    scale: float = 1.0
    out: np.ndarray | None = None


def _qw_bytes(h, w: dict) -> None:
    h.update(np.ascontiguousarray(w["qbytes"], np.uint8).tobytes())
    h.update(np.ascontiguousarray(w["scales"], np.float32).tobytes())
    h.update(np.array([w["N"], w["K"], w["bits"], int(w["signed_i8"]), w["group_size"]], np.int64).tobytes())


def linear_hash(c: LinearCase) -> str:
    h = hashlib.sha256(c.op.encode())
    _qw_bytes(h, c.w)
    if c.w2 is not None:
        _qw_bytes(h, c.w2)
    for a in (c.x, c.b, c.ids):
        if a is not None:
            h.update(np.ascontiguousarray(a).tobytes())
    h.update(np.array([c.b_off, c.scale], np.float64).tobytes())
    return h.hexdigest()


def _qw(qbytes, scales, N, K, bits, signed_i8=False, group_size=None) -> dict:
    return dict(qbytes=np.ascontiguousarray(qbytes, np.uint8).ravel(), scales=np.ascontiguousarray(scales, np.float32),
                N=N, K=K, bits=bits, signed_i8=signed_i8, group_size=group_size or K)


def linear_recipes() -> dict[str, LinearCase]:
    """The reference's quantized_kernel_parity inputs (rust/tests/gpu.rs:146-190),
    regenerated from its Lcg(9) stream: q4 and q2 linear at M = 5 and 1, q4 with
    K = 52 (not whole words), I8, and the grouped-scale q4 embedding. Then seeded
    cases of this build for the fused epilogues and Gemma-4 shapes (q_proj 4-bit
    [2048, 1536] at M = 1, a 2-bit GeGLU [256, 1536] pair at M = 3, the per-layer
    gate [256, 1536] times a column slice at M = 2, grouped-scale linear)."""
    cases: dict[str, LinearCase] = {}
    for c in synth.quant_parity_inputs():
        w = _qw(c["qbytes"], c["scales"], c["N"], c["K"], c["bits"], c["signed_i8"], c["group_size"])
        if "ids" in c:
            cases["ref_" + c["name"]] = LinearCase("embed", w, None, ids=c["ids"], scale=c["scale"])
        else:
            cases["ref_" + c["name"]] = LinearCase("linear", w, c["x"])
    qb, sc, g = synth.quant_weight(51, 2048, 1536, 4)
    cases["gemma_q_proj_q4_M1"] = LinearCase("linear", _qw(qb, sc, 2048, 1536, 4), synth.normal_f32(51, 9, 1536)
                                             .reshape(1, 1536))
    qg, sg, _ = synth.quant_weight(52, 256, 1536, 2)
    qu, su, _ = synth.quant_weight(53, 256, 1536, 2)
    cases["geglu_q2_M3"] = LinearCase("geglu", _qw(qg, sg, 256, 1536, 2), synth.normal_f32(52, 9, 3 * 1536)
                                      .reshape(3, 1536), w2=_qw(qu, su, 256, 1536, 2))
    qb, sc, _ = synth.quant_weight(54, 256, 1536, 4)
    b = synth.normal_f32(54, 8, 2 * 35 * 256).reshape(2, 35 * 256)
    cases["gelu_mul_cols_q4_M2"] = LinearCase("gelu_mul_cols", _qw(qb, sc, 256, 1536, 4),
                                              synth.normal_f32(54, 9, 2 * 1536).reshape(2, 1536), b=b, b_off=7 * 256)
    qb, sc, g = synth.quant_weight(55, 96, 256, 4, group_size=64)
    cases["linear_q4_grouped64_M2"] = LinearCase("linear", _qw(qb, sc, 96, 256, 4, group_size=g),
                                                 synth.normal_f32(55, 9, 2 * 256).reshape(2, 256))
    return cases


def oracle_qweight(oracle, w: dict):
    return oracle.QWeight(w["qbytes"], w["scales"], w["N"], w["K"], w["bits"], w["signed_i8"], w["group_size"])


def linear_eval(c: LinearCase, oracle) -> np.ndarray:
    """The oracle's output for a recipe."""
    w = oracle_qweight(oracle, c.w)
    if c.op == "linear":
        return oracle.linear_q(c.x, w)
    if c.op == "geglu":
        return oracle.linear_q_geglu(c.x, w, oracle_qweight(oracle, c.w2))
    if c.op == "gelu_mul_cols":
        return oracle.linear_q_gelu_mul_cols(c.x, w, c.b, c.b_off)
    return oracle.embed_rows_q(w, c.ids, c.scale)


def load_linear_golden() -> dict[str, LinearCase]:
    data = np.load(LINEAR_GOLDEN_PATH, allow_pickle=False)
    cases = linear_recipes()
    for name, c in cases.items():
        assert str(data[name + "__hash"]) == linear_hash(c), f"{name}: regenerated inputs differ from the fixture's"
        c.out = data[name + "__out"]
    return cases


# ---- the rest of the trait's ops ----------------------------------------------

OPS_GOLDEN_PATH = Path(__file__).resolve().parent / "backend_ops_golden.npz"


@dataclass
class OpCase:
    op: str            # add mul scale scale_by_tensor gelu_tanh geglu softcap slice_cols rms_norm
                       # add_rms_norm embed_rows linear_f32 | linear_q geglu_q gelu_mul_cols_q
    arrays: dict       # named input arrays
    params: dict       # named scalars
    out: np.ndarray | None = None


def op_hash(c: OpCase) -> str:
    h = hashlib.sha256(c.op.encode())
    for k in sorted(c.arrays):
        h.update(k.encode())
        h.update(np.ascontiguousarray(c.arrays[k]).tobytes())
    for k in sorted(c.params):
        h.update(f"{k}={c.params[k]!r}".encode())
    return h.hexdigest()


def _lcg_qw(r, n, k, bits):
    """fused_op_parity's qw closure (rust/tests/gpu.rs:303-308)."""
    vals = (np.floor(r.next(n * k) * np.float32(1 << bits)).astype(np.uint32) % (1 << bits)).astype(np.uint32)
    scales = (r.next(n) * np.float32(0.05) + np.float32(0.01)).astype(np.float32)
    return dict(qbytes=synth.pack_unsigned(vals, bits), scales=scales, N=n, K=k, bits=bits, signed_i8=False,
                group_size=k)


def _lcg_i8(r, n, k):
    qbytes = np.floor(r.next(n * k) * np.float32(256.0)).astype(np.uint32).astype(np.uint8)
    scales = (r.next(n) * np.float32(0.05) + np.float32(0.01)).astype(np.float32)
    return dict(qbytes=qbytes, scales=scales, N=n, K=k, bits=8, signed_i8=True, group_size=k)


def _qw_arrays(prefix, w):
    return {prefix + "qbytes": w["qbytes"], prefix + "scales": w["scales"]}, \
        {prefix + "N": w["N"], prefix + "K": w["K"], prefix + "bits": w["bits"], prefix + "signed_i8": w["signed_i8"]}


def ops_recipes() -> dict[str, OpCase]:
    """The reference's kernel_parity (rust/tests/gpu.rs:37-100, Lcg seed 7) and
    fused_op_parity (rust/tests/gpu.rs:298-375, Lcg seed 33) cases for the
    trait's remaining ops, regenerated in the same draw order, plus seeded
    Gemma-4-width cases of this build (hidden 1536 post-norms, the per-layer
    projection slice, an f32 projection)."""
    cases: dict[str, OpCase] = {}
    r = synth.Lcg(7)
    m, k, n = 17, 40, 23
    x, w = r.rand(m * k, 1.0).reshape(m, k), r.rand(n * k, 1.0).reshape(n, k)
    cases["kp_linear_tiled"] = OpCase("linear_f32", {"x": x, "w": w}, {})
    x1 = r.rand(k, 1.0).reshape(1, k)
    cases["kp_linear_gemv"] = OpCase("linear_f32", {"x": x1, "w": w}, {})
    t, d = 5, 48
    x, w = r.rand(t * d, 1.0).reshape(t, d), r.rand(d, 0.1)
    cases["kp_rmsNorm"] = OpCase("rms_norm", {"x": x, "w": w}, {"eps": 1e-6})
    nn = 100
    a, b = r.rand(nn, 1.0), r.rand(nn, 1.0)
    cases["kp_add"] = OpCase("add", {"a": a, "b": b}, {})
    cases["kp_mul"] = OpCase("mul", {"a": a, "b": b}, {})
    cases["kp_scale"] = OpCase("scale", {"a": a}, {"s": 3.5})
    cases["kp_geluTanh"] = OpCase("gelu_tanh", {"a": a}, {})
    cases["kp_geglu"] = OpCase("geglu", {"a": a, "b": b}, {})
    cases["kp_softcap"] = OpCase("softcap", {"a": (a * np.float32(50.0)).astype(np.float32)}, {"cap": 30.0})
    cases["kp_scaleByTensor"] = OpCase("scale_by_tensor", {"a": a, "s": np.array([0.37], np.float32)}, {})
    cases["kp_gelu_large"] = OpCase("gelu_tanh", {"a": np.array([1000.0, -1000.0, 50.0], np.float32)}, {})
    v, d = 30, 16
    table = r.rand(v * d, 1.0).reshape(v, d)
    cases["kp_embedRows"] = OpCase("embed_rows", {"table": table, "ids": np.array([3, 7, 0, 29, 12], np.uint32)},
                                   {"scale": 4.0})
    r.skip(4 * 2 * 16)  # rope(partial)
    rows, stride = 4, 20
    x = r.rand(rows * stride, 1.0).reshape(rows, stride)
    cases["kp_sliceCols"] = OpCase("slice_cols", {"x": x}, {"offset": 5, "width": 7})

    r = synth.Lcg(33)
    t, d = 5, 48
    x, res, w = r.rand(t * d, 1.0).reshape(t, d), r.rand(t * d, 1.0).reshape(t, d), r.rand(d, 0.1)
    cases["fo_add_rms_norm"] = OpCase("add_rms_norm", {"res": res, "x": x, "w": w}, {"eps": 1e-6})
    cases["fo_add_rms_norm_scalar"] = OpCase("add_rms_norm", {"res": res, "x": x, "w": w,
                                                              "s": np.array([1.37], np.float32)}, {"eps": 1e-6})
    r.skip(3 * 4 * 16 + 16 + 2 * 8 * 256 + 256 + 2 * 1 * 512 + 512)  # head_norm_rope cases
    for bits in (2, 4, 8):
        qn, qk = 70, 96
        wq = _lcg_i8(r, qn, qk) if bits == 8 else _lcg_qw(r, qn, qk, bits)
        for mm in (8, 9, 64, 70):
            x = r.rand(mm * qk, 1.0).reshape(mm, qk)
            arr, par = _qw_arrays("w_", wq)
            cases[f"fo_linear_q{bits}_M{mm}"] = OpCase("linear_q", dict(arr, x=x), par)
    for bits in (2, 4):
        qn, qk = 40, 64
        wg, wu = _lcg_qw(r, qn, qk, bits), _lcg_qw(r, qn, qk, bits)
        for mm in (1, 4, 9, 40):
            x = r.rand(mm * qk, 1.0).reshape(mm, qk)
            ag, pg = _qw_arrays("w_", wg)
            au, pu = _qw_arrays("u_", wu)
            cases[f"fo_linear_geglu_q{bits}_M{mm}"] = OpCase("geglu_q", dict(ag, **au, x=x), dict(pg, **pu))
    qn, qk, stride, off = 24, 32, 96, 48
    wi = _lcg_i8(r, qn, qk)
    for mm in (1, 6, 33):
        x = r.rand(mm * qk, 1.0).reshape(mm, qk)
        bb = r.rand(mm * stride, 1.0).reshape(mm, stride)
        arr, par = _qw_arrays("w_", wi)
        cases[f"fo_linear_gelu_mul_cols_i8_M{mm}"] = OpCase("gelu_mul_cols_q", dict(arr, x=x, b=bb),
                                                            dict(par, offset=off))

    # Gemma-4 widths (hidden 1536, 35 layers x 256 per-layer inputs)
    h = (synth.normal_f32(60, 0, 3 * 1536) * np.float32(4.0)).reshape(3, 1536)
    res = synth.normal_f32(60, 1, 3 * 1536).reshape(3, 1536)
    wn = (np.float32(1.0) + np.float32(0.1) * synth.normal_f32(60, 2, 1536)).astype(np.float32)
    cases["gemma_post_norm_layer_scalar"] = OpCase("add_rms_norm", {"res": res, "x": h, "w": wn,
                                                                    "s": np.array([0.71], np.float32)}, {"eps": 1e-6})
    cases["gemma_final_norm"] = OpCase("rms_norm", {"x": h, "w": wn}, {"eps": 1e-6})
    ple = synth.normal_f32(61, 0, 2 * 35 * 256).reshape(2, 35 * 256)
    cases["gemma_ple_slice"] = OpCase("slice_cols", {"x": ple}, {"offset": 17 * 256, "width": 256})
    wf = (synth.normal_f32(62, 0, 256 * 1536) * np.float32(0.03)).reshape(256, 1536)
    cases["gemma_f32_projection_M2"] = OpCase("linear_f32", {"x": synth.normal_f32(62, 1, 2 * 1536).reshape(2, 1536),
                                                             "w": wf}, {})
    return cases


def _qw_from(arrays, params, prefix, oracle):
    return oracle.QWeight(arrays[prefix + "qbytes"], arrays[prefix + "scales"], params[prefix + "N"],
                          params[prefix + "K"], params[prefix + "bits"], params[prefix + "signed_i8"])


def ops_eval(c: OpCase, oracle) -> np.ndarray:
    a, p = c.arrays, c.params
    if c.op == "add":
        return oracle.add(a["a"], a["b"])
    if c.op == "mul":
        return oracle.mul(a["a"], a["b"])
    if c.op == "scale":
        return oracle.scale(a["a"], p["s"])
    if c.op == "scale_by_tensor":
        return oracle.scale(a["a"], a["s"][0])
    if c.op == "gelu_tanh":
        return oracle.gelu_tanh(a["a"])
    if c.op == "geglu":
        return oracle.geglu(a["a"], a["b"])
    if c.op == "softcap":
        return oracle.softcap(a["a"], p["cap"])
    if c.op == "slice_cols":
        return oracle.slice_cols(a["x"], p["offset"], p["width"])
    if c.op == "rms_norm":
        return oracle.rms_norm(a["x"], a["w"], p["eps"])
    if c.op == "add_rms_norm":
        return oracle.add_rms_norm(a["res"], a["x"], a["w"], p["eps"], a["s"][0] if "s" in a else None)
    if c.op == "embed_rows":
        return oracle.embed_rows_f32(a["table"], a["ids"], p["scale"])
    if c.op == "linear_f32":
        return oracle.linear_f32(a["x"], a["w"])
    if c.op == "linear_q":
        return oracle.linear_q(a["x"], _qw_from(a, p, "w_", oracle))
    if c.op == "geglu_q":
        return oracle.linear_q_geglu(a["x"], _qw_from(a, p, "w_", oracle), _qw_from(a, p, "u_", oracle))
    return oracle.linear_q_gelu_mul_cols(a["x"], _qw_from(a, p, "w_", oracle), a["b"], p["offset"])


def load_ops_golden() -> dict[str, OpCase]:
    data = np.load(OPS_GOLDEN_PATH, allow_pickle=False)
    cases = ops_recipes()
    for name, c in cases.items():
        assert str(data[name + "__hash"]) == op_hash(c), f"{name}: regenerated inputs differ from the fixture's"
        c.out = data[name + "__out"]
    return cases
