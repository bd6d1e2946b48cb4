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
