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
