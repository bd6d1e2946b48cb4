"""Writes tests/golden/attention_golden.npz, norm_rope_golden.npz,
linear_golden.npz and backend_ops_golden.npz: for every
recipe in golden_io, the sha256 of its regenerated inputs and the CPU oracle's
output on them.

Run from the repository root after building the oracle:
    python tests/golden/make_golden.py
"""
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
REPO = HERE.parents[1]
sys.path[:0] = [str(HERE), str(REPO / "gemma-4-webgpu-kernels_amd"), str(REPO / "oracle")]

import numpy as np  # noqa: E402

import oracle  # noqa: E402
from golden_io import (GOLDEN_PATH, LINEAR_GOLDEN_PATH, NORM_ROPE_GOLDEN_PATH, OPS_GOLDEN_PATH,  # noqa: E402
                       input_hash, linear_eval, linear_hash, linear_recipes, norm_rope_eval, norm_rope_hash,
                       norm_rope_recipes, op_hash, ops_eval, ops_recipes, recipes)


def main():
    arrays = {}
    for name, c in recipes().items():
        out = oracle.attention(c.q, c.k, c.v, c.q_pos, c.k_pos, scale=c.scale, window=c.window, softcap=c.softcap)
        arrays[name + "__out"] = out
        arrays[name + "__hash"] = np.array(input_hash(c))
        print(f"{name}: out {out.shape}")
    np.savez_compressed(GOLDEN_PATH, **arrays)
    print("wrote", GOLDEN_PATH, GOLDEN_PATH.stat().st_size, "bytes")
    arrays = {}
    for name, c in norm_rope_recipes().items():
        out = norm_rope_eval(c, oracle)
        arrays[name + "__out"] = out
        arrays[name + "__hash"] = np.array(norm_rope_hash(c))
        print(f"{name}: out {out.shape}")
    np.savez_compressed(NORM_ROPE_GOLDEN_PATH, **arrays)
    print("wrote", NORM_ROPE_GOLDEN_PATH, NORM_ROPE_GOLDEN_PATH.stat().st_size, "bytes")
    arrays = {}
    for name, c in linear_recipes().items():
        out = linear_eval(c, oracle)
        arrays[name + "__out"] = out
        arrays[name + "__hash"] = np.array(linear_hash(c))
        print(f"{name}: out {out.shape}")
    np.savez_compressed(LINEAR_GOLDEN_PATH, **arrays)
    print("wrote", LINEAR_GOLDEN_PATH, LINEAR_GOLDEN_PATH.stat().st_size, "bytes")
    arrays = {}
    for name, c in ops_recipes().items():
        out = ops_eval(c, oracle)
        arrays[name + "__out"] = out
        arrays[name + "__hash"] = np.array(op_hash(c))
    np.savez_compressed(OPS_GOLDEN_PATH, **arrays)
    print("wrote", OPS_GOLDEN_PATH, OPS_GOLDEN_PATH.stat().st_size, "bytes")


if __name__ == "__main__":
    main()
