"""Build recipe for the MI355X attention path.

Produces, in-tree (so the files travel with the repository snapshot):
  gemma-4-webgpu-kernels_amd/_build/g4a_kernels.hsaco  gfx950 code object (hipModuleLoad)
  gemma-4-webgpu-kernels_amd/_build/libg4a.so          C-ABI host library (include/g4a.h)
  gemma-4-webgpu-kernels_amd/_build/libg4a_backend.so  C++ mirror of the Backend trait
  tests/cpp/_build/test_backend                        C++ parity driver for that mirror (test infrastructure)
  oracle/_build/liboracle.so                           CPU oracle (test infrastructure)

Every call recompiles everything (it is the "does it build" check).
"""
from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

PKG = Path(__file__).resolve().parents[1]
REPO = PKG.parent
CSRC = PKG / "csrc"
OUT = PKG / "_build"
ORACLE_DIR = REPO / "oracle"
ORACLE_OUT = ORACLE_DIR / "_build"
INCLUDE = REPO / "include"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
# Packed-FP32 VALU ops are disabled for every HIP build (they have produced
# silent wrong results on these machines); -ffp-contract=off keeps each
# multiply and add separately rounded unless the source asks for fmaf.
DEVICE_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-ffp-contract=off", "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]

HSACO = OUT / "g4a_kernels.hsaco"
LIBG4A = OUT / "libg4a.so"
LIBBACKEND = OUT / "libg4a_backend.so"
TEST_BACKEND = REPO / "tests" / "cpp" / "_build" / "test_backend"
TEST_MODEL = REPO / "tests" / "cpp" / "_build" / "test_model"
LIBORACLE = ORACLE_OUT / "liboracle.so"


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print("+", " ".join(str(c) for c in cmd), flush=True)
    r = subprocess.run([str(c) for c in cmd], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(map(str, cmd))}\n{r.stdout}\n{r.stderr}")


def build_kernels(verbose: bool = False) -> Path:
    OUT.mkdir(parents=True, exist_ok=True)
    tmp = HSACO.with_suffix(".hsaco.tmp")
    _run([HIPCC, *DEVICE_FLAGS, "--genco", f"-I{CSRC / 'kernels'}", CSRC / "kernels" / "g4a_kernels.hip", "-o", tmp], verbose)
    tmp.replace(HSACO)
    return HSACO


def build_host(verbose: bool = False) -> Path:
    OUT.mkdir(parents=True, exist_ok=True)
    tmp = LIBG4A.with_suffix(".so.tmp")
    # compiled as HIP for gfx950: the library carries one device array of its own (the
    # static scratch of g4a_attention_noalloc), registered with the HIP runtime at load
    _run([HIPCC, "-x", "hip", *DEVICE_FLAGS[:1], "-O2", "-std=c++17", *DEVICE_FLAGS[4:], "-fPIC", "-shared",
          f"-I{INCLUDE}", f"-I{CSRC}", CSRC / "g4a.cpp", "-o", tmp, "-ldl"], verbose)
    tmp.replace(LIBG4A)
    return LIBG4A


def build_backend(verbose: bool = False) -> Path:
    """The C++ HipBackend (mirror of rust/src/backend.rs) over libg4a.so, plus its parity driver."""
    OUT.mkdir(parents=True, exist_ok=True)
    tmp = LIBBACKEND.with_suffix(".so.tmp")
    _run(["g++", "-O2", "-std=c++17", "-fPIC", "-shared", f"-I{INCLUDE}", f"-I{CSRC}", CSRC / "hip_backend.cpp",
          "-o", tmp, f"-L{OUT}", "-lg4a", f"-Wl,-rpath,$ORIGIN"], verbose)
    tmp.replace(LIBBACKEND)
    TEST_BACKEND.parent.mkdir(parents=True, exist_ok=True)
    tmp = TEST_BACKEND.with_suffix(".tmp")
    oracle_obj = TEST_BACKEND.parent / "attn_oracle.o"
    linear_obj = TEST_BACKEND.parent / "linear_oracle.o"
    _run(["gcc", "-O2", "-std=gnu11", "-ffp-contract=off", "-fno-fast-math", "-c", ORACLE_DIR / "attn_oracle.c",
          "-o", oracle_obj], verbose)
    _run(["gcc", "-O2", "-std=gnu11", "-ffp-contract=off", "-fno-fast-math", "-c", ORACLE_DIR / "linear_oracle.c",
          "-o", linear_obj], verbose)
    _run(["g++", "-O2", "-std=c++17", f"-I{INCLUDE}", f"-I{CSRC}", REPO / "tests" / "cpp" / "test_backend.cpp",
          oracle_obj, linear_obj, "-o", tmp, f"-L{OUT}", "-lg4a_backend", "-lg4a", "-Wl,-rpath,$ORIGIN/../../../gemma-4-webgpu-kernels_amd/_build", "-lpthread", "-lm"],
         verbose)
    tmp.replace(TEST_BACKEND)
    # the whole-model driver: Gemma4Model's composition over HipBackend and over the oracle
    tmp = TEST_MODEL.with_suffix(".tmp")
    _run(["g++", "-O2", "-std=c++17", "-ffp-contract=off", f"-I{INCLUDE}", f"-I{CSRC}",
          REPO / "tests" / "cpp" / "test_model.cpp", oracle_obj, linear_obj, "-o", tmp, f"-L{OUT}", "-lg4a_backend",
          "-lg4a", "-Wl,-rpath,$ORIGIN/../../../gemma-4-webgpu-kernels_amd/_build", "-lpthread", "-lm"], verbose)
    tmp.replace(TEST_MODEL)
    return LIBBACKEND


def build_oracle(verbose: bool = False) -> Path:
    """CPU oracle: -ffp-contract=off and no fast-math keep the f32 arithmetic of the Rust reference."""
    ORACLE_OUT.mkdir(parents=True, exist_ok=True)
    tmp = LIBORACLE.with_suffix(".so.tmp")
    _run(["gcc", "-O2", "-std=gnu11", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math",
          ORACLE_DIR / "attn_oracle.c", ORACLE_DIR / "linear_oracle.c", "-o", tmp, "-lm", "-lpthread"], verbose)
    tmp.replace(LIBORACLE)
    return LIBORACLE


def build_all(verbose: bool = False) -> None:
    if shutil.which(HIPCC) is None and not Path(HIPCC).exists():
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    build_oracle(verbose)
    build_kernels(verbose)
    build_host(verbose)
    if (CSRC / "hip_backend.cpp").exists():
        build_backend(verbose)


if __name__ == "__main__":
    build_all(verbose=True)
