"""Host code under AddressSanitizer and UndefinedBehaviorSanitizer (CPU only):
libg4a.so rebuilt with the sanitizers on its host side only (each -fsanitize=
after -Xarch_host, so the gfx950 device code is untouched), the CPU oracle
built with them too, and tests/cpp/sanitize_host.cpp driving the host paths
that need no GPU: the dispatch planning over a sweep of shapes (trim, split
choice, workspace sizing, explicit positions, rings, forced splits), the
argument and option errors, a failed g4a_create, and the oracle's functions
on small and empty inputs. Any sanitizer report fails the run."""
import os
import subprocess

from g4a import build

OUT = build.REPO / "tests" / "cpp" / "_build" / "sanitize"
CLANG = "/opt/rocm/llvm/bin/clang++"
CLANGC = "/opt/rocm/llvm/bin/clang"
SAN = ["-fsanitize=address", "-fsanitize=undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", "-g"]


def _build() -> None:
    OUT.mkdir(parents=True, exist_ok=True)
    host_san = [flag for s in SAN for flag in (("-Xarch_host", s) if s.startswith("-f") else (s,))]
    lib = OUT / "libg4a.so"
    build._run([build.HIPCC, "-x", "hip", f"--offload-arch={build.ARCH}", "-O1", "-std=c++17",
                *build.DEVICE_FLAGS[4:], *host_san, "-fPIC", "-shared", f"-I{build.INCLUDE}", f"-I{build.CSRC}",
                build.CSRC / "g4a.cpp", "-o", lib, "-ldl"], False)
    objs = []
    for c in ("attn_oracle.c", "linear_oracle.c"):
        o = OUT / (c[:-2] + ".o")
        build._run([CLANGC, "-O1", "-std=gnu11", "-ffp-contract=off", "-fno-fast-math", *SAN, "-c",
                    build.ORACLE_DIR / c, "-o", o], False)
        objs.append(o)
    build._run([CLANG, "-O1", "-std=c++17", *SAN, f"-I{build.INCLUDE}",
                build.REPO / "tests" / "cpp" / "sanitize_host.cpp", *objs, "-o", OUT / "sanitize_host",
                f"-L{OUT}", "-lg4a", f"-Wl,-rpath,{OUT}", "-lpthread", "-lm"], False)


def test_host_code_under_address_and_undefined_behaviour_sanitizers():
    _build()
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:abort_on_error=0",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1", HIP_VISIBLE_DEVICES="")
    r = subprocess.run([str(OUT / "sanitize_host")], capture_output=True, text=True, timeout=300, env=env)
    print(r.stdout[-3000:], r.stderr[-6000:], flush=True)
    assert r.returncode == 0, "sanitizer report or failed check"
    assert "PASSED: 0 failure(s)" in r.stdout
    assert "ERROR: AddressSanitizer" not in r.stderr and "runtime error" not in r.stderr
