"""Runs the CPU test suites under AddressSanitizer and UBSan (every UB report fatal):

  1. the oracle built with gcc -fsanitize=address,undefined (`make -C oracle sanitize`), under
     tests/test_oracle.py and tests/test_goldens.py;
  2. libmantle_hip.so with the sanitizers on its host code (shape checks, launch planning,
     graph builder, model bookkeeping; `mantle_amd.build.build_hip_host_sanitized`), under
     tests/test_host.py and tests/test_checkpoint_format.py.

Python itself is not instrumented, so each run preloads the sanitizer runtime of the compiler
that built the library (gcc's libasan for the oracle, clang's for hipcc) and turns leak
detection off (the interpreter keeps allocations alive at exit by design). Usage:
    python tests/sanitize_cpu.py
Exits non-zero if a suite fails or a sanitizer reports."""
from __future__ import annotations

import glob
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _run(env_extra, tests):
    env = dict(os.environ)
    env.update(env_extra)
    env["ASAN_OPTIONS"] = "detect_leaks=0:abort_on_error=1:halt_on_error=1"
    env["UBSAN_OPTIONS"] = "print_stacktrace=1:halt_on_error=1"
    cmd = [sys.executable, "-m", "pytest", "-q", "-m", "not gpu", "-p", "no:cacheprovider", *tests]
    print("+", " ".join(f"{k}={v}" for k, v in env_extra.items()), " ".join(cmd), flush=True)
    return subprocess.run(cmd, cwd=ROOT, env=env).returncode


def main() -> int:
    sys.path.insert(0, ROOT)
    from mantle_amd import build

    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "sanitize"], check=True)
    gcc_asan = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True, text=True,
                              check=True).stdout.strip()
    gcc_ubsan = subprocess.run(["gcc", "-print-file-name=libubsan.so"], capture_output=True, text=True,
                               check=True).stdout.strip()
    rc1 = _run({"LD_PRELOAD": f"{gcc_asan}:{gcc_ubsan}",
                "MANTLE_ORACLE_LIB": os.path.join(ROOT, "oracle", "_san", "liboracle.so")},
               ["tests/test_oracle.py", "tests/test_goldens.py"])
    lib = build.build_hip_host_sanitized()
    clang_rt = sorted(glob.glob("/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    if not clang_rt:
        print("clang's ASan runtime not found", file=sys.stderr)
        return 2
    rc2 = _run({"LD_PRELOAD": clang_rt[-1], "MANTLE_TEST_HIP_LIB": lib},
               ["tests/test_host.py", "tests/test_checkpoint_format.py"])
    print(f"oracle suites: rc {rc1}; host suites: rc {rc2}")
    return 1 if (rc1 or rc2) else 0


if __name__ == "__main__":
    sys.exit(main())
