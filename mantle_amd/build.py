"""Build recipe for libmantle_hip.so (gfx950) and the CPU oracle.

``python -m mantle_amd.build`` (or ``__graft_entry__.build()``) compiles every HIP source in
``mantle_amd/csrc`` with hipcc for gfx950 and links ``mantle_amd/libmantle_hip.so`` in-tree.

Flags that carry semantics:
  -ffp-contract=off                  no a*b+c contraction: fp32 results round like the
                                     reference's separate multiply and add
  -fno-gpu-flush-denormals-to-zero   IEEE subnormals, as on the CPU
  -Xclang -target-feature -Xclang -packed-fp32-ops
                                     no packed-fp32 (v_pk_*_f32) code generation
Correctly rounded fp32 division stays on (hipcc's default); no fast-math.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libmantle_hip.so")
ARCH = "gfx950"

HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fno-fast-math",
    "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    "-I", os.path.join(ROOT, "include"),
]


def _hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libmantle_hip.so)")


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return r


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def build_hip(verbose: bool = False) -> str:
    """Compile every .hip source for gfx950 and link libmantle_hip.so (always rebuilds)."""
    hipcc = _hipcc()
    os.makedirs(BUILD, exist_ok=True)
    srcs = sources()
    objs = [os.path.join(BUILD, os.path.basename(s)[:-4] + ".o") for s in srcs]
    jobs = min(len(srcs), int(os.environ.get("MAX_JOBS", "8")) or 1)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = [ex.submit(_run, [hipcc, *HIP_FLAGS, "-c", s, "-o", o]) for s, o in zip(srcs, objs)]
        for f in futs:
            r = f.result()
            if verbose and r.stderr.strip():
                print(r.stderr, file=sys.stderr)
    tmp = LIB + ".tmp"
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-o", tmp, *objs])
    os.replace(tmp, LIB)
    return LIB


def build_hip_host_sanitized() -> str:
    """libmantle_hip.so with AddressSanitizer and UBSan on the host code only (the shape checks,
    launch planning, graph builder and model bookkeeping), into mantle_amd/_san/. The GPU code
    is built as usual (GPU sanitizers are not used). For tests/sanitize_cpu.py."""
    hipcc = _hipcc()
    out_dir = os.path.join(PKG, "_san")
    os.makedirs(out_dir, exist_ok=True)
    san = ["-g", "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
           "-Xarch_host", "-fno-sanitize-recover=undefined", "-Xarch_host", "-fno-omit-frame-pointer"]
    srcs = sources()
    objs = [os.path.join(out_dir, os.path.basename(s)[:-4] + ".o") for s in srcs]
    jobs = min(len(srcs), int(os.environ.get("MAX_JOBS", "8")) or 1)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        for f in [ex.submit(_run, [hipcc, *HIP_FLAGS, *san, "-c", s, "-o", o]) for s, o in zip(srcs, objs)]:
            f.result()
    lib = os.path.join(out_dir, "libmantle_hip.so")
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-Xarch_host", "-fsanitize=address", "-Xarch_host",
          "-fsanitize=undefined", "-o", lib, *objs])
    return lib


def build_oracle() -> str:
    """Build the CPU restatement used by the tests as the parity checker."""
    _run(["make", "-s", "-C", os.path.join(ROOT, "oracle")])
    return os.path.join(ROOT, "oracle", "liboracle.so")


def main():
    lib = build_hip(verbose=True)
    print("built", lib)
    print("built", build_oracle())


if __name__ == "__main__":
    main()
