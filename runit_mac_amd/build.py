"""Build recipe for the gfx950 code object and the C-ABI host library.

The reference compiles its Metal shaders into one .metallib at build time
(crates/kernels/build.rs:48-117).  Here the analogue is:

  csrc/kernels.hip  --hipcc --genco (gfx950)-->  lib/runit_kernels.hsaco
  csrc/runtime.cpp  --g++ -shared (libamdhip64)-> lib/librunit_hip.so

Both artefacts are built in-tree so they travel with the source tree.
"""
from __future__ import annotations

import os
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG_DIR, "csrc")
LIB_DIR = os.path.join(PKG_DIR, "lib")
REPO = os.path.dirname(PKG_DIR)
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

HSACO = os.path.join(LIB_DIR, "runit_kernels.hsaco")
HOST_LIB = os.path.join(LIB_DIR, "librunit_hip.so")

# -packed-fp32-ops: no v_pk_*_f32 (their results have been unreliable on the
# target machines); plain f32 code is fast enough for these HBM-bound kernels.
HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        ln for ln in proc.stdout.splitlines()
        if "argument unused during compilation" not in ln and "packed-fp32-ops" not in ln
    )
    if proc.returncode != 0:
        sys.stderr.write(out + "\n")
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}")


def build_kernels() -> str:
    os.makedirs(LIB_DIR, exist_ok=True)
    hipcc = os.path.join(ROCM, "bin", "hipcc")
    tmp = HSACO + ".tmp"
    _run([hipcc, *HIPCC_FLAGS, "--genco", "-o", tmp, os.path.join(CSRC, "kernels.hip")])
    os.replace(tmp, HSACO)
    return HSACO


def build_host() -> str:
    os.makedirs(LIB_DIR, exist_ok=True)
    tmp = HOST_LIB + ".tmp"
    _run([
        "g++", "-O2", "-std=c++17", "-shared", "-fPIC", "-Wall", "-Wno-unused-result",
        "-D__HIP_PLATFORM_AMD__", f"-I{ROCM}/include",
        os.path.join(CSRC, "runtime.cpp"), os.path.join(CSRC, "gguf.cpp"), "-o", tmp,
        f"-L{ROCM}/lib", "-lamdhip64", f"-Wl,-rpath,{ROCM}/lib", "-ldl",
    ])
    os.replace(tmp, HOST_LIB)
    return HOST_LIB


def build_all() -> None:
    build_kernels()
    build_host()


if __name__ == "__main__":
    build_all()
    print(HSACO)
    print(HOST_LIB)
