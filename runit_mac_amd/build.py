"""Build recipe for the gfx950 code objects and the C-ABI host library.

The reference compiles its Metal shaders into one .metallib at build time
(crates/kernels/build.rs:48-117).  Here the analogue is:

  csrc/k*.hip       --hipcc --genco (gfx950)-->  lib/kernels/<name>.hsaco
  csrc/runtime.cpp  --g++ -shared (libamdhip64)-> lib/librunit_hip.so

Each kernel translation unit becomes its own code object (compiled in
parallel); the runtime loads every code object of lib/kernels/.  Both
artefacts are built in-tree so they travel with the source tree.
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

KERNEL_DIR = os.path.join(LIB_DIR, "kernels")
# kernel translation units (csrc/<name>.hip → lib/kernels/<name>.hsaco)
KERNEL_UNITS = ("kg_q8_0", "kg_q4", "kg_q5", "kg_q6k", "kg_ggml", "kls_q8_0", "kls_q4", "kls_q5",
                "kls_q6k", "kls_ggml", "kgx_rows", "k_gemm", "k_aux", "k_decode", "k_step",
                "k_scratch", "kvs")
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


def _build_unit(name: str, force: bool) -> str:
    hipcc = os.path.join(ROCM, "bin", "hipcc")
    src = os.path.join(CSRC, name + ".hip")
    out = os.path.join(KERNEL_DIR, name + ".hsaco")
    if not force and os.path.exists(out):
        deps = [src] + [os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".h")]
        if os.path.getmtime(out) >= max(map(os.path.getmtime, deps)):
            return out
    tmp = out + ".tmp"
    _run([hipcc, *HIPCC_FLAGS, "--genco", "-o", tmp, src])
    os.replace(tmp, out)
    return out


def build_kernels(force: bool = True) -> str:
    """Compiles every kernel unit (all of them, or with force=False only those
    older than their sources), in parallel; returns the code-object directory."""
    from concurrent.futures import ThreadPoolExecutor
    os.makedirs(KERNEL_DIR, exist_ok=True)
    # stale code objects of units that no longer exist would be loaded too
    for f in os.listdir(KERNEL_DIR):
        if f.endswith(".hsaco") and f[:-6] not in KERNEL_UNITS:
            os.remove(os.path.join(KERNEL_DIR, f))
    workers = min(len(KERNEL_UNITS), max(1, min(16, os.cpu_count() or 1)))
    # the largest units first, so they do not finish last
    order = sorted(KERNEL_UNITS, key=lambda n: (not n.startswith(("kg_", "kls_", "k_gemm")), n))
    with ThreadPoolExecutor(workers) as ex:
        list(ex.map(lambda n: _build_unit(n, force), order))
    return KERNEL_DIR


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
    print(KERNEL_DIR)
    print(HOST_LIB)
