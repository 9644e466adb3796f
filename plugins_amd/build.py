"""Builds libexl3_mi355x.so (HIP kernels for gfx950 + the C ABI) in-tree.

    python -m plugins_amd.build          # or: python plugins_amd/build.py

Objects go to plugins_amd/_build/, the library to plugins_amd/lib/.  hipcc
cross-compiles gfx950 code objects without a GPU.  Device code is built with
-ffp-contract=off (the kernels reproduce the reference's f32 operation order)
and without packed-FP32 instructions.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIBDIR = os.path.join(HERE, "lib")
LIB = os.path.join(LIBDIR, "libexl3_mi355x.so")
ARCH = os.environ.get("EXL3_OFFLOAD_ARCH", "gfx950")

DEVICE_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++20", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
    # the first kernel parameters arrive in SGPRs at wave launch (gfx950)
    "-mllvm", "-amdgpu-kernarg-preload-count=8",
]
HOST_FLAGS = ["-O2", "-std=c++20", "-fPIC", "-Wall", "-Wextra", "-Wno-unused-parameter"]

# (source, object name, flags): exl3_rate.hip once per rate K (0 = any even
# n), so the rates' kernels compile in parallel.
SOURCES = [
    ("exl3_kernels.hip", "exl3_kernels", DEVICE_FLAGS),
    *[("exl3_rate.hip", f"exl3_rate_k{k}", DEVICE_FLAGS + [f"-DEXL3_INST_K={k}"]) for k in range(9)],
    ("decoder_ops.hip", "decoder_ops", DEVICE_FLAGS),
    ("exl3_noalloc.hip", "exl3_noalloc", DEVICE_FLAGS),
    ("exl3_host.cpp", "exl3_host", HOST_FLAGS),
    ("exl3_json.cpp", "exl3_json", HOST_FLAGS),
    ("exl3_codebooks.cpp", "exl3_codebooks", HOST_FLAGS),
    ("exl3_dense.cpp", "exl3_dense", HOST_FLAGS),
    ("exl3_pack.cpp", "exl3_pack", HOST_FLAGS),
    ("exl3_selfcheck.cpp", "exl3_selfcheck", HOST_FLAGS),
]


def _hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the EXL3 library cannot be built")


def _compile(src: str, name: str, flags: list[str]) -> str:
    obj = os.path.join(BUILD, name + ".o")
    cmd = [_hipcc(), *flags, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(line for line in (r.stdout + r.stderr).splitlines()
                    if "packed-fp32-ops" not in line and "--hip-link" not in line)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{out}")
    if out.strip():
        print(out, file=sys.stderr)
    return obj


def build(verbose: bool = True) -> str:
    """Compiles every source and links the shared library; returns its path."""
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    srcs = SOURCES
    lib_path = LIB
    jobs = max(1, min(len(srcs), int(os.environ.get("MAX_JOBS", os.cpu_count() or 1))))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda sf: _compile(*sf), srcs))
    tmp = lib_path + ".tmp"
    # hipBLASLt: the dense GEMMs over resident matrices (exl3_dense.cpp)
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-lhipblaslt", "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stdout + r.stderr)
    os.replace(tmp, lib_path)
    if verbose:
        print("built", lib_path)
    return lib_path


if __name__ == "__main__":
    build()
