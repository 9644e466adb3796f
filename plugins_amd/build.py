"""Builds libexl3_mi355x.so (HIP kernels for gfx950 + the C ABI) in-tree.

    python -m plugins_amd.build          # or: python plugins_amd/build.py
    python -m plugins_amd.build --timeline   # the diagnostic GEMV-timeline build
    python -m plugins_amd.build --valu-rates # the VALU instruction-rate program

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


# The diagnostic build with the GEMV phase timeline compiled in
# (EXL3_TIMELINE; plugins_amd/timeline.py reads it): a library of its own.
TIMELINE_LIB = os.path.join(LIBDIR, "libexl3_mi355x_timeline.so")


def build(verbose: bool = True, timeline: bool = False) -> str:
    """Compiles every source and links the shared library; returns its path.
    timeline: the diagnostic build (objects with a _tl suffix, TIMELINE_LIB)."""
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    srcs = SOURCES
    lib_path = LIB
    if timeline:
        device = lambda f: any(x.startswith("--offload-arch") for x in f)  # noqa: E731
        srcs = [(s, n + "_tl", f + ["-DEXL3_TIMELINE"] if device(f) else f) for s, n, f in SOURCES]
        lib_path = TIMELINE_LIB
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


# The measurement program for the VALU issue cost of the decode's integer
# multiply (csrc/valu_rates.hip): an executable, not part of the library.
VALU_RATES = os.path.join(LIBDIR, "valu_rates")


def build_valu_rates(verbose: bool = True) -> str:
    os.makedirs(LIBDIR, exist_ok=True)
    flags = [f for f in DEVICE_FLAGS if f != "-fPIC"]
    cmd = [_hipcc(), *flags, os.path.join(CSRC, "valu_rates.hip"), "-o", VALU_RATES]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("hipcc failed on valu_rates.hip:\n" + r.stdout + r.stderr)
    if verbose:
        print("built", VALU_RATES)
    return VALU_RATES


if __name__ == "__main__":
    if "--valu-rates" in sys.argv[1:]:
        build_valu_rates()
    else:
        build(timeline="--timeline" in sys.argv[1:])
