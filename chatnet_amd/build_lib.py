"""Builds the native libraries of chatnet_amd in-tree.

    lib/libchatnet_hip.so    HIP kernels + C ABI for gfx950 (hipcc)
    lib/libchatnet_synth.so  host-only synthetic weight generator (gcc)

Run as `python -m chatnet_amd.build_lib` or through __graft_entry__.build().
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG, "csrc")
LIBDIR = os.path.join(PKG, "lib")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

HIP_SOURCES = ["chatnet_api.hip", "gemv.hip", "gemv_float.hip", "gemm.hip", "prefill.hip", "decode_ops.hip", "sample.hip"]
HIP_HEADERS = ["device_common.h", "gemv_common.h", "kernels.h"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-fvisibility=hidden",
    "-Wall",
    "-Wno-unused-function",
    # packed fp32 instructions (v_pk_fma_f32 and friends) stay off
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        line for line in proc.stdout.splitlines() if "packed-fp32-ops" not in line
    )
    if proc.returncode != 0:
        sys.stderr.write(out + "\n")
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}")
    if out.strip():
        sys.stderr.write(out + "\n")


def build_hip(verbose: bool = False) -> str:
    """Compiles each translation unit to an object in parallel (no device code
    crosses translation units), then links the shared library."""
    from concurrent.futures import ThreadPoolExecutor

    hipcc = shutil.which("hipcc") or os.path.join(ROCM, "bin", "hipcc")
    os.makedirs(LIBDIR, exist_ok=True)
    objdir = os.path.join(PKG, "_build")
    os.makedirs(objdir, exist_ok=True)
    out = os.path.join(LIBDIR, "libchatnet_hip.so")
    tmp = out + ".tmp"
    srcs = [os.path.join(CSRC, s) for s in HIP_SOURCES if os.path.exists(os.path.join(CSRC, s))]
    compile_flags = [f for f in HIPCC_FLAGS if f != "-shared"]
    cmds = []
    for src in srcs:
        obj = os.path.join(objdir, os.path.basename(src) + ".o")
        cmds.append([hipcc, *compile_flags, "-I", os.path.join(PKG, "..", "include"), "-c", src, "-o", obj])
    if verbose:
        for c in cmds:
            print(" ".join(c))
    jobs = max(1, min(len(cmds), int(os.environ.get("MAX_JOBS") or os.cpu_count() or 1)))
    with ThreadPoolExecutor(jobs) as ex:
        list(ex.map(_run, cmds))
    link = [hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", *[c[-1] for c in cmds], "-o", tmp]
    if verbose:
        print(" ".join(link))
    _run(link)
    os.replace(tmp, out)
    return out


def build_synth(verbose: bool = False) -> str:
    cc = shutil.which("gcc") or "cc"
    os.makedirs(LIBDIR, exist_ok=True)
    out = os.path.join(LIBDIR, "libchatnet_synth.so")
    tmp = out + ".tmp"
    cmd = [cc, "-O2", "-std=c11", "-fPIC", "-shared", "-fopenmp", "-fvisibility=hidden",
           "-Wall", os.path.join(CSRC, "synth.c"), "-o", tmp, "-lm"]
    if verbose:
        print(" ".join(cmd))
    _run(cmd)
    os.replace(tmp, out)
    return out


def build_all(verbose: bool = False) -> list[str]:
    return [build_synth(verbose), build_hip(verbose)]


if __name__ == "__main__":
    for p in build_all(verbose=True):
        print("built", p)
