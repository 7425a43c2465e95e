"""Builds liboal_amd.so in-tree with hipcc for gfx950.

Usage: ``python -m oal_amd.build`` (``__graft_entry__.build()`` calls it).
Each source compiles to an object under oal_amd/_build/ in parallel, then one
link step writes oal_amd/liboal_amd.so.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
SOURCES = [os.path.join(PKG, "csrc", "oal_kernels.hip"), os.path.join(PKG, "csrc", "oal_mfma_fwd.hip"),
           os.path.join(PKG, "csrc", "oal_mfma_bwd.hip"), os.path.join(PKG, "csrc", "oal_mfma_local.hip"),
           os.path.join(PKG, "csrc", "oal_mfma_scan.hip"), os.path.join(PKG, "csrc", "oal_mfma_den.hip"),
           os.path.join(PKG, "csrc", "oal_mfma_pair.hip"), os.path.join(PKG, "csrc", "oal_f32_mma.hip"),
           os.path.join(PKG, "csrc", "oal_f64.hip")]
# Sources whose matrix-core accumulators the compiler would otherwise place in
# the accumulation registers (AGPRs): there every VALU use of a group sum needs
# a v_accvgpr_read copy first (256 of them per tile in the intra-chunk forward).
# In VGPRs the VALU reads them directly; each kernel in these files stays
# within 256 VGPRs without spilling.
VGPR_FORM = {"oal_mfma_fwd.hip", "oal_mfma_local.hip"}
HEADERS = [os.path.join(PKG, "csrc", "oal_common.hpp"), os.path.join(ROOT, "include", "oal_amd.h")]
OUTPUT = os.path.join(PKG, "liboal_amd.so")
OBJDIR = os.path.join(PKG, "_build")


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build oal_amd)")


def compile_flags() -> list[str]:
    return [
        "--offload-arch=gfx950",
        "-O3",
        "-std=c++20",
        "-fPIC",
        "-I" + os.path.join(ROOT, "include"),
        "-I" + os.path.join(PKG, "csrc"),
        # no packed FP32 VALU instructions (v_pk_*_f32): some of their forms have given wrong
        # results without any error on these GPUs
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    ]


def source_flags(src: str) -> list[str]:
    return ["-mllvm", "-amdgpu-mfma-vgpr-form"] if os.path.basename(src) in VGPR_FORM else []


def link_flags() -> list[str]:
    rocm = os.path.dirname(os.path.dirname(os.path.realpath(hipcc())))
    libdir = os.path.join(rocm, "lib")
    return ["-L" + libdir, "-Wl,-rpath," + libdir, "-lrocprofiler-sdk-roctx"]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"hipcc failed with exit code {proc.returncode}: {' '.join(cmd[-3:])}")


def build(verbose: bool = False) -> str:
    """Compile every HIP source into oal_amd/liboal_amd.so; returns its path."""
    os.makedirs(OBJDIR, exist_ok=True)
    objs = [os.path.join(OBJDIR, os.path.splitext(os.path.basename(s))[0] + ".o") for s in SOURCES]
    cc = hipcc()
    jobs = [[cc, *compile_flags(), *source_flags(src), "-c", src, "-o", obj] for src, obj in zip(SOURCES, objs)]
    workers = max(1, min(len(jobs), os.cpu_count() or 1))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        for fut in [pool.submit(_run, j, verbose) for j in jobs]:
            fut.result()
    tmp = OUTPUT + ".tmp"
    # librocprofiler-sdk-roctx: the host-side stage ranges (roctx) of every launch
    _run([cc, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp, *link_flags()], verbose)
    os.replace(tmp, OUTPUT)
    return OUTPUT


if __name__ == "__main__":
    print(build(verbose=True))
