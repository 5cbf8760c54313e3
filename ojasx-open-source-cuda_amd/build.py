"""Builds libojasx_e8t.so (HIP kernels + C ABI) for gfx950, in-tree.

    python ojasx-open-source-cuda_amd/build.py

Objects go to ``_build/`` and the library to ``lib/libojasx_e8t.so`` next to
this file.  hipcc cross-compiles, so no GPU is needed to build.
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
LIB = os.path.join(HERE, "lib", "libojasx_e8t.so")

SOURCES = [
    "e8t_codec.hip",
    "e8t_gemm_generic.hip",
    "e8t_gemv.hip",
    "e8t_gemm_mfma.hip",
    "e8t_hadamard.hip",
    "e8t_qat.hip",
    "e8t_noalloc.hip",
    "e8t_lora.hip",
    "e8t_capi.cpp",
]

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

# Packed-fp32 VALU instructions are disabled for all device code: hipcc would
# otherwise form v_pk_*_f32 from ordinary float code.  (The host pass warns that
# it does not know the feature; that is harmless.)
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
COMMON = ["-x", "hip", "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
          "-fvisibility=hidden", "-Wall", "-Wno-unused-function"] + DEVICE_FLAGS


# Per-file code generation options.  The decode GEMV keeps its MFMA results in ordinary
# VGPRs: its post-scaled kernel reads every result with VALU FMAs, and the accumulator
# register form would add a v_accvgpr_read per read and raise the register total.
EXTRA = {
    "e8t_gemv.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
}


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC] + COMMON + EXTRA.get(src, []) + ["-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"hipcc failed for {src}")
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(os.path.dirname(LIB), exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + objs
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("link of libojasx_e8t.so failed")
    # a kernel template the host pass could not instantiate leaves its launch stub undefined
    # (the link of a shared library does not catch it); refuse such a library
    nm = shutil.which("nm")
    if nm:
        out = subprocess.run([nm, "-D", "--undefined-only", tmp], capture_output=True,
                             text=True).stdout
        missing = [l.split()[-1] for l in out.splitlines() if "ojx" in l]
        if missing:
            raise RuntimeError("libojasx_e8t.so has undefined symbols: " + ", ".join(missing[:4]))
    os.replace(tmp, LIB)
    if verbose:
        print("built", LIB)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
