"""Build libsolattn.so (gfx950) from csrc/ with hipcc, in place.

Usage: python build.py [-v]. Every .hip file compiles in parallel to an object
under _build/, then one shared library is linked next to this file. The prep
and quant kernels are compiled with -ffp-contract=off so their fp32 arithmetic
is rounded exactly as written (the bit-exact contract of include/solattn.h).
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libsolattn.so")
ARCH = "gfx950"

SOURCES = ["capi.hip", "reorder.hip", "prep.hip", "quant.hip", "fwd_bf16.hip", "fwd_int8.hip"]
STRICT_FP = {"prep.hip", "quant.hip"}
# clang 22 (ROCm 7.2) segfaults in SimplifyCFG's common-code sinking on the
# INT8 forward; switching that one transform off builds it.
EXTRA = {"fwd_int8.hip": ["-mllvm", "-simplifycfg-sink-common=false"]}

COMMON = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-result",
    # Packed fp32 VALU ops are kept out of the generated code on this target.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libsolattn.so)")


def _compile(src: str, verbose: bool) -> str:
    obj = os.path.join(BUILD, src.replace(".hip", ".o"))
    flags = list(COMMON)
    if src in STRICT_FP:
        flags.append("-ffp-contract=off")
    flags += EXTRA.get(src, [])
    cmd = [hipcc(), *flags, "-c", os.path.join(CSRC, src), "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature; that warning is expected.
    err = "\n".join(l for l in res.stderr.splitlines() if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{err}")
    if verbose and err.strip():
        print(err, flush=True)
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), SOURCES))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
