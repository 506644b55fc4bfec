"""Build libbmx_k2b.so (gfx950: the k2b, RTN and spectral paths, prefill attention) in-tree with hipcc.

    python -m bmx_amd.build

Each .hip source compiles to an object under bmx_amd/_build/ and the objects
link into bmx_amd/libbmx_k2b.so, the library bmx_amd._lib loads.  The write
and dequant kernels are compiled without floating-point contraction so their
element-wise arithmetic matches the reference's operation order.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libbmx_k2b.so"

ARCH = "gfx950"
COMMON = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    f"-I{ROOT / 'include'}", f"-I{CSRC}",
]
SOURCES = {
    "k2b_api.hip": [],
    "k2b_decode.hip": ["-ffp-contract=fast"],
    "k2b_append.hip": ["-ffp-contract=off"],
    "k2b_dequant.hip": ["-ffp-contract=off"],
    "rtn.hip": ["-ffp-contract=off"],
    "spectral.hip": ["-ffp-contract=off"],
    "k2b_general.hip": ["-ffp-contract=off"],
    "fp16_decode.hip": ["-ffp-contract=fast"],
    "flash_prefill.hip": ["-ffp-contract=fast"],
}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libbmx_k2b.so)")


def build(verbose: bool = False) -> Path:
    BUILD.mkdir(exist_ok=True)
    cc = hipcc()
    objs = []
    for src, extra in SOURCES.items():
        obj = BUILD / (Path(src).stem + ".o")
        cmd = [cc, *COMMON, *extra, "-c", str(CSRC / src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        subprocess.run(cmd, check=True)
        objs.append(str(obj))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [cc, "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
