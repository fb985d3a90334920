"""Builds libetxmk.so (the gfx950 decode megakernel and its C ABI) in-tree with hipcc.

    python etx-megakernel_amd/build_lib.py
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
SRC = PKG / "csrc"
LIB = PKG / "lib" / "libetxmk.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-ffp-contract=off",                                  # every fma in the numerics is explicit
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mcode-object-version=5",                            # loadable by the HIP runtime torch bundles
    "-Wno-unused-command-line-argument",
]


def build(verbose: bool = False) -> Path:
    LIB.parent.mkdir(parents=True, exist_ok=True)
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, *FLAGS, f"-I{ROOT / 'include'}", f"-I{SRC}", "-o", str(tmp), str(SRC / "mk_api.hip")]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"hipcc failed ({r.returncode}) building {LIB}")
    if verbose:
        sys.stderr.write(r.stderr)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
