"""Builds libetxmk.so (the gfx950 decode megakernel and its C ABI) and libetxmk_calib.so (the grid-barrier and
streaming-read calibration kernels, outside the decode ABI) in-tree with hipcc.

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
CALIB = PKG / "lib" / "libetxmk_calib.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    "-ffp-contract=off",                                  # every fma in the numerics is explicit
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mcode-object-version=5",                            # loadable by the HIP runtime torch bundles
    "-Wno-unused-command-line-argument",
]
# translation units: the host side (C ABI, unfused and initialisation kernels) and one per persistent-kernel list
UNITS = ["mk_api.hip", "mk_fused_bf16.hip", "mk_fused_fp8.hip", "mk_batch_bf16.hip", "mk_batch_fp8.hip",
         "mk_mla.hip"]
CALIB_UNITS = ["mk_calib.hip"]


def build(verbose: bool = False) -> Path:
    """Compile every unit in parallel (one hipcc each), then link the shared library."""
    LIB.parent.mkdir(parents=True, exist_ok=True)
    obj_dir = PKG / "lib" / "obj"
    obj_dir.mkdir(parents=True, exist_ok=True)
    inc = [f"-I{ROOT / 'include'}", f"-I{SRC}"]
    procs = []
    for u in UNITS + CALIB_UNITS:
        obj = obj_dir / (Path(u).stem + ".o")
        procs.append((u, obj, subprocess.Popen([HIPCC, *FLAGS, *inc, "-c", "-o", str(obj), str(SRC / u)],
                                               stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
    failed = []
    for u, obj, pr in procs:
        out, _ = pr.communicate()
        if pr.returncode != 0:
            failed.append(u)
            sys.stderr.write(out)
        elif verbose and out:
            sys.stderr.write(out)
    if failed:
        raise RuntimeError(f"hipcc failed building {', '.join(failed)}")
    for lib, units in ((LIB, UNITS), (CALIB, CALIB_UNITS)):
        tmp = lib.with_suffix(".so.tmp")
        objs = [str(o) for u, o, _ in procs if u in units]
        cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *objs]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            sys.stderr.write(r.stdout + r.stderr)
            raise RuntimeError(f"linking {lib} failed ({r.returncode})")
        os.replace(tmp, lib)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
