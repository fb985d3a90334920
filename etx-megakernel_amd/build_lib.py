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


def build(verbose: bool = False) -> Path:
    """Compile every unit in parallel (one hipcc each), then link the shared library."""
    LIB.parent.mkdir(parents=True, exist_ok=True)
    obj_dir = PKG / "lib" / "obj"
    obj_dir.mkdir(parents=True, exist_ok=True)
    inc = [f"-I{ROOT / 'include'}", f"-I{SRC}"]
    procs = []
    for u in UNITS:
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
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *[str(o) for _, o, _ in procs]]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"linking {LIB} failed ({r.returncode})")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
