"""Makes tests/golden/mfma_bf16_gfx950.npz: outputs of gfx950's v_mfma_f32_16x16x32_bf16 on seeded operands, kept
where they tell the measured accumulation rule apart from its alternatives (tests/mfma_hypotheses.py).

Two steps:

    python tests/golden/make_mfma_fixture.py --hw gpurun_out/mfma_raw.npz      # on an MI355X: run the instruction
    python tests/golden/make_mfma_fixture.py gpurun_out/mfma_raw.npz           # on the CPU: select and write

The first runs every operand family of mfma_hypotheses.families(SEED) through the matrix-core probe of
libetxmk_calib.so and saves the hardware's D.  The second checks every element against the oracle's statement
(oracle/mk_oracle.c, orc_mfma_bf16_chain) and refuses to write if any differs; then, for each alternative rule, it
keeps up to PER_RULE elements the hardware refutes it on, plus RANDOM further elements per family."""
from __future__ import annotations

import sys
from concurrent.futures import ProcessPoolExecutor
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
for p in (str(ROOT), str(ROOT / "etx-megakernel_amd"), str(HERE.parent)):
    if p not in sys.path:
        sys.path.insert(0, p)

import mfma_hypotheses as H  # noqa: E402

SEED = 20261205
N = 16
PER_RULE = 40
RANDOM = 60
OUT = HERE / "mfma_bf16_gfx950.npz"


def hardware(path):
    from etx.runtime import calib
    res = {}
    for name, A, B, C in H.families(SEED, N):
        res[name + "_D"] = calib.mfma_bf16(A, B, C)
        print(f"{name}: {A.shape[0]} cases, {A.shape[2] // 32} steps", flush=True)
    np.savez_compressed(path, **res)


def _refuted(args):
    c, a, b, d, steps = args
    bits = 0
    for i, rule in enumerate(H.RULES[1:]):
        if np.float32(H.chain(c, a, b, steps, rule)).tobytes() != np.float32(d).tobytes():
            bits |= 1 << i
    return bits


def select(raw_path):
    from oracle import oracle as O
    L = O.lib()
    raw = np.load(raw_path)
    rng = np.random.default_rng(SEED)
    out = {"rules": np.array(H.RULES[1:])}
    for name, A, B, C in H.families(SEED, N):
        D = raw[name + "_D"]
        steps = A.shape[2] // 32
        elems = [(t, r, c) for t in range(A.shape[0]) for r in range(16) for c in range(16)]
        for t, r, c in elems:
            got = L.orc_mfma_bf16_chain(float(C[t, r, c]), np.ascontiguousarray(A[t, r]),
                                        np.ascontiguousarray(B[t, :, c]), steps)
            if np.float32(got).tobytes() != np.float32(D[t, r, c]).tobytes():
                raise SystemExit(f"{name} case {t} ({r}, {c}): oracle {got!r}, hardware {D[t, r, c]!r}")
        jobs = [(float(C[t, r, c]), A[t, r].copy(), B[t, :, c].copy(), float(D[t, r, c]), steps) for t, r, c in elems]
        with ProcessPoolExecutor(8) as ex:
            bits = list(ex.map(_refuted, jobs, chunksize=64))
        keep = []
        for i in range(len(H.RULES) - 1):
            hits = [j for j, bm in enumerate(bits) if bm >> i & 1]
            keep += list(rng.permutation(hits)[:PER_RULE])
            print(f"{name}: {H.RULES[i + 1]} refuted on {len(hits)} of {len(elems)}", flush=True)
        keep = sorted(set(keep) | set(rng.choice(len(elems), RANDOM, replace=False).tolist()))
        out[name + "_a"] = np.stack([A[elems[j][0], elems[j][1]] for j in keep])
        out[name + "_b"] = np.stack([B[elems[j][0], :, elems[j][2]] for j in keep])
        out[name + "_c"] = np.array([C[elems[j]] for j in keep], np.float32)
        out[name + "_d"] = np.array([D[elems[j]] for j in keep], np.float32)
        out[name + "_refutes"] = np.array([bits[j] for j in keep], np.uint8)
    np.savez_compressed(OUT, **out)
    print("wrote", OUT)


if __name__ == "__main__":
    if len(sys.argv) == 3 and sys.argv[1] == "--hw":
        hardware(sys.argv[2])
    elif len(sys.argv) == 2:
        select(sys.argv[1])
    else:
        raise SystemExit(__doc__)
