"""The program behind a built model artifact's `run` (etx.api.build_model): decodes the directory's rank0.json
workload on the local GPU and prints one JSON line.

    run [--tokens 1,2,3 | --prompt-len N] [--new N] [--prompt-seed S]

The prompt is the given token ids, or N seeded uniform ids in [0, vocabulary); the weights are the workload's
(seeded, or its checkpoint).  The printed line holds the prompt, the generated greedy tokens and the decode time per
token.  Reference: the model hosts' per-token loop (examples/llm/host.hip:203-229), which prints tokens and timing.
"""
from __future__ import annotations

import argparse
import json
import sys
import time
from pathlib import Path

import numpy as np


def main(directory: str, argv: list) -> int:
    ap = argparse.ArgumentParser(prog="run")
    ap.add_argument("--tokens", default="", help="comma-separated prompt token ids")
    ap.add_argument("--prompt-len", type=int, default=16)
    ap.add_argument("--prompt-seed", type=int, default=0)
    ap.add_argument("--new", type=int, default=8)
    a = ap.parse_args(argv)
    launch = json.loads((Path(directory) / "rank0.json").read_text())
    from etx.runtime import native as N
    cfg = N.ModelConfig(**launch["config"])
    run = launch["run"]
    if cfg.batch != 1:
        print(json.dumps({"error": "the launcher runs single-sequence workloads"}), flush=True)
        return 2
    dec = N.Decoder(cfg, fused=bool(launch["fused"]), workgroups=int(run.get("workgroups", 0)))
    try:
        if run.get("checkpoint"):
            from etx.models.checkpoint import Checkpoint
            Checkpoint(run["checkpoint"]).load_into(dec)
        else:
            dec.init_weights(int(run.get("seed", 0)), float(run.get("weight_scale", 0.02)))
        if a.tokens:
            prompt = [int(t) for t in a.tokens.split(",")]
        else:
            prompt = [int(t) for t in np.random.default_rng(a.prompt_seed).integers(0, cfg.V, a.prompt_len)]
        t0 = time.perf_counter()
        toks = dec.generate(prompt, a.new)
        dt = time.perf_counter() - t0
        print(json.dumps({"plan": launch["plan"], "kernel": launch["kernel"], "prompt": prompt,
                          "tokens": [int(t) for t in toks], "seconds": round(dt, 6)}), flush=True)
    finally:
        dec.close()
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1], sys.argv[2:]))
