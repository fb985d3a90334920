"""etx.api for the decode path: declare a native decode workload and run it.

The reference declares `KernelSpec(name, implementation='native', config)` but rejects native providers
("Model/imported/native providers remain rejected until their adapters land", docs/core/API.md:51); here the
native provider is the gfx950 decode megakernel (libetxmk.so).  `build_model` mirrors
etx/api/__init__.py:67-70 (plan a model workload and link it); the returned session's `run` is the
per-token loop of examples/llm/host.hip:57-244.
"""
from __future__ import annotations

from dataclasses import dataclass

from etx.api.types import SCHEMA_VERSION, Configuration, KernelSpec, WorkloadSpec

__all__ = ["SCHEMA_VERSION", "Configuration", "KernelSpec", "WorkloadSpec", "DecodeSession", "build_model",
           "decode_workload", "checkpoint_workload"]

_MODEL_KEYS = {"H", "NH", "NKV", "HD", "L", "V", "I", "E", "TOPK", "MI", "moe", "qk_norm", "norm_topk",
               "block_size", "max_ctx", "batch", "eps", "theta"}
_RUN_KEYS = {"fused", "workgroups", "seed", "weight_scale", "checkpoint"}


def decode_workload(name: str, model: dict, **run) -> WorkloadSpec:
    """A native decode workload: model dimensions plus run options (fused, workgroups, seed, weight_scale, or
    checkpoint: a packed weights.bin + llm.manifest directory, whose weights replace the seeded ones)."""
    bad = set(run) - _RUN_KEYS
    if bad:
        raise ValueError(f"unknown run options {sorted(bad)}")
    return WorkloadSpec(name, "native", {"kernel": KernelSpec("decode", "native", {}).name, "model": model, "run": run})


@dataclass
class DecodeSession:
    """A built native decode workload bound to one GPU."""
    workload: WorkloadSpec
    decoder: object

    def run(self, prompt, n_new: int):
        return self.decoder.generate(prompt, n_new)

    def close(self):
        self.decoder.close()


def build_model(workload: WorkloadSpec, device: str = "cuda:0") -> DecodeSession:
    """Check a native decode workload, allocate its buffers on `device` and fill its weights.
    Errors are ValueError / TypeError like the reference's declaration checks."""
    if not isinstance(workload, WorkloadSpec):
        raise TypeError("build_model requires a WorkloadSpec")
    if workload.kind != "native":
        raise ValueError(f"workload kind {workload.kind!r}: only 'native' decode workloads are built here")
    cfg = workload.config.to_dict()
    if cfg.get("kernel") != "decode":
        raise ValueError("native workload must name the 'decode' kernel")
    model = cfg.get("model", {})
    bad = set(model) - _MODEL_KEYS
    if bad:
        raise ValueError(f"unknown model keys {sorted(bad)}")
    run = cfg.get("run", {})
    from etx.runtime.native import Decoder, ModelConfig
    mc = ModelConfig(name=workload.name, **model)
    ck = None
    if run.get("checkpoint"):
        from etx.models.checkpoint import Checkpoint
        ck = Checkpoint(run["checkpoint"])
        ck.check(mc)                           # dimensions and tensors agree before any device memory is taken
    dec = Decoder(mc, device=device, fused=bool(run.get("fused", True)), workgroups=int(run.get("workgroups", 0)))
    if ck is not None:
        ck.load_into(dec)
    else:
        dec.init_weights(int(run.get("seed", 0)), float(run.get("weight_scale", 0.02)))
    return DecodeSession(workload, dec)


def checkpoint_workload(path, name: str = "", max_ctx: int = 0, **run) -> WorkloadSpec:
    """The native decode workload of a packed checkpoint directory (dimensions from its llm.manifest)."""
    from etx.models.checkpoint import Checkpoint
    ck = Checkpoint(path)
    mc = ck.config(max_ctx=max_ctx)
    model = {k: v for k, v in mc.as_dict().items() if k in _MODEL_KEYS}
    return decode_workload(name or mc.name, model, checkpoint=str(path), **run)
