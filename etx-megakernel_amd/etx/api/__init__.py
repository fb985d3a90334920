"""etx.api for the decode path: declare a native decode workload and run it.

The reference declares `KernelSpec(name, implementation='native', config)` but rejects native providers
("Model/imported/native providers remain rejected until their adapters land", docs/core/API.md:51); here the
native provider is the gfx950 decode megakernel (libetxmk.so).  `plan` / `emit` mirror the reference's planned
workload and source artifact records (docs/core/API.md:47-50: a deterministic identity, the plan JSON and its
decisions, a manifest written last), `build_model` mirrors etx/api/__init__.py:67-70 (plan a model workload and
link it); the returned session's `run` is the per-token loop of examples/llm/host.hip:57-244, and its
`trace_step` writes one step's phase timeline in the raw row format of the reference's timeline tool
(etx/tools/timeline.py:1-33: nine int64 per task, 10 ns ticks, with the plan's types, descs and dependencies).
"""
from __future__ import annotations

import dataclasses
import hashlib
import json
from dataclasses import dataclass
from pathlib import Path

import numpy as np

from etx.api.types import SCHEMA_VERSION, Configuration, KernelSpec, WorkloadSpec

__all__ = ["SCHEMA_VERSION", "Configuration", "KernelSpec", "WorkloadSpec", "DecodeSession", "PlannedWorkload",
           "build_model", "decode_workload", "checkpoint_workload", "plan", "emit", "load_sources"]


def _model_keys() -> set:
    from etx.runtime.native import ModelConfig
    return {f.name for f in dataclasses.fields(ModelConfig)} - {"name"}


_RUN_KEYS = {"fused", "workgroups", "seed", "weight_scale", "checkpoint"}
_CANON = dict(sort_keys=True, separators=(",", ":"), allow_nan=False)


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

    def run_batch(self, prompts, n_new: int):
        return self.decoder.generate_batch(prompts, n_new)

    def trace_step(self, directory, positions) -> Path:
        """Run one traced step at `positions` (one per sequence) and write its timeline: trace.bin (nine int64 per
        (phase, workgroup) task: type, coord[4] = (layer, workgroup, 0, 0), taken = the workgroup's arrival after
        the phase before (the launch for the first), deps ready = its barrier wait returned, body done = its
        arrival, worker = workgroup; 10 ns ticks) beside the plan artifact of this session's grid."""
        dec = self.decoder
        if not self.workload.config.to_dict().get("run", {}).get("fused", True):
            raise ValueError("the phase timeline is recorded by the persistent kernel (fused workloads)")
        pos = [int(p) for p in np.atleast_1d(positions)]
        dec.enable_trace(True)
        if dec.cfg.batch == 1 and len(pos) == 1:
            dec.step(pos[0], write_next=False)
        else:
            dec.step_batch(pos, write_next=False)
        t = dec.trace_ticks().astype(np.int64)
        dec.enable_trace(False)
        wg = t.shape[1]
        d = emit(plan(self.workload, workgroups=wg), directory)
        sched = json.loads((d / "plan.json").read_text())
        nb = t.shape[0] - 1                               # phases ending in a barrier
        rows = np.zeros((nb, wg, 9), np.int64)
        for k in range(nb):
            rows[k, :, 0] = sched["descs"][k * wg]["type"]
            rows[k, :, 1] = sched["descs"][k * wg]["coord"][0]
            rows[k, :, 2] = np.arange(wg)
            rows[k, :, 5] = t[0, :, 0] if k == 0 else t[k - 1, :, 1]
            rows[k, :, 6] = t[0, :, 0] if k == 0 else t[k, :, 0]
            rows[k, :, 7] = t[k, :, 1]
            rows[k, :, 8] = np.arange(wg)
        (d / "trace.bin").write_bytes(rows.reshape(-1, 9).astype("<i8").tobytes())
        return d

    def close(self):
        self.decoder.close()


def _checked(workload: WorkloadSpec):
    """(model config, run options) of a native decode workload; ValueError / TypeError as the reference's checks."""
    if not isinstance(workload, WorkloadSpec):
        raise TypeError("a WorkloadSpec is required")
    if workload.kind != "native":
        raise ValueError(f"workload kind {workload.kind!r}: only 'native' decode workloads are built here")
    cfg = workload.config.to_dict()
    if cfg.get("kernel") != "decode":
        raise ValueError("native workload must name the 'decode' kernel")
    model = cfg.get("model", {})
    bad = set(model) - _model_keys()
    if bad:
        raise ValueError(f"unknown model keys {sorted(bad)}")
    run = cfg.get("run", {})
    from etx.runtime import native as N
    mc = N.ModelConfig(name=workload.name, **model)
    if "prefill" not in model and bool(run.get("fused", True)):
        mc = _default_prefill(mc)
    return mc, run


def _default_prefill(mc):
    """The prompt rows per prefill launch when the model leaves them open: the most the library accepts for this
    shape (16, else 4), or none.  Prefill is bit-identical to reading the prompt token by token."""
    import dataclasses
    from etx.runtime import native as N
    for rows in (16, 4):
        cand = dataclasses.replace(mc, prefill=rows)
        try:
            N.sizes(cand)
            return cand
        except N.EtxmkError:
            continue
    return mc


@dataclass(frozen=True)
class PlannedWorkload:
    """A checked native decode workload and its plan record (kernel, grid, phases, buffers, decisions)."""
    workload: WorkloadSpec
    record: Configuration

    def to_dict(self) -> dict:
        return {"workload": self.workload.to_dict(), "plan": self.record.to_dict()}

    @property
    def identity(self) -> str:
        return hashlib.sha256(json.dumps(self.to_dict(), **_CANON).encode()).hexdigest()


def plan(workload: WorkloadSpec, workgroups: int = 256) -> PlannedWorkload:
    """Check a native decode workload against the library (no GPU needed) and record how a step runs: the
    persistent kernel (or the unfused per-phase kernels), the grid, the phases of every layer, the grid barriers,
    the three buffer sizes and the decisions behind them.  Refusals are ValueError with the library's message."""
    from etx.runtime import native as N
    mc, run = _checked(workload)
    fused = bool(run.get("fused", True))
    wg = int(run.get("workgroups", 0)) or int(workgroups)
    if wg < 8:
        raise ValueError(f"grid of {wg} workgroups is below the 8 the grid barrier needs")
    try:
        info = N.plan_info(mc, fused)
    except N.EtxmkError as e:
        raise ValueError(str(e)) from None
    phases = N.phase_names(mc)
    decisions = []
    if fused:
        decisions.append(f"one cooperative launch of {info['kernel']} per step: {wg} workgroups x {info['threads']} "
                         f"threads, {info['barriers_per_step']} grid barriers (one per phase)")
    else:
        decisions.append(f"unfused: one launch per phase ({info['barriers_per_step']} launches per step), the same "
                         f"device functions as the persistent kernel")
    decisions.append("weights: fp8 e4m3 rows with one fp32 scale per row (router, embedding, lm_head bf16)"
                     if mc.wdtype == N.W_FP8 else "weights: bf16 rows, lane-permuted in blocks of 512")
    if mc.batch > 1 or mc.arch == N.ARCH_DSV2:
        decisions.append(f"batched kernel of capacity {info['batch_capacity']} for {mc.batch} sequence(s): every "
                         f"weight row streams once per step; each (row, sequence) dot keeps the single-sequence order")
    if mc.arch == N.ARCH_DSV2:
        decisions.append("multi-head latent attention, absorbed: W_UK^T per head before the attention, W_UV after "
                         "the merge; chunk items of 8 heads x 64 positions over the latent cache")
    else:
        R = -(-mc.nqkv // wg)                             # a workgroup's QKV rows; the library's staging rule
        S = min(R, 81920 // (2 * mc.H))
        staged = (fused and mc.batch == 1 and mc.wdtype == N.W_BF16 and mc.H % 512 == 0
                  and R - S <= (16 if mc.H >= 4096 else 0))
        decisions.append((f"QKV rows staged in LDS a layer ahead ({R} rows per workgroup)" if S == R else
                          f"QKV rows: {S} of each workgroup's {R} staged in LDS a layer ahead, {R - S} loaded into "
                          f"registers before the QKV phase's wait") if staged
                         else "QKV rows streamed from HBM in the QKV phase")
        if mc.batch > 1:
            decisions.append(f"attention items: {mc.NKV} kv heads x two 64-position chunks per sequence, pipelined over "
                             f"double-buffered tiles; the merge is a phase of its own")
        else:
            decisions.append(f"attention items: {mc.NKV} kv heads x 64-position chunks, last-arriver merge")
    if fused and mc.prefill:
        decisions.append(f"prompts: {max(mc.batch, mc.prefill)} positions per prefill launch of the batched kernel, "
                         f"bit-identical to reading them token by token")
    lib = N.LIB_PATH
    record = {
        "schema_version": SCHEMA_VERSION, "workload": workload.identity, "kernel": info["kernel"], "fused": fused,
        "threads": info["threads"], "workgroups": wg, "batch_capacity": info["batch_capacity"],
        "barriers_per_step": info["barriers_per_step"], "phases": phases,
        "buffers": {"weights": info["weight_bytes"], "kv": info["kv_bytes"], "workspace": info["workspace_bytes"]},
        "decisions": decisions,
        "library": {"file": lib.name, "sha256": hashlib.sha256(lib.read_bytes()).hexdigest() if lib.exists() else None},
    }
    return PlannedWorkload(workload, Configuration(record))


def _schedule(planned: PlannedWorkload) -> dict:
    """The plan in the layout of the reference's plan.json that its timeline tool reads (etx/tools/timeline.py:
    99-139): task types, one static task per (phase, workgroup) on domain (XCD) workgroup % 8, and one event per
    grid barrier whose producers are every task of the phase before."""
    r = planned.record.to_dict()
    wg = r["workgroups"]
    flat = [(layer, name) for layer, names in enumerate(r["phases"]) for name in names]
    types = {}
    for _, name in flat:
        types.setdefault(name, {"id": len(types)})
    descs, ev_inst, task_in = [], [], []
    for k, (layer, name) in enumerate(flat):
        for w in range(wg):
            descs.append({"type": types[name]["id"], "coord": [layer, w, 0, 0], "domain": w % 8, "mode": "static"})
            task_in.append([k - 1] if k > 0 else [])
        ev_inst.append([k, "grid_barrier", list(range(k * wg, (k + 1) * wg))])
    return {"types": types, "descs": descs, "domains": 8, "workers_per_domain": -(-wg // 8), "ev_inst": ev_inst,
            "task_in": task_in}


def emit(planned: PlannedWorkload, directory) -> Path:
    """Write the planned workload's artifact into a new directory: plan.json (the record and the schedule in the
    reference's plan.json layout), decisions.txt, and manifest.json last (identity and sha256 of every payload)."""
    d = Path(directory)
    d.mkdir(parents=True, exist_ok=False)
    body = dict(planned.to_dict(), **_schedule(planned))
    payloads = {"plan.json": json.dumps(body, **_CANON).encode(),
                "decisions.txt": ("\n".join(planned.record.to_dict()["decisions"]) + "\n").encode()}
    for name, data in payloads.items():
        (d / name).write_bytes(data)
    manifest = {"identity": planned.identity, "payloads": {n: hashlib.sha256(b).hexdigest() for n, b in payloads.items()}}
    (d / "manifest.json").write_text(json.dumps(manifest, **_CANON))
    return d


def load_sources(directory) -> dict:
    """Read an emitted artifact back, checking every payload hash and the plan's identity; returns plan.json."""
    d = Path(directory)
    manifest = json.loads((d / "manifest.json").read_text())
    for name, digest in manifest["payloads"].items():
        if hashlib.sha256((d / name).read_bytes()).hexdigest() != digest:
            raise ValueError(f"{name}: payload hash mismatch")
    body = json.loads((d / "plan.json").read_text())
    ident = hashlib.sha256(json.dumps({"workload": body["workload"], "plan": body["plan"]}, **_CANON).encode()).hexdigest()
    if ident != manifest["identity"]:
        raise ValueError("plan identity mismatch")
    return body


def build_model(workload: WorkloadSpec, device: str = "cuda:0") -> DecodeSession:
    """Check a native decode workload, allocate its buffers on `device` and fill its weights.
    Errors are ValueError / TypeError like the reference's declaration checks."""
    if not isinstance(workload, WorkloadSpec):
        raise TypeError("build_model requires a WorkloadSpec")
    mc, run = _checked(workload)
    from etx.runtime.native import Decoder
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
    model = {k: v for k, v in mc.as_dict().items() if k in _model_keys()}
    return decode_workload(name or mc.name, model, checkpoint=str(path), **run)
