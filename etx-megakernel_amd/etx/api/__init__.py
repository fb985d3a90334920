"""etx.api for the decode path: the reference's declaration / plan / emit / build / run surface with the gfx950
decode megakernel (libetxmk.so) as its native provider.

The reference declares `KernelSpec(name, implementation='native', config)` but rejects native providers ("Model/
imported/native providers remain rejected until their adapters land", docs/core/API.md:51).  Here:

  model(name, config=...) / kernel(KernelSpec('decode', 'native', ...))  -> WorkloadSpec   (etx/api/__init__.py:225-228)
  plan(PlanRequest(workload, target='gfx950'))                        -> PlannedWorkload   (:216-218)
  emit(planned)                                                       -> SourceArtifact    (:186-188)
  save_sources(artifact, directory) / load_sources(directory)                              (:191-198)
  build_model(ModelBuildRequest(..., provider='native'))              -> Configuration     (:67-70)
  load_build(directory), run_artifact(ArtifactRunRequest, output=, execute_native=True) -> ArtifactRun (:160-167)

A decode workload's config is {"kernel": "decode", "model": <dimensions>, "run": <options>} (kind 'native'), or the
same without "kernel" (kind 'model').  The model dimensions are the fields of etx.runtime.native.ModelConfig; the
run options are fused, workgroups, seed, weight_scale and checkpoint (a packed weights.bin + llm.manifest directory).
Refusals are TypeError / ValueError like the reference's declaration checks (BuildRefused, a ValueError, for
builds).  `open_session` is this package's in-process form of a built workload (a Decoder on one GPU).
"""
from __future__ import annotations

import dataclasses
import hashlib
import json
import os
import platform
import subprocess
import sys
from collections.abc import Mapping
from dataclasses import dataclass
from pathlib import Path

import numpy as np

from etx.api.artifacts import SourceArtifact, payload_path
from etx.api.execution import ProcessRequest, ProcessResult
from etx.api.models import BuildRefused, ModelBuildRequest
from etx.api.runs import ArtifactRun, ArtifactRunRequest
from etx.api.types import (SCHEMA_VERSION, Configuration, Inspection, KernelSpec, PlannedWorkload, PlanRequest,
                           WorkloadSpec, canonical, digest)

__all__ = ["SCHEMA_VERSION", "Configuration", "Inspection", "KernelSpec", "PlanRequest", "PlannedWorkload",
           "WorkloadSpec", "SourceArtifact", "ModelBuildRequest", "BuildRefused", "ArtifactRunRequest", "ArtifactRun",
           "ProcessRequest", "ProcessResult", "model", "kernel", "inspect", "plan", "emit", "save_sources",
           "load_sources", "build_model", "load_build", "run_artifact", "read_artifact_run", "decode_workload",
           "checkpoint_workload", "open_session", "DecodeSession", "TARGET"]

TARGET = "gfx950"                                   # the one target this library is built for
_RUN_KEYS = {"fused", "workgroups", "seed", "weight_scale", "checkpoint"}
_BIND_KEYS = {"batch", "max_ctx", "prefill", "workgroups"}


def _model_keys() -> set:
    from etx.runtime.native import ModelConfig
    return {f.name for f in dataclasses.fields(ModelConfig)} - {"name"}


# ---------------------------------------------------------------- declarations
def model(name: str, *, config: Mapping) -> WorkloadSpec:
    """A kind='model' workload (reference etx/api/__init__.py:221-222)."""
    return WorkloadSpec(name=name, kind="model", config=Configuration(config))


def kernel(spec: KernelSpec) -> WorkloadSpec:
    """The workload of a kernel declaration (reference etx/api/__init__.py:225-228)."""
    if not isinstance(spec, KernelSpec):
        raise TypeError("kernel() takes a KernelSpec")
    return WorkloadSpec(name=spec.name, kind=spec.implementation, config=spec.config)


def inspect(subject: WorkloadSpec) -> Inspection:
    if not isinstance(subject, WorkloadSpec):
        raise TypeError("inspect() takes a WorkloadSpec")
    return Inspection(SCHEMA_VERSION, subject.identity, subject)


def decode_workload(name: str, model_dims: dict, **run) -> WorkloadSpec:
    """A native decode workload: model dimensions plus run options (fused, workgroups, seed, weight_scale, or
    checkpoint: a packed weights.bin + llm.manifest directory, whose weights replace the seeded ones)."""
    bad = set(run) - _RUN_KEYS
    if bad:
        raise ValueError(f"unknown run options {sorted(bad)}")
    return kernel(KernelSpec(name, "native", {"kernel": "decode", "model": dict(model_dims), "run": run}))


def checkpoint_workload(path, name: str = "", max_ctx: int = 0, **run) -> WorkloadSpec:
    """The native decode workload of a packed checkpoint directory (dimensions from its llm.manifest; the prompt
    rows per prefill launch are left to the library's default)."""
    from etx.models.checkpoint import Checkpoint
    ck = Checkpoint(path)
    mc = ck.config(max_ctx=max_ctx)
    dims = {k: v for k, v in mc.as_dict().items() if k in _model_keys() and k != "prefill"}
    return decode_workload(name or mc.name, dims, checkpoint=str(path), **run)


def _default_prefill(mc):
    """The prompt rows per prefill launch when the model leaves them open: the most the library accepts for this
    shape (16, else 4), or none.  Prefill is bit-identical to reading the prompt token by token."""
    from etx.runtime import native as N
    for rows in (16, 4):
        cand = dataclasses.replace(mc, prefill=rows)
        try:
            N.sizes(cand)
            return cand
        except N.EtxmkError:
            continue
    return mc


def _resolve(workload: WorkloadSpec, bindings: Mapping | None = None):
    """(ModelConfig, run options) of a decode workload, kind 'native' (kernel 'decode') or 'model'; bindings
    override batch, max_ctx, prefill and workgroups."""
    if not isinstance(workload, WorkloadSpec):
        raise TypeError("a WorkloadSpec is required")
    cfg = workload.config.to_dict()
    if workload.kind == "native":
        if cfg.get("kernel") != "decode":
            raise ValueError("a native workload here names the 'decode' kernel")
    elif workload.kind != "model":
        raise ValueError(f"workload kind {workload.kind!r}: this provider builds 'native' decode and 'model' workloads")
    extra = set(cfg) - {"kernel", "model", "run"}
    if extra:
        raise ValueError(f"unknown workload config keys {sorted(extra)}")
    dims = dict(cfg.get("model", {}))
    bad = set(dims) - _model_keys()
    if bad:
        raise ValueError(f"unknown model keys {sorted(bad)}")
    run = dict(cfg.get("run", {}))
    bad = set(run) - _RUN_KEYS
    if bad:
        raise ValueError(f"unknown run options {sorted(bad)}")
    b = dict(bindings or {})
    bad = set(b) - _BIND_KEYS
    if bad:
        raise ValueError(f"unknown bindings {sorted(bad)} (accepted: {sorted(_BIND_KEYS)})")
    for key in ("batch", "max_ctx", "prefill"):
        if key in b:
            dims[key] = b[key]
    if "workgroups" in b:
        run["workgroups"] = b["workgroups"]
    from etx.runtime import native as N
    try:
        mc = N.ModelConfig(name=workload.name, **dims)
    except TypeError as e:
        raise ValueError(str(e)) from None
    if "prefill" not in dims and bool(run.get("fused", True)):
        mc = _default_prefill(mc)
    return mc, run


# ---------------------------------------------------------------- plan
def _machine() -> dict:
    """The planning target: MI355X (gfx950) as this library is built for it."""
    return {"target": TARGET, "compute_units": 256, "xcds": 8, "wave_size": 64, "lds_bytes_per_cu": 163840,
            "hbm_bytes": 288 << 30, "hbm_GBps": 8000}


def _decisions(mc, run, info, wg) -> list:
    from etx.runtime import native as N
    fused = bool(run.get("fused", True))
    out = []
    if fused:
        out.append(f"one cooperative launch of {info['kernel']} per step: {wg} workgroups x {info['threads']} "
                   f"threads, {info['barriers_per_step']} grid barriers (one per phase)")
    else:
        out.append(f"unfused: one launch per phase ({info['barriers_per_step']} launches per step), the same device "
                   f"functions as the persistent kernel")
    out.append("weights: fp8 e4m3 rows with one fp32 scale per row (router, embedding, lm_head bf16)"
               if mc.wdtype == N.W_FP8 else "weights: bf16 rows, lane-permuted in blocks of 512")
    if mc.batch > 1 or mc.arch == N.ARCH_DSV2:
        out.append(f"batched kernel of capacity {info['batch_capacity']} for {mc.batch} sequence(s): every weight row "
                   f"streams once per step; each (row, sequence) dot keeps the single-sequence order")
    if mc.arch == N.ARCH_DSV2:
        out.append("multi-head latent attention, absorbed: W_UK^T per head before the attention, W_UV after the "
                   "merge; chunk items of 8 heads x 64 positions over the latent cache")
    else:
        R = -(-mc.nqkv // wg)                             # a workgroup's QKV rows; the library's staging rule
        S = min(R, 81920 // (2 * mc.H))
        staged = (fused and mc.batch == 1 and mc.wdtype == N.W_BF16 and mc.H % 512 == 0
                  and R - S <= (16 if mc.H >= 4096 else 0))
        out.append((f"QKV rows staged in LDS a layer ahead ({R} rows per workgroup)" if S == R else
                    f"QKV rows: {S} of each workgroup's {R} staged in LDS a layer ahead, {R - S} loaded into registers "
                    f"before the QKV phase's wait") if staged else "QKV rows streamed from HBM in the QKV phase")
        if mc.batch > 1:
            out.append(f"attention items: {mc.NKV} kv heads x two 64-position chunks per sequence, pipelined over "
                       f"double-buffered tiles; the merge is a phase of its own")
        else:
            out.append(f"attention items: {mc.NKV} kv heads x 64-position chunks x halves of the q-head group, "
                       f"last-arriver merge")
    if fused and mc.prefill:
        out.append(f"prompts: {max(mc.batch, mc.prefill)} positions per prefill launch of the batched kernel, "
                   f"bit-identical to reading them token by token")
    return out


def plan(request: PlanRequest) -> PlannedWorkload:
    """Check a decode workload against the library (no GPU needed) and record how a step runs: the persistent kernel
    (or the unfused per-phase kernels), the grid, the phases of every layer, the grid barriers, the buffer sizes and
    the decisions behind them (reference etx/api/__init__.py:216-218).  Refusals are ValueError."""
    if not isinstance(request, PlanRequest):
        raise TypeError("plan() takes a PlanRequest")
    if request.target != TARGET:
        raise ValueError(f"target {request.target!r}: this library is built for {TARGET} only")
    from etx.runtime import native as N
    mc, run = _resolve(request.workload, request.bindings)
    fused = bool(run.get("fused", True))
    wg = int(run.get("workgroups", 0)) or 256
    if wg < 8:
        raise ValueError(f"grid of {wg} workgroups is below the 8 the grid barrier needs")
    try:
        info = N.plan_info(mc, fused)
    except N.EtxmkError as e:
        raise ValueError(str(e)) from None
    lib = N.LIB_PATH
    report = {
        "devices": 1, "kernel": info["kernel"], "fused": fused, "threads": info["threads"], "workgroups": wg,
        "batch_capacity": info["batch_capacity"], "barriers_per_step": info["barriers_per_step"],
        "phases": N.phase_names(mc),
        "buffers": {"weights": info["weight_bytes"], "kv": info["kv_bytes"], "workspace": info["workspace_bytes"]},
        "config": {k: v for k, v in mc.as_dict().items()},
        "library": {"file": lib.name, "sha256": hashlib.sha256(lib.read_bytes()).hexdigest() if lib.exists() else None},
    }
    options = dict(request.options.to_dict(), run=run)
    return PlannedWorkload(request=request, machine=_machine(), options=options, report=report,
                           decisions=tuple(_decisions(mc, run, info, wg)))


# ---------------------------------------------------------------- emit / sources
def _schedule(planned: PlannedWorkload) -> dict:
    """The plan in the layout of the reference's plan.json that its timeline tool reads (etx/tools/timeline.py:
    99-139): task types, one static task per (phase, workgroup) on domain (XCD) workgroup % 8, and one event per
    grid barrier whose producers are every task of the phase before."""
    r = planned.report.to_dict()
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


_CONFIG_FIELDS = ("H", "NH", "NKV", "HD", "I", "E", "TOPK", "MI", "L", "V", "moe", "qk_norm", "norm_topk",
                  "block_size", "max_ctx", "batch", "eps", "theta", "wdtype", "arch", "kv_lora", "qk_nope", "qk_rope",
                  "v_head", "n_shared", "first_dense", "dense_I", "routed_scale", "rope_factor", "rope_mscale",
                  "rope_mscale_all", "beta_fast", "beta_slow", "rope_orig_max", "prefill")


def _rank_header(planned: PlannedWorkload) -> str:
    """A C header a host includes to launch this workload through include/etxmk.h: the etxmk_config initializer in
    the struct's field order, the kernel the step launches and the grid."""
    r = planned.report.to_dict()
    c = r["config"]
    vals = []
    for f in _CONFIG_FIELDS:
        v = c.get(f, 0)
        vals.append(repr(float(v)) + "f" if isinstance(v, float) else str(int(v)))
    guard = "ETXMK_PLAN_" + planned.identity[:16].upper()
    return (f"/* emitted by etx.api.emit for workload {planned.request.workload.name!r}; plan {planned.identity} */\n"
            f"#ifndef {guard}\n#define {guard}\n#include \"etxmk.h\"\n"
            f"#define ETXMK_PLAN_KERNEL \"{r['kernel']}\"\n#define ETXMK_PLAN_WORKGROUPS {r['workgroups']}\n"
            f"#define ETXMK_PLAN_FUSED {int(r['fused'])}\n"
            f"static const etxmk_config ETXMK_PLAN_CONFIG = {{{', '.join(vals)}}};\n#endif\n")


def emit(planned: PlannedWorkload) -> SourceArtifact:
    """The planned workload's source artifact (reference etx/api/__init__.py:186-188): plan.json (the planned record
    and its schedule in the layout of the reference's plan.json), decisions.txt, and per rank the launch record
    rank0.json and the C header rank0.h."""
    if not isinstance(planned, PlannedWorkload):
        raise TypeError("emit() takes a PlannedWorkload")
    r = planned.report.to_dict()
    body = dict(planned.to_dict(), **_schedule(planned))
    launch = {"plan": planned.identity, "workload": planned.request.workload.to_dict(), "kernel": r["kernel"],
              "fused": r["fused"], "workgroups": r["workgroups"], "config": r["config"],
              "run": planned.options.to_dict().get("run", {}), "buffers": r["buffers"], "library": r["library"]}
    files = {"plan.json": canonical(body), "decisions.txt": "\n".join(planned.decisions) + "\n",
             "rank0.json": canonical(launch), "rank0.h": _rank_header(planned)}
    return SourceArtifact(planned=planned, files=files, rank_sources=("rank0.json",), rank_headers=("rank0.h",))


def save_sources(artifact: SourceArtifact, directory) -> SourceArtifact:
    """Write the artifact's payloads into `directory` (created if needed), then manifest.json last."""
    if not isinstance(artifact, SourceArtifact):
        raise TypeError("save_sources() takes a SourceArtifact")
    d = Path(directory)
    d.mkdir(parents=True, exist_ok=True)
    for name, text in artifact.files.items():
        path = d / payload_path(name)
        path.parent.mkdir(parents=True, exist_ok=True)
        path.write_text(text)
    (d / "manifest.json").write_text(canonical(dict(artifact.manifest(), identity=artifact.identity)))
    return artifact


def load_sources(directory) -> SourceArtifact:
    """Read a saved artifact back: every payload's hash and the artifact's identity are checked (ValueError)."""
    d = Path(directory)
    man = json.loads((d / "manifest.json").read_text())
    files = {}
    for name, want in man["payloads"].items():
        text = (d / payload_path(name)).read_text()
        if hashlib.sha256(text.encode()).hexdigest() != want:
            raise ValueError(f"{name}: payload hash mismatch")
        files[name] = text
    art = SourceArtifact(planned=PlannedWorkload.from_dict(man["planned"]), files=files,
                         rank_sources=tuple(man["rank_sources"]), rank_headers=tuple(man["rank_headers"]),
                         external_sources=tuple(man["external_sources"]), status=man["status"],
                         schema_version=man["schema_version"])
    if art.identity != man.get("identity"):
        raise ValueError("artifact identity mismatch")
    return art


# ---------------------------------------------------------------- builds and runs
_LAUNCHER = '''#!{python}
"""Runs the decode workload of this directory's rank0.json on the local GPU (written by etx.api.build_model)."""
import sys
sys.path.insert(0, {pkg!r})
from etx.runtime import launcher
sys.exit(launcher.main({directory!r}, sys.argv[1:]))
'''


@dataclass(frozen=True)
class BuildRecord:
    """A built model artifact as load_build reads it: the record build_model returned, and its identity."""
    directory: str
    record: Configuration

    @property
    def status(self) -> str:
        return self.record["status"]

    @property
    def identity(self) -> str:
        return digest(self.record.to_dict())


def build_model(request: ModelBuildRequest) -> Configuration:
    """Plan a kind='model' decode workload and produce its executable (reference etx/api/__init__.py:67-70).  The
    native provider ('native') compiles nothing: it plans, saves the source artifact into request.output and writes
    `run`, a launcher over the prebuilt library that runs the workload's rank0.json.  The record names the plan and
    source identities and the executable; status 'EXECUTABLE' is not device qualification.  Other providers (the
    reference's 'host-link', 'dsv2lite') link generated code this package does not have: BuildRefused."""
    if not isinstance(request, ModelBuildRequest):
        raise TypeError("build_model() takes a ModelBuildRequest")
    if request.provider != "native":
        raise BuildRefused(f"provider {request.provider!r}: this package builds the 'native' decode provider only")
    root, out = Path(request.root), Path(request.output)
    if not root.is_dir() or not Path(request.host).is_file():
        raise BuildRefused("model build root or host file is missing")
    try:
        planned = plan(request.plan)
    except ValueError as e:
        raise BuildRefused(str(e)) from None
    artifact = emit(planned)
    out.mkdir(parents=True, exist_ok=True)
    save_sources(artifact, out)
    pkg = str(Path(__file__).resolve().parents[2])
    run = out / "run"
    run.write_text(_LAUNCHER.format(python=sys.executable, pkg=pkg, directory=str(out.resolve())))
    run.chmod(0o755)
    record = {"schema_version": SCHEMA_VERSION, "kind": "model-build", "provider": request.provider,
              "plan_identity": planned.identity, "source_identity": artifact.identity, "compiler": None,
              "host": request.host, "library": planned.report["library"], "executable": str(run),
              "executable_sha256": hashlib.sha256(run.read_bytes()).hexdigest(), "exit": 0, "status": "EXECUTABLE",
              "device_execution": False}
    (out / "build.json").write_text(canonical(record))
    return Configuration(record)


def load_build(directory) -> BuildRecord:
    d = Path(directory)
    rec = Configuration(json.loads((d / "build.json").read_text()))
    run = d / "run"
    if rec["status"] == "EXECUTABLE" and (not run.is_file() or
                                          hashlib.sha256(run.read_bytes()).hexdigest() != rec["executable_sha256"]):
        raise ValueError("the build's executable is missing or changed")
    return BuildRecord(str(d), rec)


def _write_json(path: Path, value) -> None:
    path.write_text(json.dumps(value, sort_keys=True, indent=2) + "\n")


def _execute(req: ProcessRequest, directory: Path) -> ProcessResult:
    """Run the process with its deadline; the output goes to output.log."""
    directory.mkdir(parents=True, exist_ok=True)
    env = dict(os.environ, **req.environment.to_dict())
    log = directory / "output.log"
    events = []
    with open(log, "wb") as f:
        try:
            p = subprocess.run(list(req.argv), cwd=req.cwd, env=env, stdout=f, stderr=subprocess.STDOUT,
                               timeout=req.deadline_s)
            rc, status = p.returncode, "complete" if p.returncode == 0 else "failed"
        except subprocess.TimeoutExpired:
            rc, status = 124, "deadline"
            events.append(f"deadline of {req.deadline_s} s reached")
    out = hashlib.sha256(log.read_bytes()).hexdigest()
    return ProcessResult(request_identity=req.identity, backend="host-process", status=status, returncode=rc,
                         output_sha256=out, events=tuple(events))


def run_artifact(request: ArtifactRunRequest, *, output, executor=None, execute_native=False) -> ArtifactRun:
    """Run a built model artifact (reference etx/api/__init__.py:160-162): the executable `run` of the build named by
    directory and identity, with its arguments and deadline; evidence (request.json, result.json, output.log,
    artifact_run.json) goes to `output`.  Native execution (the local GPU) must be asked for with
    execute_native=True; `executor(process_request, output_dir) -> ProcessResult` substitutes for it."""
    if not isinstance(request, ArtifactRunRequest):
        raise TypeError("run_artifact() takes an ArtifactRunRequest")
    if type(execute_native) is not bool:
        raise ValueError("execute_native must be a boolean")
    if executor is None and not execute_native:
        raise ValueError("running the artifact natively needs execute_native=True")
    if executor is not None and execute_native:
        raise ValueError("a substitute executor cannot also run natively")
    build = load_build(request.directory)
    if build.identity != request.build_identity:
        raise ValueError("artifact build identity mismatch")
    if build.status != "EXECUTABLE":
        raise ValueError("the artifact is not executable")
    if executor is None and (platform.system() != "Linux" or platform.machine() != "x86_64"):
        raise ValueError("the artifact runs on a Linux x86-64 host")
    d = Path(output).absolute()
    d.mkdir(parents=True, exist_ok=True)
    preq = request.process_request()
    _write_json(d / "request.json", preq.to_dict())
    result = executor(preq, d) if executor is not None else _execute(preq, d)
    if not isinstance(result, ProcessResult):
        raise TypeError("the executor must return a ProcessResult")
    _write_json(d / "result.json", result.to_dict())
    rec = ArtifactRun(request, result)
    _write_json(d / "artifact_run.json", dict(rec.to_dict(), identity=rec.identity))
    return rec


def read_artifact_run(directory, *, request: ArtifactRunRequest) -> ArtifactRun:
    if not isinstance(request, ArtifactRunRequest):
        raise TypeError("read_artifact_run() takes an ArtifactRunRequest")
    d = Path(directory)
    data = json.loads((d / "artifact_run.json").read_text())
    rec = ArtifactRun(ArtifactRunRequest(**{k: (tuple(v) if k == "arguments" else v) for k, v in data["request"].items()}),
                      ProcessResult(**{k: (tuple(v) if k == "events" else v) for k, v in data["process"].items()}),
                      schema_version=data["schema_version"])
    if rec.request != request or rec.identity != data["identity"]:
        raise ValueError("artifact run identity mismatch")
    if hashlib.sha256((d / "output.log").read_bytes()).hexdigest() != rec.process.output_sha256:
        raise ValueError("artifact run output does not match its evidence")
    return rec


# ---------------------------------------------------------------- in-process sessions
@dataclass
class DecodeSession:
    """A decode workload bound to one GPU in this process."""
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
        arrival, worker = workgroup; 10 ns ticks; etx/tools/timeline.py:1-33) beside the source artifact of this
        session's plan."""
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
        planned = plan(PlanRequest(self.workload, target=TARGET, bindings={"workgroups": wg}))
        d = Path(directory)
        save_sources(emit(planned), d)
        sched = _schedule(planned)
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


def open_session(workload: WorkloadSpec, device: str = "cuda:0") -> DecodeSession:
    """Check a decode workload, allocate its buffers on `device` and fill its weights (seeded, or from the
    workload's checkpoint).  Errors are ValueError / TypeError like the reference's declaration checks."""
    mc, run = _resolve(workload)
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
