"""etx.api for the decode path: declaring native decode workloads (from dimensions or from a packed checkpoint), the
reference-shaped plan / emit / build / run records, and the errors the declaration checks raise before any device
memory is taken (reference etx/api/__init__.py:55-233, types.py:1-186, artifacts.py, models.py, runs.py)."""
import hashlib
import json

import pytest

from etx import api
from etx.api.types import WorkloadSpec
from etx.models import configs


def test_decode_workload_declares_native_kernel():
    w = api.decode_workload("tiny", {"H": 512, "NH": 4}, fused=False, seed=3)
    d = w.config.to_dict()
    assert w.kind == "native" and d["kernel"] == "decode"
    assert d["model"] == {"H": 512, "NH": 4} and d["run"] == {"fused": False, "seed": 3}


def test_unknown_options_refused():
    with pytest.raises(ValueError, match="unknown run options"):
        api.decode_workload("x", {}, turbo=True)
    with pytest.raises(ValueError, match="unknown model keys"):
        api.open_session(api.decode_workload("x", {"H": 512, "colour": 1}))
    with pytest.raises(TypeError):
        api.open_session({"kind": "native"})
    with pytest.raises(TypeError):
        api.build_model({"kind": "native"})


def test_checkpoint_workload_reads_dimensions(tmp_path, oracle_lib):
    from test_checkpoint import write_from_oracle
    cfg = configs.TINY_MOE
    write_from_oracle(tmp_path / "ck", cfg)
    w = api.checkpoint_workload(tmp_path / "ck", name="tiny", fused=True)
    d = w.config.to_dict()
    assert d["run"]["checkpoint"] == str(tmp_path / "ck")
    for k in ("H", "NH", "NKV", "HD", "L", "V", "E", "TOPK", "MI", "moe", "max_ctx"):
        assert d["model"][k] == getattr(cfg, k), k


@pytest.mark.gpu
def test_checkpoint_session_generates_oracle_tokens(gpu, tmp_path):
    """A session built from a checkpoint workload decodes the same greedy tokens as the oracle on the same weights."""
    from test_checkpoint import write_from_oracle, SEED
    from oracle import oracle as O
    cfg = configs.TINY_MOE
    write_from_oracle(tmp_path / "ck", cfg)
    sess = api.open_session(api.checkpoint_workload(tmp_path / "ck"))
    prompt = O.gen_tokens(SEED, 8, cfg.V)
    got = list(sess.run(prompt, 6))
    sess.close()
    orc = O.OracleModel(cfg.as_dict(), SEED, 0.02)
    seq = list(prompt)
    for pos in range(len(prompt) + 6 - 1):
        tok = orc.step(seq[pos], pos)
        if pos + 1 >= len(prompt):
            seq.append(tok)
    orc.close()
    assert got == seq[len(prompt):]


def _wl(cfg, **run):
    return api.decode_workload(cfg.name, cfg.as_dict(), **run)


def _plan(workload, **bindings):
    return api.plan(api.PlanRequest(workload, target=api.TARGET, bindings=bindings))


def test_plan_records_kernel_grid_and_phases():
    """plan() checks a workload against the library without a GPU: the persistent kernel it launches, one grid
    barrier per phase, the buffers, and a deterministic identity."""
    p = _plan(_wl(configs.QWEN3_30B_A3B))
    r = p.report.to_dict()
    assert r["kernel"] == "etxmk_fused_h2048_a4096_moe768_e128" and r["fused"] and r["workgroups"] == 256
    assert r["devices"] == 1 and p.machine["target"] == "gfx950"
    assert r["barriers_per_step"] == 6 * 48 + 1 == sum(len(x) for x in r["phases"])
    assert r["phases"][0] == ["qkv", "attn", "oproj", "router", "expert_up", "expert_down"] and r["phases"][-1] == ["head"]
    assert r["buffers"]["weights"] > 61e9 and any("LDS" in d for d in p.decisions)
    assert _plan(_wl(configs.QWEN3_30B_A3B)).identity == p.identity
    assert _plan(_wl(configs.QWEN3_30B_A3B), workgroups=128).identity != p.identity
    assert api.PlannedWorkload.from_dict(p.to_dict()).identity == p.identity
    ds = _plan(_wl(configs.with_layers(configs.DEEPSEEK_V2_LITE, 27, batch=4))).report.to_dict()
    assert ds["kernel"].startswith("etxmk_ds_b4") and ds["batch_capacity"] == 4
    assert ds["barriers_per_step"] == 7 + 8 * 26 + 1 == sum(len(x) for x in ds["phases"])
    assert ds["phases"][0][-2:] == ["gateup", "down"] and ds["phases"][1][-3:] == ["router_shared", "expert_up", "expert_down"]
    b16 = _plan(_wl(configs.QWEN3_30B_A3B), batch=16).report.to_dict()     # a binding overrides the batch
    # the attention merge and (matrix-core experts at batch 16) the expert combine are phases of their own
    assert b16["barriers_per_step"] == 8 * 48 + 1 == sum(len(x) for x in b16["phases"])
    assert b16["phases"][0] == ["qkv", "attn", "attn_merge", "oproj", "router", "expert_up", "expert_down", "combine"]
    b4 = _plan(_wl(configs.QWEN3_30B_A3B), batch=4).report.to_dict()
    assert b4["barriers_per_step"] == 7 * 48 + 1 and b4["phases"][0][-1] == "expert_down"
    f8 = _plan(_wl(configs.with_layers(configs.QWEN3_30B_A3B, 48, batch=16, wdtype=1)))
    assert f8.report["kernel"] == "etxmk_fused_fp8_b16_h2048_a4096_moe768_e128" and any("fp8" in d for d in f8.decisions)
    un = _plan(_wl(configs.TINY_MOE, fused=False)).report.to_dict()
    assert un["kernel"] == "unfused" and un["barriers_per_step"] == 6 * configs.TINY_MOE.L + 1
    mp = _plan(api.model("q30", config={"model": configs.QWEN3_30B_A3B.as_dict()}))   # kind='model' plans alike
    assert mp.report["kernel"] == r["kernel"] and mp.request.workload.kind == "model"


def test_plan_refusals_are_value_errors():
    with pytest.raises(ValueError, match="bf16"):
        _plan(_wl(configs.with_layers(configs.DEEPSEEK_V2_LITE, 27, wdtype=1)))
    with pytest.raises(ValueError, match="unfused"):
        _plan(_wl(configs.with_layers(configs.TINY_MOE, 2, batch=4), fused=False))
    with pytest.raises(ValueError, match="8"):
        _plan(_wl(configs.TINY_MOE), workgroups=4)
    with pytest.raises(ValueError, match="gfx950"):
        api.plan(api.PlanRequest(_wl(configs.TINY_MOE)))                 # the reference's default target gfx942
    with pytest.raises(ValueError, match="bindings"):
        _plan(_wl(configs.TINY_MOE), colour=3)
    with pytest.raises(ValueError):
        api.PlanRequest(_wl(configs.TINY_MOE), bindings={"batch": -1})
    with pytest.raises(TypeError):
        api.plan(_wl(configs.TINY_MOE))
    with pytest.raises(TypeError):
        api.PlanRequest({"name": "x"})
    with pytest.raises(ValueError, match="decode"):
        _plan(api.kernel(api.KernelSpec("gemm", "native", {"kernel": "gemm"})))


def test_emit_writes_a_timeline_schedule(tmp_path):
    """emit() gives the source artifact: plan.json in the layout the reference's timeline tool reads (types, one
    static task per (phase, workgroup) with its XCD as domain, one event per grid barrier whose producers are the
    phase before), decisions.txt, the rank's launch record and C header; save_sources writes manifest.json last and
    load_sources rejects a changed payload."""
    cfg = configs.TINY_MOE
    p = _plan(_wl(cfg), workgroups=16)
    art = api.emit(p)
    assert art.rank_sources == ("rank0.json",) and art.rank_headers == ("rank0.h",) and art.status == "SOURCES"
    d = tmp_path / "art"
    api.save_sources(art, d)
    back = api.load_sources(d)
    assert back.identity == art.identity and back.planned.identity == p.identity
    body = json.loads(back.files["plan.json"])
    nb, wg = p.report["barriers_per_step"], 16
    assert len(body["descs"]) == nb * wg == len(body["task_in"]) and len(body["ev_inst"]) == nb
    assert sorted(t["id"] for t in body["types"].values()) == list(range(len(body["types"])))
    assert body["domains"] == 8 and body["workers_per_domain"] == 2
    assert body["descs"][5 * wg + 3] == {"type": body["types"]["expert_down"]["id"], "coord": [0, 3, 0, 0],
                                         "domain": 3, "mode": "static"}
    prods = [e[2] for e in body["ev_inst"]]               # the timeline tool's dependency rule
    deps = [sorted({q for ev in evs for q in prods[ev]}) for evs in body["task_in"]]
    assert deps[0] == [] and deps[wg + 7] == list(range(wg)) and deps[2 * wg] == list(range(wg, 2 * wg))
    assert (d / "decisions.txt").read_text().splitlines() == list(p.decisions)
    launch = json.loads((d / "rank0.json").read_text())
    assert launch["kernel"] == p.report["kernel"] and launch["config"]["H"] == cfg.H and launch["plan"] == p.identity
    hdr = (d / "rank0.h").read_text()
    assert "ETXMK_PLAN_CONFIG = {512, 4, 2, 128," in hdr and '"etxmk_fused_h512_a512_moe256_e16"' in hdr
    (d / "plan.json").write_text((d / "plan.json").read_text().replace('"fused":true', '"fused":false'))
    with pytest.raises(ValueError, match="hash"):
        api.load_sources(d)
    with pytest.raises(ValueError):
        api.SourceArtifact(planned=p, files={"../x": ""}, rank_sources=("../x",), rank_headers=("y",))


def test_declarations_identity_is_canonical_json():
    """Identities are the sha256 of the record's canonical JSON (sorted keys, no whitespace), so a declaration
    written against the reference names the same workload; configurations are detached and immutable."""
    w = api.model("m", config={"b": [1, 2.5, None], "a": {"y": True, "x": "s"}})
    text = json.dumps(w.to_dict(), sort_keys=True, separators=(",", ":"), allow_nan=False)
    assert w.identity == hashlib.sha256(text.encode()).hexdigest()
    assert WorkloadSpec.from_dict(w.to_dict()) == w
    c = w.config
    got = c.to_dict()
    got["a"]["x"] = "changed"
    assert c["a"]["x"] == "s" and len(c) == 2 and sorted(c) == ["a", "b"]
    for bad in ({"x": float("nan")}, {1: 2}, {"x": object()}):
        with pytest.raises(ValueError):
            api.Configuration(bad)
    with pytest.raises(ValueError):
        WorkloadSpec(" padded", "native", {})
    with pytest.raises(ValueError):
        WorkloadSpec("x", "compiled", {})
    with pytest.raises(ValueError):
        WorkloadSpec("x", "native", {}, schema_version=2)
    with pytest.raises(ValueError):
        api.KernelSpec("k", "jit", {})
    with pytest.raises(TypeError):
        api.kernel("decode")
    ins = api.inspect(w)
    assert ins.identity == w.identity and ins.status == "DECLARED"


def _build_request(tmp_path, cfg, provider="native", **run):
    from pathlib import Path
    import etx.runtime.launcher as launcher
    w = api.model(cfg.name, config={"model": cfg.as_dict(), "run": run})
    root = Path(api.__file__).resolve().parents[3]
    return api.ModelBuildRequest(plan=api.PlanRequest(w, target=api.TARGET), root=str(root),
                                 output=str(tmp_path / "build"), host=launcher.__file__, provider=provider)


def test_model_build_and_artifact_run_records(tmp_path):
    """build_model(ModelBuildRequest) plans, saves the sources and writes the executable `run`; load_build reads the
    record back by identity; run_artifact refuses native execution unless asked for it and records a substitute
    executor's process evidence; read_artifact_run checks it."""
    cfg = configs.TINY_MOE
    rec = api.build_model(_build_request(tmp_path, cfg, seed=3))
    assert rec["status"] == "EXECUTABLE" and rec["provider"] == "native" and not rec["device_execution"]
    out = tmp_path / "build"
    b = api.load_build(out)
    assert b.identity == hashlib.sha256(api.types.canonical(rec.to_dict()).encode()).hexdigest()
    assert api.load_sources(out).identity == rec["source_identity"]
    assert (out / "run").stat().st_mode & 0o111
    req = api.ArtifactRunRequest(directory=str(out), build_identity=b.identity, cwd=str(tmp_path), deadline_s=60.0,
                                 arguments=("--new", "4"))
    with pytest.raises(ValueError, match="execute_native"):
        api.run_artifact(req, output=tmp_path / "r0")

    def scripted(preq, directory):
        (directory / "output.log").write_text('{"tokens": [1, 2, 3, 4]}\n')
        digest = hashlib.sha256((directory / "output.log").read_bytes()).hexdigest()
        return api.ProcessResult(request_identity=preq.identity, backend="scripted", status="complete", returncode=0,
                                 output_sha256=digest)
    with pytest.raises(ValueError):
        api.run_artifact(req, output=tmp_path / "r0", executor=scripted, execute_native=True)
    run = api.run_artifact(req, output=tmp_path / "r1", executor=scripted)
    assert run.process.status == "complete" and run.request == req
    assert api.read_artifact_run(tmp_path / "r1", request=req).identity == run.identity
    bad = api.ArtifactRunRequest(directory=str(out), build_identity="0" * 64, cwd=str(tmp_path), deadline_s=60.0)
    with pytest.raises(ValueError, match="identity"):
        api.run_artifact(bad, output=tmp_path / "r2", executor=scripted)
    with pytest.raises(api.BuildRefused):
        api.build_model(_build_request(tmp_path, cfg, provider="host-link"))
    with pytest.raises(api.BuildRefused, match="bf16"):
        api.build_model(_build_request(tmp_path, configs.with_layers(configs.TINY_MLA, 3, wdtype=1)))
    with pytest.raises(ValueError):
        api.ModelBuildRequest(plan=api.PlanRequest(_wl(cfg), target=api.TARGET), root=str(tmp_path),
                              output=str(tmp_path), host=str(tmp_path))          # not a kind='model' workload


@pytest.mark.gpu
def test_run_artifact_native_decodes_oracle_tokens(gpu, tmp_path):
    """The built artifact run natively (a child process on the GPU) prints the oracle's greedy tokens.  The workload
    runs unfused here: a child's cooperative launch was refused (hipErrorIllegalState) while this test process held its
    own context on the GPU; the unfused per-phase kernels are the same device functions."""
    from oracle import oracle as O
    cfg = configs.TINY_MOE
    rec = api.build_model(_build_request(tmp_path, cfg, seed=11, fused=False))
    out = tmp_path / "build"
    prompt = [int(t) for t in O.gen_tokens(11, 7, cfg.V)]
    req = api.ArtifactRunRequest(directory=str(out), build_identity=api.load_build(out).identity, cwd=str(tmp_path),
                                 deadline_s=240.0, arguments=("--tokens", ",".join(map(str, prompt)), "--new", "5"))
    run = api.run_artifact(req, output=tmp_path / "run", execute_native=True)
    log = (tmp_path / "run" / "output.log").read_text()
    assert run.process.status == "complete", log[-2000:]
    line = [ln for ln in log.splitlines() if ln.startswith("{")][-1]
    got = json.loads(line)["tokens"]
    orc = O.OracleModel(cfg.as_dict(), 11, 0.02)
    seq = list(prompt)
    for pos in range(len(prompt) + 5 - 1):
        tok = orc.step(seq[pos], pos)
        if pos + 1 >= len(prompt):
            seq.append(tok)
    orc.close()
    assert got == seq[len(prompt):] and rec["plan_identity"] == json.loads(line)["plan"]


@pytest.mark.gpu
@pytest.mark.parametrize("base,B", [(configs.TINY_MOE, 1), (configs.TINY_MLA, 4)], ids=["moe-b1", "mla-b4"])
def test_trace_step_rows(gpu, tmp_path, base, B):
    """A session's traced step: one nine-int64 row per (phase, workgroup) task in plan order, taken <= ready <= done,
    worker and coordinates as the plan's descs."""
    import numpy as np
    cfg = configs.with_layers(base, base.L, batch=B)
    sess = api.open_session(api.decode_workload(cfg.name, cfg.as_dict(), seed=7))
    for b in range(B):
        sess.decoder.set_tokens([3 + b, 5, 9, 11], seq=b)
    d = sess.trace_step(tmp_path / "tr", [3] * B)
    body = json.loads(api.load_sources(d).files["plan.json"])
    rows = np.frombuffer((d / "trace.bin").read_bytes(), "<i8").reshape(-1, 9)
    assert len(rows) == len(body["descs"])
    assert np.all(rows[:, 5] > 0) and np.all(rows[:, 5] <= rows[:, 6]) and np.all(rows[:, 6] <= rows[:, 7])
    assert [int(x) for x in rows[:, 0]] == [t["type"] for t in body["descs"]]
    assert [int(x) for x in rows[:, 2]] == [t["coord"][1] for t in body["descs"]] == [int(x) for x in rows[:, 8]]
    wg = body["workers_per_domain"] * body["domains"]
    assert np.all(rows[wg:, 5] >= rows[:-wg, 7] - 1)     # a workgroup takes phase k after its arrival from k-1
    sess.close()


def test_prompt_rows_default_to_library_limit(tmp_path, oracle_lib):
    """A workload whose model leaves `prefill` open reads prompts through the largest prefill launch the library
    accepts for its shape (16 rows, 4 for Qwen3-8B and DeepSeek-V2-Lite); one that sets it, or runs unfused, keeps
    its choice; a checkpoint workload leaves it open."""
    def prompts_line(cfg, model=None, **run):
        model = model if model is not None else {k: v for k, v in cfg.as_dict().items() if k != "prefill"}
        ds = _plan(api.decode_workload(cfg.name, model, **run)).decisions
        return [d for d in ds if d.startswith("prompts:")]
    assert prompts_line(configs.QWEN3_30B_A3B)[0].startswith("prompts: 16 positions")
    assert prompts_line(configs.QWEN3_8B)[0].startswith("prompts: 4 positions")
    assert prompts_line(configs.DEEPSEEK_V2_LITE)[0].startswith("prompts: 4 positions")
    assert prompts_line(configs.QWEN3_30B_A3B, configs.QWEN3_30B_A3B.as_dict()) == []      # prefill 0 set
    assert prompts_line(configs.QWEN3_30B_A3B, fused=False) == []
    from test_checkpoint import write_from_oracle
    write_from_oracle(tmp_path / "ck", configs.TINY_MOE)
    ds = _plan(api.checkpoint_workload(tmp_path / "ck")).decisions
    assert any(d.startswith("prompts: 16 positions") for d in ds)
