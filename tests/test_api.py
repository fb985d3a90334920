"""etx.api for the decode path: declaring native decode workloads (from dimensions or from a packed checkpoint) and the
errors the declaration checks raise before any device memory is taken (etx/api/__init__.py:55-233, types.py:56-98)."""
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
        api.build_model(api.decode_workload("x", {"H": 512, "colour": 1}))
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
    sess = api.build_model(api.checkpoint_workload(tmp_path / "ck"))
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


def test_plan_records_kernel_grid_and_phases():
    """plan() checks a workload against the library without a GPU: the persistent kernel it launches, one grid
    barrier per phase, the buffers, and a deterministic identity."""
    p = api.plan(_wl(configs.QWEN3_30B_A3B))
    r = p.record.to_dict()
    assert r["kernel"] == "etxmk_fused_h2048_a4096_moe768_e128" and r["fused"] and r["workgroups"] == 256
    assert r["barriers_per_step"] == 6 * 48 + 1 == sum(len(x) for x in r["phases"])
    assert r["phases"][0] == ["qkv", "attn", "oproj", "router", "expert_up", "expert_down"] and r["phases"][-1] == ["head"]
    assert r["buffers"]["weights"] > 61e9 and any("LDS" in d for d in r["decisions"])
    assert api.plan(_wl(configs.QWEN3_30B_A3B)).identity == p.identity
    assert api.plan(_wl(configs.QWEN3_30B_A3B), workgroups=128).identity != p.identity
    ds = api.plan(_wl(configs.with_layers(configs.DEEPSEEK_V2_LITE, 27, batch=4))).record.to_dict()
    assert ds["kernel"].startswith("etxmk_ds_b4") and ds["batch_capacity"] == 4
    assert ds["barriers_per_step"] == 7 + 8 * 26 + 1 == sum(len(x) for x in ds["phases"])
    assert ds["phases"][0][-2:] == ["gateup", "down"] and ds["phases"][1][-3:] == ["router_shared", "expert_up", "expert_down"]
    b16 = api.plan(_wl(configs.with_layers(configs.QWEN3_30B_A3B, 48, batch=16))).record.to_dict()
    assert b16["barriers_per_step"] == 7 * 48 + 1 == sum(len(x) for x in b16["phases"])   # the merge phase
    assert b16["phases"][0][:4] == ["qkv", "attn", "attn_merge", "oproj"]
    f8 = api.plan(_wl(configs.with_layers(configs.QWEN3_30B_A3B, 48, batch=16, wdtype=1))).record.to_dict()
    assert f8["kernel"] == "etxmk_fused_fp8_b16_h2048_a4096_moe768_e128" and any("fp8" in d for d in f8["decisions"])
    un = api.plan(_wl(configs.TINY_MOE, fused=False)).record.to_dict()
    assert un["kernel"] == "unfused" and un["barriers_per_step"] == 6 * configs.TINY_MOE.L + 1


def test_plan_refusals_are_value_errors():
    with pytest.raises(ValueError, match="bf16"):
        api.plan(_wl(configs.with_layers(configs.DEEPSEEK_V2_LITE, 27, wdtype=1)))
    with pytest.raises(ValueError, match="unfused"):
        api.plan(_wl(configs.with_layers(configs.TINY_MOE, 2, batch=4), fused=False))
    with pytest.raises(ValueError, match="8"):
        api.plan(_wl(configs.TINY_MOE), workgroups=4)


def test_emit_writes_a_timeline_schedule(tmp_path):
    """emit() writes plan.json in the layout the reference's timeline tool reads (types, one static task per
    (phase, workgroup) with its XCD as domain, one event per grid barrier whose producers are the phase before),
    decisions.txt, and manifest.json with the payload hashes; load_sources rejects a changed payload."""
    cfg = configs.TINY_MOE
    p = api.plan(_wl(cfg), workgroups=16)
    d = api.emit(p, tmp_path / "art")
    body = api.load_sources(d)
    nb, wg = p.record["barriers_per_step"], 16
    assert len(body["descs"]) == nb * wg == len(body["task_in"]) and len(body["ev_inst"]) == nb
    assert sorted(t["id"] for t in body["types"].values()) == list(range(len(body["types"])))
    assert body["domains"] == 8 and body["workers_per_domain"] == 2
    assert body["descs"][5 * wg + 3] == {"type": body["types"]["expert_down"]["id"], "coord": [0, 3, 0, 0],
                                         "domain": 3, "mode": "static"}
    prods = [e[2] for e in body["ev_inst"]]               # the timeline tool's dependency rule
    deps = [sorted({q for ev in evs for q in prods[ev]}) for evs in body["task_in"]]
    assert deps[0] == [] and deps[wg + 7] == list(range(wg)) and deps[2 * wg] == list(range(wg, 2 * wg))
    assert (d / "decisions.txt").read_text().splitlines() == p.record["decisions"]
    (d / "plan.json").write_text((d / "plan.json").read_text().replace('"fused":true', '"fused":false'))
    with pytest.raises(ValueError, match="hash"):
        api.load_sources(d)


@pytest.mark.gpu
@pytest.mark.parametrize("base,B", [(configs.TINY_MOE, 1), (configs.TINY_MLA, 4)], ids=["moe-b1", "mla-b4"])
def test_trace_step_rows(gpu, tmp_path, base, B):
    """A session's traced step: one nine-int64 row per (phase, workgroup) task in plan order, taken <= ready <= done,
    worker and coordinates as the plan's descs."""
    import numpy as np
    cfg = configs.with_layers(base, base.L, batch=B)
    sess = api.build_model(api.decode_workload(cfg.name, cfg.as_dict(), seed=7))
    for b in range(B):
        sess.decoder.set_tokens([3 + b, 5, 9, 11], seq=b)
    d = sess.trace_step(tmp_path / "tr", [3] * B)
    body = api.load_sources(d)
    rows = np.frombuffer((d / "trace.bin").read_bytes(), "<i8").reshape(-1, 9)
    assert len(rows) == len(body["descs"])
    assert np.all(rows[:, 5] > 0) and np.all(rows[:, 5] <= rows[:, 6]) and np.all(rows[:, 6] <= rows[:, 7])
    assert [int(x) for x in rows[:, 0]] == [t["type"] for t in body["descs"]]
    assert [int(x) for x in rows[:, 2]] == [t["coord"][1] for t in body["descs"]] == [int(x) for x in rows[:, 8]]
    wg = body["workers_per_domain"] * body["domains"]
    assert np.all(rows[wg:, 5] >= rows[:-wg, 7] - 1)     # a workgroup takes phase k after its arrival from k-1
    sess.close()


def test_prompt_rows_default_to_library_limit():
    """A workload whose model leaves `prefill` open reads prompts through the largest prefill launch the library
    accepts for its shape (16 rows, 4 for Qwen3-8B and DeepSeek-V2-Lite); one that sets it, or runs unfused, keeps
    its choice."""
    def prompts_line(cfg, model=None, **run):
        model = model if model is not None else {k: v for k, v in cfg.as_dict().items() if k != "prefill"}
        ds = api.plan(api.decode_workload(cfg.name, model, **run)).record.to_dict()["decisions"]
        return [d for d in ds if d.startswith("prompts:")]
    assert prompts_line(configs.QWEN3_30B_A3B)[0].startswith("prompts: 16 positions")
    assert prompts_line(configs.QWEN3_8B)[0].startswith("prompts: 4 positions")
    assert prompts_line(configs.DEEPSEEK_V2_LITE)[0].startswith("prompts: 4 positions")
    assert prompts_line(configs.QWEN3_30B_A3B, configs.QWEN3_30B_A3B.as_dict()) == []      # prefill 0 set
    assert prompts_line(configs.QWEN3_30B_A3B, fused=False) == []
