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
