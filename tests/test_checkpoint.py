"""The packed checkpoint format (weights.bin + llm.manifest, etx/models/llm/prep.py:88-146,243-258), written from the
oracle's seeded weights and read back: every tensor bit for bit, the dimensions, and the malformed cases the reader
must refuse (layout 1, misalignment, overlap, truncation, qkv bias, a missing tensor)."""
import numpy as np
import pytest

from oracle import oracle as O
from etx.runtime import native as N
from etx.models import configs
from etx.models import checkpoint as CK

SEED = 20261201
ONE = np.uint16(0x3F80)                      # bf16 1.0, the seeded norm weights


def oracle_getter(orc, cfg):
    """get(name, shape) over the oracle's seeded tensors (the library's kinds 1..9 are the oracle's streams)."""
    plan = {name: (kind, layer) for name, kind, layer, _ in CK.tensor_plan(cfg)}

    def get(name, shape):
        kind, layer = plan.get(name, (N.T_EMBED, -1)) if name != "lm_head" else (N.T_LMHEAD, -1)
        if kind >= N.T_LN1:
            return np.full(shape, ONE, np.uint16)
        if kind in (N.T_W13, N.T_W2):
            return np.stack([orc.weight(kind, layer, e) for e in range(shape[0])])
        return orc.weight(kind, layer)
    return get


def write_from_oracle(path, cfg, tie=False):
    orc = O.OracleModel(cfg.as_dict(), SEED, 0.02)
    try:
        CK.write_checkpoint(path, cfg, oracle_getter(orc, cfg), tie=tie)
    finally:
        orc.close()
    return CK.Checkpoint(path)


@pytest.mark.parametrize("cfg", [configs.TINY_MOE, configs.TINY_DENSE], ids=["moe", "dense"])
def test_roundtrip_bit_exact(tmp_path, oracle_lib, cfg):
    ck = write_from_oracle(tmp_path / "ck", cfg)
    got = ck.config()
    for f in ("H", "NH", "NKV", "HD", "L", "V", "I", "E", "TOPK", "MI", "moe", "qk_norm", "norm_topk", "max_ctx"):
        assert getattr(got, f) == getattr(cfg, f), f
    assert got.eps == pytest.approx(cfg.eps) and got.theta == pytest.approx(cfg.theta)
    for name, (off, cnt) in ck.manifest.tensors.items():
        assert off % 256 == 0, name
    orc = O.OracleModel(cfg.as_dict(), SEED, 0.02)
    try:
        get = oracle_getter(orc, cfg)
        for name, kind, layer, shape in CK.tensor_plan(cfg):
            assert np.array_equal(ck.array(name, shape), get(name, shape)), name
    finally:
        orc.close()
    ck.check(cfg)


def test_tied_checkpoint_has_no_head(tmp_path, oracle_lib):
    ck = write_from_oracle(tmp_path / "ck", configs.TINY_DENSE, tie=True)
    assert ck.tie and "lm_head" not in ck.manifest.tensors
    ck.check(configs.TINY_DENSE)


def test_refuses_malformed(tmp_path, oracle_lib):
    cfg = configs.TINY_DENSE
    base = tmp_path / "ck"
    write_from_oracle(base, cfg)
    man = base / "llm.manifest"
    text = man.read_text()
    m = CK.read_manifest(man)

    def refused(manifest_text, exc, match, opener=CK.read_manifest):
        man.write_text(manifest_text)
        try:
            with pytest.raises(exc, match=match):
                opener(man) if opener is CK.read_manifest else opener(base)
        finally:
            man.write_text(text)

    # layout 1: gate/up rows not interleaved (host.hip:71 refuses it too)
    refused(text.replace("cfg layout 2", "cfg layout 1"), ValueError, "layout 1")
    # a tensor off the 256-byte grid
    off = m.tensors["L0.wo"][0]
    refused(text.replace(f"t L0.wo {off} ", f"t L0.wo {off + 2} "), ValueError, "offset")
    # two tensors overlapping
    refused(text.replace(f"t L0.ln2 {m.tensors['L0.ln2'][0]} ", f"t L0.ln2 {m.tensors['L0.ln1'][0]} "),
            ValueError, "overlap")
    # qkv bias is refused, not ignored
    refused(text.replace("cfg bias 0", "cfg bias 1"), ValueError, "bias", opener=lambda d: CK.Checkpoint(d).config())
    # a tensor the decoder needs is missing
    refused("\n".join(l for l in text.splitlines() if not l.startswith("t L1.wd ")) + "\n", KeyError, "L1.wd",
            opener=lambda d: CK.Checkpoint(d).check(cfg))
    # weights.bin shorter than the manifest says
    blob = (base / "weights.bin").read_bytes()
    (base / "weights.bin").write_bytes(blob[:-4096])
    with pytest.raises(ValueError, match="past weights.bin"):
        CK.Checkpoint(base)


def test_golden_file(tmp_path):
    p = tmp_path / "golden.txt"
    p.write_text("prompt: 1 2 3\ngen: 7 8\nmargin: 0.5000 1.2500\n")
    prompt, gen, margin = CK.read_golden(p)
    assert prompt == [1, 2, 3] and gen == [7, 8] and margin == [0.5, 1.25]
    (tmp_path / "empty.txt").write_text("gen: 1\n")
    with pytest.raises(ValueError):
        CK.read_golden(tmp_path / "empty.txt")
