"""The C oracle against the NumPy restatement of ref_numpy.py (the reference's evaluation order) on
seeded tiny decoders: the reference's own gate, per-layer max rel < 2e-2 (ref_numpy.py:207-212), and
identical greedy tokens."""
import numpy as np
import pytest

from oracle import oracle as O
from oracle.ref_twin import Twin

TINY_MOE = dict(H=512, NH=4, NKV=2, HD=128, I=0, E=16, TOPK=4, MI=256, L=2, V=4096, moe=1, qk_norm=1,
                norm_topk=1, block_size=16, max_ctx=256, batch=1, eps=1e-6, theta=1e6)
TINY_DENSE = dict(TINY_MOE, I=1024, E=0, TOPK=0, MI=0, moe=0)


@pytest.mark.parametrize("cfg", [TINY_MOE, TINY_DENSE], ids=["moe", "dense"])
def test_oracle_matches_numpy_reference_formulation(oracle_lib, cfg):
    m = O.OracleModel(cfg, seed=11, wscale=0.02)
    tw = Twin(m, cfg["max_ctx"])
    prompt = O.gen_tokens(11, 12, cfg["V"])
    seq = list(prompt)
    worst = 0.0
    ids_equal = ids_total = 0
    for t in range(len(prompt) + 6 - 1):
        dump_t = []
        tok_t = tw.step(seq[t], t, dump_t)
        tok_o, xo, ido, wo = m.step(seq[t], t, dump=True)
        for L in range(cfg["L"]):
            xt = dump_t[L][0]
            worst = max(worst, float(np.max(np.abs(xo[L] - xt)) / max(np.max(np.abs(xt)), 1e-12)))
            if cfg["moe"]:
                ids_total += 1
                ids_equal += int(sorted(dump_t[L][1].tolist()) == sorted(ido[L].tolist()))
        assert tok_o == tok_t, f"step {t}: oracle {tok_o} vs numpy formulation {tok_t}"
        if t >= len(prompt) - 1:
            seq.append(tok_o)
    assert worst < 2e-2
    if cfg["moe"]:
        assert ids_equal == ids_total
    m.close()
