"""etx.operators.moe_layer: the native MoE-layer provider (reference interface etx/operators/moe_layer.py:31-185).
CPU: the record's dimensions, the deterministic input and the grouping arithmetic of runtime(); GPU: the layer built
from the provider against the CPU oracle's layer step on the same seeded weights and cache, bit for bit."""
import numpy as np
import pytest

from etx.models import configs
from etx.operators import moe_layer


def test_provider_record_and_inputs():
    p = moe_layer.provider(small=True)
    assert (p.D, p.H, p.HD, p.NE, p.K, p.FF) == (512, 4, 128, 16, 4, 256) and p.S == 128
    assert p.T == "etxmk_fused_h512_a512_moe256_e16"
    big = moe_layer.provider()
    assert (big.D, big.NE, big.K, big.FF, big.S) == (2048, 128, 8, 768, 1024)
    with pytest.raises(ValueError):
        moe_layer.provider(small=1)
    x = np.array(p.lcg_x(3, seed=7), np.float32)
    assert x.shape == (3, 512) and np.array_equal(x, np.array(p.lcg_x(3, seed=7), np.float32))
    assert np.all(np.abs(x) <= 1.0) and np.all(x * 128 == np.round(x * 128))     # integers / 128: bf16-exact
    # the first value follows the 32-bit LCG: state = 7 * 1664525 + 1013904223 (mod 2^32)
    s = (7 * 1664525 + 1013904223) & 0xFFFFFFFF
    assert x[0, 0] == ((s >> 8) % 257 - 128) / 128.0


def test_runtime_grouping_arithmetic():
    p = moe_layer.provider(small=True)
    rng = np.random.default_rng(1)
    topk = [sorted(int(e) for e in rng.choice(p.NE, p.K, replace=False)) for _ in range(9)]
    r = p.runtime({"B": 9}, topk)
    assert sum(r["expert_counts"]) == 9 * p.K
    assert r["tok_indptr"][-1] == 9 * p.K and r["indptr"][-1] == sum(-(-c // p.TPT) for c in r["expert_counts"])
    slots = sorted(s for row in r["tok_slot"] for s in row)
    assert slots == list(range(9 * p.K))                  # every (token, slot) pair gets one grouped row
    for row, sl in zip(topk, r["tok_slot"]):
        for e, q in zip(row, sl):
            assert r["tok_indptr"][e] <= q < r["tok_indptr"][e + 1]
    assert len(r["tile_expert"]) == r["indptr"][-1]
    assert p.bindings(topk=topk, B=9)["n_gg"] == r["indptr"][-1]


@pytest.mark.gpu
def test_native_layer_matches_oracle(gpu):
    """provider(small=True).build(): each input row through the layer equals the oracle's layer step on the same
    seeded weights and cache (output residual, top-k ids and weights bit for bit); routing() is those ids sorted."""
    from oracle import oracle as O
    p = moe_layer.provider(small=True)
    layer = p.build(seed=5)
    x = p.lcg_x(3, seed=9)
    outs, ids, wts = layer.forward(x)
    cfg = configs.with_layers(configs.TINY_MOE, 1, max_ctx=p.S + 16)
    orc = O.OracleModel(cfg.as_dict(), 5, 0.02)
    orc.fill_kv_random(p.S)
    for r in range(3):
        xo, ido, wo, _ = orc.layer_step(0, np.array(x[r], np.float32), p.S)
        assert np.array_equal(outs[r], xo), f"row {r}: layer output differs"
        assert np.array_equal(ids[r], ido) and np.array_equal(wts[r], wo), f"row {r}: routing differs"
    assert p.routing(x, layer) == [sorted(int(e) for e in row) for row in ids]
    orc.close()
    layer.close()
