"""etxmk_step_static, the allocation-free step: the same step as etxmk_step with its scratch in the library's static
device array.  Two calls in a row on one GPU, the second with a smaller input (a smaller model at a shorter context,
so it uses less of the array and reads none of what the first left there), each against etxmk_step on a twin handle:
per-layer residuals, top-k ids and weights, the greedy tokens and the KV cache, bit for bit."""
import numpy as np
import pytest

from etx.runtime import native as N
from etx.models import configs
from progress_log import say

pytestmark = pytest.mark.gpu

SEED = 20261204


def _pair(cfg, ctx):
    decs = []
    for _ in range(2):
        d = N.Decoder(cfg)
        d.init_weights(SEED, 0.02)
        d.fill_kv_seeded(SEED, ctx)
        row = np.zeros(ctx + 1, np.int32)
        row[ctx] = 7 % cfg.V
        d.set_tokens(row)
        d.enable_dumps(True)
        decs.append(d)
    return decs


@pytest.mark.parametrize("name,ctx", [("qwen3-30b-a3b-L2", 900), ("tiny-moe", 40)])
def test_static_step_equals_step(gpu, name, ctx):
    cfg = configs.with_layers(configs.QWEN3_30B_A3B, 2) if name.startswith("qwen3") else configs.TINY_MOE
    say(f"[gpu] allocation-free step {cfg.name} at context {ctx}")
    ref, st = _pair(cfg, ctx)
    for pos in (ctx, ctx + 1):
        ref.step(pos, write_next=True)
        st.step_static(pos, write_next=True)
        a, b = ref.dumps(), st.dumps()
        for key in ("x", "ids", "w"):
            assert np.array_equal(a[key], b[key]), f"position {pos}: {key} differs"
    ref.sync()
    st.sync()
    assert np.array_equal(ref.read_tokens(ctx + 2), st.read_tokens(ctx + 2))
    for L in range(cfg.L):
        ka, va = ref.kv_layer(L)
        kb, vb = st.kv_layer(L)
        assert np.array_equal(ka, kb) and np.array_equal(va, vb), f"layer {L}: KV cache differs"
    ref.close()
    st.close()


def test_static_step_refusals(gpu):
    dec = N.Decoder(configs.with_layers(configs.TINY_MOE, 2, batch=2))
    with pytest.raises(N.EtxmkError, match="single-sequence"):
        dec.step_static(0)
    dec.close()
