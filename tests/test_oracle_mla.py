"""The oracle's DeepSeek-V2 decode: yarn RoPE tables, the DeepSeek RoPE interleave, the
unnormalised router, and whole decode steps against a NumPy restatement of the reference's MLA specification that
uses the non-absorbed attention form (oracle/ref_twin_mla.py)."""
import math

import numpy as np
import pytest

from oracle import oracle as O
from oracle.ref_twin_mla import TwinMLA, yarn_cos_sin
from etx.models import configs

SEED = 20261201


def test_yarn_tables(oracle_lib):
    c = configs.DEEPSEEK_V2_LITE.as_dict()
    ctx = 2112
    cs, sn = O.yarn_tables(c, ctx)
    assert np.all(cs[0] == 1.0) and np.all(sn[0] == 0.0)
    # the reference's float32 numpy steps: numpy's float32 power is not correctly rounded (4 of the 32 base powers
    # differ from powf, which equals the rounded double), so its angles drift by a few ulps and its tables differ
    # by up to ~1e-4 at the far positions; the oracle's tables are the correctly rounded ones
    rc, rs = yarn_cos_sin(c, ctx)
    assert np.max(np.abs(cs - rc[:, :32])) < 1e-4 and np.max(np.abs(sn - rs[:, :32])) < 1e-4
    assert np.array_equal(rc[:, :32], rc[:, 32:])
    # the same float32 steps with correctly rounded powers, cos/sin in float64: within a float32 rounding
    pw = (1e4 ** (np.arange(0, 64, 2, dtype=np.float32) / 64).astype(np.float64)).astype(np.float32)
    low_, high_ = 10, 23
    ramp_ = np.clip((np.arange(32, dtype=np.float32) - low_) / np.float32(high_ - low_), 0, 1).astype(np.float32)
    mask_ = (np.float32(1) - ramp_).astype(np.float32)
    inv_ = ((np.float32(1) / (np.float32(40) * pw)) * (np.float32(1) - mask_) + (np.float32(1) / pw) * mask_).astype(np.float32)
    ang = (np.arange(ctx, dtype=np.float32)[:, None] * inv_[None, :]).astype(np.float32)
    assert np.max(np.abs(cs - np.cos(ang.astype(np.float64)))) < 1e-7
    assert np.max(np.abs(sn - np.sin(ang.astype(np.float64)))) < 1e-7
    # float64 mathematics of the yarn blend (beta 32 / 1 over 4096 positions, factor 40)
    dim, base = 64, 1e4
    corr = lambda r: (dim * math.log(4096 / (r * 2 * math.pi))) / (2 * math.log(base))
    low, high = max(math.floor(corr(32)), 0), min(math.ceil(corr(1)), dim - 1)
    i = np.arange(32)
    ramp = np.clip((i - low) / (high - low), 0, 1)
    inv = (1 - (1 - ramp)) / (40 * base ** (2 * i / dim)) + (1 - ramp) / base ** (2 * i / dim)
    t = np.arange(ctx)[:, None]
    assert np.max(np.abs(cs - np.cos(t * inv))) < 3e-4 and np.max(np.abs(sn - np.sin(t * inv))) < 3e-4
    assert 0 < low < high < 31                             # both ends of the ramp are inside the 32 frequencies


def test_rope_interleave(oracle_lib):
    rng = np.random.default_rng(1)
    x = O.bf16_bits_to_f32(O.f32_to_bf16_bits(rng.standard_normal(64).astype(np.float32)))
    ang = rng.uniform(0, 6, 32)
    cs, sn = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    out = O.rope_ds(x, cs, sn)
    # pair (2i, 2i+1) rotated by angle i, written to (i, i + 32)
    ex = np.concatenate([x[0::2] * cs - x[1::2] * sn, x[1::2] * cs + x[0::2] * sn])
    assert np.allclose(out, ex, rtol=2 ** -7, atol=1e-6)
    assert abs(np.linalg.norm(out) - np.linalg.norm(x)) < 0.02 * np.linalg.norm(x)
    ident = O.rope_ds(x, np.ones(32, np.float32), np.zeros(32, np.float32))
    assert np.array_equal(ident, np.concatenate([x[0::2], x[1::2]]))


def test_router_unnormalised(oracle_lib):
    rng = np.random.default_rng(2)
    lg = rng.standard_normal(64).astype(np.float32)
    lg[5] = lg[9] = lg.max() + 1                           # a tie: the lower id first
    ids, w = np.zeros(6, np.int32), np.zeros(6, np.float32)
    O.lib().orc_route_ds(lg, 64, 6, 0, 1.0, ids, w)
    p = np.exp(lg.astype(np.float64) - lg.max()); p /= p.sum()
    assert list(ids[:2]) == [5, 9]
    assert list(ids) == list(np.argsort(-p, kind="stable")[:6])
    assert np.allclose(w, p[ids], rtol=1e-6)              # probabilities, not renormalised, not rounded
    O.lib().orc_route_ds(lg, 64, 6, 0, 2.5, ids, w)
    assert np.allclose(w, 2.5 * p[ids], rtol=1e-6)


@pytest.mark.parametrize("ctx0", [0, 70], ids=["prompt", "filled"])
def test_decode_against_reference_restatement(oracle_lib, ctx0):
    """Greedy decode of the tiny MLA decoder: the C oracle (absorbed, fixed order) and the NumPy twin (non-absorbed,
    numpy order) read the same tokens; per-layer residuals within 2e-2, the same routing, the same greedy tokens."""
    cfg = configs.TINY_MLA
    orc = O.OracleModel(cfg.as_dict(), SEED)
    tw = TwinMLA(orc, cfg.max_ctx)
    if ctx0:                                               # a filled latent cache, mirrored into the twin
        orc.fill_kv_random(ctx0)
        CD = cfg.kv_lora + cfg.qk_rope
        for l in range(cfg.L):
            k, _ = orc.kv(l)
            blk = k.reshape(-1, CD // 8, cfg.block_size, 8)
            lat = blk.transpose(0, 2, 1, 3).reshape(-1, CD)
            tw.cache[l][:ctx0] = O.bf16_bits_to_f32(lat[:ctx0])
    toks = list(O.gen_tokens(SEED, 6, cfg.V))
    worst = 0.0
    for s in range(10):
        pos = ctx0 + s
        t_o, xo, ido, _ = orc.step(toks[s], pos, dump=True)
        t_w, xw, idw = tw.step(toks[s], pos)
        for L in range(cfg.L):
            worst = max(worst, float(np.max(np.abs(xo[L] - xw[L])) / np.max(np.abs(xw[L]))))
            if L >= cfg.first_dense:
                assert list(np.sort(ido[L])) == list(idw[L]), f"step {s} layer {L}: routing"
        assert t_o == t_w, f"step {s}: greedy token {t_o} vs {t_w}"
        if s + 1 >= len(toks):
            toks.append(t_o)
    assert worst < 2e-2, worst
    orc.close()
