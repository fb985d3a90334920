"""GPU parity of the batched step (etxmk_step_batch): B sequences at their own positions, with their own token rows
and block-table rows into one paged-KV pool, decoded by one persistent launch per step.  Each sequence is compared
with the CPU oracle's step of that sequence (a batched oracle holds the same pool and computes the batch's rows in one
pass over the weights, each row equal to its single-sequence step): per-layer residuals bit for bit
(the 2e-2 gate reported), top-k ids and weights exactly, greedy tokens identical, and the whole pool's K and V
caches bit for bit."""
import sys

import numpy as np
import pytest

from oracle import oracle as O
from etx.runtime import native as N
from etx.models import configs
from progress_log import say

pytestmark = pytest.mark.gpu

SEED = 20261201


def rel(a, b):
    return float(np.max(np.abs(a - b)) / max(float(np.max(np.abs(b))), 1e-30))


def check_layers(cfg, d, b, xo, ido, wo, what):
    for L in range(cfg.L):
        assert rel(d["x"][L][b], xo[L]) < 2e-2, f"{what} layer {L}: max rel {rel(d['x'][L][b], xo[L]):.3e}"
        assert np.array_equal(d["x"][L][b], xo[L]), f"{what} layer {L}: residual differs in {np.sum(d['x'][L][b] != xo[L])}"
        if cfg.moe:
            assert np.array_equal(d["ids"][L][b], ido[L]), f"{what} layer {L}: top-k ids {d['ids'][L][b]} vs {ido[L]}"
            assert np.array_equal(d["w"][L][b], wo[L]), f"{what} layer {L}: top-k weights differ"


def check_pool(cfg, dec, orc):
    for L in range(cfg.L):
        kg, vg = dec.kv_layer(L)
        ko, vo = orc.kv(L)
        assert np.array_equal(kg, ko), f"layer {L}: paged K pool differs"
        assert np.array_equal(vg, vo), f"layer {L}: paged V pool differs"


def run_contexts(cfg, ctx, n_steps, shuffle=False, check_every=1, pool=True):
    """Sequence b holds ctx[b] cached positions (seeded KV), reads one seeded token at position ctx[b], then decodes
    greedily for n_steps positions; every step is one batched launch."""
    import time
    B = cfg.batch
    t0 = time.time()
    say(f"[gpu] batch {B} {cfg.name}: contexts {list(ctx)}, {n_steps} steps, shuffled={shuffle}")
    dec = N.Decoder(cfg)
    dec.init_weights(SEED, 0.02)
    orc = O.OracleModel(cfg.as_dict(), SEED, 0.02)
    if shuffle:
        bt = np.random.default_rng(B).permutation(B * dec.blocks_per_seq).astype(np.int32)
        dec.set_block_table(bt)
        orc.set_block_table(bt)
    first = O.gen_tokens(SEED + 1, B, cfg.V)
    for b in range(B):
        dec.fill_kv_seeded(SEED, int(ctx[b]), seq=b)
        orc.fill_kv_random(int(ctx[b]), seq=b)
        row = np.zeros(int(ctx[b]) + 1, np.int32)
        row[-1] = first[b]
        dec.set_tokens(row, seq=b)
        if cfg.L > 2:
            say(f"[gpu]   sequence {b}: {int(ctx[b])} cached positions filled ({time.time() - t0:.0f}s)")
    dec.enable_dumps(True)
    toks = [[int(first[b])] for b in range(B)]
    pos = np.asarray(ctx, np.int32).copy()
    for s in range(n_steps):
        dec.step_batch(pos, write_next=True)
        check = s % check_every == 0 or s == n_steps - 1
        d = dec.dumps() if check else None
        if d is not None and B == 1:                        # single-sequence handles dump [layer][...]
            d = {k: v[:, None] for k, v in d.items()}
        # the oracle's batched step: every sequence's row in one pass over the weights (each row equals the
        # single-sequence step, tests/test_oracle_prefill.py)
        r = orc.step_rows(list(range(B)), [toks[b][-1] for b in range(B)], pos, dump=check)
        for b in range(B):
            if check:
                check_layers(cfg, d, b, r[1][b], r[2][b], r[3][b], f"step {s} sequence {b} (position {pos[b]})")
            toks[b].append(int(r[0][b] if check else r[b]))
        if cfg.L > 2:
            say(f"[gpu]   step {s}: oracle tokens {[tk[-1] for tk in toks]} ({time.time() - t0:.0f}s)")
        pos += 1
    dec.sync()
    for b in range(B):
        got = dec.read_tokens(int(pos[b]), seq=b)[int(ctx[b]):]
        assert list(got) == toks[b][1:], f"sequence {b}: greedy tokens {list(got)} vs {toks[b][1:]}"
    if pool:
        check_pool(cfg, dec, orc)
    orc.close()
    dec.close()


@pytest.mark.parametrize("base,B", [(configs.TINY_MOE, 4), (configs.TINY_MOE, 3), (configs.TINY_MOE, 16),
                                    (configs.TINY_DENSE, 4)], ids=["moe-b4", "moe-b3", "moe-b16", "dense-b4"])
def test_tiny_batch_contexts_bit_exact(gpu, base, B):
    cfg = configs.with_layers(base, base.L, batch=B)
    ctx = np.random.default_rng(100 + B).integers(1, 200, B)
    run_contexts(cfg, ctx, n_steps=5, shuffle=True)


def test_tiny_batch_prompts_mixed_lengths(gpu):
    """Prompts of different lengths read token by token in the same launches (the write-next mask keeps each
    sequence's prompt), then greedy decoding; against the oracle's single-sequence decode of each prompt."""
    cfg = configs.with_layers(configs.TINY_MOE, configs.TINY_MOE.L, batch=4)
    say(f"[gpu] batch prompts {cfg.name}")
    dec = N.Decoder(cfg)
    dec.init_weights(SEED, 0.02)
    prompts = [O.gen_tokens(SEED + b, 3 + 5 * b, cfg.V) for b in range(4)]
    got = dec.generate_batch(prompts, 6, prefill=False)
    orc = O.OracleModel(configs.TINY_MOE.as_dict(), SEED, 0.02)
    for b, p in enumerate(prompts):
        o = O.OracleModel(configs.TINY_MOE.as_dict(), SEED, 0.02)
        toks = list(p)
        for pos in range(len(p) + 5):
            t = o.step(toks[pos], pos)
            if pos + 1 >= len(p):
                toks.append(t)
        assert list(got[b]) == toks[len(p):], f"sequence {b}"
        o.close()
    orc.close()
    dec.close()


def test_qwen3_30b_a3b_batch4_two_layers(gpu):
    """Real Qwen3-30B-A3B shapes at batch 4 (two layers): contexts across several chunks, shuffled pool."""
    cfg = configs.with_layers(configs.QWEN3_30B_A3B, 2, batch=4)
    run_contexts(cfg, [97, 530, 1000, 5], n_steps=3, shuffle=True)


def test_qwen3_30b_a3b_batch16_two_layers(gpu):
    """Batch 16 (two layers): 128 routed pairs, more than one LDS pass of expert rows in the down projection."""
    cfg = configs.with_layers(configs.QWEN3_30B_A3B, 2, batch=16)
    ctx = np.random.default_rng(16).integers(512, 1080, 16)
    run_contexts(cfg, ctx, n_steps=2, pool=False)


def test_qwen3_8b_batch4_two_layers(gpu):
    """Qwen3-8B shapes at batch 4 (two dense layers, H 4096, 12288-long down rows in the long-row batched GEMV)."""
    cfg = configs.with_layers(configs.QWEN3_8B, 2, batch=4)
    run_contexts(cfg, [300, 64, 1000, 7], n_steps=3, shuffle=True)


@pytest.mark.timeout(900)
def test_qwen3_30b_a3b_batch4_full_depth(gpu):
    """48 layers at batch 4 with per-sequence contexts: 8 greedy steps of every sequence identical to the oracle,
    last step's per-layer residuals and routing bit for bit."""
    cfg = configs.with_layers(configs.QWEN3_30B_A3B, 48, batch=4)
    run_contexts(cfg, [600, 811, 1024, 700], n_steps=8, check_every=7, pool=False)


@pytest.mark.parametrize("B", [1, 2], ids=["b1", "b2"])
def test_tiny_contexts_past_4096(gpu, B):
    """More than 64 chunks of 64 positions: the merge's second chunk per lane (contexts up to 8192)."""
    cfg = configs.with_layers(configs.TINY_MOE, configs.TINY_MOE.L, batch=B, max_ctx=4700)
    run_contexts(cfg, [4500, 4100][:B], n_steps=3, check_every=2)
