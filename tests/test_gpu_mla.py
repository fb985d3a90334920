"""GPU parity of the DeepSeek-V2 decode step (multi-head latent attention, shared experts, a dense first layer): one
persistent launch per step for up to 4 sequences, each compared with the CPU oracle's single-sequence step on the
same seeded weights and latent cache: per-layer residuals bit for bit (the 2e-2 gate reported first), top-k ids and
fp32 weights of the MoE layers exactly, greedy tokens identical, and the latent cache bit for bit."""
import sys
import time

import numpy as np
import pytest

from oracle import oracle as O
from etx.runtime import native as N
from etx.models import configs
from progress_log import say

pytestmark = pytest.mark.gpu

SEED = 20261202


def rel(a, b):
    return float(np.max(np.abs(a - b)) / max(float(np.max(np.abs(b))), 1e-30))


def check_layers(cfg, d, b, xo, ido, wo, what):
    for L in range(cfg.L):
        assert rel(d["x"][L][b], xo[L]) < 2e-2, f"{what} layer {L}: max rel {rel(d['x'][L][b], xo[L]):.3e}"
        assert np.array_equal(d["x"][L][b], xo[L]), f"{what} layer {L}: residual differs in {np.sum(d['x'][L][b] != xo[L])}"
        if L >= cfg.first_dense:
            assert np.array_equal(d["ids"][L][b], ido[L]), f"{what} layer {L}: top-k ids {d['ids'][L][b]} vs {ido[L]}"
            assert np.array_equal(d["w"][L][b], wo[L]), f"{what} layer {L}: top-k weights {d['w'][L][b]} vs {wo[L]}"


def check_latent(cfg, dec, orc):
    for L in range(cfg.L):
        assert np.array_equal(dec.kv_layer(L)[0], orc.kv(L)[0]), f"layer {L}: latent cache differs"


def run_contexts(cfg, ctx, n_steps, shuffle=False, check_every=1, cache=True):
    """Sequence b holds ctx[b] cached latent rows (seeded), reads one seeded token at position ctx[b], then decodes
    greedily for n_steps positions; every step is one launch."""
    B = cfg.batch
    t0 = time.time()
    say(f"[gpu] mla batch {B} {cfg.name}: contexts {list(ctx)}, {n_steps} steps, shuffled={shuffle}")
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
    say(f"[gpu]   caches filled ({time.time() - t0:.0f}s)")
    dec.enable_dumps(True)
    toks = [[int(first[b])] for b in range(B)]
    pos = np.asarray(ctx, np.int32).copy()
    for s in range(n_steps):
        if B == 1:
            dec.step(int(pos[0]))
        else:
            dec.step_batch(pos, write_next=True)
        check = s % check_every == 0 or s == n_steps - 1
        d = dec.dumps() if check else None
        if d is not None and B == 1:
            d = {k: v[:, None] for k, v in d.items()}
        for b in range(B):
            if check:
                t, xo, ido, wo = orc.step(toks[b][-1], int(pos[b]), dump=True, seq=b)
                check_layers(cfg, d, b, xo, ido, wo, f"step {s} sequence {b} (position {pos[b]})")
            else:
                t = orc.step(toks[b][-1], int(pos[b]), seq=b)
            toks[b].append(t)
        if cfg.L > 3:
            say(f"[gpu]   step {s}: oracle tokens {[tk[-1] for tk in toks]} ({time.time() - t0:.0f}s)")
        pos += 1
    dec.sync()
    for b in range(B):
        got = dec.read_tokens(int(pos[b]), seq=b)[int(ctx[b]):]
        assert list(got) == toks[b][1:], f"sequence {b}: greedy tokens {list(got)} vs {toks[b][1:]}"
    if cache:
        check_latent(cfg, dec, orc)
    orc.close()
    dec.close()


def test_tiny_mla_single_from_empty_cache(gpu):
    """One sequence from position 0: the first chunk fills position by position (the current row patched in)."""
    cfg = configs.TINY_MLA
    run_contexts(cfg, [0], n_steps=6)


@pytest.mark.parametrize("B", [4, 3, 1], ids=["b4", "b3", "b1"])
def test_tiny_mla_batch_contexts_bit_exact(gpu, B):
    cfg = configs.with_layers(configs.TINY_MLA, configs.TINY_MLA.L, batch=B)
    ctx = np.random.default_rng(200 + B).integers(1, 200, B)
    run_contexts(cfg, ctx, n_steps=4, shuffle=True)


def test_tiny_mla_prompts_mixed_lengths(gpu):
    """Prompts of different lengths read token by token in the same launches, then greedy decoding; against the
    oracle's single-sequence decode of each prompt."""
    cfg = configs.with_layers(configs.TINY_MLA, configs.TINY_MLA.L, batch=4)
    say(f"[gpu] mla batch prompts {cfg.name}")
    dec = N.Decoder(cfg)
    dec.init_weights(SEED, 0.02)
    prompts = [O.gen_tokens(SEED + b, 3 + 7 * b, cfg.V) for b in range(4)]
    got = dec.generate_batch(prompts, 5, prefill=False)
    for b, p in enumerate(prompts):
        o = O.OracleModel(configs.TINY_MLA.as_dict(), SEED, 0.02)
        toks = list(p)
        for q in range(len(p) + 4):
            t = o.step(toks[q], q)
            if q + 1 >= len(p):
                toks.append(t)
        assert list(got[b]) == toks[len(p):], f"sequence {b}"
        o.close()
    dec.close()


def test_deepseek_v2_lite_batch4_two_layers(gpu):
    """Real DeepSeek-V2-Lite shapes (the dense layer 0 with its padded 10944-wide down rows, one MoE layer), batch 4,
    contexts across several chunks, shuffled block table."""
    cfg = configs.with_layers(configs.DEEPSEEK_V2_LITE, 2, batch=4)
    run_contexts(cfg, [97, 530, 1000, 5], n_steps=3, shuffle=True)


@pytest.mark.timeout(900)
def test_deepseek_v2_lite_batch4_full_depth(gpu):
    """27 layers at batch 4 with contexts in [512, 2048]: 32 greedy steps of every sequence
    identical to the oracle, the first and last step's per-layer residuals and routing bit for bit."""
    cfg = configs.with_layers(configs.DEEPSEEK_V2_LITE, 27, batch=4)
    run_contexts(cfg, [1500, 620, 2040, 1024], n_steps=32, check_every=31, cache=False)
