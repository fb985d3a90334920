"""GPU parity of batched prefill (etxmk_prefill): a prompt's positions go n per launch through the batched persistent
kernel, one row per position, the rows attending to the cache below the launch's first position and to the launch's
own K/V rows.  Compared with the CPU oracle's token-by-token decode of the same prompt (the reference's prompt loop,
examples/llm/host.hip:203-213): every layer's paged K and V cache bit for bit, every prompt position's greedy token,
and the greedy continuation decoded after the prompt."""
import time

import numpy as np
import pytest

from oracle import oracle as O
from etx.runtime import native as N
from etx.models import configs
from progress_log import say

pytestmark = pytest.mark.gpu

SEED = 20261203


def check_cache(cfg, dec, orc):
    for L in range(cfg.L):
        kg, vg = dec.kv_layer(L)
        ko, vo = orc.kv(L)
        assert np.array_equal(kg, ko), f"layer {L}: paged K cache differs in {np.sum(kg != ko)} entries"
        assert np.array_equal(vg, vo), f"layer {L}: paged V cache differs in {np.sum(vg != vo)} entries"


def run_prefill(cfg, prompt_len, n_new, rows, start=0):
    """Positions [0, start) come from the seeded KV fill; the prompt covers [start, start + prompt_len) in launches
    of `rows` positions, the last launch writing the first greedy token; then n_new - 1 decode steps."""
    t0 = time.time()
    say(f"[gpu] prefill {cfg.name}: {start} cached + {prompt_len} prompt positions, {rows} per launch, {n_new} new")
    dec = N.Decoder(cfg)
    dec.init_weights(SEED, 0.02)
    orc = O.OracleModel(cfg.as_dict(), SEED, 0.02)
    if start:
        dec.fill_kv_seeded(SEED, start)
        orc.fill_kv_random(start)
    prompt = O.gen_tokens(SEED + start, prompt_len, cfg.V)
    row = np.zeros(start + prompt_len, np.int32)
    row[start:] = prompt
    dec.set_tokens(row)
    end = start + prompt_len
    for p0 in range(start, end, rows):
        n = min(rows, end - p0)
        dec.prefill(p0, n, write_next=p0 + n == end)
    for pos in range(end, end + n_new - 1):
        dec.step(pos, write_next=True)
    dec.sync()
    say(f"[gpu]   device done ({time.time() - t0:.1f}s)")
    seq = list(row)
    greedy = []                                            # the oracle's greedy token at every position
    for pos in range(start, end + n_new - 1):
        t = orc.step(seq[pos], pos)
        greedy.append(t)
        if pos + 1 >= end:
            seq.append(t)
    say(f"[gpu]   oracle done ({time.time() - t0:.1f}s)")
    got = dec.read_tokens(end + n_new - 1)[start:]
    bad = [start + i for i in range(len(greedy)) if got[i] != greedy[i]]
    assert not bad, f"greedy tokens differ at positions {bad[:10]}"
    check_cache(cfg, dec, orc)
    orc.close()
    dec.close()


@pytest.mark.parametrize("base,pf,rows,plen", [(configs.TINY_MOE, 16, 16, 150), (configs.TINY_MOE, 16, 12, 150),
                                               (configs.TINY_MOE, 16, 3, 40), (configs.TINY_DENSE, 4, 3, 70)],
                         ids=["moe-16", "moe-12", "moe-3", "dense-3"])
def test_tiny_prefill_bit_exact(gpu, base, pf, rows, plen):
    """Launches of 12 and 3 positions straddle the 64-position chunks and the two-chunk attention items (at 64, 128);
    the last launch is ragged."""
    run_prefill(configs.with_layers(base, base.L, prefill=pf), plen, n_new=6, rows=rows)


def test_tiny_prefill_after_cached_context(gpu):
    """A prompt continuing 300 cached positions: the launches' rows read several cached chunks and patch the rest."""
    run_prefill(configs.with_layers(configs.TINY_MOE, configs.TINY_MOE.L, prefill=16, max_ctx=512), 45, n_new=4,
                rows=16, start=300)


def test_tiny_prefill_fp8(gpu):
    cfg = configs.with_layers(configs.TINY_MOE, configs.TINY_MOE.L, prefill=16, wdtype=N.W_FP8)
    run_prefill(cfg, 40, n_new=4, rows=16)


@pytest.mark.parametrize("B", [4, 16], ids=["b4", "b16"])
def test_tiny_batched_handle_prefill_per_sequence(gpu, B):
    """A batch-B handle: each prompt prefilled on its own (B positions per launch, other sequences untouched), then
    batched decode from the end of each prompt; against the oracle's token-by-token decode of every prompt.  At
    batch 16 the handle's projections run on the matrix cores, the ragged last launches of fewer than 8 positions
    included, and the oracle (a model of the same batch capacity) follows the tile order."""
    cfg = configs.with_layers(configs.TINY_MOE, configs.TINY_MOE.L, batch=B)
    say(f"[gpu] prefill per sequence, batch-{B} handle {cfg.name}")
    dec = N.Decoder(cfg)
    dec.init_weights(SEED, 0.02)
    assert dec.prefill_rows == B
    prompts = [O.gen_tokens(SEED + b, 5 + (9 if B == 4 else 7) * b, cfg.V) for b in range(B)]
    got = dec.generate_batch(prompts, 5, prefill=True)
    for b, p in enumerate(prompts):
        o = O.OracleModel(cfg.as_dict(), SEED, 0.02)
        toks = list(p)
        for q in range(len(p) + 4):
            t = o.step(toks[q], q)
            if q + 1 >= len(p):
                toks.append(t)
        assert list(got[b]) == toks[len(p):], f"sequence {b}"
        o.close()
    dec.close()


def test_qwen3_30b_a3b_prefill_two_layers(gpu):
    """Real Qwen3-30B-A3B shapes (two layers, vocab 151936): 16 positions per launch of the batch-16 kernel."""
    run_prefill(configs.with_layers(configs.QWEN3_30B_A3B, 2, prefill=16), 70, n_new=4, rows=16)


def test_qwen3_8b_prefill_two_layers(gpu):
    """Qwen3-8B shapes (two dense layers, 12288-long down rows): 4 positions per launch of its batch-4 kernel."""
    run_prefill(configs.with_layers(configs.QWEN3_8B, 2, prefill=4), 22, n_new=4, rows=4)


def run_prefill_mla(cfg, prompt_len, n_new, rows):
    """DeepSeek-V2: the prompt in launches of `rows` positions, then n_new - 1 decode steps (a batch-1 handle runs
    its batched kernel as a batch of one); the latent cache and every position's greedy token against the oracle."""
    t0 = time.time()
    say(f"[gpu] prefill {cfg.name}: {prompt_len} prompt positions, {rows} per launch, {n_new} new")
    dec = N.Decoder(cfg)
    dec.init_weights(SEED, 0.02)
    orc = O.OracleModel(cfg.as_dict(), SEED, 0.02)
    prompt = O.gen_tokens(SEED, prompt_len, cfg.V)
    dec.set_tokens(prompt)
    dec.feed_prompt(prompt_len, rows=rows)
    for pos in range(prompt_len, prompt_len + n_new - 1):
        dec.step(pos, write_next=True)
    dec.sync()
    seq, greedy = list(prompt), []
    for pos in range(prompt_len + n_new - 1):
        t = orc.step(seq[pos], pos)
        greedy.append(t)
        if pos + 1 >= prompt_len:
            seq.append(t)
    say(f"[gpu]   device and oracle done ({time.time() - t0:.1f}s)")
    got = dec.read_tokens(prompt_len + n_new - 1)
    bad = [i for i in range(len(greedy)) if got[i] != greedy[i]]
    assert not bad, f"greedy tokens differ at positions {bad[:10]}"
    for L in range(cfg.L):
        assert np.array_equal(dec.kv_layer(L)[0], orc.kv(L)[0]), f"layer {L}: latent cache differs"
    orc.close()
    dec.close()


@pytest.mark.parametrize("rows,plen", [(4, 90), (3, 70)], ids=["rows4", "rows3"])
def test_tiny_mla_prefill_bit_exact(gpu, rows, plen):
    """Launches of 3 positions straddle the 64-position chunk boundary; the last launch is ragged."""
    run_prefill_mla(configs.with_layers(configs.TINY_MLA, configs.TINY_MLA.L, prefill=4), plen, n_new=5, rows=rows)


def test_tiny_mla_batched_handle_prefill(gpu):
    cfg = configs.with_layers(configs.TINY_MLA, configs.TINY_MLA.L, batch=4)
    say(f"[gpu] mla prefill per sequence, batch-4 handle {cfg.name}")
    dec = N.Decoder(cfg)
    dec.init_weights(SEED, 0.02)
    prompts = [O.gen_tokens(SEED + b, 6 + 11 * b, cfg.V) for b in range(4)]
    got = dec.generate_batch(prompts, 5, prefill=True)
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


def test_deepseek_v2_lite_prefill_two_layers(gpu):
    """DeepSeek-V2-Lite shapes (the dense layer 0 and one MoE layer): 4 positions per launch."""
    run_prefill_mla(configs.with_layers(configs.DEEPSEEK_V2_LITE, 2, prefill=4), 26, n_new=4, rows=4)


def test_prefill_refusals(gpu):
    """Rows beyond the handle's prefill rows, positions past max_ctx, a sequence outside the batch and the unfused
    mode are refused before anything is launched."""
    cfg = configs.with_layers(configs.TINY_MOE, configs.TINY_MOE.L, prefill=4)
    dec = N.Decoder(cfg)
    dec.init_weights(SEED, 0.02)
    for args, kw, msg in [((0, 5), {}, "prefill positions"), ((0, 0), {}, "prefill positions"),
                          ((cfg.max_ctx - 2, 4), {}, "outside"), ((0, 2), {"seq": 1}, "sequence")]:
        with pytest.raises(N.EtxmkError, match=msg):
            dec.prefill(*args, **kw)
    dec.close()
    unf = N.Decoder(cfg, fused=False)
    with pytest.raises(N.EtxmkError, match="persistent kernel"):
        unf.prefill(0, 2)
    assert unf.prefill_rows == 0
    unf.close()
