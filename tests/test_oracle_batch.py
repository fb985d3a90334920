"""The oracle's batch: sequences share the weights and one paged-KV pool through their own block-table rows, and
nothing else.  Each sequence of a batched oracle must decode exactly as a single-sequence oracle does, whatever
physical blocks its table names."""
import numpy as np

from oracle import oracle as O
from etx.models import configs

SEED = 20261201


def _decode(orc, seq, prompt, n_new):
    toks = list(prompt)
    for pos in range(len(prompt) + n_new - 1):
        t = orc.step(toks[pos], pos, seq=seq)
        if pos + 1 >= len(prompt):
            toks.append(t)
    return toks[len(prompt):]


def test_sequences_are_independent(oracle_lib):
    cfg = configs.TINY_MOE
    prompts = [O.gen_tokens(SEED + b, 5 + 3 * b, cfg.V) for b in range(3)]
    single = []
    for p in prompts:
        o1 = O.OracleModel(cfg.as_dict(), SEED)
        single.append(_decode(o1, 0, p, 4))
        o1.close()
    ob = O.OracleModel(configs.with_layers(cfg, cfg.L, batch=3).as_dict(), SEED)
    assert ob.num_blocks == 3 * ob.blocks_per_seq
    # a shuffled pool: sequence b's blocks are scattered over the whole pool
    bt = np.random.default_rng(7).permutation(ob.num_blocks).astype(np.int32).reshape(3, -1)
    ob.set_block_table(bt)
    got = [None] * 3
    for b in (2, 0, 1):                                    # order of sequences does not matter
        got[b] = _decode(ob, b, prompts[b], 4)
    assert got == single
    ob.close()


def test_kv_fill_streams_are_per_sequence(oracle_lib):
    cfg = configs.with_layers(configs.TINY_DENSE, 1, batch=2)
    orc = O.OracleModel(cfg.as_dict(), SEED)
    orc.fill_kv_random(64, seq=0)
    orc.fill_kv_random(64, seq=1)
    k, _ = orc.kv(0)
    per_block = cfg.block_size * cfg.NKV * cfg.HD
    nbps = orc.blocks_per_seq
    s0, s1 = k[:4 * per_block], k[nbps * per_block:(nbps + 4) * per_block]
    assert np.any(s0 != 0) and np.any(s1 != 0) and not np.array_equal(s0, s1)
    # sequence 0's stream is the single-sequence one
    o1 = O.OracleModel(configs.with_layers(configs.TINY_DENSE, 1).as_dict(), SEED)
    o1.fill_kv_random(64)
    assert np.array_equal(o1.kv(0)[0][:4 * per_block], s0)
    o1.close()
    orc.close()
