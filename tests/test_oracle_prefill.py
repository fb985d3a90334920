"""The oracle's many-position form (orc_prefill_seq) against its one-step form (orc_step_seq).

A prompt fed through OracleModel.prefill in pieces of any length must leave the same KV cache, and give every
position the same greedy token, as feeding it one decode step per token (the prompt loop of
examples/llm/host.hip:203-213).  The one-step form is the restatement of examples/llm/ref_numpy.py:105-158 that the
other oracle tests pin; this file pins the many-position form to it, bit for bit, over the dense, MoE and fp8 paths,
a shuffled block table, and pieces that start and end inside 64-position attention chunks and 16-position blocks."""
import numpy as np
import pytest

from oracle import oracle as O
from etx.models import configs
from etx.runtime import native as N

SEED = 20261202


def _stepwise(orc, prompt, seq=0):
    return np.array([orc.step(int(t), pos, seq=seq) for pos, t in enumerate(prompt)], np.int32)


def _caches(orc, L):
    return [orc.kv(layer) for layer in range(L)]


@pytest.mark.parametrize("name,pieces", [
    ("tiny-moe", [70, 1, 13, 64, 2]),
    ("tiny-dense", [150]),
    ("tiny-moe-fp8", [17, 47, 86]),
])
def test_prefill_equals_stepwise(oracle_lib, name, pieces):
    base = configs.TINY_DENSE if name == "tiny-dense" else configs.TINY_MOE
    cfg = configs.with_layers(base, base.L, wdtype=N.W_FP8) if name.endswith("fp8") else base
    n = sum(pieces)
    prompt = O.gen_tokens(SEED, n, cfg.V)
    a = O.OracleModel(cfg.as_dict(), SEED)
    b = O.OracleModel(cfg.as_dict(), SEED)
    bt = np.random.default_rng(3).permutation(a.num_blocks).astype(np.int32)
    a.set_block_table(bt)
    b.set_block_table(bt)
    want = _stepwise(a, prompt)
    got, p0 = [], 0
    for k in pieces:
        got.append(b.prefill(prompt[p0:p0 + k], p0))
        p0 += k
    got = np.concatenate(got)
    assert np.array_equal(got, want), f"greedy tokens differ at {np.flatnonzero(got != want)[:8]}"
    for layer, ((ka, va), (kb, vb)) in enumerate(zip(_caches(a, cfg.L), _caches(b, cfg.L))):
        assert np.array_equal(ka, kb) and np.array_equal(va, vb), f"layer {layer}: KV cache differs"
    # decoding continues identically from either cache
    t = int(want[-1])
    for pos in range(n, n + 3):
        ta, tb = a.step(t, pos, dump=True), b.step(t, pos, dump=True)
        assert ta[0] == tb[0] and np.array_equal(ta[1], tb[1]) and np.array_equal(ta[2], tb[2])
        t = ta[0]
    a.close()
    b.close()


def test_prefill_second_sequence_of_a_batch(oracle_lib):
    """A batched oracle's sequence 1 prefilled in one piece equals its single-step decode; sequence 0 is untouched."""
    cfg = configs.with_layers(configs.TINY_MOE, 2, batch=2)
    prompt = O.gen_tokens(SEED + 1, 40, cfg.V)
    a = O.OracleModel(cfg.as_dict(), SEED)
    b = O.OracleModel(cfg.as_dict(), SEED)
    want = _stepwise(a, prompt, seq=1)
    got = b.prefill(prompt, 0, seq=1)
    assert np.array_equal(got, want)
    ka, _ = a.kv(0)
    kb, _ = b.kv(0)
    assert np.array_equal(ka, kb)
    a.close()
    b.close()


def test_prefill_refuses_bad_ranges(oracle_lib):
    cfg = configs.TINY_DENSE
    o = O.OracleModel(cfg.as_dict(), SEED)
    with pytest.raises(ValueError):
        o.prefill(np.zeros(4, np.int32), cfg.max_ctx - 2)
    o.close()


@pytest.mark.parametrize("name", ["tiny-moe", "tiny-dense", "tiny-moe-fp8"])
def test_step_rows_equals_batched_single_steps(oracle_lib, name):
    """A batched step of several sequences (shuffled pool, contexts across chunks) through step_rows equals one
    step() per sequence: tokens, per-layer residuals, top-k ids and weights, and the pool."""
    base = configs.TINY_DENSE if name == "tiny-dense" else configs.TINY_MOE
    kw = dict(batch=5) if not name.endswith("fp8") else dict(batch=5, wdtype=N.W_FP8)
    cfg = configs.with_layers(base, base.L, **kw)
    a = O.OracleModel(cfg.as_dict(), SEED)
    b = O.OracleModel(cfg.as_dict(), SEED)
    bt = np.random.default_rng(11).permutation(a.num_blocks).astype(np.int32)
    a.set_block_table(bt)
    b.set_block_table(bt)
    ctx = [3, 130, 64, 200, 0]
    for s, n in enumerate(ctx):
        a.fill_kv_random(n, seq=s)
        b.fill_kv_random(n, seq=s)
    toks = [int(t) for t in O.gen_tokens(SEED + 5, 5, cfg.V)]
    pos = list(ctx)
    order = [3, 0, 4, 1, 2]                                # rows in any order of sequences
    for step in range(3):
        want = {s: a.step(toks[s], pos[s], dump=True, seq=s) for s in range(5)}
        out, x, ids, w = b.step_rows(order, [toks[s] for s in order], [pos[s] for s in order], dump=True)
        for r, s in enumerate(order):
            t, xo, ido, wo = want[s]
            assert out[r] == t, f"step {step} sequence {s}: token"
            assert np.array_equal(x[r], xo), f"step {step} sequence {s}: residuals"
            if cfg.moe:
                assert np.array_equal(ids[r], ido) and np.array_equal(w[r], wo), f"step {step} sequence {s}: routing"
        toks = [int(want[s][0]) for s in range(5)]
        pos = [p + 1 for p in pos]
    for layer in range(cfg.L):
        ka, va = a.kv(layer)
        kb, vb = b.kv(layer)
        assert np.array_equal(ka, kb) and np.array_equal(va, vb), f"layer {layer}: pool differs"
    a.close()
    b.close()


@pytest.mark.parametrize("K", [64, 128, 512, 768, 2048, 4096])
def test_vector_dot_equals_scalar_dot(oracle_lib, K):
    """The rows form's AVX2 dot (orc_dot64f: fp32 weight images, 8 ymm accumulators, hadd tree) against the scalar
    canonical dot (orc_dot64: bf16 weights, 64 accumulators, lanes_reduce) on the same values: equal bit for bit.
    The inputs span 40 binades so that the lane tree's shape decides the rounding: a plain left-to-right sum of the
    same 64 lane values differs from the tree on most rows, which the test also checks (it could not tell the two
    orders apart otherwise)."""
    L = O.lib()
    rng = np.random.default_rng(K)
    differs = 0
    for trial in range(200):
        w = O.f32_to_bf16_bits((rng.standard_normal(K) * np.exp2(rng.uniform(-20, 20, K))).astype(np.float32))
        x = O.bf16_bits_to_f32(O.f32_to_bf16_bits((rng.standard_normal(K) * np.exp2(rng.uniform(-20, 20, K)))
                                                  .astype(np.float32)))
        wf = O.bf16_bits_to_f32(w)
        got = L.orc_dot64f(np.ascontiguousarray(wf), np.ascontiguousarray(x), K)
        want = L.orc_dot64(np.ascontiguousarray(w), np.ascontiguousarray(x), K)
        assert np.float32(got).tobytes() == np.float32(want).tobytes(), f"trial {trial}: {got!r} vs {want!r}"
        acc = np.zeros(64, np.float32)
        for k in range(K):                                 # the per-lane fma chains, rounded per step
            acc[k % 64] = np.float32(np.float64(acc[k % 64]) + np.float64(wf[k]) * np.float64(x[k]))
        seq = np.float32(0)
        for v in acc:
            seq = np.float32(seq + v)
        differs += seq != np.float32(want)
    assert differs > 20, "the inputs do not separate the tree from a sequential lane sum"
