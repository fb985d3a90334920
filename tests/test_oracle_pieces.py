"""Oracle functions pinned against closed forms, brute force in float64, and the reference's own fixtures."""
import math

import numpy as np
import pytest

from oracle import oracle as O


def bf(x):
    return O.bf16_bits_to_f32(O.f32_to_bf16_bits(np.asarray(x, np.float32)))


@pytest.mark.parametrize("K", [64, 256, 768, 2048, 4096])
def test_dot64_against_float64(oracle_lib, K):
    rng = np.random.default_rng(K)
    w = O.f32_to_bf16_bits(rng.normal(0, 0.02, K))
    x = bf(rng.normal(0, 1, K))
    exact = float(O.bf16_bits_to_f32(w).astype(np.float64) @ x.astype(np.float64))
    got = O.dot64(w, x)
    bound = np.sum(np.abs(O.bf16_bits_to_f32(w).astype(np.float64) * x)) * 2.0 ** -24 * (K // 64 + 6)
    assert abs(got - exact) <= bound
    # a single nonzero term is exact wherever it sits (every lane and every butterfly stage carries it)
    for k in (0, 1, 63, K - 1):
        e = np.zeros(K, np.float32); e[k] = 1.0
        assert O.dot64(w, e) == float(O.bf16_bits_to_f32(w[k:k + 1])[0])


def test_rmsnorm_closed_form(oracle_lib):
    rng = np.random.default_rng(1)
    x = bf(rng.normal(0, 3, 2048))
    y = O.rmsnorm(x, 1e-6)
    r = 1 / math.sqrt(float(np.mean(x.astype(np.float64) ** 2)) + 1e-6)
    assert np.allclose(y, x * r, rtol=2 ** -7, atol=0)                  # bf16 twice
    assert abs(np.sqrt(np.mean(y.astype(np.float64) ** 2)) - 1) < 5e-3  # output RMS is one
    # a constant vector normalises to (almost) +-1
    c = np.full(128, 5.0, np.float32)
    assert np.all(O.rmsnorm(c, 1e-6) == 1.0)
    # with a weight the result is bfr(w * bfr(x r)); w = 2 doubles it exactly
    w2 = O.f32_to_bf16_bits(np.full(2048, 2.0, np.float32))
    assert np.array_equal(O.rmsnorm(x, 1e-6, w2), 2 * y)


def test_rope_position_zero_is_identity_and_rotation_preserves_norm(oracle_lib):
    cos, sin = O.rope_tables(1e6, 128, 1100)
    assert np.all(cos[0] == 1) and np.all(sin[0] == 0)
    rng = np.random.default_rng(2)
    v = bf(rng.normal(0, 1, 128))
    assert np.array_equal(O.apply_rope(v, cos[0], sin[0]), v)
    for p in (1, 17, 1023):
        r = O.apply_rope(v, cos[p], sin[p])
        assert abs(np.linalg.norm(r) / np.linalg.norm(v) - 1) < 1e-2
        # rotate_half pairs (d, d+64): the rotation angle of pair i is p * theta^(-2i/128)
        i = 5
        ang = p * 1e6 ** (-2 * i / 128)
        a, b = float(v[i]), float(v[i + 64])
        assert abs(float(r[i]) - (a * math.cos(ang) - b * math.sin(ang))) < 0.03
        assert abs(float(r[i + 64]) - (b * math.cos(ang) + a * math.sin(ang))) < 0.03


def test_rope_tables_match_reference_formula(oracle_lib):
    from oracle import ref_twin as T
    c, s = O.rope_tables(1e6, 128, 1100)
    tc, ts = T.rope_tables(1e6, 128, 1100)
    # same fp32 frequencies; cos/sin from libm vs numpy differ by at most one bf16 step on rare entries
    assert np.mean(c != tc) < 1e-3 and np.mean(s != ts) < 1e-3
    assert np.max(np.abs(c - tc)) <= 2 ** -8 and np.max(np.abs(s - ts)) <= 2 ** -8


def _paged(K, V, NKV, HD, BS, btab):
    """K,V [n][NKV][HD] float -> paged bf16 caches, by the layout of etx/importer/spec.py:274-281."""
    n = K.shape[0]
    nb = max(btab) + 1
    kc = np.zeros(nb * NKV * HD * BS, np.uint16); vc = np.zeros_like(kc)
    kb = O.f32_to_bf16_bits(K); vb = O.f32_to_bf16_bits(V)
    for t in range(n):
        blk, off = btab[t // BS], t % BS
        for h in range(NKV):
            for d in range(HD):
                kc[((((blk * NKV + h) * (HD // 8)) + d // 8) * BS + off) * 8 + d % 8] = kb[t, h, d]
                vc[(((blk * NKV + h) * HD) + d) * BS + off] = vb[t, h, d]
    return kc, vc


def test_kv_index_closed_form(oracle_lib):
    L = O.lib()
    NKV, HD, BS = 4, 128, 16
    for blk, off, h, d in [(0, 0, 0, 0), (3, 15, 2, 127), (7, 5, 3, 64), (1, 1, 1, 9)]:
        assert L.orc_kv_k_index(blk, off, h, d, NKV, HD, BS) == ((((blk * NKV + h) * 16) + d // 8) * 16 + off) * 8 + d % 8
        assert L.orc_kv_v_index(blk, off, h, d, NKV, HD, BS) == ((blk * NKV + h) * HD + d) * 16 + off
    # the K map is a bijection onto one block's [NKV][HD/8][BS][8] cube
    idx = {L.orc_kv_k_index(0, o, h, d, NKV, HD, BS) for o in range(BS) for h in range(NKV) for d in range(HD)}
    assert idx == set(range(NKV * HD * BS))


@pytest.mark.parametrize("n", [1, 5, 64, 65, 200])
def test_attention_brute_force(oracle_lib, n):
    rng = np.random.default_rng(n)
    NKV, HD, BS = 2, 128, 16
    K = bf(rng.normal(0, 1, (n, NKV, HD))); V = bf(rng.normal(0, 1, (n, NKV, HD)))
    btab = list(rng.permutation((n + BS - 1) // BS + 3))               # a shuffled block table
    kc, vc = _paged(K, V, NKV, HD, BS, btab)
    q = bf(rng.normal(0, 1, HD))
    for h in range(NKV):
        got = O.attention_head(q, kc, vc, np.array(btab, np.int32), n, h, NKV, HD, BS)
        s = K[:, h].astype(np.float64) @ q.astype(np.float64) / math.sqrt(HD)
        p = np.exp(s - s.max()); p /= p.sum()
        ref = p @ V[:, h].astype(np.float64)
        assert np.allclose(got, ref, rtol=2 ** -7, atol=1e-6)
    if n == 1:                                                          # one position: o = v exactly
        assert np.array_equal(O.attention_head(q, kc, vc, np.array(btab, np.int32), 1, 0, NKV, HD, BS), V[0, 0])


def test_route_ties_lower_id_and_renorm(oracle_lib):
    # etx/bench/numerical.py fixture rule (tests/test_cpu_numerical.py:16-23): equal logits -> ids [0, 1]
    ids, w = O.route(np.zeros(8, np.float32), 2, True)
    assert list(ids) == [0, 1] and np.all(w == 0.5)
    ids, w = O.route(np.zeros(8, np.float32), 2, False)
    assert list(ids) == [0, 1] and np.all(w == bf(0.125))
    lg = bf(np.array([1.0, 3.0, 3.0, -2.0, 3.0, 0.5], np.float32))
    ids, w = O.route(lg, 3, True)
    assert list(ids) == [1, 2, 4] and np.all(w == bf(1 / 3))
    rng = np.random.default_rng(4)
    for _ in range(50):
        lg = bf(rng.normal(0, 1, 128))
        ids, w = O.route(lg, 8, True)
        p = np.exp(lg.astype(np.float64) - lg.max()); p /= p.sum()
        ref = sorted(range(128), key=lambda i: (-p[i], i))[:8]
        assert list(ids) == ref
        assert np.allclose(w, p[ref] / p[ref].sum(), rtol=2 ** -7)


def test_moe_block_fixture_against_scalar_float64(oracle_lib):
    """The reference's synthetic MoE fixture (etx/bench/numerical.py:31-39: seed 17, N(0, 0.15) weights,
    E in {8, 128}, top-k {2, 8}, renorm on/off), bf16-quantised, through the oracle's layer with the
    attention path made neutral, against an independent float64 scalar reference of the same block."""
    from oracle.oracle import OracleModel
    for E, K in ((8, 2), (128, 8)):
        for renorm in (False, True):
            rng = np.random.default_rng(17)
            H, MI = 64, 64                  # the fixture's hidden 8 / intermediate 12 padded to the 64-lane unit
            wt = lambda shape: bf(rng.normal(0, 0.15, shape))
            x, router = wt(H), wt((E, H))
            gate, up, down = wt((E, MI, H)), wt((E, MI, H)), wt((E, H, MI))
            xs = O.rmsnorm(x, 1e-5)
            logits = bf(np.array([O.dot64(O.f32_to_bf16_bits(router[e]), xs) for e in range(E)], np.float32))
            ids, wts = O.route(logits, K, renorm)
            # float64 scalar reference (fsum, own routing) on the same normalised input
            lg = [math.fsum(float(a) * float(b) for a, b in zip(row, xs)) for row in router]
            ex = [math.exp(v - max(lg)) for v in lg]
            pr = [v / math.fsum(ex) for v in ex]
            sel = sorted(range(E), key=lambda i: (-pr[i], i))[:K]
            assert list(ids) == sel
            den = math.fsum(pr[i] for i in sel) if renorm else 1.0
            assert np.allclose(wts, [pr[i] / den for i in sel], rtol=2e-2)   # logits are bf16 before the softmax
            out = np.zeros(H)
            got = np.zeros(H, np.float32)
            acc = np.zeros(H, np.float32)
            for slot in sorted(range(K), key=lambda s: ids[s]):
                e = ids[slot]
                g = bf([O.dot64(O.f32_to_bf16_bits(gate[e, j]), xs) for j in range(MI)])
                u = bf([O.dot64(O.f32_to_bf16_bits(up[e, j]), xs) for j in range(MI)])
                hh = bf(bf(np.array([O.lib().orc_silu(float(v)) for v in g], np.float32)) * u)
                y = bf(bf([O.dot64(O.f32_to_bf16_bits(down[e, i]), hh) for i in range(H)]) * np.float32(wts[slot]))
                acc = bf(acc + y)
                g64 = np.array([math.fsum(float(a) * float(b) for a, b in zip(r, xs)) for r in gate[e]])
                u64 = np.array([math.fsum(float(a) * float(b) for a, b in zip(r, xs)) for r in up[e]])
                m64 = g64 / (1 + np.exp(-g64)) * u64
                out += pr[e] / den * (down[e].astype(np.float64) @ m64)
            got = bf(x + acc)
            ref = x.astype(np.float64) + out
            assert np.max(np.abs(got - ref)) / np.max(np.abs(ref)) < 2e-2
