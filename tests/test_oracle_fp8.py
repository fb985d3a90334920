"""The oracle's fp8 weights: the e4m3 codec, per-row quantisation, the scaled dot, and the
fp8 model against the dequantised-bf16 reference within the north star's 5e-2 gate.

The codec is pinned against torch's float8_e4m3fn (an independent implementation: decode of all 256 codes, and
round-to-nearest-even encoding of values inside the range); saturation at +-448 is this build's rule, checked on
its own.  The scaled dot is pinned to the bf16 canonical dot (pinned elsewhere), since every e4m3 value is a bf16
value."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from etx.models import configs

SEED = 20261201


def test_decode_all_codes_matches_torch(oracle_lib):
    L = O.lib()
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    got = np.array([L.orc_e4m3_to_f32(int(c)) for c in codes], np.float32)
    finite = ~np.isnan(ref)
    assert np.sum(~finite) == 2                                # 0x7F and 0xFF
    assert np.array_equal(got[finite], ref[finite])
    assert got[0x7E] == 448.0 and got[0x08] == 2.0 ** -6 and got[0x01] == 2.0 ** -9 and got[0x38] == 1.0


def test_encode_matches_torch_inside_the_range(oracle_lib):
    L = O.lib()
    rng = np.random.default_rng(3)
    mags = np.concatenate([rng.uniform(0, 448, 20000), 2.0 ** rng.uniform(-12, 8.8, 20000)]).astype(np.float32)
    mags = mags[mags < 448]
    x = np.concatenate([mags, -mags]).astype(np.float32)
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    got = np.array([L.orc_f32_to_e4m3(float(v)) for v in x], np.uint8)
    assert np.array_equal(got, ref), f"{np.sum(got != ref)} encodings differ"
    # the midpoints between neighbouring codes round to the even one
    for c in range(1, 0x7D):
        lo, hi = L.orc_e4m3_to_f32(c), L.orc_e4m3_to_f32(c + 1)
        mid = np.float32((np.float64(lo) + np.float64(hi)) / 2)
        assert L.orc_f32_to_e4m3(float(mid)) == (c if c % 2 == 0 else c + 1)


def test_saturation(oracle_lib):
    L = O.lib()
    for v in (448.0, 449.0, 465.0, 1e9, float("inf")):
        assert L.orc_f32_to_e4m3(v) == 0x7E and L.orc_f32_to_e4m3(-v) == 0xFE


def test_quantize_rows_error_bound(oracle_lib):
    L = O.lib()
    R, K = 64, 768
    w = O.gen_normal_bf16(SEED, 99, R * K, scale=0.02)
    q = np.zeros(R * K, np.uint8)
    s = np.zeros(R, np.float32)
    L.orc_quantize_rows(w, R, K, q, s)
    wf = O.bf16_bits_to_f32(w).reshape(R, K)
    dec = np.array([L.orc_e4m3_to_f32(int(c)) for c in range(256)], np.float32)[q].reshape(R, K)
    assert np.allclose(s, np.abs(wf).max(axis=1) / np.float32(448))
    assert np.all(np.abs(dec).max(axis=1) == 448.0)            # the row maximum lands on the top code
    err = np.abs(dec * s[:, None] - wf)
    # round to nearest: half a step of 3 mantissa bits (relative 2^-4), or half the subnormal step 2^-9
    bound = np.maximum(np.abs(wf) * 2.0 ** -4, s[:, None] * 2.0 ** -10) * (1 + 1e-6)
    assert np.all(err <= bound)


def test_scaled_dot_is_the_canonical_dot_over_decoded_weights(oracle_lib):
    L = O.lib()
    K = 2048
    rng = np.random.default_rng(5)
    q = rng.integers(0, 256, K, dtype=np.uint8)
    q[(q & 0x7F) == 0x7F] = 0x10                               # no NaN codes
    x = O.bf16_bits_to_f32(O.gen_normal_bf16(SEED, 7, K, scale=1.0))
    dec = np.array([L.orc_e4m3_to_f32(int(c)) for c in q], np.float32)
    assert L.orc_dot64_q(q, x, K) == L.orc_dot64(O.f32_to_bf16_bits(dec), x, K)


@pytest.mark.parametrize("base", [configs.TINY_MOE, configs.TINY_DENSE], ids=["moe", "dense"])
def test_fp8_model_within_gate_of_dequantised_reference(oracle_lib, base):
    """Greedy decode with fp8 weights (scaled dots) against the same weights dequantised into bf16 (HF-style):
    per-layer residuals within max rel 5e-2 while both read the same tokens."""
    d8 = dict(base.as_dict(), wdtype=O.W_FP8)
    dq = dict(base.as_dict(), wdtype=O.W_FP8_DEQ)
    m8, mq = O.OracleModel(d8, SEED), O.OracleModel(dq, SEED)
    prompt = O.gen_tokens(SEED, 10, base.V)
    worst = 0.0
    for pos, tok in enumerate(prompt):
        _, x8, i8, _ = m8.step(int(tok), pos, dump=True)
        _, xq, iq, _ = mq.step(int(tok), pos, dump=True)
        for L in range(base.L):
            worst = max(worst, float(np.max(np.abs(x8[L] - xq[L])) / np.max(np.abs(xq[L]))))
    assert worst < 5e-2, worst
    # and the fp8 matrices are what quantize_rows makes of the seeded bf16 rows
    mb = O.OracleModel(base.as_dict(), SEED)
    qq, ss = m8.weight_fp8(O.S_WQKV, 0)
    wb = mb.weight(O.S_WQKV, 0)
    q2 = np.zeros(wb.size, np.uint8)
    s2 = np.zeros(wb.shape[0], np.float32)
    O.lib().orc_quantize_rows(np.ascontiguousarray(wb.reshape(-1)), wb.shape[0], wb.shape[1], q2, s2)
    assert np.array_equal(qq.reshape(-1), q2) and np.array_equal(ss, s2)
    for m in (m8, mq, mb):
        m.close()
