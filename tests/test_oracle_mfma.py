"""The oracle's statement of the gfx950 bf16 matrix-core step (orc_mfma_bf16_k32 / _chain in oracle/mk_oracle.c)
against the instruction's own outputs, kept in tests/golden/mfma_bf16_gfx950.npz (made by
tests/golden/make_mfma_fixture.py on an MI355X): every kept element bit for bit, and each plausible alternative rule
(tests/mfma_hypotheses.py) refuted by some of them, so that the fixture pins every part of the statement."""
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle as O
import mfma_hypotheses as H

FIX = np.load(Path(__file__).parent / "golden" / "mfma_bf16_gfx950.npz")
FAMILIES = ("wide", "narrow", "czero", "cancel", "chain8", "chain4_wide")


def _elems(name):
    a, b, c, d = (FIX[f"{name}_{k}"] for k in "abcd")
    return a, b, c, d, a.shape[1] // 32


@pytest.mark.parametrize("name", FAMILIES)
def test_oracle_matches_hardware(name):
    L = O.lib()
    a, b, c, d, steps = _elems(name)
    for i in range(len(c)):
        got = L.orc_mfma_bf16_chain(float(c[i]), np.ascontiguousarray(a[i]), np.ascontiguousarray(b[i]), steps)
        assert np.float32(got).tobytes() == np.float32(d[i]).tobytes(), f"{name} element {i}: {got!r} vs {d[i]!r}"


def test_fixture_refutes_every_alternative():
    rules = list(FIX["rules"])
    assert rules == list(H.RULES[1:])
    for i, rule in enumerate(rules):
        n = sum(int(np.sum(FIX[f"{name}_refutes"] >> i & 1)) for name in FAMILIES)
        assert n >= 5, f"the fixture refutes {rule} on {n} elements only"


@pytest.mark.parametrize("name", FAMILIES)
def test_recorded_refutations_hold(name):
    """For two elements per alternative: the alternative (exact rational statement) differs from the hardware, and
    the measured rule in the same statement equals it."""
    a, b, c, d, steps = _elems(name)
    ref = FIX[f"{name}_refutes"]
    for i, rule in enumerate(H.RULES[1:]):
        for j in np.flatnonzero(ref >> i & 1)[:2]:
            want = np.float32(d[j]).tobytes()
            assert np.float32(H.chain(c[j], a[j], b[j], steps, rule)).tobytes() != want
            assert np.float32(H.chain(c[j], a[j], b[j], steps, "measured")).tobytes() == want


def test_small_integers_are_exact():
    L = O.lib()
    rng = np.random.default_rng(3)
    for _ in range(200):
        a = rng.integers(-40, 41, 32).astype(np.float32)
        b = rng.integers(-40, 41, 32).astype(np.float32)
        c = float(rng.integers(-1000, 1000))
        got = L.orc_mfma_bf16_k32(c, H.bf16_bits(a), H.bf16_bits(b))
        assert got == c + float(np.dot(a.astype(np.float64), b.astype(np.float64)))


def test_zero_products_leave_the_accumulator():
    L = O.lib()
    z = np.zeros(32, np.uint16)
    for c in (0.0, 1.5, -3.25e-20, 7.0e30):
        assert np.float32(L.orc_mfma_bf16_k32(c, z, z)).tobytes() == np.float32(c).tobytes()
