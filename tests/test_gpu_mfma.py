"""The gfx950 bf16 matrix-core step on fresh seeded operands (tests/mfma_hypotheses.families, a seed the committed
fixture does not use) through the probe of libetxmk_calib.so, against the oracle's statement of it bit for bit:
wide-range, narrow, zero-accumulator and cancelling operands, 8-step chains at weight and activation scales, and
4-step wide chains."""
import numpy as np
import pytest

from oracle import oracle as O
from etx.runtime import calib
import mfma_hypotheses as H
from progress_log import say

pytestmark = pytest.mark.gpu


def test_matrix_core_step_matches_the_oracle(gpu):
    L = O.lib()
    for name, A, B, C in H.families(20261206, 8):
        say(f"[gpu] mfma probe {name}: {A.shape[0]} cases, {A.shape[2] // 32} steps")
        D = calib.mfma_bf16(A, B, C)
        steps = A.shape[2] // 32
        bad = 0
        for t in range(A.shape[0]):
            for r in range(16):
                for c in range(16):
                    want = L.orc_mfma_bf16_chain(float(C[t, r, c]), np.ascontiguousarray(A[t, r]),
                                                 np.ascontiguousarray(B[t, :, c]), steps)
                    bad += np.float32(want).tobytes() != np.float32(D[t, r, c]).tobytes()
        assert bad == 0, f"{name}: {bad} of {A.shape[0] * 256} elements differ from the oracle"


def test_probe_refuses_bad_arguments(gpu):
    with pytest.raises(ValueError):
        calib.mfma_bf16(np.zeros((1, 16, 30), np.uint16), np.zeros((1, 30, 16), np.uint16), np.zeros((1, 16, 16)))
