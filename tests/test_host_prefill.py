"""Host logic of prompt reading (etx/runtime/native.py Decoder.feed_prompt / generate / generate_batch) with the
launches recorded instead of run: the chunking of a prompt into prefill launches, the write-next flag on the last
one only, the token-by-token fallback, and the positions of the batched steps that follow."""
import numpy as np
import pytest

from etx.runtime import native as N
from etx.models import configs


class Recorder(N.Decoder):
    """A Decoder whose launches are recorded; no device, no library."""

    def __init__(self, cfg, fused=True):                  # noqa: D401 - no base initialisation on purpose
        self.cfg, self.fused, self.calls = cfg, fused, []

    def prefill(self, pos0, n, write_next=True, seq=0):
        self.calls.append(("prefill", seq, pos0, n, bool(write_next)))

    def step(self, pos, write_next=True):
        self.calls.append(("step", pos, bool(write_next)))

    def step_batch(self, positions, write_next=True):
        self.calls.append(("batch", list(positions), write_next))

    def set_tokens(self, tokens, seq=0):
        self.calls.append(("tokens", seq, len(tokens)))

    def sync(self):
        pass

    def read_tokens(self, n, seq=0):
        return np.arange(n, dtype=np.int32)


def test_prefill_rows_of_a_handle():
    assert Recorder(configs.TINY_MOE).prefill_rows == 0
    assert Recorder(configs.with_layers(configs.TINY_MOE, 2, prefill=16)).prefill_rows == 16
    assert Recorder(configs.with_layers(configs.TINY_MOE, 2, batch=4)).prefill_rows == 4
    assert Recorder(configs.with_layers(configs.TINY_MOE, 2, batch=4, prefill=16)).prefill_rows == 16
    assert Recorder(configs.with_layers(configs.TINY_MOE, 2, prefill=16), fused=False).prefill_rows == 0


def test_feed_prompt_chunks_and_flags():
    d = Recorder(configs.with_layers(configs.TINY_MOE, 2, prefill=16))
    d.feed_prompt(37, seq=0)
    assert d.calls == [("prefill", 0, 0, 16, False), ("prefill", 0, 16, 16, False), ("prefill", 0, 32, 5, True)]
    d.calls.clear()
    d.feed_prompt(32, rows=16)                            # an exact multiple: the last full launch writes next
    assert d.calls == [("prefill", 0, 0, 16, False), ("prefill", 0, 16, 16, True)]
    d.calls.clear()
    d.feed_prompt(3, rows=1)                              # token by token on a single-sequence handle
    assert d.calls == [("step", 0, False), ("step", 1, False), ("step", 2, True)]


def test_feed_prompt_without_rows_on_a_batched_handle_is_refused():
    d = Recorder(configs.with_layers(configs.TINY_MOE, 2, batch=4))
    with pytest.raises(ValueError):
        d.feed_prompt(5, rows=1)


def test_generate_uses_prefill_then_steps():
    d = Recorder(configs.with_layers(configs.TINY_MOE, 2, prefill=4))
    out = d.generate(list(range(6)), 3)
    assert d.calls == [("tokens", 0, 6), ("prefill", 0, 0, 4, False), ("prefill", 0, 4, 2, True),
                       ("step", 6, True), ("step", 7, True)]
    assert list(out) == [5, 6, 7]                         # out_tokens[P-1 .. P+n-2]
    d.calls.clear()
    d.generate(list(range(3)), 2, prefill=False)
    assert d.calls == [("tokens", 0, 3), ("step", 0, False), ("step", 1, False), ("step", 2, True), ("step", 3, True)]


def test_generate_batch_prefills_each_sequence_then_steps_together():
    d = Recorder(configs.with_layers(configs.TINY_MOE, 2, batch=2))
    out = d.generate_batch([[1, 2, 3], [4, 5, 6, 7, 8]], 3, prefill=True)
    pf = [c for c in d.calls if c[0] == "prefill"]
    assert pf == [("prefill", 0, 0, 2, False), ("prefill", 0, 2, 1, True),
                  ("prefill", 1, 0, 2, False), ("prefill", 1, 2, 2, False), ("prefill", 1, 4, 1, True)]
    assert [c for c in d.calls if c[0] == "batch"] == [("batch", [3, 5], True), ("batch", [4, 6], True)]
    assert out.shape == (2, 3) and list(out[0]) == [2, 3, 4] and list(out[1]) == [4, 5, 6]
