"""Failure handling of a step (reference: etx_host::wait_stream / after_wait, etx/runtime/include/etx/host.h:351-417:
the host polls the stream with a timeout and writes the abort word; the kernel's waits are bounded by spin_limit).

Every case is forced from the host so that every kernel still exits normally: a spin limit of one clock tick makes
the kernel's own bounded waits give up, a stop request makes them leave, a zero timeout makes the host watchdog fire.
After each, the handle is reset by the sync that reports it, and re-running the interrupted positions gives exactly
the oracle's tokens, residuals and routing."""
import numpy as np
import pytest

from oracle import oracle as O
from etx.runtime import native as N
from etx.models import configs
from progress_log import say

pytestmark = pytest.mark.gpu

SEED = 20261203


def _oracle_run(cfg, prompt, n_new):
    """The oracle after decoding the prompt and n_new tokens, its token row and the dumps of each position."""
    orc = O.OracleModel(cfg.as_dict(), SEED, 0.02)
    seq, dumps = list(prompt), {}
    for pos in range(len(prompt) + n_new - 1):
        t, x, ids, w = orc.step(seq[pos], pos, dump=True)
        dumps[pos] = (x, ids, w)
        if pos + 1 >= len(prompt):
            seq.append(t)
    return orc, seq, dumps


def _check_step(dec, cfg, dumps, pos):
    d = dec.dumps()
    x, ids, w = dumps[pos]
    for L in range(cfg.L):
        assert np.array_equal(d["x"][L], x[L]), f"pos {pos} layer {L}: residual differs"
        assert np.array_equal(d["ids"][L], ids[L]), f"pos {pos} layer {L}: top-k ids differ"


def test_abort_paths_then_recovery(gpu):
    cfg = configs.TINY_MOE
    P, n_new = 8, 10
    prompt = O.gen_tokens(SEED, P, cfg.V)
    orc, seq, dumps = _oracle_run(cfg, prompt, n_new)
    dec = N.Decoder(cfg)
    dec.init_weights(SEED, 0.02)
    dec.enable_dumps(True)
    dec.set_tokens(prompt)

    def run(pos):
        dec.step(pos, write_next=pos + 1 >= P)

    for pos in range(4):
        run(pos)
    dec.sync()
    _check_step(dec, cfg, dumps, 3)

    say("[gpu] watchdog: device spin limit of one tick")
    dec.set_spin_limit(1, 1)
    run(4)
    with pytest.raises(N.DeviceAbort, match="exceeded its limit"):
        dec.sync()
    dec.set_spin_limit(0, 0)
    run(4)
    dec.sync()
    _check_step(dec, cfg, dumps, 4)

    say("[gpu] watchdog: host stop request")
    dec.set_spin_limit(0, 1)                               # waits look at the stop word at every poll
    dec.abort()
    run(5)
    with pytest.raises(N.DeviceAbort, match="host stop"):
        dec.sync()
    dec.set_spin_limit(0, 0)
    run(5)                                                 # the stop word was cleared by the sync that reported it
    dec.sync()
    _check_step(dec, cfg, dumps, 5)

    say("[gpu] watchdog: host timeout stops queued steps")
    dec.set_spin_limit(0, 1)
    for pos in range(6, 10):
        run(pos)
    with pytest.raises(N.StepTimeout):
        dec.sync(timeout_ms=0)
    dec.set_spin_limit(0, 0)
    for pos in range(6, 10):
        run(pos)
    dec.sync()
    _check_step(dec, cfg, dumps, 9)

    say("[gpu] watchdog: a timeout that the steps outlive without being stuck")
    for pos in range(10, P + n_new - 1):
        run(pos)
    try:
        dec.sync(timeout_ms=0)                             # default cadence: running steps finish and stand
    except N.StepTimeout:
        pass
    dec.sync()
    _check_step(dec, cfg, dumps, P + n_new - 2)
    got = dec.read_tokens(P + n_new - 1)
    assert list(got[P - 1:]) == seq[P:], "greedy tokens differ after the aborted steps were re-run"
    for L in range(cfg.L):
        kg, vg = dec.kv_layer(L)
        ko, vo = orc.kv(L)
        assert np.array_equal(kg, ko) and np.array_equal(vg, vo), f"layer {L}: KV cache differs"
    orc.close()
    dec.close()


def test_spin_limit_arguments(gpu):
    dec = N.Decoder(configs.TINY_DENSE)
    with pytest.raises(N.EtxmkError):
        dec.set_spin_limit(0, 3)                           # not a power of two
    with pytest.raises(N.EtxmkError):
        dec.set_spin_limit(0, 512)
    dec.set_spin_limit(0, 0)
    dec.close()
