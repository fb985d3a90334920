"""The unfused step (one launch per phase, parameters by value, no memory set or copied) recorded in a HIP graph
and replayed: every replay gives the eager step's next token, final residual and KV slot bit for bit, with eager
steps of the same handle run between the replays (a replay of position P reads positions 0..P only, so a step at
P + 1 between two replays leaves what it reads unchanged)."""
import numpy as np
import pytest

from oracle import oracle as O
from etx.runtime import native as N
from etx.models import configs
from progress_log import say

pytestmark = pytest.mark.gpu

SEED = 20261204


@pytest.mark.parametrize("base", [configs.TINY_MOE, configs.TINY_DENSE], ids=["moe", "dense"])
def test_unfused_step_graph_replays(gpu, base):
    import torch
    cfg = base
    say(f"[gpu] graph replay of the unfused {cfg.name} step")
    P = 37
    prompt = O.gen_tokens(SEED, P, cfg.V)
    dec = N.Decoder(cfg, fused=False)
    dec.init_weights(SEED, 0.02)
    dec.set_tokens(prompt)
    for pos in range(P - 1):
        dec.step(pos, write_next=False)
    dec.step(P - 1, write_next=True)                       # the token at P
    dec.sync()
    dec.step(P, write_next=True)                           # eager reference: the step at P ...
    dec.sync()
    want_tok = dec.read_tokens(P + 1)[P]                   # out_tokens[q]: the greedy output of step q
    want_x = dec.read_residual()
    dec.step(P + 1, write_next=True)                       # ... and the step at P + 1 after it
    dec.sync()
    want_tok2 = dec.read_tokens(P + 2)[P + 1]
    want_kv = [dec.kv_layer(L) for L in range(cfg.L)]
    # the residual tells a replay from no work at all: after the step at P + 1 it is that step's
    assert not np.array_equal(dec.read_residual(), want_x)

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        dec.step(P, write_next=True)
    torch.cuda.synchronize()
    for r in range(4):
        graph.replay()
        torch.cuda.synchronize()
        assert dec.read_tokens(P + 1)[P] == want_tok, f"replay {r}: next token differs"
        assert np.array_equal(dec.read_residual(), want_x), f"replay {r}: final residual differs"
        dec.step(P + 1, write_next=True)                   # eager work between replays
        dec.sync()
        assert dec.read_tokens(P + 2)[P + 1] == want_tok2, f"eager step after replay {r}: token differs"
    for L in range(cfg.L):
        for g, w in zip(dec.kv_layer(L), want_kv[L]):
            assert np.array_equal(g, w), f"layer {L}: KV after the replays differs"
    del graph
    dec.close()
