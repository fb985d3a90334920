"""GPU parity of fp8 e4m3 weights with per-row scales: the quantised tensors bit for bit,
single-sequence and batched decode bit for bit against the oracle's fp8 arithmetic, and the north star's fp8 gate
(per-layer max rel 5e-2) against the dequantised-bf16 reference (the oracle's wdtype 2)."""
import numpy as np
import pytest

from oracle import oracle as O
from etx.runtime import native as N
from etx.models import configs
from test_gpu_batch import SEED, run_contexts, say, rel

pytestmark = pytest.mark.gpu


def fp8(cfg, L=None, **kw):
    return configs.with_layers(cfg, cfg.L if L is None else L, wdtype=N.W_FP8, **kw)


@pytest.mark.parametrize("base", [configs.TINY_MOE, configs.TINY_DENSE], ids=["moe", "dense"])
def test_fp8_weights_bit_exact(gpu, base):
    """Seeded quantisation on the device equals the oracle's quantize_rows, codes and scales; load_tensor of natural
    bf16 rows quantises the same way."""
    cfg = fp8(base)
    say(f"[gpu] fp8 weights {cfg.name}")
    dec = N.Decoder(cfg)
    dec.init_weights(SEED, 0.02)
    orc = O.OracleModel(cfg.as_dict(), SEED, 0.02)
    specs = [(N.T_WQKV, l) for l in range(cfg.L)] + [(N.T_WO, l) for l in range(cfg.L)]
    if cfg.moe:
        specs += [(k, l, e) for l in range(cfg.L) for e in (0, 3, cfg.E - 1) for k in (N.T_W13, N.T_W2)]
    else:
        specs += [(k, l) for l in range(cfg.L) for k in (N.T_WGU, N.T_WD)]
    for spec in specs:
        q, sc = dec.tensor_fp8(*spec)
        qo, so = orc.weight_fp8(*spec)
        assert np.array_equal(sc, so), f"{spec}: scales differ"
        assert np.array_equal(q, qo), f"{spec}: {np.sum(q != qo)} codes differ"
    assert dec.tensor_format(N.T_ROUTER if cfg.moe else N.T_EMBED, 0)[0] == N.W_BF16
    # load_tensor: natural bf16 rows in, the same quantisation
    import torch
    bf = O.OracleModel(base.as_dict(), SEED, 0.02)
    w = bf.weight(O.S_WQKV, 1)
    src = torch.from_numpy(w.view(np.int16).copy()).to(dec.device)
    dec.load_tensor(N.T_WQKV, 1, 0, src)
    dec.sync()
    q, sc = dec.tensor_fp8(N.T_WQKV, 1)
    qo, so = orc.weight_fp8(O.S_WQKV, 1)
    assert np.array_equal(q, qo) and np.array_equal(sc, so)
    for m in (orc, bf):
        m.close()
    dec.close()


@pytest.mark.parametrize("base,B", [(configs.TINY_MOE, 1), (configs.TINY_DENSE, 1), (configs.TINY_MOE, 4),
                                    (configs.TINY_MOE, 16), (configs.TINY_DENSE, 4)],
                         ids=["moe-b1", "dense-b1", "moe-b4", "moe-b16", "dense-b4"])
def test_fp8_decode_bit_exact(gpu, base, B):
    cfg = fp8(base, batch=B)
    ctx = np.random.default_rng(200 + B).integers(1, 200, B)
    run_contexts(cfg, ctx, n_steps=5, shuffle=B > 1)


def test_fp8_gate_against_dequantised_reference(gpu):
    """The north star's fp8 gate: per-layer residuals within max rel 5e-2 of the reference that dequantises the same
    codes into bf16 weights, fed the same tokens."""
    cfg = fp8(configs.TINY_MOE, batch=4)
    say(f"[gpu] fp8 gate {cfg.name}")
    dec = N.Decoder(cfg)
    dec.init_weights(SEED, 0.02)
    ref = O.OracleModel(dict(cfg.as_dict(), wdtype=O.W_FP8_DEQ), SEED, 0.02)
    ctx = [40, 120, 7, 199]
    first = O.gen_tokens(SEED + 1, 4, cfg.V)
    for b in range(4):
        dec.fill_kv_seeded(SEED, ctx[b], seq=b)
        ref.fill_kv_random(ctx[b], seq=b)
        row = np.zeros(ctx[b] + 1, np.int32)
        row[-1] = first[b]
        dec.set_tokens(row, seq=b)
    dec.enable_dumps(True)
    pos = np.array(ctx, np.int32)
    toks = [int(t) for t in first]
    worst = 0.0
    for s in range(4):
        dec.step_batch(pos, write_next=True)
        d = dec.dumps()
        out = [dec.read_tokens(int(pos[b]) + 1, seq=b)[int(pos[b])] for b in range(4)]
        for b in range(4):
            _, xo, _, _ = ref.step(toks[b], int(pos[b]), dump=True, seq=b)
            for L in range(cfg.L):
                worst = max(worst, rel(d["x"][L][b], xo[L]))
        toks = out
        pos += 1
    say(f"[gpu]   worst per-layer max rel vs dequantised reference {worst:.3e}")
    assert worst < 5e-2
    ref.close()
    dec.close()


@pytest.mark.parametrize("B", [1, 16], ids=["b1", "b16"])
def test_qwen3_30b_a3b_fp8_two_layers(gpu, B):
    cfg = fp8(configs.QWEN3_30B_A3B, L=2, batch=B)
    ctx = np.random.default_rng(300 + B).integers(512, 1080, B)
    run_contexts(cfg, ctx, n_steps=3, pool=B == 1)


@pytest.mark.timeout(1100)
def test_qwen3_30b_a3b_fp8_b16_full_greedy_32(gpu):
    """BASELINE.json configs[4] at full depth: 48 layers, fp8 weights, batch 16, per-sequence contexts uniform in
    [512, 4096], 32 greedy steps of every sequence identical to the oracle; first and last step's per-layer
    residuals and routing bit for bit."""
    ctx = np.random.default_rng(5).integers(512, 4097, 16)
    cfg = fp8(configs.QWEN3_30B_A3B, batch=16, max_ctx=int(ctx.max()) + 40)
    run_contexts(cfg, ctx, n_steps=32, check_every=31, pool=False)
