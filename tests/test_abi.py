"""The C ABI library: loads, exports every declared symbol, sizes and refuses shapes without a GPU."""
import ctypes as C

import numpy as np
import pytest

from etx.runtime import native as N
from etx.models import configs


def test_library_exports_every_declared_symbol():
    L = N.load()
    names = N.declared_functions()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing
    assert L.etxmk_abi_version() == N.ABI_VERSION == 3


def test_calibration_library_exports():
    from etx.runtime import calib
    lib = calib.load()                                     # loads without a GPU; nothing is launched
    assert hasattr(lib, "etxmk_calib_barrier") and hasattr(lib, "etxmk_calib_stream")
    assert hasattr(lib, "etxmk_calib_stream_tiles") and hasattr(lib, "etxmk_calib_mfma_bf16")


def test_sizes_of_real_configurations():
    s = N.sizes(configs.QWEN3_30B_A3B)
    c = configs.QWEN3_30B_A3B
    per_layer = ((c.NH + 2 * c.NKV) * c.HD * c.H + c.H * c.NH * c.HD + c.E * c.H + c.E * 3 * c.MI * c.H) * 2
    assert s["weights"] >= per_layer * c.L + 2 * c.V * c.H * 2
    assert s["weights"] < per_layer * c.L * 1.01 + 2 * c.V * c.H * 2 + 1e6
    assert s["kv"] == 2 * 2 * c.L * ((c.max_ctx + 15) // 16) * 16 * c.NKV * c.HD
    s8 = N.sizes(configs.QWEN3_8B)
    assert 15.0e9 < s8["weights"] < 16.5e9


@pytest.mark.parametrize("bad", [dict(HD=64), dict(H=3000), dict(batch=0), dict(batch=17), dict(block_size=48), dict(block_size=8), dict(block_size=32),
                                 dict(max_ctx=10**6), dict(TOPK=9), dict(E=0), dict(NKV=3), dict(prefill=17),
                                 dict(prefill=-1)])
def test_config_refused(bad):
    d = configs.TINY_MOE.as_dict()
    d.update(bad)
    cfg = N.ModelConfig(**d)
    with pytest.raises(N.EtxmkError) as e:
        N.sizes(cfg)
    assert e.value.code == N.EINVAL


def test_batch_needs_a_batched_kernel():
    # Qwen3-8B's dense down projection (12288 long) has a batch-4 kernel only: beyond it refused, not run wrongly
    N.sizes(configs.with_layers(configs.QWEN3_8B, 36, batch=4))
    for kw in (dict(batch=5), dict(prefill=16)):
        with pytest.raises(N.EtxmkError) as e:
            N.sizes(configs.with_layers(configs.QWEN3_8B, 36, **kw))
        assert e.value.code == N.EINVAL and "batched" in str(e.value), kw


def test_prefill_rows_size_the_activations_only():
    one = N.sizes(configs.QWEN3_30B_A3B)
    pf = N.sizes(configs.with_layers(configs.QWEN3_30B_A3B, 48, prefill=16))
    b16 = N.sizes(configs.with_layers(configs.QWEN3_30B_A3B, 48, batch=16))
    assert pf["weights"] == one["weights"] and pf["kv"] == one["kv"]     # one sequence's cache
    assert one["workspace"] < pf["workspace"] < b16["workspace"]         # 16 activation rows, one token row


def test_batch_sizes_scale_per_sequence():
    one, four = N.sizes(configs.QWEN3_30B_A3B), N.sizes(configs.with_layers(configs.QWEN3_30B_A3B, 48, batch=4))
    assert four["weights"] == one["weights"]              # weights are shared by the sequences
    assert four["kv"] == 4 * one["kv"]                    # one block pool, max_ctx positions per sequence
    assert four["workspace"] > one["workspace"]


def test_unpermute_inverts_the_lane_permutation():
    for K in (256, 768, 2048):
        rng = np.random.default_rng(K)
        nat = rng.integers(0, 2 ** 16, (3, K), dtype=np.uint16)
        stored = np.empty_like(nat)
        for base in range(0, K, 512):
            S = min(512, K - base)
            m = S // 64
            for p in range(S):
                lane, e = divmod(p, m)
                stored[:, base + p] = nat[:, base + lane + 64 * e]
        assert np.array_equal(N.unpermute_rows(stored), nat)


def test_fp8_weights_shrink_the_arena():
    bf, f8 = configs.QWEN3_30B_A3B, configs.with_layers(configs.QWEN3_30B_A3B, 48, wdtype=N.W_FP8)
    c = bf
    sb, s8 = N.sizes(bf)["weights"], N.sizes(f8)["weights"]
    fp8_elems = c.L * ((c.NH + 2 * c.NKV) * c.HD * c.H + c.H * c.NH * c.HD + c.E * 3 * c.MI * c.H)
    fp8_rows = c.L * ((c.NH + 2 * c.NKV) * c.HD + c.H + c.E * (2 * c.MI + c.H))
    # every fp8 element saves one byte; every fp8 row gains its 16-byte scale slot (up to 256-byte padding per tensor)
    assert abs((sb - s8) - (fp8_elems - 16 * fp8_rows)) < 256 * 8 * c.L


@pytest.mark.parametrize("bad", [dict(wdtype=2), dict(wdtype=-1)])
def test_unknown_weight_type_refused(bad):
    with pytest.raises(N.EtxmkError) as e:
        N.sizes(N.ModelConfig(**dict(configs.TINY_MOE.as_dict(), **bad)))
    assert e.value.code == N.EINVAL


def test_fp8_needs_a_persistent_kernel():
    # Qwen3-8B's dense rows (12288) have no fp8 kernel: refused, not run wrongly
    with pytest.raises(N.EtxmkError) as e:
        N.sizes(configs.with_layers(configs.QWEN3_8B, 36, wdtype=N.W_FP8))
    assert e.value.code == N.EINVAL and "fp8" in str(e.value)


def test_deepseek_v2_lite_sizes():
    """Weights: every DeepSeek-V2-Lite tensor once (the dense layer's down rows padded to 11264), bf16."""
    c = configs.DEEPSEEK_V2_LITE
    SI, IP, NQA = c.n_shared * c.MI, (c.dense_I + 511) // 512 * 512, c.nqkv
    attn = NQA * c.H + c.NH * (c.qk_nope + c.v_head) * c.kv_lora + c.H * c.NH * c.v_head + c.kv_lora + 2 * c.H
    dense = 2 * c.dense_I * c.H + c.H * IP
    moe = c.E * c.H + c.E * 3 * c.MI * c.H + 3 * SI * c.H
    elems = c.L * attn + c.first_dense * dense + (c.L - c.first_dense) * moe + 2 * c.V * c.H + c.H
    s = N.sizes(c)
    assert elems * 2 <= s["weights"] < elems * 2 + 256 * 20 * c.L
    assert 31.0e9 < s["weights"] < 31.6e9                  # 15.7B parameters
    assert s["kv"] == 2 * c.L * ((c.max_ctx + 15) // 16) * 16 * (c.kv_lora + c.qk_rope)   # one latent pool


@pytest.mark.parametrize("bad", [dict(wdtype=1), dict(batch=5), dict(kv_lora=256), dict(block_size=8),
                                 dict(HD=128), dict(NH=12), dict(MI=1024), dict(prefill=5)])
def test_deepseek_config_refused(bad):
    d = configs.DEEPSEEK_V2_LITE.as_dict()
    d.update(bad)
    with pytest.raises(N.EtxmkError) as e:
        N.sizes(N.ModelConfig(**d))
    assert e.value.code == N.EINVAL
