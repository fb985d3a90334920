"""Decoder configurations of the decode path.

The real shapes are those of examples/llm/configs/{qwen3-8b,qwen3-30b-a3b}.json in the reference, read
through the same rules as examples/llm/model.py:95-140 (load_dims); the tiny ones exist so the CPU oracle
can check every phase in seconds.
"""
from __future__ import annotations

import json
from pathlib import Path

from etx.runtime.native import ARCH_DSV2, ModelConfig

QWEN3_8B = ModelConfig(name="qwen3-8b", H=4096, NH=32, NKV=8, HD=128, L=36, V=151936, I=12288,
                       moe=0, qk_norm=1, eps=1e-6, theta=1e6, max_ctx=1088)
QWEN3_30B_A3B = ModelConfig(name="qwen3-30b-a3b", H=2048, NH=32, NKV=4, HD=128, L=48, V=151936,
                            E=128, TOPK=8, MI=768, moe=1, qk_norm=1, norm_topk=1, eps=1e-6, theta=1e6, max_ctx=1088)
# one Qwen3-8B layer (the single-layer configuration; the vocabulary is irrelevant there)
QWEN3_8B_LAYER = ModelConfig(name="qwen3-8b-layer", H=4096, NH=32, NKV=8, HD=128, L=1, V=1024, I=12288,
                             moe=0, qk_norm=1, eps=1e-6, theta=1e6, max_ctx=1088)
TINY_MOE = ModelConfig(name="tiny-moe", H=512, NH=4, NKV=2, HD=128, L=2, V=4096, E=16, TOPK=4, MI=256,
                       moe=1, qk_norm=1, norm_topk=1, max_ctx=256)
TINY_DENSE = ModelConfig(name="tiny-dense", H=512, NH=4, NKV=2, HD=128, L=2, V=4096, I=1024,
                         moe=0, qk_norm=1, max_ctx=256)

# DeepSeek-V2-Lite (the shapes of its HF config, which the reference's MLA host uses):
# MLA with kv_lora 512, qk_nope 128, qk_rope 64, v_head 128 and no q LoRA; layer 0 dense (10944), then 64 routed
# experts top-6 (softmax, not renormalised, scaling 1.0) plus 2 shared, each 1408 wide; yarn RoPE factor 40 over
# 4096 positions (beta 32 / 1, mscale 0.707 for both).  HD is the query head dim (qk_nope + qk_rope).
DEEPSEEK_V2_LITE = ModelConfig(name="deepseek-v2-lite", H=2048, NH=16, NKV=1, HD=192, L=27, V=102400, E=64, TOPK=6,
                               MI=1408, moe=1, qk_norm=0, norm_topk=0, eps=1e-6, theta=1e4, max_ctx=2112,
                               arch=ARCH_DSV2, kv_lora=512, qk_nope=128, qk_rope=64, v_head=128, n_shared=2,
                               first_dense=1, dense_I=10944, routed_scale=1.0, rope_factor=40.0, rope_mscale=0.707,
                               rope_mscale_all=0.707, beta_fast=32.0, beta_slow=1.0, rope_orig_max=4096)
# a tiny MLA decoder for the oracle checks: the real head dims, fewer heads and experts, a 960-wide dense layer 0
# (its rows are padded to 1024 on the device)
TINY_MLA = ModelConfig(name="tiny-mla", H=512, NH=4, NKV=1, HD=192, L=3, V=4096, E=16, TOPK=6, MI=256, moe=1,
                       qk_norm=0, norm_topk=0, eps=1e-6, theta=1e4, max_ctx=256, arch=ARCH_DSV2, kv_lora=512,
                       qk_nope=128, qk_rope=64, v_head=128, n_shared=2, first_dense=1, dense_I=960, routed_scale=1.0,
                       rope_factor=40.0, rope_mscale=0.707, rope_mscale_all=0.707, beta_fast=32.0, beta_slow=1.0,
                       rope_orig_max=4096)

CONFIGS = {c.name: c for c in (QWEN3_8B, QWEN3_30B_A3B, QWEN3_8B_LAYER, TINY_MOE, TINY_DENSE, DEEPSEEK_V2_LITE,
                               TINY_MLA)}


def with_layers(cfg: ModelConfig, L: int, **kw) -> ModelConfig:
    d = cfg.as_dict()
    d.update(L=L, **kw)
    return ModelConfig(name=f"{cfg.name}-L{L}", **d)


def from_hf_config(path: str | Path, max_ctx: int = 1088, layers: int = 0) -> ModelConfig:
    """Dimensions from a Hugging Face config.json (the subset examples/llm/model.py:95-140 accepts for
    Qwen3 dense and Qwen3-MoE); anything else is refused rather than guessed."""
    c = json.loads(Path(path).read_text())
    mt = c.get("model_type", "")
    if not mt.startswith("qwen3"):
        raise ValueError(f"{path}: model_type {mt!r} is not a Qwen3 dense/MoE decoder")
    E = int(c.get("num_experts", 0) or 0)
    if E and (c.get("mlp_only_layers") or c.get("decoder_sparse_step", 1) != 1):
        raise ValueError("mixed dense / MoE layer layouts are not supported")
    if c.get("tie_word_embeddings"):
        raise ValueError("tied embeddings are not supported by this path")
    H, NH = c["hidden_size"], c["num_attention_heads"]
    return ModelConfig(name=Path(path).stem, H=H, NH=NH, NKV=c.get("num_key_value_heads", NH), HD=c.get("head_dim", H // NH),
                       L=min(layers or c["num_hidden_layers"], c["num_hidden_layers"]), V=c["vocab_size"],
                       I=0 if E else c["intermediate_size"], E=E, TOPK=int(c.get("num_experts_per_tok", 0)) if E else 0,
                       MI=int(c.get("moe_intermediate_size", 0)) if E else 0, moe=int(E > 0), qk_norm=1,
                       norm_topk=int(bool(c.get("norm_topk_prob", True))), eps=float(c.get("rms_norm_eps", 1e-6)),
                       theta=float(c.get("rope_theta", 1e6)), max_ctx=max_ctx)
