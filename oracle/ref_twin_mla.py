"""NumPy restatement of the reference's DeepSeek-V2 MLA decode (TEST INFRASTRUCTURE ONLY).

A second, independent CPU statement of one DeepSeek-V2 decoder step, in numpy's own evaluation order with bf16
rounding where the reference rounds: examples/dsv2lite/results/2026-10-14-k1/b_alld4r0l1kvs_stamps/fleet_src/host/
reference_decode.py (a snapshot the reference keeps of its MLA host's numerical specification).  Unlike that file
and the C oracle, the attention here is written in the non-absorbed form (per-head keys and values materialised
from kv_b_proj), so agreement also pins the absorption algebra.  It pins the C oracle (one fixed fp32 order) to the
reference's formulas within the per-layer gate of 2e-2 at small sizes.

Every function cites the line of reference_decode.py it restates; the weights come from the oracle's seeded
generator in natural layout; norm weights are 1.0.
"""
from __future__ import annotations

import math

import numpy as np

from oracle import oracle as O
from oracle.ref_twin import bfr


def rms_norm(x, eps):                                     # :51-65 (bf16: two roundings, weight 1.0)
    x32 = x.astype(np.float32)
    var = np.mean(x32 * x32, axis=-1, keepdims=True)
    y = bfr(x32 * (np.float32(1.0) / np.sqrt(var + np.float32(eps))))
    return bfr(y * np.float32(1.0))


def silu(x):                                              # :68-69
    return x / (np.float32(1.0) + np.exp(-x, dtype=np.float32))


def softmax(x):                                           # :72-75
    m = np.max(x, axis=-1, keepdims=True)
    e = np.exp(x - m)
    return e / np.sum(e, axis=-1, keepdims=True)


def yarn_mscale(scale, mscale):                           # :78-82
    return 1.0 if scale <= 1 else 0.1 * mscale * math.log(scale) + 1.0


def yarn_cos_sin(c, seq_len):                             # :85-117
    dim, base, scale = c["qk_rope"], float(c["theta"]), float(c["rope_factor"])

    def corr(n_rot):
        return (dim * math.log(c["rope_orig_max"] / (n_rot * 2 * math.pi))) / (2 * math.log(base))

    low = max(math.floor(corr(c["beta_fast"])), 0)
    high = min(math.ceil(corr(c["beta_slow"])), dim - 1)
    if low == high:
        high += 0.001
    ramp = np.clip((np.arange(dim // 2, dtype=np.float32) - low) / (high - low), 0, 1)
    mask = 1.0 - ramp
    ex = np.arange(0, dim, 2, dtype=np.float32) / dim
    extra = 1.0 / (base ** ex)
    inter = 1.0 / (scale * base ** ex)
    inv = inter * (1 - mask) + extra * mask
    freqs = np.outer(np.arange(seq_len, dtype=np.float32), inv)
    emb = np.concatenate([freqs, freqs], axis=-1)
    ms = yarn_mscale(scale, c["rope_mscale"]) / yarn_mscale(scale, c["rope_mscale_all"])
    return (np.cos(emb) * ms).astype(np.float32), (np.sin(emb) * ms).astype(np.float32)


def apply_rope(x, cos, sin):                              # :120-136 (interleave, then rotate_half)
    d = x.shape[-1]
    x = x.reshape(*x.shape[:-1], d // 2, 2).swapaxes(-1, -2).reshape(*x.shape[:-1], d)
    rot = np.concatenate([-x[..., d // 2:], x[..., :d // 2]], axis=-1)
    return x * cos + rot * sin


class TwinMLA:
    """decoder_layer (:294-302) over the oracle model's seeded weights, with a float32 latent cache per sequence."""

    def __init__(self, model: "O.OracleModel", ctx: int):
        c = self.c = model.cfg
        f = O.bf16_bits_to_f32
        self.m = model
        self.embed = f(model.weight(O.S_EMBED))
        self.lm = f(model.weight(O.S_LMHEAD))
        self.cos, self.sin = yarn_cos_sin(c, ctx)
        qd = c["qk_nope"] + c["qk_rope"]
        m = yarn_mscale(c["rope_factor"], c["rope_mscale_all"])
        self.scale = qd ** -0.5 * m * m                   # :198-206
        self.layers = []
        for l in range(c["L"]):
            d = dict(wqa=f(model.weight(O.S_WQKV, l)), wo=f(model.weight(O.S_WO, l)),
                     wkvb=f(model.weight(O.S_WKVB, l)))
            if l < c["first_dense"]:
                d.update(wgu=f(model.weight(O.S_WGU, l)), wd=f(model.weight(O.S_WD, l)))
            else:
                d.update(wr=f(model.weight(O.S_ROUTER, l)), wsgu=f(model.weight(O.S_WSGU, l)),
                         wsd=f(model.weight(O.S_WSD, l)), experts={})
            self.layers.append(d)
        self.cache = [np.zeros((ctx, c["kv_lora"] + c["qk_rope"]), np.float32) for _ in range(c["L"])]

    def expert(self, l, e):
        d = self.layers[l]["experts"]
        if e not in d:
            f = O.bf16_bits_to_f32
            d[e] = (f(self.m.weight(O.S_W13, l, e)), f(self.m.weight(O.S_W2, l, e)))
        return d[e]

    def mlp_unit(self, gu, down, x_n):                    # :259-265 (gate/up rows interleaved)
        g, u = gu[0::2], gu[1::2]
        h = bfr(bfr(silu(bfr(g @ x_n))) * bfr(u @ x_n))
        return bfr(down @ h)

    def attention(self, l, x, pos):                       # :210-256 in non-absorbed form
        c, w = self.c, self.layers[l]
        NH, Dk, Dr, Dv, Lr = c["NH"], c["qk_nope"], c["qk_rope"], c["v_head"], c["kv_lora"]
        x_n = rms_norm(x, c["eps"])
        qa = bfr(w["wqa"] @ x_n)
        q = qa[:NH * (Dk + Dr)].reshape(NH, Dk + Dr)
        q_nope, q_pe = q[:, :Dk], q[:, Dk:]
        kv_a = qa[NH * (Dk + Dr):]
        c_new = rms_norm(kv_a[:Lr], c["eps"])
        k_pe_new = bfr(apply_rope(kv_a[Lr:][None, :], self.cos[pos][None, :], self.sin[pos][None, :])[0])
        q_pe = bfr(apply_rope(q_pe, self.cos[pos][None, :], self.sin[pos][None, :]))
        cache = self.cache[l]
        cache[pos, :Lr], cache[pos, Lr:] = c_new, k_pe_new
        cl, kpe = cache[:pos + 1, :Lr], cache[:pos + 1, Lr:]
        out = np.empty(NH * Dv, np.float32)
        for h in range(NH):
            base = h * (Dk + Dv)
            w_uk, w_uv = w["wkvb"][base:base + Dk], w["wkvb"][base + Dk:base + Dk + Dv]
            k_nope = cl @ w_uk.T                          # [S, Dk]: the keys the absorbed form never builds
            v = cl @ w_uv.T                               # [S, Dv]
            s = (k_nope @ q_nope[h] + kpe @ q_pe[h]) * np.float32(self.scale)
            out[h * Dv:(h + 1) * Dv] = softmax(s) @ v
        return bfr(w["wo"] @ bfr(out))

    def moe(self, l, x_n):                                # :268-287
        c, w = self.c, self.layers[l]
        scores = softmax(w["wr"] @ x_n)
        idx = np.argsort(-scores, kind="stable")[:c["TOPK"]]
        wts = scores[idx]
        wts = wts / (wts.sum() + 1e-20) if c["norm_topk"] else wts * np.float32(c["routed_scale"])
        y = np.zeros_like(x_n)
        for k, e in enumerate(idx):
            gu, down = self.expert(l, int(e))
            y += bfr(wts[k] * self.mlp_unit(gu, down, x_n))
        shared = self.mlp_unit(w["wsgu"], w["wsd"], x_n)
        return bfr(bfr(y) + shared), idx

    def step(self, tok: int, pos: int):
        """(greedy token, per-layer residuals [L][H], top-k ids per MoE layer)"""
        c = self.c
        x = self.embed[tok].astype(np.float32)
        xs, ids = [], []
        for l in range(c["L"]):                           # :294-302
            x = bfr(x + self.attention(l, x, pos))
            x_n2 = rms_norm(x, c["eps"])
            if l < c["first_dense"]:
                w = self.layers[l]
                x = bfr(x + self.mlp_unit(w["wgu"], w["wd"], x_n2))
                ids.append(None)
            else:
                y, idx = self.moe(l, x_n2)
                x = bfr(x + y)
                ids.append(np.sort(idx))
            xs.append(x.copy())
        logits = bfr(self.lm @ rms_norm(x, c["eps"]))
        return int(np.argmax(logits)), np.stack(xs), ids
