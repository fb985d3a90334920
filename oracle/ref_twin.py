"""NumPy restatement of examples/llm/ref_numpy.py (TEST INFRASTRUCTURE ONLY).

A second, independent CPU statement of the decode step: numpy's own evaluation order (`@`, np.mean,
.sum(), np.exp) exactly as the reference writes it, with bf16 rounding at the reference's points.  It
pins the C oracle (which fixes one canonical fp32 order) to the reference's formulas within the
reference's own per-layer gate (ref_numpy.py:207-212: max rel < 2e-2) at small sizes.

Every function cites the line of ref_numpy.py it restates; the weights come from the oracle's seeded
generator in natural layout.
"""
from __future__ import annotations

import numpy as np

from oracle import oracle as O


def bfr(x):                                               # ref_numpy.py:26-32
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = x.view(np.uint32)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) & 0xFFFF0000).astype(np.uint32)
    return r.view(np.float32)


def rmsnorm(x, w, eps):                                   # ref_numpy.py:71-73
    r = np.float32(1.0) / np.sqrt(np.float32(np.mean(x.astype(np.float32) ** 2)) + np.float32(eps))
    return bfr(w * bfr(x * r))


def rope_tables(theta, hd, ctx):                          # ref_numpy.py:76-81
    inv = (1.0 / (np.float32(theta) ** (np.arange(0, hd, 2, dtype=np.float32) / np.float32(hd)))).astype(np.float32)
    pos = np.arange(ctx, dtype=np.float32)[:, None]
    f = pos * inv[None, :]
    return bfr(np.cos(f)), bfr(np.sin(f))


def apply_rope(v, cos, sin):                              # ref_numpy.py:84-88
    half = v.shape[-1] // 2
    rot = np.concatenate([-v[half:], v[:half]])
    c = np.concatenate([cos, cos]); s = np.concatenate([sin, sin])
    return bfr(bfr(v * c) + bfr(rot * s))


def silu(g):                                              # ref_numpy.py:91-92
    return g / (np.float32(1.0) + np.exp(-g))


class Twin:
    """Ref (ref_numpy.py:95-158) over the oracle model's seeded weights; norm weights are 1.0."""

    def __init__(self, model: "O.OracleModel", ctx: int):
        c = self.c = model.cfg
        self.m = model
        f = lambda b: O.bf16_bits_to_f32(b)
        self.embed = f(model.weight(O.S_EMBED))
        self.lm = f(model.weight(O.S_LMHEAD))
        self.layers = []
        for l in range(c["L"]):
            d = dict(wqkv=f(model.weight(O.S_WQKV, l)), wo=f(model.weight(O.S_WO, l)))
            if c["moe"]:
                d["wr"] = f(model.weight(O.S_ROUTER, l))
            else:
                d["wgu"] = f(model.weight(O.S_WGU, l)); d["wd"] = f(model.weight(O.S_WD, l))
            self.layers.append(d)
        self.cos, self.sin = rope_tables(c["theta"], c["HD"], ctx)
        self.kc = np.zeros((c["L"], ctx, c["NKV"], c["HD"]), np.float32)
        self.vc = np.zeros((c["L"], ctx, c["NKV"], c["HD"]), np.float32)
        self.ones_h = np.ones(c["H"], np.float32)
        self.ones_hd = np.ones(c["HD"], np.float32)

    def expert(self, l, e):
        f = lambda b: O.bf16_bits_to_f32(b)
        return f(self.m.weight(O.S_W13, l, e)), f(self.m.weight(O.S_W2, l, e))

    def step(self, tok: int, pos: int, dump=None) -> int:   # ref_numpy.py:105-158
        c = self.c
        NH, NKV, HD = c["NH"], c["NKV"], c["HD"]
        G = NH // NKV
        x = self.embed[tok].copy()
        for L in range(c["L"]):
            Ly = self.layers[L]
            xs = rmsnorm(x, self.ones_h, c["eps"])
            qkv = bfr(Ly["wqkv"] @ xs)
            q = qkv[:NH * HD].reshape(NH, HD); k = qkv[NH * HD:(NH + NKV) * HD].reshape(NKV, HD)
            v = qkv[(NH + NKV) * HD:].reshape(NKV, HD)
            if c["qk_norm"]:
                q = np.stack([rmsnorm(h, self.ones_hd, c["eps"]) for h in q])
                k = np.stack([rmsnorm(h, self.ones_hd, c["eps"]) for h in k])
            q = np.stack([apply_rope(h, self.cos[pos], self.sin[pos]) for h in q])
            k = np.stack([apply_rope(h, self.cos[pos], self.sin[pos]) for h in k])
            self.kc[L, pos] = k; self.vc[L, pos] = v
            scale = np.float32(1.0 / np.sqrt(HD))
            o = np.zeros((NH, HD), np.float32)
            for h in range(NH):
                kvh = h // G
                K = self.kc[L, :pos + 1, kvh]; V = self.vc[L, :pos + 1, kvh]
                s = (K @ q[h]) * scale
                s = s - s.max(); pr = np.exp(s); pr = pr / pr.sum()
                o[h] = bfr(pr @ V)
            x = bfr(x + bfr(Ly["wo"] @ o.reshape(-1)))
            xs = rmsnorm(x, self.ones_h, c["eps"])
            ids = wts = None
            if c["moe"]:
                E, TOPK = c["E"], c["TOPK"]
                logits = bfr(Ly["wr"] @ xs)
                pr = np.exp(logits - logits.max()); pr = pr / pr.sum()
                order = np.lexsort((np.arange(E), -pr))[:TOPK]
                wts = pr[order]
                if c["norm_topk"]:
                    wts = wts / wts.sum()
                wts = bfr(wts)
                ids = order
                acc = np.float32(0.0)
                for e, we in sorted(zip(order.tolist(), wts.tolist())):
                    w13, w2 = self.expert(L, e)
                    g = bfr(w13[0::2] @ xs); u = bfr(w13[1::2] @ xs)     # gate/up rows interleaved
                    hh = bfr(bfr(silu(g)) * u)
                    y = bfr(bfr(w2 @ hh) * np.float32(we))
                    acc = bfr(acc + y)
                x = bfr(x + acc)
            else:
                g = bfr(Ly["wgu"][0::2] @ xs); u = bfr(Ly["wgu"][1::2] @ xs)
                hh = bfr(bfr(silu(g)) * u)
                x = bfr(x + bfr(Ly["wd"] @ hh))
            if dump is not None:
                dump.append((x.copy(), None if ids is None else np.array(ids), None if wts is None else np.array(wts)))
        xs = rmsnorm(x, self.ones_h, c["eps"])
        logits = bfr(self.lm @ xs)
        return int(np.argmax(logits))
