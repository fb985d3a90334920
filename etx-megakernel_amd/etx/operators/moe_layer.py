"""One MoE transformer layer at decode time as an operator provider, with the gfx950 megakernel as its native body
(reference interface: etx/operators/moe_layer.py:31-185, `provider(small=...)` returning a record of the layer's
dimensions, its builder, a deterministic input generator, the routing, the runtime grouping arrays and the
bindings).

The reference's provider builds an IR graph of toy tiles (norm -> qkv -> attention over a KV cache -> o_proj ->
router -> grouping -> gather -> grouped expert GEMM -> down -> combine).  The native provider's layer is a Qwen3-MoE
decoder layer of this library (the same structure, with the model's real top-k softmax routing, renormalised, and
SiLU-gated experts) run through etxmk_step_layers: build() returns a MoELayer bound to one GPU, whose forward() maps
B residual rows to the layer's outputs, one single-layer step per row at its KV position.  Routing is a function of
the layer's weights and input; routing(x_rows) therefore runs the layer (it needs the GPU), and runtime() derives
the grouping arrays (expert counts, tiles of TPT tokens, CSR offsets, token slots, tile-to-expert) from any routing,
exactly as the reference's runtime() does from its own.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Callable

import numpy as np


@dataclass(frozen=True)
class MoEProvider:
    _SMALL: bool
    D: int        # hidden size
    H: int        # query heads
    HD: int       # head dim
    S: int        # KV context each row attends to (seeded cache)
    NE: int       # routed experts
    K: int        # experts per token
    FF: int       # expert intermediate size
    TPT: int      # tokens per grouped-GEMM tile (runtime grouping)
    T: str        # the persistent kernel symbol that runs the layer
    build: Callable
    lcg_x: Callable
    routing: Callable
    runtime: Callable
    bindings: Callable


class MoELayer:
    """A native MoE decoder layer on one GPU: seeded weights, a seeded KV cache of S positions (stream as the
    library's etxmk_fill_kv_seeded), forward() over residual rows."""

    def __init__(self, cfg, seed: int, context: int, device: str = "cuda:0"):
        from etx.runtime import native as N
        self.cfg, self.context = cfg, context
        self.dec = N.Decoder(cfg, device=device)
        self.dec.init_weights(seed, 0.02)
        self.dec.fill_kv_seeded(seed, context)
        self.dec.enable_dumps(True)

    def forward(self, x_rows):
        """Each row through the layer at position S (the cache holds S positions; every row sees the same cache):
        returns (outputs [B][D] fp32 holding bf16 values, top-k ids [B][K] in selection order, weights [B][K])."""
        x_rows = np.asarray(x_rows, np.float32)
        outs, ids, wts = [], [], []
        for row in x_rows:
            self.dec.set_residual(row)
            self.dec.step_layers(self.context, 0, 1)
            outs.append(self.dec.read_residual())
            d = self.dec.dumps()
            ids.append(d["ids"][0].copy())
            wts.append(d["w"][0].copy())
        return np.stack(outs), np.stack(ids), np.stack(wts)

    def close(self):
        self.dec.close()


def provider(*, small: bool = False) -> MoEProvider:
    """Dimensions bound per request: small is the tiny MoE decoder's layer, else a Qwen3-30B-A3B layer."""
    if type(small) is not bool:
        raise ValueError("small must be a boolean")
    from etx.models import configs
    base = configs.TINY_MOE if small else configs.QWEN3_30B_A3B
    S = 128 if small else 1024
    cfg = configs.with_layers(base, 1, max_ctx=S + 16)
    from etx.runtime import native as N
    T = N.plan_info(cfg)["kernel"]
    D, H, HD, NE, K, FF, TPT = cfg.H, cfg.NH, cfg.HD, cfg.E, cfg.TOPK, cfg.MI, 4

    def build(seed: int = 12345, device: str = "cuda:0") -> MoELayer:
        return MoELayer(cfg, seed, S, device)

    def lcg_x(B: int, seed: int = 12345) -> list:
        """B input rows of D bf16-exact values (integer / 128, |integer| <= 128) from a 32-bit linear congruential
        generator (multiplier 1664525, increment 1013904223): the reference's deterministic input rule."""
        state = seed & 0xFFFFFFFF
        rows = []
        for _ in range(B):
            row = []
            for _ in range(D):
                state = (state * 1664525 + 1013904223) & 0xFFFFFFFF
                row.append(((state >> 8) % 257 - 128) / 128.0)
            rows.append(row)
        return rows

    def routing(x_rows, layer: MoELayer | None = None) -> list:
        """The experts each row is routed to, stored ascending by expert id: the layer's own top-k (run on the GPU)."""
        own = layer is None
        lyr = build() if own else layer
        try:
            _, ids, _ = lyr.forward(x_rows)
        finally:
            if own:
                lyr.close()
        return [sorted(int(e) for e in r) for r in ids]

    def runtime(bindings: dict, topk: list | None = None) -> dict:
        """Grouping arrays of a routing (default: the routing of lcg_x(B, seed) through the layer): per-expert token
        counts, tiles of TPT tokens, CSR offsets of tokens and tiles, each (token, slot)'s row in the grouped order,
        and the expert of each tile."""
        B = bindings["B"]
        if topk is None:
            topk = routing(lcg_x(B, bindings.get("seed", 12345)))
        counts = [0] * NE
        for row in topk:
            for e in row:
                counts[e] += 1
        tiles = [-(-c // TPT) for c in counts]
        tok_indptr, indptr = [0], [0]
        for e in range(NE):
            tok_indptr.append(tok_indptr[-1] + counts[e])
            indptr.append(indptr[-1] + tiles[e])
        fill = [0] * NE
        tok_slot = []
        for row in topk:
            slots = []
            for e in row:
                slots.append(tok_indptr[e] + fill[e])
                fill[e] += 1
            tok_slot.append(slots)
        tile_expert = [[e] for e in range(NE) for _ in range(tiles[e])]
        return {"topk": topk, "expert_counts": counts, "expert_tiles": tiles, "tok_indptr": tok_indptr,
                "indptr": indptr, "tok_slot": tok_slot, "tile_expert": tile_expert}

    def bindings(topk: list | None = None, **overrides) -> dict:
        b = {"B": 8, "seed": 12345}
        b.update(overrides)
        b["n_gg"] = runtime(b, topk)["indptr"][-1]
        return b

    return MoEProvider(small, D, H, HD, S, NE, K, FF, TPT, T, build, lcg_x, routing, runtime, bindings)
