"""The reference's packed checkpoint: weights.bin + llm.manifest (+ golden*.txt), read and written here.

Format (written by etx/models/llm/prep.py:88-146 and :243-258, read by examples/llm/host.hip:70-121):

  llm.manifest   text, one record per line:
                   "cfg <key> <value>"  H NH NKV HD INTER L V E TOPK MI CTX CHUNK qk_norm bias moe norm_topk tie eps
                                        theta active_bytes layout (and per-XCD rpt_* entries, ignored here)
                   "t <name> <byte offset> <element count>"
  weights.bin    the tensors as bf16, each starting on a 256-byte boundary (zero bytes between)
  golden*.txt    "prompt: <ids>", "gen: <ids>", "margin: <floats>" (HF greedy decode of the checkpoint)

Tensor names: embed [V][H], final_norm [H], lm_head [V][H] (absent when tie), and per layer L<l>.:
ln1, ln2 [H]; wqkv [(NH+2NKV)*HD][H] (q, k, v rows); bqkv (bias, optional); qn, kn [HD] (optional); wo [H][NH*HD];
MoE: wr [E][H], egu [E][2*MI][H] (gate and up rows interleaved), ed [E][H][MI]; dense: wgu [2*I][H] (interleaved),
wd [H][I].  Layout 2 is the interleaved one; the reference host refuses layout 1 (host.hip:71), and so does this reader.

The library takes each tensor in natural row-major order and lays it out itself (etxmk_load_tensor), so loading is a
copy per tensor (per expert for the expert stacks) from the memory-mapped file.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

from etx.runtime import native as N
from etx.runtime.native import ModelConfig

ALIGN = 256                                  # prep.py:100-102
LAYOUT = 2


@dataclass
class Manifest:
    cfg: dict = field(default_factory=dict)          # key -> value text
    tensors: dict = field(default_factory=dict)      # name -> (byte offset, element count)

    def geti(self, key: str) -> int:
        if key not in self.cfg:
            raise ValueError(f"manifest lacks cfg {key}")
        return int(float(self.cfg[key]))

    def getf(self, key: str) -> float:
        if key not in self.cfg:
            raise ValueError(f"manifest lacks cfg {key}")
        return float(self.cfg[key])


def read_manifest(path: str | Path) -> Manifest:
    """Parse and check llm.manifest: layout 2, every tensor 256-byte aligned, no two tensors overlapping."""
    m = Manifest()
    for n, line in enumerate(Path(path).read_text().splitlines(), 1):
        f = line.split()
        if not f:
            continue
        if f[0] == "cfg" and len(f) == 3:
            m.cfg[f[1]] = f[2]
        elif f[0] == "t" and len(f) == 4:
            off, cnt = int(f[2]), int(f[3])
            if off % ALIGN or cnt <= 0:
                raise ValueError(f"{path}:{n}: tensor {f[1]} at offset {off} with {cnt} elements")
            if f[1] in m.tensors:
                raise ValueError(f"{path}:{n}: tensor {f[1]} listed twice")
            m.tensors[f[1]] = (off, cnt)
        else:
            raise ValueError(f"{path}:{n}: unrecognised record {line!r}")
    if int(float(m.cfg.get("layout", 1))) < LAYOUT:
        raise ValueError(f"{path}: weights are layout 1 (gate/up not interleaved); repack with layout 2")
    spans = sorted((o, o + 2 * c, k) for k, (o, c) in m.tensors.items())
    for (o0, e0, k0), (o1, e1, k1) in zip(spans, spans[1:]):
        if o1 < e0:
            raise ValueError(f"{path}: tensors {k0} and {k1} overlap")
    return m


def model_config(m: Manifest, name: str = "checkpoint", max_ctx: int = 0, layers: int = 0) -> ModelConfig:
    """The decoder dimensions a manifest describes (host.hip:77-83).  Features this path does not compute (qkv bias)
    are refused rather than ignored."""
    if m.geti("bias"):
        raise ValueError("qkv bias is not supported by this decode path")
    moe = m.geti("moe")
    L = m.geti("L")
    return ModelConfig(name=name, H=m.geti("H"), NH=m.geti("NH"), NKV=m.geti("NKV"), HD=m.geti("HD"),
                       L=min(layers or L, L), V=m.geti("V"), I=0 if moe else m.geti("INTER"),
                       E=m.geti("E") if moe else 0, TOPK=m.geti("TOPK") if moe else 0, MI=m.geti("MI") if moe else 0,
                       moe=moe, qk_norm=m.geti("qk_norm"), norm_topk=m.geti("norm_topk"),
                       eps=m.getf("eps"), theta=m.getf("theta"), max_ctx=max_ctx or m.geti("CTX"))


def tensor_plan(cfg: ModelConfig, tie: bool = False) -> list:
    """(manifest name, library kind, layer, shape) of every tensor of a decoder, in prep.py's order."""
    H, HD, V = cfg.H, cfg.HD, cfg.V
    out = [("embed", N.T_EMBED, -1, (V, H)), ("final_norm", N.T_FINAL_NORM, -1, (H,))]
    if not tie:
        out.append(("lm_head", N.T_LMHEAD, -1, (V, H)))
    for l in range(cfg.L):
        p = f"L{l}."
        out += [(p + "ln1", N.T_LN1, l, (H,)), (p + "ln2", N.T_LN2, l, (H,)),
                (p + "wqkv", N.T_WQKV, l, (cfg.nqkv, H))]
        if cfg.qk_norm:
            out += [(p + "qn", N.T_QNORM, l, (HD,)), (p + "kn", N.T_KNORM, l, (HD,))]
        out.append((p + "wo", N.T_WO, l, (H, cfg.NH * HD)))
        if cfg.moe:
            out += [(p + "wr", N.T_ROUTER, l, (cfg.E, H)), (p + "egu", N.T_W13, l, (cfg.E, 2 * cfg.MI, H)),
                    (p + "ed", N.T_W2, l, (cfg.E, H, cfg.MI))]
        else:
            out += [(p + "wgu", N.T_WGU, l, (2 * cfg.I, H)), (p + "wd", N.T_WD, l, (H, cfg.I))]
    return out


class Checkpoint:
    """A packed checkpoint directory; weights.bin is memory-mapped, never read whole."""

    def __init__(self, path: str | Path):
        self.dir = Path(path)
        self.manifest = read_manifest(self.dir / "llm.manifest")
        self.blob = np.memmap(self.dir / "weights.bin", dtype=np.uint8, mode="r")
        for name, (off, cnt) in self.manifest.tensors.items():
            if off + 2 * cnt > self.blob.size:
                raise ValueError(f"{self.dir}: tensor {name} ends past weights.bin ({off + 2 * cnt} > {self.blob.size})")

    @property
    def tie(self) -> bool:
        return bool(int(float(self.manifest.cfg.get("tie", 0))))

    def config(self, **kw) -> ModelConfig:
        return model_config(self.manifest, name=self.dir.name, **kw)

    def array(self, name: str, shape=None) -> np.ndarray:
        """A tensor's bf16 bits (uint16, a view of the mapped file), reshaped when shape is given."""
        if name not in self.manifest.tensors:
            raise KeyError(f"manifest lacks tensor {name}")
        off, cnt = self.manifest.tensors[name]
        a = self.blob[off:off + 2 * cnt].view(np.uint16)
        if shape is not None:
            if int(np.prod(shape)) != cnt:
                raise ValueError(f"tensor {name}: {cnt} elements, expected shape {tuple(shape)}")
            a = a.reshape(shape)
        return a

    def check(self, cfg: ModelConfig):
        """Every tensor the decoder needs is present with the element count its shape implies."""
        for name, _, _, shape in tensor_plan(cfg, self.tie):
            self.array(name, shape)

    def load_into(self, dec: "N.Decoder"):
        """Copy every tensor into a bound Decoder (etxmk_load_tensor per tensor, per expert for the stacks).  A tied
        checkpoint fills the head from the embedding (prep.py:106-107 writes no lm_head then)."""
        import torch
        cfg = dec.cfg
        self.check(cfg)
        staging = None

        def put(kind, layer, expert, a):
            nonlocal staging
            a = np.array(a, dtype=np.uint16, order="C", copy=True)   # the mapped file is read-only
            n = a.size
            if staging is None or staging.numel() < n:
                staging = torch.empty(n, dtype=torch.int16, device=dec.device)
            staging[:n].copy_(torch.from_numpy(a.view(np.int16).reshape(-1)))   # same stream as the library's copy
            dec.load_tensor(kind, layer, expert, staging[:n])

        for name, kind, layer, shape in tensor_plan(cfg, self.tie):
            a = self.array(name, shape)
            if kind in (N.T_W13, N.T_W2):
                for e in range(shape[0]):
                    put(kind, layer, e, a[e])
            else:
                put(kind, layer, 0, a)
            if kind == N.T_EMBED and self.tie:
                put(N.T_LMHEAD, -1, 0, a)
        dec.sync()


def write_checkpoint(path: str | Path, cfg: ModelConfig, get, tie: bool = False, ctx: int = 0, chunk: int = 64):
    """Write weights.bin + llm.manifest the way prep.py does; get(name, shape) returns a tensor's bf16 bits (uint16).
    ctx is the CTX recorded (default: cfg.max_ctx)."""
    d = Path(path)
    d.mkdir(parents=True, exist_ok=True)
    lines, off = [], 0
    with open(d / "weights.bin", "wb") as wf:
        for name, _, _, shape in tensor_plan(cfg, tie):
            pad = (-off) % ALIGN
            if pad:
                wf.write(b"\0" * pad)
                off += pad
            a = np.ascontiguousarray(get(name, shape), dtype=np.uint16)
            if a.shape != tuple(shape):
                raise ValueError(f"{name}: shape {a.shape}, expected {tuple(shape)}")
            wf.write(a.tobytes())
            lines.append(f"t {name} {off} {a.size}")
            off += a.nbytes
    attn = (cfg.nqkv * cfg.H + cfg.H * cfg.NH * cfg.HD) * 2
    mlp = (cfg.E * cfg.H + cfg.TOPK * 3 * cfg.MI * cfg.H) * 2 if cfg.moe else 3 * cfg.I * cfg.H * 2
    keys = dict(H=cfg.H, NH=cfg.NH, NKV=cfg.NKV, HD=cfg.HD, INTER=0 if cfg.moe else cfg.I, L=cfg.L, V=cfg.V, E=cfg.E,
                TOPK=cfg.TOPK, MI=cfg.MI, CTX=ctx or cfg.max_ctx, CHUNK=chunk, qk_norm=int(cfg.qk_norm), bias=0,
                moe=int(cfg.moe), norm_topk=int(cfg.norm_topk), tie=int(tie), eps=cfg.eps, theta=cfg.theta,
                active_bytes=cfg.L * (attn + mlp) + cfg.V * cfg.H * 2, layout=LAYOUT)
    (d / "llm.manifest").write_text("\n".join([f"cfg {k} {v}" for k, v in keys.items()] + lines) + "\n")
    return off


def read_golden(path: str | Path):
    """prompt ids, greedy ids and margins of a golden*.txt (prep.py:231-234; host.hip:72-74)."""
    rows = {}
    for line in Path(path).read_text().splitlines():
        f = line.split()
        if f and f[0].endswith(":"):
            rows[f[0][:-1]] = f[1:]
    prompt = [int(t) for t in rows.get("prompt", [])]
    gen = [int(t) for t in rows.get("gen", [])]
    margin = [float(t) for t in rows.get("margin", [])]
    if not prompt:
        raise ValueError(f"{path}: no prompt line")
    return prompt, gen, margin
