"""ctypes binding of libetxmk.so, the gfx950 decode megakernel (include/etxmk.h).

PyTorch is used only to allocate the device buffers the library borrows and to pick the HIP stream.
There is no fallback: if the library is missing or a call fails, an exception says so.

Reference counterparts: etx_host (etx/runtime/include/etx/host.h:22-692) and the per-token loop of
examples/llm/host.hip:57-244 (prompt fed token by token through the decode step, :203-213).
"""
from __future__ import annotations

import ctypes as C
import re
from dataclasses import dataclass, field, asdict
from pathlib import Path

import numpy as np

PKG = Path(__file__).resolve().parents[2]
LIB_PATH = PKG / "lib" / "libetxmk.so"
HEADER = PKG.parent / "include" / "etxmk.h"

ABI_VERSION = 3
OK, EINVAL, EHIP, ABORTED, EUNBOUND, TIMEOUT = 0, 1, 2, 3, 4, 5
T_EMBED, T_LMHEAD, T_WQKV, T_WO, T_ROUTER, T_W13, T_W2, T_WGU, T_WD = 1, 2, 3, 4, 5, 6, 7, 8, 9
T_LN1, T_LN2, T_QNORM, T_KNORM, T_FINAL_NORM = 20, 21, 22, 23, 24
T_WKVB, T_WSGU, T_WSD = 14, 15, 16             # DeepSeek-V2: kv_b_proj, shared experts' gate/up and down


class EtxmkError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"etxmk error {code}: {msg}")
        self.code = code


class DeviceAbort(EtxmkError):
    pass


class StepTimeout(EtxmkError):
    """etxmk_sync_timeout: the stream outlived the limit; a stopped step's outputs are void."""


class EtxmkConfig(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("H", "NH", "NKV", "HD", "I", "E", "TOPK", "MI", "L", "V",
                                          "moe", "qk_norm", "norm_topk", "block_size", "max_ctx", "batch")] + \
               [("eps", C.c_float), ("theta", C.c_float), ("wdtype", C.c_int32), ("arch", C.c_int32)] + \
               [(n, C.c_int32) for n in ("kv_lora", "qk_nope", "qk_rope", "v_head", "n_shared", "first_dense",
                                         "dense_I")] + \
               [(n, C.c_float) for n in ("routed_scale", "rope_factor", "rope_mscale", "rope_mscale_all", "beta_fast",
                                         "beta_slow")] + [("rope_orig_max", C.c_int32), ("prefill", C.c_int32)]


class EtxmkPlanInfo(C.Structure):
    _fields_ = [("kernel", C.c_char * 96), ("barriers_per_step", C.c_int32), ("threads", C.c_int32),
                ("batch_capacity", C.c_int32), ("matrix_cores", C.c_int32), ("weight_bytes", C.c_uint64),
                ("kv_bytes", C.c_uint64), ("workspace_bytes", C.c_uint64)]


W_BF16, W_FP8 = 0, 1          # weight types of etxmk_config.wdtype
ARCH_QWEN3, ARCH_DSV2 = 0, 1  # etxmk_config.arch


@dataclass(frozen=True)
class ModelConfig:
    """Decoder dimensions (the fields of examples/llm/model.py:45-93 Dims that the decode step uses)."""
    H: int
    NH: int
    NKV: int
    HD: int
    L: int
    V: int
    I: int = 0
    E: int = 0
    TOPK: int = 0
    MI: int = 0
    moe: int = 0
    qk_norm: int = 1
    norm_topk: int = 1
    block_size: int = 16
    max_ctx: int = 1088
    batch: int = 1
    eps: float = 1e-6
    theta: float = 1e6
    wdtype: int = W_BF16          # W_FP8: QKV / O / MLP matrices as e4m3 with per-row scales
    # DeepSeek-V2 (arch = ARCH_DSV2): multi-head latent attention, shared experts, leading dense layers, yarn RoPE
    arch: int = ARCH_QWEN3
    kv_lora: int = 0
    qk_nope: int = 0
    qk_rope: int = 0
    v_head: int = 0
    n_shared: int = 0
    first_dense: int = 0
    dense_I: int = 0
    routed_scale: float = 1.0
    rope_factor: float = 1.0
    rope_mscale: float = 1.0
    rope_mscale_all: float = 1.0
    beta_fast: float = 32.0
    beta_slow: float = 1.0
    rope_orig_max: int = 4096
    prefill: int = 0              # rows per prefill launch (<= 16; DeepSeek-V2 <= 4); 0: prompts token by token
    name: str = field(default="custom", compare=False)

    def as_struct(self) -> EtxmkConfig:
        return EtxmkConfig(**{k: getattr(self, k) for k, _ in EtxmkConfig._fields_})

    def as_dict(self) -> dict:
        d = asdict(self)
        d.pop("name")
        return d

    @property
    def nqkv(self) -> int:
        """Rows of the fused input projection: Q, K, V heads, or (DeepSeek-V2) q_proj and kv_a_proj_with_mqa."""
        if self.arch == ARCH_DSV2:
            return self.NH * (self.qk_nope + self.qk_rope) + self.kv_lora + self.qk_rope
        return (self.NH + 2 * self.NKV) * self.HD


_lib = None


def declared_functions() -> list[str]:
    """Every function include/etxmk.h declares."""
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(etxmk_\w+)\s*\(", text, re.M)))


def load(path: Path | None = None):
    """Load libetxmk.so (torch first, so the process holds the one HIP runtime torch brings)."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    import torch  # noqa: F401  (binds libamdhip64 before the library resolves it)
    p = Path(path or LIB_PATH)
    if not p.exists():
        raise FileNotFoundError(f"{p} is not built; run etx-megakernel_amd/build_lib.py (no fallback path exists)")
    L = C.CDLL(str(p))
    vp, i32, u64 = C.c_void_p, C.c_int32, C.c_uint64
    sig = {
        "etxmk_abi_version": [],
        "etxmk_last_error": [],
        "etxmk_weight_bytes": [C.POINTER(EtxmkConfig), C.POINTER(u64)],
        "etxmk_kv_bytes": [C.POINTER(EtxmkConfig), C.POINTER(u64)],
        "etxmk_workspace_bytes": [C.POINTER(EtxmkConfig), C.POINTER(u64)],
        "etxmk_create": [C.POINTER(EtxmkConfig), C.POINTER(vp)],
        "etxmk_destroy": [vp],
        "etxmk_bind": [vp, vp, vp, vp],
        "etxmk_tensor_info": [vp, i32, i32, i32, C.POINTER(u64), C.POINTER(i32), C.POINTER(i32), C.POINTER(i32)],
        "etxmk_tensor_format": [vp, i32, i32, C.POINTER(i32), C.POINTER(u64)],
        "etxmk_init_weights_seeded": [vp, u64, C.c_float, vp],
        "etxmk_load_tensor": [vp, i32, i32, i32, vp, vp],
        "etxmk_set_block_table": [vp, C.POINTER(i32), i32, vp],
        "etxmk_fill_kv_seeded": [vp, u64, i32, vp],
        "etxmk_fill_kv_seeded_seq": [vp, u64, i32, i32, vp],
        "etxmk_set_tokens": [vp, C.POINTER(i32), i32, vp],
        "etxmk_read_tokens": [vp, C.POINTER(i32), i32, vp],
        "etxmk_set_tokens_seq": [vp, i32, C.POINTER(i32), i32, vp],
        "etxmk_read_tokens_seq": [vp, i32, C.POINTER(i32), i32, vp],
        "etxmk_step": [vp, i32, i32, vp],
        "etxmk_step_batch": [vp, C.POINTER(i32), i32, vp],
        "etxmk_step_static": [vp, i32, i32, vp],
        "etxmk_prefill": [vp, i32, i32, i32, i32, vp],
        "etxmk_step_layers": [vp, i32, i32, i32, vp],
        "etxmk_set_residual": [vp, C.POINTER(C.c_float), vp],
        "etxmk_read_residual": [vp, C.POINTER(C.c_float), vp],
        "etxmk_sync": [vp, vp],
        "etxmk_sync_timeout": [vp, vp, C.c_int64],
        "etxmk_abort": [vp],
        "etxmk_set_spin_limit": [vp, u64, i32],
        "etxmk_set_fused": [vp, i32],
        "etxmk_set_dump": [vp, vp, vp, vp, vp],
        "etxmk_set_grid": [vp, i32],
        "etxmk_barriers_per_step": [vp, C.POINTER(i32)],
        "etxmk_set_trace": [vp, vp],
        "etxmk_plan": [C.POINTER(EtxmkConfig), i32, C.POINTER(EtxmkPlanInfo)],
    }
    for name, args in sig.items():
        f = getattr(L, name)
        f.argtypes = args
        f.restype = C.c_char_p if name == "etxmk_last_error" else C.c_int
    if L.etxmk_abi_version() != ABI_VERSION:
        raise EtxmkError(EINVAL, f"ABI version {L.etxmk_abi_version()} != {ABI_VERSION}")
    if path is None:
        _lib = L
    return L


def _check(L, rc: int):
    if rc != OK:
        msg = L.etxmk_last_error().decode(errors="replace")
        if rc == ABORTED:
            raise DeviceAbort(rc, msg)
        if rc == TIMEOUT:
            raise StepTimeout(rc, msg)
        raise EtxmkError(rc, msg)


def sizes(cfg: ModelConfig) -> dict:
    """Bytes of the weight arena, KV cache and workspace (no GPU needed)."""
    L = load()
    c = cfg.as_struct()
    out = {}
    for key, fn in (("weights", L.etxmk_weight_bytes), ("kv", L.etxmk_kv_bytes), ("workspace", L.etxmk_workspace_bytes)):
        v = C.c_uint64()
        _check(L, fn(C.byref(c), C.byref(v)))
        out[key] = int(v.value)
    return out


def plan_info(cfg: ModelConfig, fused: bool = True) -> dict:
    """The library's plan of a configuration (no GPU needed): the persistent kernel symbol (or "unfused"), grid
    barriers per step, threads per workgroup, the kernel's batch capacity and the buffer sizes."""
    L = load()
    c = cfg.as_struct()
    out = EtxmkPlanInfo()
    _check(L, L.etxmk_plan(C.byref(c), int(fused), C.byref(out)))
    return {"kernel": out.kernel.decode(), "barriers_per_step": int(out.barriers_per_step), "threads": int(out.threads),
            "batch_capacity": int(out.batch_capacity), "matrix_cores": bool(out.matrix_cores),
            "weight_bytes": int(out.weight_bytes),
            "kv_bytes": int(out.kv_bytes), "workspace_bytes": int(out.workspace_bytes)}


def phase_names(cfg: ModelConfig) -> list[list[str]]:
    """The phases of one step, layer by layer (each ends in a grid barrier), then ["head"] (the lm_head phase; the
    token write after it ends the step)."""
    if cfg.arch == ARCH_DSV2:
        att = ["qkv", "absorb", "attn", "wuv", "oproj"]
        layers = [att + (["gateup", "down"] if l < cfg.first_dense else ["router_shared", "expert_up", "expert_down"])
                  for l in range(cfg.L)]
    else:                                   # batched kernels merge the attention partials in a phase of its own
        att = ["qkv", "attn"] + (["attn_merge"] if cfg.batch > 1 else []) + ["oproj"]
        mlp = ["router", "expert_up", "expert_down"] if cfg.moe else ["gateup", "down"]
        # handles on the matrix cores combine the expert outputs in a phase of their own (the library's plan says
        # which)
        if cfg.moe and plan_info(cfg)["matrix_cores"]:
            mlp = mlp + ["combine"]
        layers = [att + mlp for _ in range(cfg.L)]
    return layers + [["head"]]


def unpermute_rows(stored: np.ndarray, block: int = 512) -> np.ndarray:
    """Natural row order from the lane-permuted storage (blocks of 512 for bf16 rows, 1024 for fp8 codes; lane l
    holds l, l+64, ...)."""
    rows, K = stored.shape
    out = np.empty_like(stored)
    for base in range(0, K, block):
        S = min(block, K - base)
        m = S // 64
        blk = stored[:, base:base + S].reshape(rows, 64, m)           # [row][lane][e]
        out[:, base:base + S] = blk.transpose(0, 2, 1).reshape(rows, S)  # element l + 64 e
    return out


class Decoder:
    """One model on one GPU: owns the torch buffers the library borrows."""

    def __init__(self, cfg: ModelConfig, device: str = "cuda:0", fused: bool = True, workgroups: int = 0):
        import torch
        self.torch = torch
        self.cfg = cfg
        self.device = torch.device(device)
        self.L = load()
        sz = sizes(cfg)
        self.sizes = sz
        self.weights = torch.empty(sz["weights"], dtype=torch.uint8, device=self.device)
        self.kv = torch.zeros(sz["kv"], dtype=torch.uint8, device=self.device)
        self.workspace = torch.zeros(sz["workspace"], dtype=torch.uint8, device=self.device)
        h = C.c_void_p()
        c = cfg.as_struct()
        with torch.cuda.device(self.device):
            _check(self.L, self.L.etxmk_create(C.byref(c), C.byref(h)))
            self.h = h
            _check(self.L, self.L.etxmk_bind(h, self.weights.data_ptr(), self.kv.data_ptr(), self.workspace.data_ptr()))
            _check(self.L, self.L.etxmk_set_fused(h, int(fused)))
            _check(self.L, self.L.etxmk_set_grid(h, int(workgroups)))
        self._nwg = int(workgroups)
        self.fused = bool(fused)
        self._dumps = None

    # ---- plumbing
    def _stream(self):
        return C.c_void_p(self.torch.cuda.current_stream(self.device).cuda_stream)

    def close(self):
        if getattr(self, "h", None):
            self.L.etxmk_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---- weights / cache
    def init_weights(self, seed: int, scale: float = 0.02):
        _check(self.L, self.L.etxmk_init_weights_seeded(self.h, seed, scale, self._stream()))

    def tensor_info(self, kind: int, layer: int = -1, expert: int = 0):
        off, r, c, p = C.c_uint64(), C.c_int32(), C.c_int32(), C.c_int32()
        _check(self.L, self.L.etxmk_tensor_info(self.h, kind, layer, expert, C.byref(off), C.byref(r), C.byref(c), C.byref(p)))
        return int(off.value), int(r.value), int(c.value), bool(p.value)

    def tensor_format(self, kind: int, layer: int = -1):
        """(weight type W_BF16 / W_FP8, bytes per row) of a tensor kind."""
        wt, rb = C.c_int32(), C.c_uint64()
        _check(self.L, self.L.etxmk_tensor_format(self.h, kind, layer, C.byref(wt), C.byref(rb)))
        return int(wt.value), int(rb.value)

    def tensor_fp8(self, kind: int, layer: int = -1, expert: int = 0):
        """Host copy of an fp8 tensor: (e4m3 codes [rows][cols] uint8 in natural order, scales [rows] fp32)."""
        wt, rb = self.tensor_format(kind, layer)
        if wt != W_FP8:
            raise ValueError(f"tensor kind {kind} is not held as fp8")
        off, r, c, _ = self.tensor_info(kind, layer, expert)
        raw = self.weights[off:off + r * rb].cpu().numpy().reshape(r, rb)
        return unpermute_rows(raw[:, :c].copy(), 1024), raw[:, c:c + 4].copy().view(np.float32).reshape(r)

    def tensor(self, kind: int, layer: int = -1, expert: int = 0, natural: bool = True) -> np.ndarray:
        """Host copy of one bf16 tensor as uint16 bits [rows][cols] (natural row order unless natural=False)."""
        if self.tensor_format(kind, layer)[0] != W_BF16:
            raise ValueError(f"tensor kind {kind} is held as fp8: use tensor_fp8")
        off, r, c, perm = self.tensor_info(kind, layer, expert)
        if kind == T_WKVB and self.cfg.arch == ARCH_DSV2:
            raise ValueError("kv_b_proj is stored split (W_UK^T, W_UV): read it with kv_b()")
        cs = self.tensor_format(kind, layer)[1] // 2          # stored row length (padded rows are longer than c)
        t = self.weights[off:off + r * cs * 2].view(self.torch.int16).cpu().numpy().view(np.uint16).reshape(r, cs)
        return (unpermute_rows(t) if (perm and natural) else t)[:, :c] if natural else t

    def kv_b(self, layer: int) -> np.ndarray:
        """DeepSeek-V2 kv_b_proj of a layer in its natural layout [NH*(qk_nope + v_head)][kv_lora] (uint16 bits),
        rebuilt from the stored W_UK^T and W_UV."""
        c = self.cfg
        off, r, kvl, _ = self.tensor_info(T_WKVB, layer)
        raw = self.weights[off:off + r * kvl * 2].view(self.torch.int16).cpu().numpy().view(np.uint16)
        NH, nope, vh = c.NH, c.qk_nope, c.v_head
        uk = unpermute_rows(raw[:NH * kvl * nope].reshape(NH * kvl, nope)).reshape(NH, kvl, nope)
        uv = unpermute_rows(raw[NH * kvl * nope:].reshape(NH * vh, kvl)).reshape(NH, vh, kvl)
        out = np.empty((NH, nope + vh, kvl), np.uint16)
        out[:, :nope] = uk.transpose(0, 2, 1)
        out[:, nope:] = uv
        return out.reshape(NH * (nope + vh), kvl)

    def load_tensor(self, kind: int, layer: int, expert: int, src):
        """src: torch bf16/int16 tensor on the device in natural [rows][cols] layout."""
        _check(self.L, self.L.etxmk_load_tensor(self.h, kind, layer, expert, src.data_ptr(), self._stream()))

    @property
    def blocks_per_seq(self) -> int:
        return -(-self.cfg.max_ctx // self.cfg.block_size)

    def set_block_table(self, table):
        """One sequence's table, or [batch][blocks_per_seq] (flattened row by row)."""
        t = np.ascontiguousarray(np.asarray(table, np.int32).reshape(-1))
        _check(self.L, self.L.etxmk_set_block_table(self.h, t.ctypes.data_as(C.POINTER(C.c_int32)), len(t), self._stream()))

    def fill_kv_seeded(self, seed: int, npos: int, seq: int = 0):
        _check(self.L, self.L.etxmk_fill_kv_seeded_seq(self.h, seed, seq, npos, self._stream()))

    def kv_layer(self, layer: int):
        """(K, V) of one layer as uint16 bf16 bits, paged layout, flat; DeepSeek-V2: (latent cache, None)."""
        if self.cfg.arch == ARCH_DSV2:
            n = self.sizes["kv"] // 2 // self.cfg.L
            return self.kv.view(self.torch.int16)[layer * n:(layer + 1) * n].cpu().numpy().view(np.uint16), None
        n = self.sizes["kv"] // 2 // self.cfg.L // 2
        base = layer * 2 * n
        flat = self.kv.view(self.torch.int16)
        return (flat[base:base + n].cpu().numpy().view(np.uint16), flat[base + n:base + 2 * n].cpu().numpy().view(np.uint16))

    # ---- dumps
    def enable_dumps(self, on: bool = True):
        torch = self.torch
        cfg = self.cfg
        if not on:
            _check(self.L, self.L.etxmk_set_dump(self.h, None, None, None, None))
            self._dumps = None
            return
        k = max(cfg.TOPK, 1)
        lb = (cfg.L,) if cfg.batch == 1 else (cfg.L, cfg.batch)      # batched handles: [layer][sequence][...]
        self._dumps = dict(
            x=torch.zeros(lb + (cfg.H,), dtype=torch.float32, device=self.device),
            ids=torch.full(lb + (k,), -1, dtype=torch.int32, device=self.device),
            w=torch.zeros(lb + (k,), dtype=torch.float32, device=self.device),
            logits=torch.zeros(lb + (max(cfg.E, 1),), dtype=torch.float32, device=self.device))
        d = self._dumps
        moe = bool(cfg.moe)
        _check(self.L, self.L.etxmk_set_dump(self.h, d["x"].data_ptr(), d["ids"].data_ptr() if moe else None,
                                             d["w"].data_ptr() if moe else None, d["logits"].data_ptr() if moe else None))

    def dumps(self) -> dict:
        self.sync()
        return {k: v.cpu().numpy().copy() for k, v in self._dumps.items()}

    # ---- steps
    def set_tokens(self, tokens, seq: int = 0):
        t = np.ascontiguousarray(tokens, np.int32)
        _check(self.L, self.L.etxmk_set_tokens_seq(self.h, seq, t.ctypes.data_as(C.POINTER(C.c_int32)), len(t),
                                                   self._stream()))

    def read_tokens(self, n: int, seq: int = 0) -> np.ndarray:
        out = np.zeros(n, np.int32)
        _check(self.L, self.L.etxmk_read_tokens_seq(self.h, seq, out.ctypes.data_as(C.POINTER(C.c_int32)), n,
                                                    self._stream()))
        return out

    def step(self, pos: int, write_next: bool = True):
        _check(self.L, self.L.etxmk_step(self.h, pos, int(write_next), self._stream()))

    def step_static(self, pos: int, write_next: bool = True):
        """etxmk_step with its scratch in the library's static device array (no workspace scratch, no allocation)."""
        _check(self.L, self.L.etxmk_step_static(self.h, pos, int(write_next), self._stream()))

    def step_batch(self, positions, write_next=True):
        """One step of every sequence; write_next: one flag for all, or one per sequence."""
        pos = np.ascontiguousarray(positions, np.int32)
        if pos.shape != (self.cfg.batch,):
            raise ValueError(f"{pos.shape[0] if pos.ndim else 0} positions for batch {self.cfg.batch}")
        flags = [write_next] * self.cfg.batch if np.isscalar(write_next) else list(write_next)
        mask = sum(1 << b for b, f in enumerate(flags) if f)
        _check(self.L, self.L.etxmk_step_batch(self.h, pos.ctypes.data_as(C.POINTER(C.c_int32)), mask, self._stream()))

    def prefill(self, pos0: int, n: int, write_next: bool = True, seq: int = 0):
        """Positions pos0 .. pos0 + n - 1 of sequence seq in one launch, one row per position."""
        _check(self.L, self.L.etxmk_prefill(self.h, seq, pos0, n, int(write_next), self._stream()))

    @property
    def prefill_rows(self) -> int:
        """Positions one prefill launch takes (0: this handle reads prompts token by token)."""
        c = self.cfg
        if not self.fused:
            return 0
        return max(c.batch, c.prefill) if (c.batch > 1 or c.prefill > 0) else 0

    def feed_prompt(self, n: int, seq: int = 0, rows: int | None = None):
        """Positions 0 .. n - 1 of sequence seq (its tokens set), the last one writing the greedy token at n: in
        launches of `rows` positions (default prefill_rows; 0 or 1 = one decode step per position)."""
        rows = self.prefill_rows if rows is None else rows
        if rows > 1:
            for p0 in range(0, n, rows):
                self.prefill(p0, min(rows, n - p0), write_next=p0 + rows >= n, seq=seq)
        elif self.cfg.batch == 1:
            for pos in range(n):
                self.step(pos, write_next=pos + 1 >= n)
        else:
            raise ValueError("a batched handle without prefill rows reads prompts through generate_batch")

    def step_layers(self, pos: int, l0: int, l1: int):
        _check(self.L, self.L.etxmk_step_layers(self.h, pos, l0, l1, self._stream()))

    def set_residual(self, x):
        x = np.ascontiguousarray(x, np.float32)
        _check(self.L, self.L.etxmk_set_residual(self.h, x.ctypes.data_as(C.POINTER(C.c_float)), self._stream()))

    def read_residual(self) -> np.ndarray:
        x = np.zeros(self.cfg.H, np.float32)
        _check(self.L, self.L.etxmk_read_residual(self.h, x.ctypes.data_as(C.POINTER(C.c_float)), self._stream()))
        return x

    def sync(self, timeout_ms: int | None = None):
        """Wait for the handle's work; with timeout_ms, stop a step still running past it (StepTimeout)."""
        if timeout_ms is None:
            _check(self.L, self.L.etxmk_sync(self.h, self._stream()))
        else:
            _check(self.L, self.L.etxmk_sync_timeout(self.h, self._stream(), int(timeout_ms)))

    def abort(self):
        """Ask the running (or next) step to stop; the next sync raises DeviceAbort."""
        _check(self.L, self.L.etxmk_abort(self.h))

    def set_spin_limit(self, ticks: int = 0, check_every: int = 0):
        """Bounds of the kernel's barrier waits (100 MHz ticks, 0 = default 2 s; check cadence in polls)."""
        _check(self.L, self.L.etxmk_set_spin_limit(self.h, int(ticks), int(check_every)))

    def enable_trace(self, on: bool = True):
        """Per-phase, per-workgroup s_memrealtime stamps of the fused kernel; read with trace()."""
        if on:
            n = (self.barriers_per_step() + 1) * self.workgroups() * 3
            self._trace = self.torch.zeros(n, dtype=self.torch.int64, device=self.device)
            _check(self.L, self.L.etxmk_set_trace(self.h, self._trace.data_ptr()))
        else:
            _check(self.L, self.L.etxmk_set_trace(self.h, None))
            self._trace = None

    def trace_ticks(self) -> np.ndarray:
        """Raw stamps of the last traced step: uint64 [barriers + 1][workgroups][3] of the 100 MHz clock."""
        self.sync()
        return self._trace.cpu().numpy().view(np.uint64).reshape(self.barriers_per_step() + 1, self.workgroups(), 3)

    def trace(self) -> np.ndarray:
        """Stamps of the last traced step in microseconds from the launch:
        [phase][workgroup][wait done, arrive, first weight loads issued (GEMV phases; nan otherwise)]."""
        self.sync()
        t = self._trace.cpu().numpy().reshape(self.barriers_per_step() + 1, self.workgroups(), 3).astype(np.float64)
        t0 = t[0, :, 0].min()
        out = (t - t0) / 100.0
        out[t == 0] = np.nan
        return out

    def workgroups(self) -> int:
        import torch
        return self._nwg or torch.cuda.get_device_properties(self.device).multi_processor_count

    def barriers_per_step(self) -> int:
        n = C.c_int32()
        _check(self.L, self.L.etxmk_barriers_per_step(self.h, C.byref(n)))
        return int(n.value)

    def generate_batch(self, prompts, n_new: int, prefill: bool | None = None) -> np.ndarray:
        """Batched greedy decode; returns [batch][n_new] ids.  With prefill (the default where the handle has
        prefill rows) each prompt goes through prefill launches, then every sequence decodes from the end of its
        prompt; without, sequence b reads prompts[b] token by token inside the batched steps and every sequence moves
        one position per step (sequences with shorter prompts start decoding earlier)."""
        B = self.cfg.batch
        prompts = [list(int(t) for t in p) for p in prompts]
        if len(prompts) != B or min(len(p) for p in prompts) < 1:
            raise ValueError(f"{len(prompts)} prompts for batch {B}")
        lens = [len(p) for p in prompts]
        T = max(lens) + n_new - 1
        if T + 1 > self.cfg.max_ctx + 1 or max(lens) + n_new > self.cfg.max_ctx:
            raise ValueError(f"prompts + {n_new} new tokens exceed max_ctx {self.cfg.max_ctx}")
        for b, p in enumerate(prompts):
            self.set_tokens(p, seq=b)
        if prefill is None:
            prefill = self.prefill_rows > 1
        if prefill:
            for b in range(B):
                self.feed_prompt(lens[b], seq=b)
            for s in range(n_new - 1):
                self.step_batch([lens[b] + s for b in range(B)], write_next=True)
            self.sync()
            return np.stack([self.read_tokens(lens[b] + n_new - 1, seq=b)[lens[b] - 1:] for b in range(B)])
        # sequence b decodes positions [0, lens[b] + n_new - 1); it waits (repeats its last step's position) once
        # done, which rewrites the same cache entry with the same values
        for s in range(T):
            pos = [min(s, lens[b] + n_new - 2) for b in range(B)]
            self.step_batch(pos, write_next=[pos[b] + 1 >= lens[b] for b in range(B)])
        self.sync()
        return np.stack([self.read_tokens(lens[b] + n_new - 1, seq=b)[lens[b] - 1:lens[b] - 1 + n_new]
                         for b in range(B)])

    def generate(self, prompt, n_new: int, prefill: bool | None = None) -> np.ndarray:
        """Feed the prompt (prefill launches where the handle has prefill rows, else token by token), then n_new
        greedy steps; returns the generated ids (examples/llm/host.hip:203-213 and ref_numpy.py:181-186 drive the
        same loop token by token; prefill reproduces it bit for bit)."""
        prompt = list(int(t) for t in prompt)
        P = len(prompt)
        if P < 1 or P + n_new > self.cfg.max_ctx:
            raise ValueError(f"prompt {P} + {n_new} new tokens exceed max_ctx {self.cfg.max_ctx}")
        if self.cfg.batch != 1:
            raise ValueError("batched handles generate through generate_batch")
        self.set_tokens(prompt)
        if prefill is None:
            prefill = self.prefill_rows > 1
        self.feed_prompt(P, rows=None if prefill else 1)
        for pos in range(P, P + n_new - 1):
            self.step(pos, write_next=True)
        self.sync()
        out = self.read_tokens(P + n_new - 1)
        return out[P - 1:P - 1 + n_new]
