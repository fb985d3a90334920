"""ctypes view of the CPU oracle (oracle/mk_oracle.c).  TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module; it is the
checker the HIP library is compared against, never part of the product path.  It restates
examples/llm/ref_numpy.py (Ref.step, :105-158) of the reference; see mk_oracle.c for the fixed
evaluation order.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "build" / "liboracle.so"

# tensor kinds of the seeded generator (stream id = kind << 48 | (layer + 1) << 24 | expert)
S_EMBED, S_LMHEAD, S_WQKV, S_WO, S_ROUTER, S_W13, S_W2, S_WGU, S_WD, S_KINIT, S_VINIT, S_XIN, S_PROMPT = range(1, 14)


class OrcConfig(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("H", "NH", "NKV", "HD", "I", "E", "TOPK", "MI", "L", "V",
                                          "moe", "qk_norm", "norm_topk", "block_size", "max_ctx", "batch")] + \
               [("eps", C.c_float), ("theta", C.c_float), ("wdtype", C.c_int32), ("arch", C.c_int32)] + \
               [(n, C.c_int32) for n in ("kv_lora", "qk_nope", "qk_rope", "v_head", "n_shared", "first_dense",
                                         "dense_I")] + \
               [(n, C.c_float) for n in ("routed_scale", "rope_factor", "rope_mscale", "rope_mscale_all", "beta_fast",
                                         "beta_slow")] + [("rope_orig_max", C.c_int32)]

ARCH_QWEN3, ARCH_DSV2 = 0, 1
S_WKVB, S_WSGU, S_WSD = 14, 15, 16

# weight types: bf16; fp8 e4m3 rows with per-row fp32 scales; (oracle only) fp8 dequantised into bf16 before the dot
W_BF16, W_FP8, W_FP8_DEQ = 0, 1, 2


def build(force: bool = False) -> Path:
    if force or not LIB.exists() or LIB.stat().st_mtime < (HERE / "mk_oracle.c").stat().st_mtime:
        subprocess.run(["make", "-s", "-C", str(HERE)] + (["-B"] if force else []), check=True)
    return LIB


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        L = C.CDLL(str(LIB))
        u16p, f32p, i32p, u8p = (np.ctypeslib.ndpointer(t, flags="C_CONTIGUOUS")
                                 for t in (np.uint16, np.float32, np.int32, np.uint8))
        sig = {
            "orc_splitmix64": (C.c_uint64, [C.c_uint64, C.c_uint64]),
            "orc_stream_key": (C.c_uint64, [C.c_uint64, C.c_uint64]),
            "orc_stream_id": (C.c_uint64, [C.c_int, C.c_int, C.c_int]),
            "orc_expf": (C.c_float, [C.c_float]),
            "orc_logf": (C.c_float, [C.c_float]),
            "orc_silu": (C.c_float, [C.c_float]),
            "orc_sincos_q": (None, [C.c_float, C.POINTER(C.c_float), C.POINTER(C.c_float)]),
            "orc_gen_normal_bf16": (None, [C.c_uint64, C.c_uint64, C.c_uint64, C.c_uint64, C.c_float, u16p]),
            "orc_gen_normal_f32": (None, [C.c_uint64, C.c_uint64, C.c_uint64, C.c_uint64, f32p]),
            "orc_gen_tokens": (None, [C.c_uint64, C.c_uint64, C.c_uint64, C.c_uint32, i32p]),
            "orc_dot64": (C.c_float, [u16p, f32p, C.c_int]),
            "orc_dot64_q": (C.c_float, [u8p, f32p, C.c_int]),
            "orc_dot64f": (C.c_float, [f32p, f32p, C.c_int]),
            "orc_mfma_bf16_k32": (C.c_float, [C.c_float, u16p, u16p]),
            "orc_mfma_bf16_chain": (C.c_float, [C.c_float, u16p, u16p, C.c_int]),
            "orc_mfma_tile_dot": (C.c_float, [f32p, f32p, C.c_int]),
            "orc_mfma_proj_dot": (C.c_float, [f32p, f32p, C.c_int, C.c_int]),
            "orc_mfma_down_dot": (C.c_float, [f32p, f32p, C.c_int, C.c_int]),
            "orc_e4m3_to_f32": (C.c_float, [C.c_uint8]),
            "orc_f32_to_e4m3": (C.c_uint8, [C.c_float]),
            "orc_quantize_rows": (None, [u16p, C.c_int64, C.c_int, u8p, f32p]),
            "orc_weight_q": (C.POINTER(C.c_uint8), [C.c_void_p, C.c_int, C.c_int, C.c_int]),
            "orc_yarn_tables": (None, [C.c_void_p, C.c_int, f32p, f32p]),
            "orc_rope_ds": (None, [f32p, C.c_int, f32p, f32p, f32p]),
            "orc_attn_scale": (C.c_float, [C.c_void_p]),
            "orc_route_ds": (None, [f32p, C.c_int, C.c_int, C.c_int, C.c_float, i32p, f32p]),
            "orc_weight_scale": (C.POINTER(C.c_float), [C.c_void_p, C.c_int, C.c_int, C.c_int]),
            "orc_sum64": (C.c_float, [f32p, C.c_int]),
            "orc_rmsnorm": (None, [f32p, C.c_void_p, C.c_int, C.c_float, f32p]),
            "orc_rope_tables": (None, [C.c_float, C.c_int, C.c_int, f32p, f32p]),
            "orc_apply_rope": (None, [f32p, C.c_int, f32p, f32p]),
            "orc_attention_head": (None, [f32p, u16p, u16p, i32p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, f32p]),
            "orc_route": (None, [f32p, C.c_int, C.c_int, C.c_int, i32p, f32p]),
            "orc_kv_k_index": (C.c_int64, [C.c_int] * 7),
            "orc_kv_v_index": (C.c_int64, [C.c_int] * 7),
            "orc_model_create": (C.c_void_p, [C.POINTER(OrcConfig), C.c_uint64, C.c_float]),
            "orc_model_destroy": (None, [C.c_void_p]),
            "orc_set_block_table": (None, [C.c_void_p, i32p, C.c_int]),
            "orc_num_blocks": (C.c_int, [C.c_void_p]),
            "orc_blocks_per_seq": (C.c_int, [C.c_void_p]),
            "orc_fill_kv_random_seq": (None, [C.c_void_p, C.c_int, C.c_int]),
            "orc_step_seq": (C.c_int32, [C.c_void_p, C.c_int, C.c_int32, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p]),
            "orc_layer_step_seq": (None, [C.c_void_p, C.c_int, C.c_int, f32p, C.c_int, C.c_void_p, C.c_void_p,
                                          C.c_void_p]),
            "orc_kcache": (C.POINTER(C.c_uint16), [C.c_void_p, C.c_int]),
            "orc_vcache": (C.POINTER(C.c_uint16), [C.c_void_p, C.c_int]),
            "orc_fill_kv_random": (None, [C.c_void_p, C.c_int]),
            "orc_step": (C.c_int32, [C.c_void_p, C.c_int32, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p]),
            "orc_layer_step": (None, [C.c_void_p, C.c_int, f32p, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p]),
            "orc_weight": (C.POINTER(C.c_uint16), [C.c_void_p, C.c_int, C.c_int, C.c_int]),
            "orc_num_threads": (C.c_int, []),
            "orc_materialize_experts": (None, [C.c_void_p]),
            "orc_prefill_seq": (C.c_int, [C.c_void_p, C.c_int, i32p, C.c_int, C.c_int, i32p]),
            "orc_step_rows": (C.c_int, [C.c_void_p, C.c_int, i32p, i32p, i32p, i32p, C.c_void_p, C.c_void_p,
                                        C.c_void_p]),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype, f.argtypes = res, args
        _lib = L
    return _lib


# ---------------------------------------------------------------- element helpers
def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(np.asarray(x, np.float32)).view(np.uint32)
    return ((u + np.uint32(0x7FFF) + ((u >> 16) & np.uint32(1))) >> 16).astype(np.uint16)


def stream_id(kind: int, layer: int, expert: int = 0) -> int:
    return (kind << 48) | ((layer + 1) << 24) | expert


def gen_normal_bf16(seed: int, stream: int, n: int, start: int = 0, scale: float = 0.02) -> np.ndarray:
    out = np.empty(n, np.uint16)
    lib().orc_gen_normal_bf16(seed, stream, start, n, scale, out)
    return out


def gen_normal_f32(seed: int, stream: int, n: int, start: int = 0) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_gen_normal_f32(seed, stream, start, n, out)
    return out


def gen_tokens(seed: int, n: int, bound: int, stream: int | None = None) -> np.ndarray:
    out = np.empty(n, np.int32)
    lib().orc_gen_tokens(seed, stream_id(S_PROMPT, -1) if stream is None else stream, n, bound, out)
    return out


def dot64(w_bits: np.ndarray, x: np.ndarray) -> float:
    return float(lib().orc_dot64(np.ascontiguousarray(w_bits, np.uint16), np.ascontiguousarray(x, np.float32), len(x)))


def rmsnorm(x: np.ndarray, eps: float, w_bits: np.ndarray | None = None) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    wp = None if w_bits is None else np.ascontiguousarray(w_bits, np.uint16).ctypes.data
    lib().orc_rmsnorm(x, wp, len(x), eps, out)
    return out


def rope_tables(theta: float, hd: int, ctx: int):
    c = np.empty((ctx, hd // 2), np.float32)
    s = np.empty((ctx, hd // 2), np.float32)
    lib().orc_rope_tables(theta, hd, ctx, c, s)
    return c, s


def apply_rope(v: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    v = np.array(v, np.float32)
    lib().orc_apply_rope(v, len(v), np.ascontiguousarray(cos, np.float32), np.ascontiguousarray(sin, np.float32))
    return v


def route(logits: np.ndarray, k: int, renorm: bool):
    logits = np.ascontiguousarray(logits, np.float32)
    ids = np.empty(k, np.int32)
    w = np.empty(k, np.float32)
    lib().orc_route(logits, len(logits), k, int(renorm), ids, w)
    return ids, w


def attention_head(q, kc, vc, btab, n, h, NKV, HD, BS):
    o = np.empty(HD, np.float32)
    lib().orc_attention_head(np.ascontiguousarray(q, np.float32), np.ascontiguousarray(kc, np.uint16),
                             np.ascontiguousarray(vc, np.uint16), np.ascontiguousarray(btab, np.int32),
                             n, h, NKV, HD, BS, o)
    return o


# ---------------------------------------------------------------- model
class OracleModel:
    """Seeded random-init decoder held on the CPU; step() is ref_numpy.py's Ref.step."""

    def __init__(self, cfg: dict, seed: int, wscale: float = 0.02):
        self.cfg = dict(cfg)
        c = OrcConfig(**{k: cfg.get(k, 0) for k, _ in OrcConfig._fields_})
        self._h = lib().orc_model_create(C.byref(c), seed, wscale)
        if not self._h:
            raise MemoryError("oracle model allocation failed")

    def close(self):
        if self._h:
            lib().orc_model_destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def set_block_table(self, bt):
        """bt: one sequence's table, or [batch][blocks per sequence] (flattened row by row)."""
        bt = np.ascontiguousarray(np.asarray(bt, np.int32).reshape(-1))
        lib().orc_set_block_table(self._h, bt, len(bt))

    @property
    def num_blocks(self) -> int:
        return lib().orc_num_blocks(self._h)

    @property
    def blocks_per_seq(self) -> int:
        return lib().orc_blocks_per_seq(self._h)

    def fill_kv_random(self, n: int, seq: int = 0):
        lib().orc_fill_kv_random_seq(self._h, int(seq), int(n))

    def kv(self, layer: int):
        """(K, V) of one layer's paged pool, flat; DeepSeek-V2: (latent cache [blk][CD/8][BS][8], None)."""
        c = self.cfg
        if c.get("arch", 0) == ARCH_DSV2:
            n = self.num_blocks * c["block_size"] * (c["kv_lora"] + c["qk_rope"])
            return np.ctypeslib.as_array(lib().orc_kcache(self._h, layer), shape=(n,)).copy(), None
        n = self.num_blocks * c["block_size"] * c["NKV"] * c["HD"]
        k = np.ctypeslib.as_array(lib().orc_kcache(self._h, layer), shape=(n,)).copy()
        v = np.ctypeslib.as_array(lib().orc_vcache(self._h, layer), shape=(n,)).copy()
        return k, v

    def weight(self, kind: int, layer: int = -1, expert: int = 0, shape=None) -> np.ndarray:
        c = self.cfg
        H, NQKV = c["H"], (c["NH"] + 2 * c["NKV"]) * c["HD"]
        shapes = {S_EMBED: (c["V"], H), S_LMHEAD: (c["V"], H), S_WQKV: (NQKV, H), S_WO: (H, c["NH"] * c["HD"]),
                  S_ROUTER: (c["E"], H), S_W13: (2 * c["MI"], H), S_W2: (H, c["MI"]),
                  S_WGU: (2 * c["I"], H), S_WD: (H, c["I"])}
        if c.get("arch", 0) == ARCH_DSV2:
            NH, QD, KVL, R = c["NH"], c["qk_nope"] + c["qk_rope"], c["kv_lora"], c["qk_rope"]
            SI = c["n_shared"] * c["MI"]
            shapes.update({S_WQKV: (NH * QD + KVL + R, H), S_WO: (H, NH * c["v_head"]),
                           S_WKVB: (NH * (c["qk_nope"] + c["v_head"]), KVL), S_WSGU: (2 * SI, H), S_WSD: (H, SI),
                           S_WGU: (2 * c["dense_I"], H), S_WD: (H, c["dense_I"])})
        shp = shape or shapes[kind]
        p = lib().orc_weight(self._h, kind, layer, expert)
        return np.ctypeslib.as_array(p, shape=(int(np.prod(shp)),)).reshape(shp).copy()

    @property
    def attn_scale(self) -> float:
        return float(lib().orc_attn_scale(self._h))

    def weight_fp8(self, kind: int, layer: int = -1, expert: int = 0):
        """(e4m3 codes [rows][cols] uint8, per-row scales [rows] fp32) of a matrix the model holds as fp8."""
        c = self.cfg
        H, NQKV = c["H"], (c["NH"] + 2 * c["NKV"]) * c["HD"]
        shapes = {S_WQKV: (NQKV, H), S_WO: (H, c["NH"] * c["HD"]), S_W13: (2 * c["MI"], H), S_W2: (H, c["MI"]),
                  S_WGU: (2 * c["I"], H), S_WD: (H, c["I"])}
        R, K = shapes[kind]
        q = lib().orc_weight_q(self._h, kind, layer, expert)
        sc = lib().orc_weight_scale(self._h, kind, layer, expert)
        if not q or not sc:
            raise ValueError(f"tensor kind {kind} is not held as fp8")
        return (np.ctypeslib.as_array(q, shape=(R * K,)).reshape(R, K).copy(),
                np.ctypeslib.as_array(sc, shape=(R,)).copy())

    def step(self, tok: int, pos: int, dump: bool = False, seq: int = 0):
        """Sequence `seq`'s decode step (a batched step is one call per sequence: they share only weights)."""
        c = self.cfg
        if not dump:
            return int(lib().orc_step_seq(self._h, int(seq), int(tok), int(pos), None, None, None))
        x = np.empty((c["L"], c["H"]), np.float32)
        k = max(c["TOPK"], 1)
        ids = np.zeros((c["L"], k), np.int32)
        w = np.zeros((c["L"], k), np.float32)
        t = int(lib().orc_step_seq(self._h, int(seq), int(tok), int(pos), x.ctypes.data, ids.ctypes.data,
                                   w.ctypes.data))
        return t, x, ids, w

    def materialize_experts(self):
        lib().orc_materialize_experts(self._h)

    def step_rows(self, seqs, tokens, positions, dump: bool = False):
        """Rows of decode steps computed together, every weight row read once for all of them (Qwen3 architecture):
        row r is sequence seqs[r]'s step with token tokens[r] at position positions[r].  Rows of distinct sequences
        are one batched step; each row's result equals step(tokens[r], positions[r], seq=seqs[r]).  Returns the
        greedy tokens [n], and with dump the residuals [n][L][H], top-k ids and weights [n][L][TOPK]."""
        c = self.cfg
        sq = np.ascontiguousarray(np.asarray(seqs, np.int32).reshape(-1))
        tk = np.ascontiguousarray(np.asarray(tokens, np.int32).reshape(-1))
        ps = np.ascontiguousarray(np.asarray(positions, np.int32).reshape(-1))
        n = len(sq)
        if len(tk) != n or len(ps) != n or n < 1:
            raise ValueError("step_rows needs one sequence, token and position per row")
        out = np.zeros(n, np.int32)
        k = max(c["TOPK"], 1)
        x = np.empty((n, c["L"], c["H"]), np.float32) if dump else None
        ids = np.zeros((n, c["L"], k), np.int32) if dump else None
        w = np.zeros((n, c["L"], k), np.float32) if dump else None
        ptr = (lambda a: a.ctypes.data if a is not None else None)
        if lib().orc_step_rows(self._h, n, sq, tk, ps, out, ptr(x), ptr(ids), ptr(w)) != 0:
            raise ValueError("oracle step_rows refused (architecture, sequence, position or token out of range)")
        return (out, x, ids, w) if dump else out

    def prefill(self, tokens, pos0: int, seq: int = 0) -> np.ndarray:
        """Positions pos0 .. pos0+n-1 of sequence `seq` with input tokens `tokens` (n of them), computed with every
        weight row read once for the n positions: the KV cache afterwards and the returned greedy token of every
        position equal n step() calls (Qwen3 architecture)."""
        toks = np.ascontiguousarray(np.asarray(tokens, np.int32).reshape(-1))
        out = np.zeros(len(toks), np.int32)
        if lib().orc_prefill_seq(self._h, int(seq), toks, int(pos0), len(toks), out) != 0:
            raise ValueError(f"oracle prefill of {len(toks)} positions at {pos0} refused")
        return out

    def layer_step(self, layer: int, x: np.ndarray, pos: int, seq: int = 0):
        c = self.cfg
        x = np.array(x, np.float32)
        k = max(c["TOPK"], 1)
        ids = np.zeros(k, np.int32)
        w = np.zeros(k, np.float32)
        lg = np.zeros(max(c["E"], 1), np.float32)
        lib().orc_layer_step_seq(self._h, int(seq), layer, x, pos, ids.ctypes.data, w.ctypes.data, lg.ctypes.data)
        return x, ids, w, lg


def yarn_tables(cfg: dict, ctx: int):
    """The oracle's fp32 yarn cos / sin tables [ctx][qk_rope / 2] of a DeepSeek-V2 configuration."""
    c = OrcConfig(**{k: cfg.get(k, 0) for k, _ in OrcConfig._fields_})
    half = cfg["qk_rope"] // 2
    cs, sn = np.zeros(ctx * half, np.float32), np.zeros(ctx * half, np.float32)
    lib().orc_yarn_tables(C.addressof(c), ctx, cs, sn)
    return cs.reshape(ctx, half), sn.reshape(ctx, half)


def rope_ds(x: np.ndarray, cs: np.ndarray, sn: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros_like(x)
    lib().orc_rope_ds(x, len(x), np.ascontiguousarray(cs, np.float32), np.ascontiguousarray(sn, np.float32), out)
    return out


def num_threads() -> int:
    return int(lib().orc_num_threads())


def env_threads() -> int:
    return int(os.environ.get("OMP_NUM_THREADS", "0")) or num_threads()
