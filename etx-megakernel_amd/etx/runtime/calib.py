"""Bindings of libetxmk_calib.so: the grid barrier of the persistent decode kernels timed alone, and the HBM read
bandwidth of their streaming load pattern (non-temporal 1 KiB-per-wave loads) at several loads in flight per wave.
These are the two machine figures the decode step's time is built from (barriers x barrier cost + weight bytes /
streaming bandwidth); they are measured, not taken from a data sheet."""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parents[2] / "lib" / "libetxmk_calib.so"
BAR_WORDS = 17 * 64                       # 8 group counters, the global counter, 8 release flags (a 256 B line each)

_lib = None


def load():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built (python etx-megakernel_amd/build_lib.py)")
        lib = C.CDLL(str(LIB_PATH))
        lib.etxmk_calib_barrier.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_void_p]
        lib.etxmk_calib_barrier.restype = C.c_int
        lib.etxmk_calib_stream.argtypes = [C.c_void_p, C.c_size_t, C.c_int, C.c_int, C.c_void_p, C.c_void_p]
        lib.etxmk_calib_stream.restype = C.c_int
        lib.etxmk_calib_mfma_bf16.argtypes = [C.c_void_p] * 4 + [C.c_int, C.c_int, C.c_void_p]
        lib.etxmk_calib_mfma_bf16.restype = C.c_int
        lib.etxmk_calib_stream_tiles.argtypes = [C.c_void_p] + [C.c_int] * 5 + [C.c_void_p, C.c_void_p]
        lib.etxmk_calib_stream_tiles.restype = C.c_int
        _lib = lib
    return _lib


def _stream(torch, dev):
    return C.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def barrier(nwg: int, iters: int, device="cuda:0"):
    """One cooperative launch of `nwg` workgroups running `iters` grid barriers back to back.  Returns
    (microseconds per barrier, the barrier words after the launch, the abort word)."""
    import torch
    lib = load()
    dev = torch.device(device)
    bar = torch.zeros(BAR_WORDS, dtype=torch.int32, device=dev)
    ab = torch.zeros(1, dtype=torch.int32, device=dev)
    st = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    rc = lib.etxmk_calib_barrier(C.c_void_p(bar.data_ptr()), C.c_void_p(ab.data_ptr()), int(nwg), int(iters),
                                 _stream(torch, dev))
    if rc != 0:
        raise RuntimeError(f"etxmk_calib_barrier: HIP error {rc}")
    e1.record(st)
    e1.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / max(iters, 1)
    return us, bar.cpu().numpy().view("uint32"), int(ab.item())


def stream(src, inflight: int, nwg: int):
    """One streaming read of the device tensor `src` (a multiple of 1 KiB).  Returns (seconds, the per-thread sums
    of the words read, mod 2^32)."""
    import torch
    lib = load()
    dev = src.device
    sink = torch.empty(nwg * 512, dtype=torch.int32, device=dev)
    st = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    rc = lib.etxmk_calib_stream(C.c_void_p(src.data_ptr()), src.numel() * src.element_size(), int(inflight),
                                int(nwg), C.c_void_p(sink.data_ptr()), _stream(torch, dev))
    if rc != 0:
        raise RuntimeError(f"etxmk_calib_stream: HIP error {rc}")
    e1.record(st)
    e1.synchronize()
    return e0.elapsed_time(e1) * 1e-3, sink


def stream_tiles(src, row_bytes: int, nblk: int, inflight: int, nwg: int):
    """One read of the device tensor `src` as tiles of 16 rows of `row_bytes` (nblk blocks of 1024 bytes each) with
    the matrix-core tiles' load pattern (a load: 64 bytes of each of 16 rows), 1 or 2 blocks of 16 KB per wave in
    flight.  Returns (seconds, the bytes of the blocks read, the per-thread sums of the words read)."""
    import torch
    lib = load()
    dev = src.device
    nbytes = src.numel() * src.element_size()
    ntile = nbytes // (16 * row_bytes)
    sink = torch.empty(nwg * 512, dtype=torch.int32, device=dev)
    st = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    rc = lib.etxmk_calib_stream_tiles(C.c_void_p(src.data_ptr()), int(ntile), int(nblk), int(row_bytes), int(inflight),
                                      int(nwg), C.c_void_p(sink.data_ptr()), _stream(torch, dev))
    if rc != 0:
        raise RuntimeError(f"etxmk_calib_stream_tiles: HIP error {rc}")
    e1.record(st)
    e1.synchronize()
    return e0.elapsed_time(e1) * 1e-3, ntile * 16 * nblk * 1024, sink


def word_sum(t) -> int:
    """Sum of a device tensor's 32-bit words mod 2^32 (what the stream kernel's sinks add up to)."""
    import torch
    w = t.view(torch.int32).reshape(-1)
    total = 0
    step = 1 << 26
    for i in range(0, w.numel(), step):
        total += int((w[i:i + step].to(torch.int64) & 0xFFFFFFFF).sum().item())
    return total & 0xFFFFFFFF


def mfma_bf16(a_bits, b_bits, c, device="cuda:0"):
    """D = C + A B through chained v_mfma_f32_16x16x32_bf16, one wave per case: a_bits [n][16][32 s] and b_bits
    [n][32 s][16] bf16 bit patterns (uint16), c [n][16][16] fp32; returns D [n][16][16] fp32.  Step i takes k in
    [32 i, 32 i + 32); within a step, lane l holds A row l % 16 and B column l % 16 at k = 8 (l // 16) .. + 7, and
    D rows 4 (l // 16) .. + 3 of column l % 16."""
    import numpy as np
    import torch
    lib = load()
    a_bits = np.asarray(a_bits, np.uint16); b_bits = np.asarray(b_bits, np.uint16); c = np.asarray(c, np.float32)
    n, K = a_bits.shape[0], a_bits.shape[2]
    if a_bits.shape != (n, 16, K) or b_bits.shape != (n, K, 16) or c.shape != (n, 16, 16) or K % 32:
        raise ValueError("shapes: a [n][16][32 s], b [n][32 s][16], c [n][16][16]")
    steps = K // 32
    lane = np.arange(64)
    row, quad = lane % 16, lane // 16
    # k index of lane l, step s, element j: 32 s + 8 quad + j
    k = (32 * np.arange(steps)[None, :, None] + 8 * quad[:, None, None] + np.arange(8)[None, None, :])   # [64][s][8]
    a = a_bits[:, row[:, None, None], k]                     # [n][64][s][8]
    b = np.transpose(b_bits, (0, 2, 1))[:, row[:, None, None], k]
    cr = c[:, 4 * quad[:, None] + np.arange(4)[None, :], row[:, None]]       # [n][64][4]
    dev = torch.device(device)
    ta = torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(dev)
    tb = torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).to(dev)
    tc = torch.from_numpy(np.ascontiguousarray(cr)).to(dev)
    td = torch.empty_like(tc)
    rc = lib.etxmk_calib_mfma_bf16(C.c_void_p(ta.data_ptr()), C.c_void_p(tb.data_ptr()), C.c_void_p(tc.data_ptr()),
                                   C.c_void_p(td.data_ptr()), n, steps, _stream(torch, dev))
    if rc != 0:
        raise RuntimeError(f"etxmk_calib_mfma_bf16: HIP error {rc}")
    torch.cuda.synchronize(dev)
    dr = td.cpu().numpy()
    D = np.zeros((n, 16, 16), np.float32)
    D[:, 4 * quad[:, None] + np.arange(4)[None, :], row[:, None]] = dr
    return D
