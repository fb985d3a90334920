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


def word_sum(t) -> int:
    """Sum of a device tensor's 32-bit words mod 2^32 (what the stream kernel's sinks add up to)."""
    import torch
    w = t.view(torch.int32).reshape(-1)
    total = 0
    step = 1 << 26
    for i in range(0, w.numel(), step):
        total += int((w[i:i + step].to(torch.int64) & 0xFFFFFFFF).sum().item())
    return total & 0xFFFFFFFF
