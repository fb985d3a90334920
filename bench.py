#!/usr/bin/env python3
"""Headline benchmark: Qwen3-30B-A3B-shaped bf16 decode at batch 1 on one MI355X.

    python bench.py [--gpus 1] [--steps 32] [--warmup 4] [--ctx 1024] [--no-cpu] [--unfused]
    python bench.py --batch 16 [--ctx-lo 512 --ctx-hi 4096]      (batched step; not the headline line)
    python bench.py --model deepseek-v2-lite --batch 4 --ctx-lo 512 --ctx-hi 2048   (BASELINE.json configs[3])

Setup (untimed): seeded random-init weights N(0, 0.02) in HBM, a prompt of `ctx` seeded random token ids fed
token by token through the decode step (as examples/llm/host.hip:203-213 does), then `warmup` greedy steps.
Timed: `steps` greedy decode steps (one persistent megakernel launch each), bracketed by synchronisation and
HIP events on the launch stream.  One JSON line on stdout; progress on stderr.

Bytes per token follow the reference's ledger rules (etx/models/vllm_llm/byte_ledger.py:121-178): every
non-expert weight once, the TOPK active experts, the KV cache read over the context plus one position written.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (str(ROOT), str(ROOT / "etx-megakernel_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "decode ms/token at batch 1, Qwen3-30B-A3B shape; achieved HBM GB/s vs peak"
HBM_PEAK_GBPS = 8000.0
REFERENCE_MI300X_MS = 4.087415          # docs/qwen/QWEN-BATCH-BASELINE-2026-10-18.md:17 (MI300X, not comparable hardware)
METRIC_8B = "decode ms/token at batch 1, Qwen3-8B shape; achieved HBM GB/s vs peak"
REFERENCE_MI300X_8B_TILES_MS = 10.07    # README.md:140-146: the generic hand-written tiles at context 1024 (MI300X)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def mat_bytes(cfg, rows: int, cols: int) -> int:
    """Algorithmic bytes of a rows x cols matrix of the model's weight type: bf16, or fp8 codes plus one fp32 scale
    per row."""
    return rows * (cols + 4) if cfg.wdtype else rows * cols * 2


def bytes_per_token(cfg, context: int) -> dict:
    """Algorithmic HBM bytes of one decode step at `context` cached positions."""
    H, HD, NH, NKV, V = cfg.H, cfg.HD, cfg.NH, cfg.NKV, cfg.V
    bf = 2
    glob = (H + H + V * H) * bf                     # embedding row, final norm, lm_head
    layer = (2 * H + 2 * HD) * bf                   # ln1, ln2, q/k norm
    layer += mat_bytes(cfg, (NH + 2 * NKV) * HD, H) + mat_bytes(cfg, H, NH * HD)
    if cfg.moe:
        layer += cfg.E * H * bf + cfg.TOPK * (mat_bytes(cfg, 2 * cfg.MI, H) + mat_bytes(cfg, H, cfg.MI))
    else:
        layer += mat_bytes(cfg, 2 * cfg.I, H) + mat_bytes(cfg, H, cfg.I)
    kv_pos = 2 * NKV * HD * bf
    kv = cfg.L * (context * kv_pos + kv_pos)
    weights = glob + cfg.L * layer
    return {"weights": weights, "kv": kv, "total": weights + kv}


def bytes_per_step_ds(cfg, contexts, union) -> dict:
    """DeepSeek-V2 step (the ledger of BASELINE.json configs[3]): every attention weight once (q_proj and
    kv_a rows, kv_b_proj, o_proj, norms), the dense layers' MLP, the MoE layers' router and shared experts once and
    their distinct routed experts once (union[l], measured), the latent cache read over each context plus one row
    written, one embedding row per sequence, lm_head."""
    H, V, NH, bf = cfg.H, cfg.V, cfg.NH, 2
    B = len(contexts)
    glob = (B * H + H + V * H) * bf
    attn = (2 * H + cfg.kv_lora) * bf + cfg.nqkv * H * bf + NH * (cfg.qk_nope + cfg.v_head) * cfg.kv_lora * bf \
        + H * NH * cfg.v_head * bf
    dense = 3 * cfg.dense_I * H * bf
    SI = cfg.n_shared * cfg.MI
    moe = cfg.E * H * bf + 3 * SI * H * bf
    expert = 3 * cfg.MI * H * bf
    weights = glob + cfg.L * attn + cfg.first_dense * dense + (cfg.L - cfg.first_dense) * moe \
        + sum(int(u) * expert for u in union[cfg.first_dense:])
    row = (cfg.kv_lora + cfg.qk_rope) * bf
    kv = cfg.L * sum((int(c) + 1) * row for c in contexts)
    return {"weights": weights, "kv": kv, "total": weights + kv}


def bytes_per_step(cfg, contexts, union) -> dict:
    """Algorithmic HBM bytes of one batched step: every non-expert weight once, each layer's distinct routed experts
    once (union[l], measured), each sequence's KV read over its context plus one position written, one embedding
    row per sequence (byte_ledger.py:121-178 rules with the expert union of a batch)."""
    from etx.runtime import native as N
    if cfg.arch == N.ARCH_DSV2:
        return bytes_per_step_ds(cfg, contexts, union)
    H, HD, NH, NKV, V = cfg.H, cfg.HD, cfg.NH, cfg.NKV, cfg.V
    bf = 2
    B = len(contexts)
    glob = (B * H + H + V * H) * bf
    layer = (2 * H + 2 * HD) * bf + mat_bytes(cfg, (NH + 2 * NKV) * HD, H) + mat_bytes(cfg, H, NH * HD)
    experts = 0
    if cfg.moe:
        layer += cfg.E * H * bf
        experts = sum(int(u) * (mat_bytes(cfg, 2 * cfg.MI, H) + mat_bytes(cfg, H, cfg.MI)) for u in union)
    else:
        layer += mat_bytes(cfg, 2 * cfg.I, H) + mat_bytes(cfg, H, cfg.I)
    kv_pos = 2 * NKV * HD * bf
    kv = cfg.L * sum((int(c) + 1) * kv_pos for c in contexts)
    weights = glob + cfg.L * layer + experts
    return {"weights": weights, "kv": kv, "total": weights + kv}


def main_batch(a):
    """Batched decode (BASELINE.json configs[4] shape with bf16 weights): `batch` sequences with per-sequence contexts
    drawn uniform in [ctx_lo, ctx_hi] (seeded N(0,1) KV; the reference prefills by decoding), one seeded token each,
    `warmup` then `steps` batched greedy steps (one persistent launch each)."""
    import torch
    from etx.runtime import native as N
    from etx.models import configs
    B = a.batch
    ds = a.model == "deepseek-v2-lite"
    rng = np.random.default_rng(a.seed + 4)
    ctx = rng.integers(a.ctx_lo, a.ctx_hi + 1, B).astype(np.int32)
    max_ctx = int(ctx.max()) + a.warmup + a.steps + 2
    base = configs.DEEPSEEK_V2_LITE if ds else configs.QWEN3_30B_A3B
    cfg = configs.with_layers(base, base.L, batch=B, max_ctx=max_ctx, wdtype=N.W_FP8 if a.fp8 else N.W_BF16)
    wname = "fp8 e4m3 (per-row scales; router, embedding, lm_head bf16)" if a.fp8 else "bf16"
    dev = torch.device("cuda:0")
    if a.calib_copy:
        calib_copy(dev)
    t0 = time.time()
    dec = N.Decoder(cfg, device="cuda:0", workgroups=a.workgroups)
    dec.init_weights(a.seed, 0.02)
    first = rng.integers(0, cfg.V, B).astype(np.int32)
    for b in range(B):
        dec.fill_kv_seeded(a.seed, int(ctx[b]), seq=b)
        row = np.zeros(int(ctx[b]) + 1, np.int32)
        row[-1] = first[b]
        dec.set_tokens(row, seq=b)
    dec.sync()
    log(f"[gpu] batch {B}: weights {dec.sizes['weights'] / 1e9:.2f} GB, KV pool {dec.sizes['kv'] / 1e9:.2f} GB, "
        f"contexts {list(ctx)} ready in {time.time() - t0:.1f}s")
    pos = ctx.copy()
    for _ in range(a.warmup):
        dec.step_batch(pos)
        pos += 1
    dec.sync()
    stream = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    first_timed = pos.copy()
    w0 = time.perf_counter()
    e0.record(stream)
    for _ in range(a.steps):
        dec.step_batch(pos)
        pos += 1
    e1.record(stream)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - w0) * 1e3
    dec.sync()
    ms = e0.elapsed_time(e1) / a.steps
    # distinct routed experts per layer, from one more (untimed) step with the routing dumps on
    dec.enable_dumps(True)
    dec.step_batch(pos)
    pos += 1
    d = dec.dumps()
    dec.enable_dumps(False)
    phase_us = None
    if a.trace:
        dec.enable_trace(True)
        dec.step_batch(pos)
        pos += 1
        t = dec.trace()
        dec.enable_trace(False)
        if a.trace_out:
            np.save(a.trace_out, t)
        phase_us = trace_summary(t, cfg)
    union = [len(np.unique(d["ids"][l])) if l >= cfg.first_dense else 0 for l in range(cfg.L)]
    mean_ctx = (first_timed + pos - 1) / 2.0
    by = bytes_per_step(cfg, np.round(mean_ctx).astype(int), union)
    gbps = by["total"] / (ms * 1e-3) / 1e9
    umean = float(np.mean(union[cfg.first_dense:]))
    log(f"[gpu] {a.steps} batched steps: {ms:.4f} ms/step ({ms / B:.4f} ms/token, {B * 1e3 / ms:.1f} tokens/s), "
        f"{gbps:.1f} GB/s = {gbps / HBM_PEAK_GBPS:.3f} of 8 TB/s; expert union per MoE layer mean {umean:.1f}")
    shape = "DeepSeek-V2-Lite" if ds else "Qwen3-30B-A3B"
    if ds:
        workload = (f"{a.model} decode, batch {B}, bf16 weights, multi-head latent attention over a paged latent "
                    f"cache, contexts uniform in [{a.ctx_lo}, {a.ctx_hi}], greedy (BASELINE.json configs[3])")
    else:
        workload = (f"{a.model} decode, batch {B}, {wname} weights, contexts uniform in [{a.ctx_lo}, {a.ctx_hi}], "
                    f"greedy" + (" (BASELINE.json configs[4])" if a.fp8 else " (configs[4] shape with bf16 weights)"))
    out = {
        "metric": f"decode ms/step at batch {B}, {shape} shape; tokens/s; achieved HBM GB/s vs peak",
        "value": round(ms, 4), "unit": "ms/step", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(ms, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp8-e4m3 weights x bf16 activations, fp32 accumulation" if a.fp8 else "bf16",
        "data": f"synthetic: seeded random-init weights N(0,0.02) ({wname}); per-sequence "
                f"{'latent cache' if ds else 'KV'} of seeded N(0,1) values",
        "config": {"workload": workload, "batch": B, "contexts": [int(c) for c in ctx], "layers": cfg.L, "experts": cfg.E,
                   "top_k": cfg.TOPK, "vocab": cfg.V, "mode": "fused megakernel", "seed": a.seed},
        "tokens_per_s": round(B * 1e3 / ms, 2), "ms_per_token": round(ms / B, 4),
        "host_wall_ms_per_step": round(wall / a.steps, 4), "expert_union_mean": round(umean, 2),
        "bytes_per_step": by["total"], "achieved_GBps": round(gbps, 1),
        "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": None,
                     "kernel": "etxmk_ds_b4*" if ds else "etxmk_fused_b*"},
        "cpu_baseline": None,
    }
    if phase_us:
        out["phase_us"] = phase_us
    if (a.ctx_lo, a.seed) == (512, 20261201):             # the workloads the counter passes were taken on
        if ds and B == 4 and a.ctx_hi == 2048:
            attach_traffic(out, "etxmk_ds_b4_deepseek-v2-lite_ctx512-2048_hbm_traffic.json")
        elif not ds and B == 16 and a.fp8 and a.ctx_hi == 4096:
            attach_traffic(out, "etxmk_fused_fp8_b16_qwen3-30b-a3b_ctx512-4096_hbm_traffic.json")
    dec.close()                                           # release the handle before the CPU leg and the exit
    del dec
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    if not a.no_cpu:
        try:
            out["cpu_baseline"] = cpu_baseline_batch(cfg, ctx, a.seed)
        except Exception as e:  # the baseline is reported, never gating
            log(f"[cpu] baseline failed: {e!r}")
    print(json.dumps(out), flush=True)


def calib_copy(dev):
    """A 1 GiB device-to-device copy: the known-size reference the HBM counter passes are scaled by."""
    import torch
    src = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    log("[gpu] calibration copy: 1 GiB read + 1 GiB written")


def calibrate(dev) -> dict:
    """The machine figures a decode step is built from, measured with the decode kernels' own code: the grid
    barrier (grid_arrive / grid_wait, one 512-thread workgroup per CU, 2000 back to back per cooperative launch,
    best of 3 launches) and the streaming read (non-temporal 1 KiB-per-wave loads over 4 GiB, 1 or 2 workgroups
    per CU, 1 to 16 loads in flight per wave, best of 3).  Every barrier launch is checked (no wait gave up, every
    counter at its final generation) and one stream pass is checked against a sum of the words it read."""
    import torch
    from etx.runtime import calib
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    iters = 2000
    calib.barrier(cus, 100, dev)                           # warm
    best = None
    for _ in range(3):
        us, bar, ab = calib.barrier(cus, iters, dev)
        if ab != 0 or int(bar[64 * 8]) != 8 * iters or any(int(bar[64 * (9 + j)]) != iters for j in range(8)):
            raise RuntimeError(f"barrier calibration: abort word {ab}, counters {bar[64 * 8]} / {bar[64 * 9]}")
        best = us if best is None else min(best, us)
    log(f"[gpu] grid barrier: {best:.3f} us ({cus} workgroups, {iters} per launch)")
    gib = 4
    src = torch.randint(-2**31, 2**31 - 1, (gib << 28,), dtype=torch.int32, device=dev)
    nbytes = src.numel() * 4
    want = calib.word_sum(src)
    rows = []
    for per_cu in (1, 2):
        for inflight in (1, 2, 4, 8, 16):
            calib.stream(src, inflight, per_cu * cus)
            t = min(calib.stream(src, inflight, per_cu * cus)[0] for _ in range(3))
            rows.append({"workgroups_per_cu": per_cu, "loads_in_flight_per_wave": inflight,
                         "GBps": round(nbytes / t / 1e9, 1)})
            log(f"[gpu] stream {per_cu} WG/CU, {inflight:2d} x 1 KiB per wave in flight: {rows[-1]['GBps']} GB/s")
    _, sink = calib.stream(src, 4, cus)
    got = calib.word_sum(sink)
    if got != want:
        raise RuntimeError(f"stream calibration read {got:#x}, words sum to {want:#x}")
    # the matrix-core tiles' pattern over the same words: 16 rows of 2064 bytes (an fp8 row of 2048 codes and its
    # scale), two 1 KiB blocks of each row, 64 bytes of each of 16 rows per load
    tiles = []
    for inflight in (1, 2):
        calib.stream_tiles(src, 2064, 2, inflight, cus)
        t, used, _ = min((calib.stream_tiles(src, 2064, 2, inflight, cus) for _ in range(3)), key=lambda r: r[0])
        tiles.append({"blocks_in_flight_per_wave": inflight, "GBps": round(used / t / 1e9, 1)})
        log(f"[gpu] tile stream, {inflight} x 16 KiB per wave in flight: {tiles[-1]['GBps']} GB/s")
    del src, sink
    return {"calibration": "gfx950 grid barrier and streaming read", "cus": cus,
            "barrier_us": round(best, 3), "barriers_per_launch": iters, "stream_bytes": nbytes,
            "stream": rows, "stream_checksum_ok": True, "tile_stream": tiles,
            "kernels": "etx-megakernel_amd/csrc/mk_calib.hip (grid_arrive/grid_wait of mk_device.h)"}


def attach_traffic(out, name):
    """HBM bytes per launch of this workload from its committed counter passes (rocprofv3 --pmc FETCH_SIZE and
    WRITE_SIZE of the same command, each scaled by that counter's reading for the calibration copy), if present."""
    tf = ROOT / "profiles" / name
    if tf.exists():
        t = json.loads(tf.read_text())
        out["roofline"]["traffic"] = t["traffic_bytes_per_launch"]
        out["roofline"]["traffic_source"] = f"profiles/{tf.name} (FETCH x{t['fetch_factor']}, WRITE x{t['write_factor']})"


def cpu_baseline(cfg, ctx: int, seed: int, reps: int = 5) -> dict:
    """The CPU oracle on a bounded sample of the same workload: the full-depth model (every layer, lm_head) with a
    seeded KV cache of `ctx` positions; one untimed step at position ctx generates the experts it routes to, then
    `reps` timed repeats of that step (each a whole decode step of the oracle: same token, same position, same
    routing)."""
    import numpy as np
    from oracle import oracle as O
    t0 = time.time()
    m = O.OracleModel(cfg.as_dict(), seed, 0.02)
    m.fill_kv_random(ctx)
    tok = int(O.gen_tokens(seed, 1, cfg.V)[0])
    m.step(tok, ctx)
    log(f"[cpu] oracle model ({cfg.L} layers) and its first step ready in {time.time() - t0:.1f}s "
        f"({O.num_threads()} threads)")
    t1 = time.time()
    for _ in range(reps):
        m.step(tok, ctx)
    ms = (time.time() - t1) / reps * 1e3
    m.close()
    import platform
    return {"value": round(ms, 3), "unit": "ms/token", "cores": O.num_threads(), "kind": "port",
            "sample": f"CPU oracle (C, OpenMP): {reps} full-depth decode steps ({cfg.L} layers + lm_head) at context "
                      f"{ctx}, timed after one untimed step of the same token and position "
                      f"({platform.processor() or platform.machine()})",
            "tokens_per_s": round(1e3 / ms, 3), "effective_GBps": round(bytes_per_token(cfg, ctx)["total"] / ms / 1e6, 2)}


def cpu_baseline_batch(cfg, contexts, seed: int, reps: int = 2) -> dict:
    """The CPU oracle's batched step on a bounded sample: the batch's rows (each sequence at its context, seeded KV)
    through slices of 2 and 4 layers plus lm_head (DeepSeek-V2: 2 and 3 layers, the dense layer first, one
    sequence at a time); per layer = the difference / the extra layers, head = the rest; ms/step = head + L x per
    layer."""
    import numpy as np
    from oracle import oracle as O
    from etx.models.configs import with_layers
    from etx.runtime import native as N
    ds = cfg.arch == N.ARCH_DSV2
    B = len(contexts)
    lo, hi = (2, 3) if ds else (2, 4)
    toks = [int(t) for t in O.gen_tokens(seed + 1, B, cfg.V)]
    times = {}
    for L in (lo, hi):
        m = O.OracleModel(with_layers(cfg, L).as_dict(), seed, 0.02)
        for b, c in enumerate(contexts):
            m.fill_kv_random(int(c), seq=b)

        def step():
            if ds:
                for b in range(B):
                    m.step(toks[b], int(contexts[b]), seq=b)
            else:
                m.step_rows(list(range(B)), toks, [int(c) for c in contexts])
        step()                                              # untimed: generates the routed experts
        t = time.time()
        for _ in range(reps):
            step()
        times[L] = (time.time() - t) / reps
        m.close()
    per_layer = (times[hi] - times[lo]) / (hi - lo)
    head = max(times[lo] - lo * per_layer, 0.0)
    ms = (head + cfg.L * per_layer) * 1e3
    import platform
    return {"value": round(ms, 3), "unit": "ms/step", "cores": O.num_threads(), "kind": "port",
            "sample": f"CPU oracle (C, OpenMP): the batch's {B} rows at their contexts through {lo}- and {hi}-layer "
                      f"slices + lm_head, {reps} timed steps each after an untimed one; ms/step = head + {cfg.L} x "
                      f"per-layer time ({platform.processor() or platform.machine()})",
            "ms_per_token": round(ms / B, 3), "tokens_per_s": round(B * 1e3 / ms, 3)}


def trace_summary(t, cfg):
    """Per-phase timeline of one traced step.  t[k][wg] = (wait for phase k's inputs returned, arrived after phase k,
    first weight loads issued (GEMV phases) / chunk partials issued (attention)), microseconds from the launch."""
    from etx.runtime import native as N
    per_layer = N.phase_names(cfg)[:-1]
    flat = [n for names_l in per_layer for n in names_l]
    names = list(dict.fromkeys(flat))
    nb = len(flat)
    end = np.nanmax(t[:, :, 1], axis=1)                   # phase k complete: last arrival
    span = np.diff(np.concatenate([[0.0], end[:nb + 1]]))
    idx = {n: np.array([k for k, m in enumerate(flat) if m == n]) for n in names}
    phase_us = {n: round(float(span[idx[n]].mean()), 2) for n in names}
    phase_us["head"] = round(float(span[nb]), 2)
    avg = lambda v: {n: round(float(np.nanmean(v[idx[n]])), 2) for n in names}
    lag = np.full(nb, np.nan)
    lag[1:] = np.nanmedian(t[1:nb, :, 0], axis=1) - end[:nb - 1]
    lagmax = np.full(nb, np.nan)
    lagmax[1:] = np.nanmax(t[1:nb, :, 0], axis=1) - end[:nb - 1]
    work = np.full(nb, np.nan)
    work[1:] = np.nanmedian(t[1:nb, :, 1] - t[1:nb, :, 0], axis=1)
    wmax = np.full(nb, np.nan)
    wmax[1:] = np.nanmax(t[1:nb, :, 1] - t[1:nb, :, 0], axis=1)
    s2 = np.full(nb, np.nan)
    s2[1:] = np.nanmedian(t[1:nb, :, 2] - t[1:nb, :, 0], axis=1)
    phase_us["barrier_median"] = round(float(np.nanmedian(lag)), 2)
    log(f"[gpu] traced step {end[-2]:.1f} us; per-layer phase spans (us) {phase_us}")
    log("[gpu] barrier (us), last arrival -> wait returned, median / last workgroup: "
        + str({n: (avg(lag)[n], avg(lagmax)[n]) for n in names}))
    log("[gpu] work after the wait (us), median / max workgroup: " + str({n: (avg(work)[n], avg(wmax)[n]) for n in names}))
    log("[gpu] slot 2 relative to the wait (us; GEMV: weight loads issued, negative = before; attention: partials "
        "issued): " + str(avg(s2)))
    return phase_us


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=32)
    ap.add_argument("--warmup", type=int, default=4)
    ap.add_argument("--ctx", type=int, default=1024)
    ap.add_argument("--seed", type=int, default=20261201)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--unfused", action="store_true")
    ap.add_argument("--graph", action="store_true",
                    help="with --unfused: capture one step's per-phase launches in a HIP graph and time replays of it "
                         "(each replay a whole step at the context the warmup ends on)")
    ap.add_argument("--workgroups", type=int, default=0)
    ap.add_argument("--trace", action="store_true", help="after timing, trace one fused step per phase (stderr)")
    ap.add_argument("--trace-out", default="", help="with --trace: also save the raw stamps (.npy)")
    ap.add_argument("--calibrate", action="store_true",
                    help="measure the grid barrier and the streaming read bandwidth (libetxmk_calib.so), print them "
                         "as one JSON line and exit")
    ap.add_argument("--calib-copy", action="store_true",
                    help="profiling runs: first copy 1 GiB device to device, the known-size reference for HBM counters")
    ap.add_argument("--kv-fill", action="store_true",
                    help="profiling runs: fill the KV cache with seeded N(0,1) instead of prefilling the prompt")
    ap.add_argument("--prefill-rows", type=int, default=16,
                    help="prompt positions per prefill launch (batched kernel); 0 or 1: one decode step per position")
    ap.add_argument("--batch", type=int, default=1, help="sequences per step (> 1: the batched step, not the headline)")
    ap.add_argument("--ctx-lo", type=int, default=512)
    ap.add_argument("--ctx-hi", type=int, default=0,
                    help="batched contexts' upper bound (default 4096; 2048 for deepseek-v2-lite, BASELINE configs[3])")
    ap.add_argument("--fp8", action="store_true", help="fp8 e4m3 weights with per-row scales (BASELINE.json configs[4])")
    ap.add_argument("--model", default="qwen3-30b-a3b", choices=["qwen3-30b-a3b", "qwen3-8b", "deepseek-v2-lite"],
                    help="qwen3-8b: the dense model of BASELINE.json configs[1] at batch 1; deepseek-v2-lite: the "
                         "batched multi-head latent attention step (configs[3])")
    a = ap.parse_args()
    if a.ctx_hi <= 0:
        a.ctx_hi = 2048 if a.model == "deepseek-v2-lite" else 4096
    if a.gpus != 1:
        print(f"bench.py: this build runs on exactly one GPU (asked for {a.gpus}); multi-GPU sharding is a design "
              f"note only", file=sys.stderr)
        sys.exit(2)
    if a.model == "qwen3-8b" and a.batch > 1:
        raise SystemExit("the Qwen3-8B workload (BASELINE.json configs[1]) is batch 1")
    if a.calibrate:
        import torch
        print(json.dumps(calibrate(torch.device("cuda:0"))), flush=True)
        return
    if a.graph and not a.unfused:
        raise SystemExit("--graph replays the unfused step; the persistent kernel's barrier generations advance per "
                         "launch and are not replayable")
    if a.batch > 1 or a.model == "deepseek-v2-lite":
        return main_batch(a)

    import numpy as np
    import torch
    from etx.runtime import native as N
    from etx.models import configs

    dense = a.model == "qwen3-8b"
    cfg = configs.QWEN3_8B if dense else configs.QWEN3_30B_A3B
    if a.fp8:
        if dense:
            raise SystemExit("fp8 weights are built for the Qwen3-30B-A3B shape (BASELINE.json configs[4])")
        cfg = configs.with_layers(cfg, cfg.L, wdtype=N.W_FP8)
    rows = a.prefill_rows if a.prefill_rows > 1 and not a.unfused else 0
    if dense:
        rows = min(rows, 4)                               # the Qwen3-8B batched kernel holds 4 rows
    if rows:
        cfg = configs.with_layers(cfg, cfg.L, prefill=rows)
    if a.ctx + a.warmup + a.steps + 1 > cfg.max_ctx:
        raise SystemExit(f"ctx {a.ctx} + warmup + steps exceeds max_ctx {cfg.max_ctx}")
    dev = torch.device("cuda:0")
    if a.calib_copy:
        calib_copy(dev)
    t0 = time.time()
    dec = N.Decoder(cfg, device="cuda:0", fused=not a.unfused, workgroups=a.workgroups)
    dec.init_weights(a.seed, 0.02)
    torch.cuda.synchronize()
    log(f"[gpu] weights {dec.sizes['weights'] / 1e9:.2f} GB initialised in {time.time() - t0:.1f}s; "
        f"{dec.barriers_per_step()} grid barriers per step")
    prompt = np.random.default_rng(a.seed).integers(0, cfg.V, a.ctx).astype(np.int32)
    t1 = time.time()
    prefill = None
    if a.kv_fill:
        dec.fill_kv_seeded(a.seed, a.ctx)
        toks = np.zeros(a.ctx + 1, np.int32)
        toks[a.ctx] = prompt[-1]
        dec.set_tokens(toks)
        log(f"[gpu] KV cache filled with {a.ctx} seeded positions")
    else:
        dec.set_tokens(prompt)
        dec.sync()
        stream = torch.cuda.current_stream(dev)
        p0, p1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        p0.record(stream)
        if rows:
            for q in range(0, a.ctx, rows):
                n = min(rows, a.ctx - q)
                dec.prefill(q, n, write_next=q + n == a.ctx)
                if q // rows % 16 == 15:
                    dec.sync()
                    log(f"[gpu] prefill {q + n}/{a.ctx} ({(time.time() - t1) / (q + n) * 1e3:.3f} ms/token)")
        else:
            for pos in range(a.ctx):
                dec.step(pos, write_next=pos + 1 >= a.ctx)
                if pos % 256 == 255:
                    dec.sync()
                    log(f"[gpu] prefill {pos + 1}/{a.ctx} ({(time.time() - t1) / (pos + 1) * 1e3:.3f} ms/token)")
        p1.record(stream)
        dec.sync()
        pms = p0.elapsed_time(p1)
        prefill = {"tokens": a.ctx, "positions_per_launch": rows or 1, "launches": -(-a.ctx // (rows or 1)),
                   "ms": round(pms, 2), "ms_per_token": round(pms / a.ctx, 4),
                   "tokens_per_s": round(a.ctx / (pms * 1e-3), 1),
                   "kernel": "batched persistent kernel, one row per position" if rows else "decode step per token"}
        log(f"[gpu] prefill of {a.ctx} positions: {pms:.1f} ms ({pms / a.ctx:.4f} ms/token, "
            f"{rows or 1} per launch)")
    dec.sync()
    pos = a.ctx
    for _ in range(a.warmup):
        dec.step(pos, write_next=True)
        pos += 1
    dec.sync()
    stream = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    graph = None
    if a.graph:
        # the step at position pos (its per-phase launches, parameters by value) recorded once and replayed; a
        # replay rewrites the same KV slot and next token with the same values, so every replay is the same step
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            dec.step(pos, write_next=True)
        for _ in range(a.warmup):
            graph.replay()
        torch.cuda.synchronize()
        log(f"[gpu] one step at position {pos} captured in a HIP graph "
            f"({cfg.L * (6 if cfg.moe else 5) + 2} kernel nodes)")
    torch.cuda.synchronize()
    w0 = time.perf_counter()
    e0.record(stream)
    first_timed = pos
    for _ in range(a.steps):
        if graph is not None:
            graph.replay()
        else:
            dec.step(pos, write_next=True)
            pos += 1
    e1.record(stream)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - w0) * 1e3
    dec.sync()
    ms = e0.elapsed_time(e1) / a.steps
    if graph is not None:
        pos += 1
    toks = dec.read_tokens(pos)
    ctx_mean = (first_timed + pos - 1) / 2.0
    b = bytes_per_token(cfg, int(round(ctx_mean)))
    gbps = b["total"] / (ms * 1e-3) / 1e9
    log(f"[gpu] {a.steps} steps: {ms:.4f} ms/token (events), host wall {wall / a.steps:.4f} ms/token, "
        f"{gbps:.1f} GB/s = {gbps / HBM_PEAK_GBPS:.3f} of 8 TB/s; last tokens {list(toks[-4:])}")
    phase_us = None
    if a.trace and not a.unfused:
        dec.enable_trace(True)
        dec.step(pos, write_next=True)
        pos += 1
        t = dec.trace()                                   # [phase][wg][wait done, arrive, loads issued], us
        dec.enable_trace(False)
        if a.trace_out:
            np.save(a.trace_out, t)
        phase_us = trace_summary(t, cfg)
    out = {
        "metric": METRIC_8B if dense else METRIC, "value": round(ms, 4), "unit": "ms/token", "n_gpus": 1,
        "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(ms, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp8-e4m3 weights x bf16 activations, fp32 accumulation" if a.fp8 else "bf16",
        "data": "synthetic: seeded random-init " + ("fp8 (quantised from bf16 N(0,0.02))" if a.fp8 else "bf16")
                + " weights N(0,0.02); " + ("KV cache of seeded N(0,1) values"
                if a.kv_fill else "prompt of seeded uniform token ids, prefilled " +
                (f"{rows} positions per launch (bit-identical to token by token)" if rows else "token by token")),
        "config": {"workload": f"{a.model} decode, batch 1, context {a.ctx} (+{a.warmup} warmup), greedy "
                               f"(BASELINE.json configs[{1 if dense else 2}])",
                   "batch": 1, "context": a.ctx, "layers": cfg.L, "experts": cfg.E, "top_k": cfg.TOPK,
                   "vocab": cfg.V, "mode": ("unfused, HIP graph replay" if a.graph else "unfused")
                   if a.unfused else "fused megakernel",
                   "workgroups": a.workgroups or "one per CU", "seed": a.seed},
        "tokens_per_s": round(1e3 / ms, 2), "host_wall_ms_per_token": round(wall / a.steps, 4),
        "bytes_per_token": b["total"], "achieved_GBps": round(gbps, 1),
        ("reference_mi300x_generic_tiles_ms_per_token" if dense else "reference_mi300x_ms_per_token"):
            REFERENCE_MI300X_8B_TILES_MS if dense else REFERENCE_MI300X_MS,
        "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": None,
                     "kernel": "etxmk_fused" if not a.unfused else "etxmk_phase (all phases)"},
        "cpu_baseline": None,
    }
    if phase_us:
        out["phase_us"] = phase_us
    if prefill:
        out["prefill"] = prefill
    if not a.unfused and not a.fp8 and a.ctx == 1024:      # the workloads the counter passes were taken on
        attach_traffic(out, f"etxmk_fused_{'qwen3-8b' if dense else 'qwen3-30b-a3b'}_b1_ctx1024_hbm_traffic.json")
    del graph
    dec.close()                                           # release the handle before the CPU leg and the exit
    del dec
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    if not a.no_cpu:
        try:
            out["cpu_baseline"] = cpu_baseline(cfg, a.ctx, a.seed)
        except Exception as e:  # the baseline is reported, never gating
            log(f"[cpu] baseline failed: {e!r}")
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
