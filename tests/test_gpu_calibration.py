"""The calibration kernels (libetxmk_calib.so) that the barrier and streaming figures are measured with: the grid
barrier runs to completion with every counter at its final generation, and the streaming read reads every word
exactly once (its per-thread sums add up to the sum of the buffer's words, mod 2^32), at every load depth."""
import numpy as np
import pytest

from etx.runtime import calib
from progress_log import say

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("per_cu_groups", [1.0, 0.25], ids=["one-per-cu", "quarter"])
def test_barrier_counts(gpu, per_cu_groups):
    import torch
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    nwg = max(8, int(cus * per_cu_groups))
    iters = 300
    say(f"[gpu] calibration barrier: {nwg} workgroups x {iters}")
    us, bar, ab = calib.barrier(nwg, iters)
    assert ab == 0, f"a wait gave up (abort word {ab})"
    for g in range(8):
        ng = (nwg - g + 7) // 8
        assert int(bar[64 * g]) == iters * ng, f"group {g}: {bar[64 * g]} arrivals, expected {iters * ng}"
    assert int(bar[64 * 8]) == iters * 8
    assert all(int(bar[64 * (9 + j)]) == iters for j in range(8))
    assert 0 < us < 1000


def test_barrier_refuses_oversized_grid(gpu):
    import torch
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    with pytest.raises(RuntimeError, match="HIP error"):
        calib.barrier(cus * 64, 1)                         # more workgroups than can be co-resident
    with pytest.raises(RuntimeError, match="HIP error"):
        calib.barrier(4, 1)                                # the barrier spreads arrivals over 8 groups


@pytest.mark.parametrize("inflight", [1, 2, 4, 8, 16])
def test_stream_reads_every_word_once(gpu, inflight):
    import torch
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    g = torch.Generator(device="cuda:0").manual_seed(inflight)
    n = (64 << 20) // 4 + 256 * 7                          # 64 MiB + 7 KiB: a ragged last round
    src = torch.randint(-2**31, 2**31 - 1, (n,), dtype=torch.int32, device="cuda:0", generator=g)
    say(f"[gpu] calibration stream: {n * 4} bytes, {inflight} in flight")
    secs, sink = calib.stream(src, inflight, cus)
    assert calib.word_sum(sink) == calib.word_sum(src)
    assert secs > 0
    with pytest.raises(RuntimeError, match="HIP error"):
        calib.stream(src, 3, cus)                          # not one of the built depths


@pytest.mark.parametrize("inflight", [1, 2])
def test_tile_stream_reads_every_block_word_once(gpu, inflight):
    """The tiles' pattern reads the 16 rows' first nblk KiB each exactly once: the sinks add up to the sum of those
    words (a tile count that is not a multiple of the waves leaves some waves with fewer tiles)."""
    import torch
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    row_bytes, nblk, ntile = 2064, 2, 3 * cus * 8 + 5
    g = torch.Generator(device="cuda:0").manual_seed(10 + inflight)
    src = torch.randint(-2**31, 2**31 - 1, (ntile * 16 * row_bytes // 4,), dtype=torch.int32, device="cuda:0",
                        generator=g)
    say(f"[gpu] calibration tile stream: {ntile} tiles, {inflight} in flight")
    secs, used, sink = calib.stream_tiles(src, row_bytes, nblk, inflight, cus)
    assert used == ntile * 16 * nblk * 1024 and secs > 0
    blocks = src.view(ntile * 16, row_bytes // 4)[:, : nblk * 256]
    assert calib.word_sum(sink) == calib.word_sum(blocks.contiguous())
    with pytest.raises(RuntimeError, match="HIP error"):
        calib.stream_tiles(src, row_bytes, nblk, 3, cus)   # not one of the built depths
