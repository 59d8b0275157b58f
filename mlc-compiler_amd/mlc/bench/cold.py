"""Launch durations with the caches cold.

A kernel launched back to back on the same buffers reads them from the
256 MB Infinity Cache (MALL) after the first launch, so a loop of launches
measures partly cache bandwidth. Inside a forward a kernel's inputs were
usually written long enough before (or by a library GEMM whose output does
not stay cached) that they come from HBM. ``cold_launch_us`` times one launch
right after a 1 GiB fill, which evicts both the L2s and the MALL: the HBM
figure.
"""

from __future__ import annotations

import statistics

FLUSH_BYTES = 1 << 30


def cold_launch_us(launch, reps: int = 30, flush_bytes: int = FLUSH_BYTES) -> float:
    """Median duration (us) of ``launch()`` (which enqueues one kernel on
    torch's current stream) right after a fill of ``flush_bytes``: hipEvents
    around the launch alone, less the median of the same event pair around
    nothing (also after a fill)."""
    import torch

    flush = torch.empty(flush_bytes, dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream()

    def sample(body) -> list[float]:
        pairs = []
        for i in range(reps):
            flush.fill_(i & 0x7F)
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record(stream)
            body()
            b.record(stream)
            pairs.append((a, b))
        torch.cuda.synchronize()
        return [a.elapsed_time(b) * 1e3 for a, b in pairs]

    launch()  # load, warm the instruction cache
    torch.cuda.synchronize()
    timed = sample(launch)
    empty = sample(lambda: None)
    del flush
    return statistics.median(timed) - statistics.median(empty)
