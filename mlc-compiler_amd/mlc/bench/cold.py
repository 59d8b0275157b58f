"""Launch durations with the caches cold.

A kernel launched back to back on the same buffers reads them from the
256 MB Infinity Cache (MALL) after the first launch, so a loop of launches
measures partly cache bandwidth. Inside a forward a kernel's inputs were
usually written long enough before (or by a library GEMM whose output does
not stay cached) that they come from HBM. ``cold_launch_us`` times one launch
right after a 1 GiB fill, which evicts both the L2s and the MALL: the HBM
figure. The fill leaves the MALL full of dirty lines, so the launch also pays
for writing some of them back, as a kernel inside a forward does for the
output of the kernels before it.
"""

from __future__ import annotations

import statistics

FLUSH_BYTES = 1 << 30


def cold_launch_us(launch, reps: int = 30, flush_bytes: int = FLUSH_BYTES) -> float:
    """Median duration (us) of ``launch()`` (which enqueues one kernel on
    torch's current stream) right after a fill of ``flush_bytes``: hipEvents
    around the launch, less the same event pair around nothing. The two are
    interleaved (fill, timed pair, fill, empty pair, ...) so that both see the
    same conditions; the median of the per-repetition differences is taken."""
    import torch

    flush = torch.empty(flush_bytes, dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream()

    def pair(body, i):
        flush.fill_(i & 0x7F)
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(stream)
        body()
        b.record(stream)
        return a, b

    launch()  # load the module, warm the instruction cache
    torch.cuda.synchronize()
    samples = [(pair(launch, i), pair(lambda: None, i + 1)) for i in range(reps)]
    torch.cuda.synchronize()
    del flush
    return statistics.median((t[0].elapsed_time(t[1]) - e[0].elapsed_time(e[1])) * 1e3
                             for t, e in samples)
