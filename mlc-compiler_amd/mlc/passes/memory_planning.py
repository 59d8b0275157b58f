"""The arena: every intermediate buffer at a fixed byte offset of one slab.

Shapes are static and each intermediate buffer is written by one kernel and
read by known later ones, so its lifetime is an interval of kernel indices.
Buffers whose intervals are disjoint may share bytes. On the GPU the arena is
one ``hipMalloc`` slab, and because every offset is fixed at compile time
every kernel argument is the same pointer on every call -- what lets the whole
schedule be captured once as a hipGraph and replayed.

Placement contract (kept bit-exact with the reference planner,
``mlc/passes/memory_planning.py:35-240``, so offsets match its golden
fixtures): buffers are taken largest first, ties by first-write index, then
name; each goes to the lowest offset whose bytes no time-overlapping buffer
already placed occupies; offsets and buffer sizes are multiples of 256 bytes.

Besides placement the planner reports the lower bound no placement can beat
(the most bytes live at one kernel) and checks its own result: any two
buffers live at the same time must not share a byte.
"""

from __future__ import annotations

from collections import defaultdict
from dataclasses import dataclass, field
from itertools import accumulate

from ..config import Config
from ..ir.graph import Graph
from ..ir.types import Buffer
from ..kernels import Schedule

#: byte alignment of every arena offset (16-byte packs, library GEMM operands)
ALIGNMENT = 256


def _round_up(n: int) -> int:
    return -(-n // ALIGNMENT) * ALIGNMENT


@dataclass
class LiveRange:
    buffer: Buffer
    #: index of the kernel that first writes the buffer
    start: int
    #: index of the last kernel touching it (len(schedule) for a graph output)
    end: int
    #: bytes reserved (the buffer's size rounded up to ALIGNMENT)
    size: int

    def overlaps(self, other: "LiveRange") -> bool:
        return self.start <= other.end and other.start <= self.end


@dataclass
class AllocationPlan:
    #: "arena" (placed in one slab) or "eager" (allocated around each kernel)
    mode: str
    arena_bytes: int = 0
    offsets: dict[str, int] = field(default_factory=dict)
    #: eager mode: kernel index -> buffers to allocate before it runs
    alloc_at: dict[int, list[Buffer]] = field(default_factory=dict)
    #: eager mode: kernel index -> buffer names to drop after it runs
    free_at: dict[int, list[str]] = field(default_factory=dict)
    live_ranges: dict[str, LiveRange] = field(default_factory=dict)
    #: most bytes live at any one kernel: the bound no placement can beat
    peak_bytes: int = 0
    #: bytes if every buffer had memory of its own
    total_bytes: int = 0

    @property
    def efficiency(self) -> float:
        """Arena size over the lower bound (1.0 is optimal)."""
        return self.arena_bytes / self.peak_bytes if self.peak_bytes else 1.0

    def summary(self) -> str:
        kib = lambda n: f"{n / 1024:.1f} KiB"  # noqa: E731
        if self.mode == "arena":
            return (f"memory: arena {kib(self.arena_bytes)}, lower bound {kib(self.peak_bytes)} "
                    f"({self.efficiency:.2f}x), unplanned would be {kib(self.total_bytes)}")
        return f"memory: unplanned, peak {kib(self.peak_bytes)} of {kib(self.total_bytes)} total"


# --------------------------------------------------------------------------
# lifetimes
# --------------------------------------------------------------------------

def compute_live_ranges(graph: Graph, schedule: Schedule) -> list[LiveRange]:
    """Lifetimes of the plannable buffers, per *buffer* (a view keeps its
    whole buffer alive), in order of first appearance in the schedule."""
    first: dict[str, int] = {}
    last: dict[str, int] = {}
    by_name: dict[str, Buffer] = {}

    def touch(buf: Buffer, i: int, writes: bool) -> None:
        by_name.setdefault(buf.name, buf)
        if writes:
            first.setdefault(buf.name, i)
        last[buf.name] = max(last.get(buf.name, i), i)

    for i, k in enumerate(schedule.kernels):
        for v in k.writes():
            touch(v.buffer, i, True)
        for v in k.reads():
            touch(v.buffer, i, False)
    for v in graph.outputs:  # results outlive the schedule
        by_name.setdefault(v.buffer.name, v.buffer)
        last[v.buffer.name] = len(schedule.kernels)

    return [LiveRange(buf, first[name], last[name], _round_up(buf.nbytes))
            for name, buf in by_name.items() if buf.plannable and name in first]


def peak_live_bytes(ranges: list[LiveRange], n_kernels: int) -> int:
    """Most bytes live at one kernel index (a lower bound on the arena)."""
    delta: dict[int, int] = defaultdict(int)
    for r in ranges:
        delta[r.start] += r.size
        delta[r.end + 1] -= r.size
    return max(accumulate(delta[t] for t in sorted(delta)), default=0) if ranges else 0


# --------------------------------------------------------------------------
# placement
# --------------------------------------------------------------------------

def _lowest_fit(busy: list[tuple[int, int]], size: int) -> int:
    """Lowest offset with ``size`` free bytes below the next busy extent;
    ``busy`` are ``[lo, hi)`` byte extents (overlapping allowed)."""
    at = 0
    for lo, hi in sorted(busy):
        if lo - at >= size:
            break
        at = max(at, hi)
    return at


def pack(ranges: list[LiveRange]) -> tuple[dict[str, int], int]:
    """Offsets of every range and the arena size they need."""
    order = sorted(ranges, key=lambda r: (-r.size, r.start, r.buffer.name))
    offsets: dict[str, int] = {}
    placed: list[tuple[LiveRange, int]] = []
    arena = 0
    for r in order:
        busy = [(off, _round_up(off + p.size)) for p, off in placed if p.overlaps(r)]
        off = _lowest_fit(busy, r.size)
        offsets[r.buffer.name] = off
        placed.append((r, off))
        arena = max(arena, off + r.size)
    return offsets, arena


def verify(ranges: list[LiveRange], offsets: dict[str, int]) -> list[str]:
    """Every pair of buffers live at one time that share a byte, described.
    Two lifetimes overlap exactly when both are live at the later start, so
    the check runs once per distinct start time over the buffers live then."""
    found: list[str] = []
    reported: set[tuple[str, str]] = set()
    for t in sorted({r.start for r in ranges}):
        live = sorted(((offsets[r.buffer.name], r) for r in ranges if r.start <= t <= r.end),
                      key=lambda e: e[0])
        for i, (off_a, a) in enumerate(live):
            for off_b, b in live[i + 1:]:
                if off_b >= off_a + a.size:
                    break
                if off_a >= off_b + b.size:  # b is empty and sits at a's start
                    continue
                pair = tuple(sorted((a.buffer.name, b.buffer.name)))
                if pair in reported:
                    continue
                reported.add(pair)
                found.append(f"{a.buffer.name} bytes [{off_a}, {off_a + a.size}) kernels "
                             f"[{a.start}, {a.end}] share memory with {b.buffer.name} bytes "
                             f"[{off_b}, {off_b + b.size}) kernels [{b.start}, {b.end}]")
    return found


def plan_memory(graph: Graph, schedule: Schedule, cfg: Config) -> AllocationPlan:
    """Place (or, with ``memory_planning`` off, schedule the allocation of)
    every intermediate; records the plan on ``schedule`` and each buffer."""
    ranges = compute_live_ranges(graph, schedule)
    plan = AllocationPlan(mode="arena" if cfg.memory_planning else "eager",
                          live_ranges={r.buffer.name: r for r in ranges},
                          peak_bytes=peak_live_bytes(ranges, len(schedule.kernels)),
                          total_bytes=sum(r.size for r in ranges))
    if plan.mode == "eager":
        for r in ranges:
            plan.alloc_at.setdefault(r.start, []).append(r.buffer)
            if r.end < len(schedule.kernels):
                plan.free_at.setdefault(r.end, []).append(r.buffer.name)
    else:
        plan.offsets, plan.arena_bytes = pack(ranges)
        clashes = verify(ranges, plan.offsets)
        if clashes:
            raise AssertionError("arena placement overlaps live buffers:\n" + "\n".join(clashes))
    for b in graph.buffers():
        b.arena_offset = plan.offsets.get(b.name)
    schedule.arena_bytes = plan.arena_bytes
    schedule.plan = plan
    return plan
