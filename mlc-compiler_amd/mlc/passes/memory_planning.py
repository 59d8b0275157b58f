"""Memory planning: pack every intermediate buffer into one arena.

Live ranges are kernel-index intervals per buffer (first write to last read;
graph outputs live past the end). Packing is greedy: largest first (ties by
first write, then name), each at the lowest 256-byte-aligned offset clear of
every already-placed buffer whose range overlaps. The arena is then one
``hipMalloc`` slab on the device, and these offsets are the byte offsets of
each buffer inside it.

Reference behaviour followed: ``mlc/passes/memory_planning.py:35-240``. The
packing order and the gap search are the reference's, so offsets and the
arena size are bit-identical for the same schedule.
"""

from __future__ import annotations

from dataclasses import dataclass, field

from ..config import Config
from ..ir.graph import Graph
from ..ir.types import Buffer
from ..kernels import Schedule

#: byte alignment of every arena offset
ALIGNMENT = 256


def _align(n: int, to: int = ALIGNMENT) -> int:
    return -(-n // to) * to


@dataclass
class LiveRange:
    buffer: Buffer
    start: int
    end: int
    size: int

    def overlaps(self, other: "LiveRange") -> bool:
        return self.start <= other.end and other.start <= self.end


@dataclass
class AllocationPlan:
    mode: str  # "arena" | "eager"
    arena_bytes: int = 0
    offsets: dict[str, int] = field(default_factory=dict)
    #: eager mode: kernel index -> buffers allocated just before it
    alloc_at: dict[int, list[Buffer]] = field(default_factory=dict)
    #: eager mode: kernel index -> buffer names released just after it
    free_at: dict[int, list[str]] = field(default_factory=dict)
    live_ranges: dict[str, LiveRange] = field(default_factory=dict)
    #: most bytes live at once: a lower bound for any arena
    peak_bytes: int = 0
    #: sum of all plannable buffers
    total_bytes: int = 0

    @property
    def efficiency(self) -> float:
        return self.arena_bytes / self.peak_bytes if self.peak_bytes else 1.0

    def summary(self) -> str:
        if self.mode != "arena":
            return (f"memory: unplanned, peak {self.peak_bytes / 1024:.1f} KiB "
                    f"of {self.total_bytes / 1024:.1f} KiB total")
        return (f"memory: arena {self.arena_bytes / 1024:.1f} KiB, "
                f"lower bound {self.peak_bytes / 1024:.1f} KiB ({self.efficiency:.2f}x), "
                f"unplanned would be {self.total_bytes / 1024:.1f} KiB")


def compute_live_ranges(graph: Graph, schedule: Schedule) -> list[LiveRange]:
    """Per-buffer [first write, last read] over kernel indices."""
    first_write: dict[str, int] = {}
    last_use: dict[str, int] = {}
    by_name: dict[str, Buffer] = {}
    for i, k in enumerate(schedule.kernels):
        for v in k.writes():
            nm = v.buffer.name
            by_name.setdefault(nm, v.buffer)
            first_write.setdefault(nm, i)
            last_use[nm] = max(last_use.get(nm, i), i)
        for v in k.reads():
            nm = v.buffer.name
            by_name.setdefault(nm, v.buffer)
            last_use[nm] = max(last_use.get(nm, i), i)
    horizon = len(schedule.kernels)
    for v in graph.outputs:
        last_use[v.buffer.name] = horizon
        by_name.setdefault(v.buffer.name, v.buffer)

    ranges: list[LiveRange] = []
    for nm, buf in by_name.items():
        if not buf.plannable or nm not in first_write:
            continue
        start = first_write[nm]
        ranges.append(LiveRange(buf, start, last_use.get(nm, start), _align(buf.nbytes)))
    return ranges


def peak_live_bytes(ranges: list[LiveRange], n_kernels: int) -> int:
    if not ranges:
        return 0
    events = sorted([(r.start, r.size) for r in ranges] + [(r.end + 1, -r.size) for r in ranges])
    live = peak = 0
    for _, delta in events:
        live += delta
        peak = max(peak, live)
    return peak


def pack(ranges: list[LiveRange]) -> tuple[dict[str, int], int]:
    """Greedy largest-first, lowest-fit placement."""
    placed: list[tuple[int, LiveRange]] = []
    offsets: dict[str, int] = {}
    arena = 0
    for r in sorted(ranges, key=lambda r: (-r.size, r.start, r.buffer.name)):
        blockers = sorted(((off, p) for off, p in placed if p.overlaps(r)), key=lambda t: t[0])
        at = 0
        for off, p in blockers:
            if off >= at + r.size:
                break
            at = max(at, _align(off + p.size))
        offsets[r.buffer.name] = at
        placed.append((at, r))
        arena = max(arena, at + r.size)
    return offsets, arena


def verify(ranges: list[LiveRange], offsets: dict[str, int]) -> list[str]:
    """Every pair of simultaneously live buffers must be byte-disjoint."""
    problems: list[str] = []
    for i, a in enumerate(ranges):
        oa = offsets[a.buffer.name]
        for b in ranges[i + 1:]:
            if not a.overlaps(b):
                continue
            ob = offsets[b.buffer.name]
            if oa < ob + b.size and ob < oa + a.size:
                problems.append(
                    f"{a.buffer.name}[{oa}:{oa + a.size}] live [{a.start},{a.end}] overlaps "
                    f"{b.buffer.name}[{ob}:{ob + b.size}] live [{b.start},{b.end}]")
    return problems


def plan_memory(graph: Graph, schedule: Schedule, cfg: Config) -> AllocationPlan:
    ranges = compute_live_ranges(graph, schedule)
    peak = peak_live_bytes(ranges, len(schedule.kernels))
    total = sum(r.size for r in ranges)
    by_name = {r.buffer.name: r for r in ranges}

    if not cfg.memory_planning:
        plan = AllocationPlan(mode="eager", peak_bytes=peak, total_bytes=total, live_ranges=by_name)
        for r in ranges:
            plan.alloc_at.setdefault(r.start, []).append(r.buffer)
            if r.end < len(schedule.kernels):
                plan.free_at.setdefault(r.end, []).append(r.buffer.name)
        for b in graph.buffers():
            b.arena_offset = None
        schedule.arena_bytes = 0
        schedule.plan = plan
        return plan

    offsets, arena = pack(ranges)
    problems = verify(ranges, offsets)
    if problems:
        raise AssertionError("memory planner produced overlapping buffers:\n" + "\n".join(problems))
    for b in graph.buffers():
        b.arena_offset = offsets.get(b.name)
    plan = AllocationPlan(mode="arena", arena_bytes=arena, offsets=offsets, live_ranges=by_name,
                          peak_bytes=peak, total_bytes=total)
    schedule.arena_bytes = arena
    schedule.plan = plan
    return plan
