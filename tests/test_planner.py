"""The arena planner: known answers, the closed form of the BERT arena, and
invariants on seeded random interval sets (``tests/test_memory_planning.py``
of the reference)."""

from __future__ import annotations

import random

import pytest
import torch

from mlc.api import build_pipeline
from mlc.config import Config
from mlc.ir.capture import capture
from mlc.ir.types import Buffer, Layout
from mlc.passes.memory_planning import ALIGNMENT, LiveRange, pack, peak_live_bytes, verify
from models import all_models
from oracle import compile_reference
from workload_cache import graph_of

PLANNED = Config(reduction_fusion=False, cuda_graphs=False)
UNPLANNED = Config(reduction_fusion=False, cuda_graphs=False, memory_planning=False)


def test_alignment_is_256():
    assert ALIGNMENT == 256


def test_packing_is_optimal_on_a_chain():
    ranges = [LiveRange(Buffer(f"b{i}", (256,), torch.float32), i, i, 1024) for i in range(8)]
    offsets, total = pack(ranges)
    assert total == 1024
    assert set(offsets.values()) == {0}


def test_packing_stacks_simultaneous_buffers():
    ranges = [LiveRange(Buffer(f"b{i}", (256,), torch.float32), 0, 5, 1024) for i in range(4)]
    offsets, total = pack(ranges)
    assert total == 4096
    assert sorted(offsets.values()) == [0, 1024, 2048, 3072]


def _random_ranges(n, rng, horizon=40):
    out = []
    for i in range(n):
        start = rng.randrange(horizon)
        end = min(horizon, start + rng.randrange(1, 8))
        size = rng.choice([256, 512, 1024, 4096, 16384])
        out.append(LiveRange(Buffer(f"b{i}", (size // 4,), torch.float32), start, end, size))
    return out


@pytest.mark.parametrize("seed", range(25))
def test_packing_never_aliases_on_random_intervals(seed):
    rng = random.Random(seed)
    ranges = _random_ranges(rng.randrange(1, 40), rng)
    offsets, total = pack(ranges)
    assert not verify(ranges, offsets)
    assert total >= peak_live_bytes(ranges, 40)
    assert total <= sum(r.size for r in ranges)
    for r in ranges:
        assert offsets[r.buffer.name] % ALIGNMENT == 0
        assert offsets[r.buffer.name] + r.size <= total


def test_verify_reports_a_planted_overlap():
    a = LiveRange(Buffer("a", (256,), torch.float32), 0, 3, 1024)
    b = LiveRange(Buffer("b", (256,), torch.float32), 2, 5, 1024)
    assert verify([a, b], {"a": 0, "b": 512})
    assert not verify([a, b], {"a": 0, "b": 1024})


@pytest.mark.parametrize("name", [m[0] for m in all_models()])
def test_planned_schedule_invariants(name):
    _, model, args = next(t for t in all_models() if t[0] == name)
    sched = build_pipeline(capture(model, args), PLANNED)
    plan = sched.plan
    assert not verify(list(plan.live_ranges.values()), plan.offsets)
    assert plan.peak_bytes <= plan.arena_bytes <= plan.total_bytes
    outs = {v.buffer.name for v in sched.graph.outputs}
    assert not (outs & set(plan.offsets)), "graph outputs must never be packed"


@pytest.mark.parametrize("name", [m[0] for m in all_models()])
def test_planning_does_not_change_results(name):
    """Planned and unplanned execution are bit-identical (oracle runner)."""
    _, model, args = next(t for t in all_models() if t[0] == name)
    planned = compile_reference(model, args, PLANNED)(*args)
    unplanned = compile_reference(model, args, UNPLANNED)(*args)
    torch.testing.assert_close(planned, unplanned, rtol=0, atol=0)


def _bert_closed_form(B, T, e, D=768, FF=3072):
    """fc1 mm-out and GELU-out live together, plus the residual, plus the mask:
    B*(2*T*FF + T*D)*e + align256(B*T*e)."""
    return B * (2 * T * FF + T * D) * e + -(-(B * T * e) // 256) * 256


@pytest.mark.parametrize("key,B,e", [("C2", 1, 2)])
def test_bert_arena_closed_form(key, B, e):
    sched = build_pipeline(graph_of(key), Config())
    assert sched.arena_bytes == _bert_closed_form(B, 128, e) == 1769728
    assert sched.plan.arena_bytes == sched.plan.peak_bytes


def test_layout_respects_a_non_zero_storage_offset():
    arena = torch.arange(64, dtype=torch.float32)
    piece = arena[16:32]
    lay = Layout.contiguous((4, 4))
    assert torch.equal(lay.as_torch(piece), arena[16:32].reshape(4, 4))
    strided = Layout((2, 4), (8, 1), 0)
    assert torch.equal(strided.as_torch(piece), arena[16:32].reshape(4, 4)[::2])
