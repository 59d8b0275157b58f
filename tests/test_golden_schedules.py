"""The kernel schedule and the arena are bit-exact with the reference's.

``tests/golden/reference_schedules.json`` was written by
``tests/golden/dump_reference.py`` from the reference compiler itself (same
torch version as this image). Per case it holds every kernel (kind, order,
operand buffers, rendered index strings, bodies / steps, reduce kinds, row
outputs) and the planner's result (arena size, lower bound, unplanned total,
every offset). This build's front end, fusion, lowering and planner must
reproduce all of it exactly, for every toy model under every pass
configuration and for the benchmark models at every BASELINE shape.
"""

from __future__ import annotations

import json
import pathlib
import sys

import pytest
import torch

from mlc.api import build_pipeline
from mlc.bench.models import build
from mlc.config import Config
from mlc.ir.capture import capture
from models import all_models

GOLDEN = pathlib.Path(__file__).parent / "golden" / "reference_schedules.json"
sys.path.insert(0, str(GOLDEN.parent))
from dump_reference import _describe, _plan  # noqa: E402

CONFIGS = {
    "no_fusion": Config(elementwise_fusion=False, recompute=False, reduction_fusion=False,
                        memory_planning=False, cuda_graphs=False),
    "elementwise": Config(reduction_fusion=False, recompute=False, memory_planning=False,
                          cuda_graphs=False),
    "planned": Config(reduction_fusion=False, cuda_graphs=False),
    "all_passes": Config(cuda_graphs=False),
    "streamed": Config(cuda_graphs=False, max_persistent_row=4),
    "graphs": Config(),
}


@pytest.fixture(scope="module")
def golden():
    data = json.loads(GOLDEN.read_text())
    if data["torch"] != torch.__version__:
        pytest.skip(f"fixtures were written with torch {data['torch']}, this is {torch.__version__}")
    return data


def _compare(got, want):
    assert len(got["kernels"]) == len(want["kernels"])
    for g, w in zip(got["kernels"], want["kernels"]):
        assert g == w, f"kernel {w['name']} differs"
    assert got["plan"] == want["plan"]


@pytest.mark.parametrize("cname", list(CONFIGS))
@pytest.mark.parametrize("name", [m[0] for m in all_models()])
def test_toy_schedule_matches_reference(golden, name, cname):
    _, model, args = next(t for t in all_models() if t[0] == name)
    sched = build_pipeline(capture(model, args), CONFIGS[cname])
    _compare({"kernels": _describe(sched), "plan": _plan(sched)}, golden["toy"][name][cname])


BENCH_KEYS = [
    "bert-base|b1|s128|float16|graphs",
    "bert-base|b1|s128|float16|streamed64",
    "bert-base|b32|s128|float16|graphs",
    "bert-base|b1|s128|float32|graphs",
    "gpt2-small|b1|s128|float16|graphs",
    "gpt2-small|b32|s128|float16|graphs",
    "gpt2-small|b32|s512|float16|graphs",
    "bert-small|b1|s32|float32|graphs",
    "bert-small|b2|s32|float32|graphs",
    "gpt-small|b1|s32|float32|graphs",
    "gpt-small|b2|s32|float32|graphs",
]


@pytest.mark.parametrize("key", BENCH_KEYS)
def test_bench_schedule_matches_reference(golden, key):
    mname, b, s, dt, cname = key.split("|")
    model, args = build(mname, int(b[1:]), int(s[1:]), "cpu", getattr(torch, dt))
    cfg = Config() if cname == "graphs" else Config(max_persistent_row=64)
    sched = build_pipeline(capture(model, args), cfg)
    want = golden["bench"][key]
    _compare({"kernels": _describe(sched), "plan": _plan(sched)}, want)
    assert sched.counts() == want["counts"]


def test_published_counts_and_arenas(golden):
    """The A40 log's published kernel counts and arenas
    (results/gpu_check.log:57-100 of the reference) are in the fixtures too."""
    b = golden["bench"]
    assert b["bert-base|b1|s128|float16|graphs"]["counts"] == {"extern": 100, "pointwise": 63,
                                                              "reduction": 37}
    assert b["bert-base|b32|s128|float16|graphs"]["counts"] == {"extern": 100, "pointwise": 99,
                                                               "reduction": 37}
    assert b["bert-base|b1|s128|float16|graphs"]["plan"]["arena_bytes"] == 1769728
    assert b["bert-base|b32|s128|float16|graphs"]["plan"]["arena_bytes"] == 56631296
    assert b["bert-base|b1|s128|float32|graphs"]["plan"]["arena_bytes"] == 3539456
    assert b["gpt2-small|b1|s128|float16|graphs"]["plan"]["arena_bytes"] == 1966080


CONFIG1 = pathlib.Path(__file__).parent / "golden" / "reference_config1.json"


def test_config1_schedule_and_arena_match_reference():
    """BASELINE config 1 (the FFN block, fp32, seeded 0): the reference
    compiler's schedule -- one LayerNorm reduction with the residual add, two
    GEMMs, the fc1 bias + tanh-GELU and the fc2 bias -- and its arena,
    3,145,728 B (the fc1 GEMM output and the GELU output live together:
    2 x 128 x 3072 x 4 B), written by ``dump_reference.py --config1``."""
    from mlc.bench.workloads import make

    want = json.loads(CONFIG1.read_text())
    if want["torch"] != torch.__version__:
        pytest.skip(f"fixture was written with torch {want['torch']}, this is {torch.__version__}")
    model, args = make("C1", "cpu")
    sched = build_pipeline(capture(model, args), Config())
    _compare({"kernels": _describe(sched), "plan": _plan(sched)}, want)
    assert sched.counts() == want["counts"] == {"extern": 2, "pointwise": 2, "reduction": 1}
    assert sched.plan.arena_bytes == 3145728 == 2 * 128 * 3072 * 4
