"""Layout selection (``Config.layout_selection``, an opt-in schedule change):
index-map composition, what the pass merges, and that the merged schedule
computes exactly what the reference schedule computes (oracle, bit for bit)."""

from __future__ import annotations

import torch

from mlc.api import build_pipeline
from mlc.bench.models import build
from mlc.codegen.hip_backend import build_module
from mlc.codegen.index import flat_index
from mlc.config import Config
from mlc.ir.types import Layout
from mlc.kernels import PointwiseKernel
from mlc.passes.layout import compose
from mlc.passes.memory_planning import verify
from oracle import compile_reference
from workload_cache import graph_of

LAYOUT = Config(layout_selection=True)


def test_compose_transpose_and_broadcast():
    # producer space [4, 6, 8] (flat), copy view = permute to [4, 8, 6]
    view = Layout.contiguous((4, 6, 8)).permute([0, 2, 1])
    ident = flat_index((4, 6, 8), Layout.contiguous((4, 6, 8)))
    lay = compose(view, ident)
    assert lay == view
    # a bias broadcast along the producer's rows, indexed (idx % 8)
    bias = flat_index((4, 6, 8), Layout.contiguous((8,)).expand((4, 6, 8)))
    lay = compose(view, bias)
    assert lay.shape == (4, 8, 6) and lay.strides == (0, 1, 0) and lay.offset == 0


def test_compose_refuses_a_non_affine_read():
    # producer reads its input at (idx % 5) over a 12-element space: wrapping
    # inside a dimension of the view cannot be written as one stride
    from mlc.codegen.index import Axis, IndexMap

    wrap = IndexMap((Axis("idx", 12, ((5, 1, 1),)),), 0)
    view = Layout.contiguous((3, 4)).permute([1, 0])
    assert compose(view, wrap) is None


def _pointwise(s):
    return [k for k in s.kernels if isinstance(k, PointwiseKernel)]


def test_bert_b32_copies_merge_into_bias_adds():
    base = build_pipeline(graph_of("C4"), Config())
    sched = build_pipeline(graph_of("C4"), LAYOUT)
    assert sched.counts() == {"extern": 100, "pointwise": 63, "reduction": 37}
    merged = [k for k in _pointwise(sched)
              if [n.op for n in k.nodes] == ["aten.add.Tensor", "aten.clone.default"]]
    assert len(merged) == 36
    assert not verify(list(sched.plan.live_ranges.values()), sched.plan.offsets)
    mod = build_module(sched, LAYOUT)
    kinds = [mod.launches[k.name].meta["kind"] for k in merged]
    assert kinds.count("transpose") == 12 and kinds.count("pointwise") == 24
    assert base.counts()["pointwise"] == 99


def test_gpt2_b32_fused_qkv_add_splits_into_three_merged_kernels():
    sched = build_pipeline(graph_of("C5"), LAYOUT)
    assert sched.counts() == {"extern": 75, "reduction": 37, "pointwise": 60}
    assert sched.arena_bytes < build_pipeline(graph_of("C5"), Config()).arena_bytes


def test_batch_one_has_nothing_to_merge():
    assert build_pipeline(graph_of("C2"), LAYOUT).counts()["pointwise"] == 63


def test_merged_schedule_is_bit_identical_to_the_reference_schedule():
    for name in ("bert-small", "gpt-small"):
        model, args = build(name, 2, 32, "cpu", torch.float32)
        base = compile_reference(model, args, Config(cuda_graphs=False))(*args)
        got = compile_reference(model, args, Config(layout_selection=True, cuda_graphs=False))(*args)
        assert torch.equal(got, base)
        both = compile_reference(model, args, Config(layout_selection=True, gemm_epilogue=True,
                                                     cuda_graphs=False))(*args)
        torch.testing.assert_close(both, base, rtol=1e-5, atol=1e-6)
