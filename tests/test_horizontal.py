"""Parallel-GEMM merging (``Config.merge_parallel_gemms``, an opt-in graph
rewrite): what merges, the rewritten graph stays well-formed, results match
eager, and a group whose downstream views would stop being expressible is
left exactly as it was."""

from __future__ import annotations

import torch
import torch.nn as nn

from mlc.api import build_pipeline
from mlc.bench.models import build
from mlc.config import Config
from mlc.ir.capture import capture
from mlc.kernels import ExternKernel
from mlc.passes.horizontal import merge_parallel_gemms
from oracle import compile_reference
from workload_cache import graph_of

MERGE = Config(merge_parallel_gemms=True, cuda_graphs=False)


def test_bert_qkv_become_one_gemm_per_layer():
    g = graph_of("C2")
    n_params = len(g.params)
    assert merge_parallel_gemms(g) == 24
    g.topo_check()
    assert len(g.params) == n_params - 12 * 6 + 12 * 2
    sched = build_pipeline(g, Config())
    assert sched.counts() == {"extern": 76, "pointwise": 39, "reduction": 37}
    mms = [k for k in sched.kernels if isinstance(k, ExternKernel)
           and k.node.op == "aten.mm.default" and k.outputs[0].shape == (128, 2304)]
    assert len(mms) == 12


def test_with_the_epilogue_the_merged_bias_folds_too():
    sched = build_pipeline(graph_of("C2"), Config(merge_parallel_gemms=True,
                                                        gemm_epilogue=True))
    assert sched.counts() == {"extern": 76, "pointwise": 27, "reduction": 37}


def test_gpt2_is_already_merged():
    assert merge_parallel_gemms(graph_of("C3")) == 0


def test_merged_model_matches_eager():
    for name, b in (("bert-small", 1), ("bert-small", 2)):
        model, args = build(name, b, 32, "cpu", torch.float32)
        with torch.no_grad():
            want = model(*args)
        for cfg in (MERGE, Config(merge_parallel_gemms=True, gemm_epilogue=True,
                                  layout_selection=True, cuda_graphs=False)):
            got = compile_reference(model, args, cfg)(*args)
            torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-6)


class _Flattened(nn.Module):
    """Two linears on one input; one output is flattened, which a column
    slice of a merged product cannot express as a view."""

    def __init__(self):
        super().__init__()
        self.a = nn.Linear(16, 8)
        self.b = nn.Linear(16, 8)

    def forward(self, x):
        return self.a(x).reshape(-1), self.b(x)


def test_inexpressible_views_leave_the_group_untouched():
    x = torch.randn(4, 16)
    g = capture(_Flattened(), (x,))
    before = [(n.op, [o.name for o in n.outputs]) for n in g.nodes]
    layouts = {v.name: (v.buffer.name, v.layout) for v in g.values()}
    assert merge_parallel_gemms(g) == 0
    assert [(n.op, [o.name for o in n.outputs]) for n in g.nodes] == before
    assert {v.name: (v.buffer.name, v.layout) for v in g.values()} == layouts
    model = _Flattened()
    with torch.no_grad():
        want = model(x)
    got = compile_reference(model, (x,), MERGE)(x)
    for gt, w in zip(got, want):
        torch.testing.assert_close(gt, w, rtol=1e-5, atol=1e-6)
