"""The GEMM bias-epilogue pass (``Config.gemm_epilogue``, an opt-in schedule
change): what it folds, what it must leave alone, and that the folded
schedule computes the same function (oracle against eager)."""

from __future__ import annotations

import torch
import torch.nn as nn

from mlc.api import build_pipeline
from mlc.bench.models import build
from mlc.config import Config
from mlc.ir.capture import capture
from mlc.kernels import ExternKernel, PointwiseKernel
from mlc.passes.memory_planning import verify
from models import all_models
from oracle import compile_reference
from workload_cache import graph_of

EPI = Config(gemm_epilogue=True, cuda_graphs=False)


def _addmms(sched):
    return [k for k in sched.kernels if isinstance(k, ExternKernel)
            and k.node.op == "aten.addmm.default"]


def test_bert_qkv_bias_adds_fold_into_the_gemm():
    base = build_pipeline(graph_of("C2"), Config())
    sched = build_pipeline(graph_of("C2"), Config(gemm_epilogue=True))
    assert len(_addmms(sched)) == 36
    assert sched.counts() == {"extern": 100, "pointwise": 27, "reduction": 37}
    assert base.counts()["pointwise"] - sched.counts()["pointwise"] == 36
    # biases that fuse with more work stay where they are: LayerNorm (attention
    # output, fc2) and GELU (fc1) keep their adds
    assert sum(1 for k in sched.kernels if isinstance(k, PointwiseKernel)
               and any(n.op == "aten.erf.default" for n in k.nodes)) == 12
    plan = sched.plan
    assert not verify(list(plan.live_ranges.values()), plan.offsets)
    for k in _addmms(sched):
        bias, a, w = k.node.args
        assert bias.shape == (768,) and k.outputs[0].shape == (128, 768)


def test_gpt2_fused_qkv_bias_folds():
    sched = build_pipeline(graph_of("C3"), Config(gemm_epilogue=True))
    assert len(_addmms(sched)) == 12
    assert all(k.outputs[0].shape == (128, 2304) for k in _addmms(sched))


def test_default_config_keeps_the_reference_schedule():
    sched = build_pipeline(graph_of("C2"), Config())
    assert not _addmms(sched)


def test_folded_schedule_matches_eager():
    model, args = build("bert-small", 2, 32, "cpu", torch.float32)
    with torch.no_grad():
        want = model(*args)
    got = compile_reference(model, args, EPI)(*args)
    torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-6)
    for name, m, a in all_models():
        with torch.no_grad():
            w = m(*a)
        torch.testing.assert_close(compile_reference(m, a, EPI)(*a), w, rtol=1e-5, atol=1e-6)


class _SharedMM(nn.Module):
    """The mm output is read twice: folding would drop the plain product."""

    def __init__(self):
        super().__init__()
        self.w = nn.Parameter(torch.randn(16, 32))
        self.b = nn.Parameter(torch.randn(32))

    def forward(self, x):
        y = x @ self.w
        return y + self.b, y * 2.0


def test_no_fold_when_the_product_has_another_reader():
    x = torch.randn(8, 16)
    sched = build_pipeline(capture(_SharedMM(), (x,)), Config(gemm_epilogue=True))
    assert not _addmms(sched)
