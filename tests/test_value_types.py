"""Value types: the tensor type each scalar value has in the reference's torch
evaluation (``mlc/codegen/torch_backend.py:53-118`` of the reference), which
decides where a generated kernel rounds to fp16 or bf16.

Pinned against the oracle's own evaluation (which restates that backend and
reproduces the reference's outputs bit for bit): every temporary of every
kernel of the seeded random programs gets the dtype and dimensionality the
oracle's tensors have. Known answers cover torch's promotion rules that the
random programs may not reach."""

from __future__ import annotations

import pytest
import torch

import fuzz_programs as fp
from mlc.api import build_pipeline
from mlc.codegen.hip_backend import build_module
from mlc.codegen.value_types import call_type, expr_type, kernel_types, load_type
from mlc.config import Config
from mlc.ir.capture import capture
from mlc.ir.scalar import Call, Cast, Const, Load, Ref, walk
from mlc.kernels import Bind, PointwiseKernel, Reduce, ReductionKernel
from oracle.torch_reference import _REDUCE, _promote, eval_expr
from workload_cache import graph_of

F16, BF16, F32, I64, B = torch.float16, torch.bfloat16, torch.float32, torch.int64, torch.bool


def _oracle_types(k):
    """Temporary name -> (dtype, has dims) of the oracle's tensors for ``k``,
    evaluated over a 2 x 3 block of ones."""
    loads = [_promote(torch.ones(2, 3, dtype=a.dtype)) for a in k.inputs]
    like = loads[0] if loads else torch.ones(2, 3, dtype=torch.int64)
    refs, out = {}, {}
    steps = ([Bind(n, e) for n, e in k.body] if isinstance(k, PointwiseKernel) else k.steps)
    for s in steps:
        v = eval_expr(s.expr, loads, refs, like)
        if not torch.is_tensor(v):
            v = torch.as_tensor(v)
        if isinstance(s, Reduce):
            v = _REDUCE[s.kind](v.expand(2, 3) if v.dim() < 2 else v)
        refs[s.name] = v
        out[s.name] = (v.dtype, v.dim() > 0)
    return out


@pytest.mark.parametrize("seed,wide", [(s, False) for s in range(12)] + [(s, True) for s in range(3)])
def test_kernel_types_match_the_oracles_tensors(seed, wide):
    model, args = fp.program(seed, wide=wide)
    sched = build_pipeline(capture(model, args), Config(cuda_graphs=False))
    checked = 0
    for k in sched.kernels:
        if not isinstance(k, (PointwiseKernel, ReductionKernel)):
            continue
        want = _oracle_types(k)
        got = kernel_types(k)
        assert got == want, (k.name, {n: (got[n], want[n]) for n in want if got[n] != want[n]})
        checked += len(want)
    assert checked > 0


def _t(e, inputs=(F32,), temps=None):
    return expr_type(e, lambda s: load_type(inputs[s]), (temps or {}).__getitem__)


def test_known_answers():
    x = Load(0)
    # narrow loads are promoted: arithmetic on them is fp32
    assert _t(Call("add", (x, Const(1.0, F16))), (F16,)) == (F32, True)
    assert _t(Call("mul", (x, x)), (BF16,)) == (F32, True)
    # an explicit cast makes what follows narrow; a 0-dim fp32 constant does not widen it
    h = Cast(x, F16)
    assert _t(Call("add", (h, Const(1.0, F32))), (F32,)) == (F16, True)
    assert _t(Call("log", (h,))) == (F16, True)
    assert _t(Call("where", (Const(True), h, Const(0.5, F32)))) == (F16, True)
    # a dimensioned fp32 operand widens it; fp16 against bf16 is fp32
    assert _t(Call("add", (h, x))) == (F32, True)
    assert _t(Call("add", (h, Cast(x, BF16)))) == (F32, True)
    # a 0-dim operand of a higher category decides: int64 tensor + fp16 constant
    assert _t(Call("add", (x, Const(0.5, F16))), (I64,)) == (F16, True)
    assert _t(Call("add", (x, Const(2, I64))), (I64,)) == (I64, True)
    # true division and float functions of integers are fp32; comparisons bool
    assert _t(Call("div", (x, x)), (I64,)) == (F32, True)
    assert _t(Call("exp", (x,)), (I64,)) == (F32, True)
    assert _t(Call("gt", (h, Const(0.0, F32)))) == (B, True)
    # constants alone stay 0-dim; a boolean constant is a full tensor
    assert _t(Call("add", (Const(1.0, F16), Const(2.0, F16)))) == (F16, False)
    assert _t(Const(False)) == (B, True)
    assert call_type("sigmoid", ((BF16, True),)) == (BF16, True)
    # what torch refuses is typed fp32 (no rounding), not an error
    assert call_type("neg", ((B, True),)) == (F32, True)


def test_reductions_keep_their_operand_type():
    x = Load(0)
    steps = [Bind("h", Cast(x, F16)), Reduce("s", "sum", Ref("h")), Reduce("m", "max", Ref("h")),
             Reduce("c", "sum", Call("gt", (x, Const(0.0, F32)))), Reduce("f", "sum", x)]
    k = ReductionKernel.__new__(ReductionKernel)
    object.__setattr__(k, "steps", steps)
    object.__setattr__(k, "inputs", [type("A", (), {"dtype": F16})()])
    types = kernel_types(k)
    assert types["s"] == (F16, True) and types["m"] == (F16, True)
    assert types["c"] == (I64, True) and types["f"] == (F32, True)
    # the streamed form's online-softmax max and sum are fp32 tensors
    assert kernel_types(k, frozenset({"s", "m"}))["s"] == (F32, True)


class _NarrowTail(torch.nn.Module):
    def forward(self, x):
        s = torch.softmax(x.float(), dim=-1).half()
        return torch.log(s.abs() + 1.0), (x.half() * 0.1).sum(dim=-1)


def test_narrow_arithmetic_is_rounded_in_the_generated_code():
    """After a cast to fp16 each arithmetic result is rounded to fp16, as the
    reference's torch evaluation rounds it; the row sum of fp16 values too."""
    args = (torch.randn(8, 96),)
    cfg = Config(cuda_graphs=False)
    src = build_module(build_pipeline(capture(_NarrowTail(), args), cfg), cfg).source
    assert "mlc::round_f16(mlc::log_(" in src
    assert "mlc::round_f16(mlc::row_reduce<" in src


class _NarrowConstants(torch.nn.Module):
    def forward(self, x):
        h = x.half()
        return h - 0.1, h * 0.1


def test_narrow_add_rounds_its_constant_and_mul_does_not():
    """torch's CPU kernels add an fp16 tensor and a constant in fp16 (the
    constant converted first) but multiply by the constant's fp32 value."""
    args = (torch.randn(4, 64),)
    cfg = Config(cuda_graphs=False)
    src = build_module(build_pipeline(capture(_NarrowConstants(), args), cfg), cfg).source
    lines = [ln for ln in src.splitlines() if "0x1.99" in ln]
    assert len(lines) == 2
    assert any("0x1.9980000000000p-4f" in ln and "neg_one_" in ln for ln in lines)  # fp16(0.1)
    assert any("0x1.99999a0000000p-4f" in ln and "neg_zero_" in ln for ln in lines)  # fp32(0.1)


@pytest.mark.parametrize("key", ["C1", "C2", "C3", "C4"])
def test_benchmark_kernels_have_no_narrow_arithmetic(key):
    """The BASELINE models cast to fp16 only right before a store: none of
    their kernels rounds in between, so this typing adds no instruction to
    them."""
    full = Config(merge_parallel_gemms=True, gemm_epilogue=True, layout_selection=True,
                  fused_attention=True)
    for cfg in (Config(), full):
        sched = build_pipeline(graph_of(key), cfg)
        for k in sched.kernels:
            if not isinstance(k, (PointwiseKernel, ReductionKernel)):
                continue
            types = kernel_types(k)
            steps = k.body if isinstance(k, PointwiseKernel) else [(s.name, s.expr) for s in k.steps]
            for name, e in steps + list(k.out_expr.items()):
                if isinstance(k, ReductionKernel) and name in types and any(
                        isinstance(s, Reduce) and s.name == name for s in k.steps):
                    assert types[name][0] not in (F16, BF16), (k.name, name)
                for x in walk(e):
                    if isinstance(x, Call):
                        t = expr_type(x, lambda s: load_type(k.inputs[s].dtype), types.__getitem__)
                        assert t[0] not in (F16, BF16), (k.name, x.fn)
