"""Front-end properties the reference's suite checks (its ``tests/test_layout.py``,
``test_fusion.py``, ``test_capture.py``, ``test_dtypes.py``,
``test_bench_reporting.py``): view layouts against torch's own views, schedule
invariants, fp16/bf16 numerics of the kernel IR, binding externs without
running them, and the pointwise tail guard."""

from __future__ import annotations

import random

import pytest
import torch

from mlc.api import build_pipeline
from mlc.codegen.hip_backend import emit_pointwise
from mlc.config import Config
from mlc.ir.capture import capture
from mlc.ir.shapes import infer_view
from mlc.ir.types import Layout
from mlc.kernels import ExternKernel, PointwiseKernel
from mlc.runtime.executor import bind_extern, run_bound_extern
from models import all_models
from oracle import compile_reference

CONFIGS = {
    "no_fusion": Config(elementwise_fusion=False, reduction_fusion=False, memory_planning=False,
                        cuda_graphs=False),
    "all_passes": Config(cuda_graphs=False),
    "streamed": Config(max_persistent_row=4, cuda_graphs=False),
    "every_variant": Config(merge_parallel_gemms=True, gemm_epilogue=True, layout_selection=True,
                            fused_attention=True, cuda_graphs=False),
}


class _Arg:
    def __init__(self, layout):
        self.layout = layout


def _random_view(rng: random.Random, t: torch.Tensor):
    """One view op valid for ``t``: (aten op name, args after the tensor, torch fn)."""
    shape = list(t.shape)
    r = len(shape)
    # (a 0-d view is re-viewed through unsqueeze: the restride rule, like the
    # reference's, reports shapes over no old dims as needing a copy)
    choices = ["permute", "unsqueeze"] + (["view"] if r else [])
    if r >= 2:
        choices += ["transpose", "t"] if r == 2 else ["transpose"]
    if r >= 1:
        choices += ["slice", "select", "expand"]
    if 1 in shape:
        choices.append("squeeze")
    op = rng.choice(choices)
    if op == "permute":
        dims = list(range(r))
        rng.shuffle(dims)
        return "aten.permute.default", [dims], lambda x: x.permute(dims)
    if op == "transpose":
        a, b = rng.sample(range(r), 2)
        return "aten.transpose.int", [a, b], lambda x: x.transpose(a, b)
    if op == "t":
        return "aten.t.default", [], lambda x: x.t()
    if op == "unsqueeze":
        d = rng.randint(0, r)
        return "aten.unsqueeze.default", [d], lambda x: x.unsqueeze(d)
    if op == "squeeze":
        d = rng.choice([i for i, n in enumerate(shape) if n == 1])
        return "aten.squeeze.dim", [d], lambda x: x.squeeze(d)
    if op == "slice":
        d = rng.randrange(r)
        n = shape[d]
        start = rng.randint(0, max(0, n - 1))
        end = rng.randint(start, n)
        step = rng.choice([1, 1, 2])
        return ("aten.slice.Tensor", [d, start, end, step],
                lambda x: x[(slice(None),) * d + (slice(start, end, step),)])
    if op == "select":
        d = rng.choice([i for i, n in enumerate(shape) if n > 0])
        i = rng.randrange(shape[d])
        return "aten.select.int", [d, i], lambda x: x.select(d, i)
    if op == "expand":
        new = [rng.choice([n, 3]) if n == 1 else n for n in shape]
        return "aten.expand.default", [new], lambda x: x.expand(new)
    # view: regroup the trailing dims of a contiguous-compatible shape
    numel = t.numel()
    merged = shape[:-2] + [shape[-2] * shape[-1]] if r >= 2 else [numel, 1]
    for cand in (merged, [numel], [1, numel]):
        try:
            t.view(cand)
        except RuntimeError:
            continue
        return "aten.view.default", [cand], lambda x, c=cand: x.view(c)
    return "aten.unsqueeze.default", [0], lambda x: x.unsqueeze(0)


@pytest.mark.parametrize("seed", range(8))
def test_view_layouts_match_torch(seed):
    """Every view rule against torch's own view on random chains: same shape,
    strides and storage offset (reference ``tests/test_layout.py:35-78``)."""
    rng = random.Random(seed)
    for _ in range(60):
        shape = [rng.randint(1, 5) for _ in range(rng.randint(1, 4))]
        t = torch.arange(int(torch.tensor(shape).prod())).reshape(shape)
        lay = Layout.contiguous(tuple(shape))
        for _ in range(rng.randint(1, 6)):
            if t.numel() == 0:
                break
            op, args, fn = _random_view(rng, t)
            t = fn(t)
            lay = infer_view(op, [_Arg(lay)] + args, {})
            assert lay.shape == tuple(t.shape), (op, args)
            assert lay.strides == tuple(t.stride()) or t.numel() <= 1, (op, args)
            if t.numel() > 1:
                assert lay.offset == t.storage_offset(), (op, args)


@pytest.mark.parametrize("cname", sorted(CONFIGS))
@pytest.mark.parametrize("name", [m[0] for m in all_models()])
def test_schedule_invariants(name, cname):
    """One writer per buffer; every read is of a graph input, a parameter or a
    buffer an earlier kernel wrote; views never allocate (reference
    ``tests/test_fusion.py:51-76``, ``tests/test_capture.py:37-45``). Also
    under every schedule variant, whose passes rewrite the schedule."""
    _, model, args = next(t for t in all_models() if t[0] == name)
    graph = capture(model, args)
    for n in graph.nodes:
        if n.meta.get("is_view"):
            src = n.args[0]
            assert all(o.buffer is src.buffer for o in n.outputs), f"view {n.op} allocated"
    sched = build_pipeline(graph, CONFIGS[cname])
    ready = {v.buffer.name for v in graph.inputs} | {v.buffer.name for v in graph.params}
    ready |= {v.buffer.name for v in graph.values() if v.buffer.kind in ("param", "const")}
    written: set[str] = set()
    for k in sched.kernels:
        for v in k.reads():
            assert v.buffer.name in ready or v.buffer.name in written, \
                f"{k.summary()} reads {v.buffer.name} before it is written"
        for name_ in {v.buffer.name for v in k.writes()}:
            assert name_ not in written, f"{name_} has two writers"
            written.add(name_)
    for v in graph.outputs:
        assert v.buffer.name in written or v.buffer.name in ready


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("name", ["two_input_chain", "feed_forward", "masked_softmax", "norm_affine", "pre_norm_block"])
def test_narrow_float_models(name, dtype):
    """fp16/bf16 storage through the kernel IR (fp32 math inside kernels):
    within 1e-2/5e-2 of eager in the same dtype and 2e-2/5e-2 of eager fp32
    (reference ``tests/test_dtypes.py:35-58``)."""
    _, model, args = next(t for t in all_models() if t[0] == name)
    narrow_model = model.to(dtype)
    narrow = tuple(a.to(dtype) for a in args)
    got = compile_reference(narrow_model, narrow, Config(cuda_graphs=False))(*narrow)
    with torch.no_grad():
        eager = narrow_model(*narrow)
        ref32 = model.float()(*(a.float() for a in narrow))
    assert got.dtype == dtype
    torch.testing.assert_close(got.float(), eager.float(), rtol=1e-2, atol=5e-2)
    torch.testing.assert_close(got.float(), ref32, rtol=2e-2, atol=5e-2)


def test_binding_an_extern_never_runs_it():
    """Resolving an extern against the buffer table leaves its outputs
    untouched; only running the bound call writes them (reference
    ``tests/test_bench_reporting.py:77-111``)."""
    _, model, args = next(t for t in all_models() if t[0] == "feed_forward")
    graph = capture(model, args)
    sched = build_pipeline(graph, Config(memory_planning=False, cuda_graphs=False))
    externs = [k for k in sched.kernels if isinstance(k, ExternKernel)]
    assert externs
    buffers = {}
    for k in sched.kernels:
        for v in list(k.reads()) + list(k.writes()):
            if v.buffer.name not in buffers:
                fill = torch.randn(v.buffer.numel) if v.buffer.dtype.is_floating_point else \
                    torch.zeros(v.buffer.numel, dtype=v.buffer.dtype)
                buffers[v.buffer.name] = fill.to(v.buffer.dtype)
    for k in externs:
        for v in k.writes():
            buffers[v.buffer.name].fill_(float("nan"))
        bound = bind_extern(k, buffers)
        for v in k.writes():
            assert torch.isnan(buffers[v.buffer.name]).all(), f"binding {k.node.op} ran it"
        run_bound_extern(bound)
        for v in k.writes():
            assert torch.isfinite(buffers[v.buffer.name]).all()


@pytest.mark.parametrize("n,tail", [(4096, False), (4100, True), (8, False), (12, True)])
def test_pointwise_tail_path_only_when_packs_do_not_divide(n, tail):
    """The scalar tail exists only when 8-element fp16 packs do not divide the
    element count (the reference omits its mask when BLOCK divides numel,
    ``tests/test_codegen.py:82-87``)."""

    class AddOne(torch.nn.Module):
        def forward(self, x):
            return x * 3.0 + 1.0

    x = torch.randn(n).half()
    sched = build_pipeline(capture(AddOne(), (x,)), Config(cuda_graphs=False))
    (k,) = [k for k in sched.kernels if isinstance(k, PointwiseKernel)]
    src, spec = emit_pointwise(k)
    assert spec.meta["vec"] == 8
    assert ("if (e0 + V <= N)" in src) == tail


@pytest.mark.parametrize("name", [m[0] for m in all_models()])
def test_every_variant_matches_eager_on_toy_models(name):
    """The schedule variants compute the same function: every toy model with
    all of them on, through the oracle, against eager at the fp32 bar."""
    _, model, args = next(t for t in all_models() if t[0] == name)
    with torch.no_grad():
        want = model(*args)
    got = compile_reference(model, args, CONFIGS["every_variant"])(*args)
    for g, w in zip(got if isinstance(got, (list, tuple)) else [got],
                    want if isinstance(want, (list, tuple)) else [want]):
        torch.testing.assert_close(g, w, rtol=1e-5, atol=1e-6)
