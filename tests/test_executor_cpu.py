"""Executor behaviour on the CPU, with the oracle as the kernel runner (the
product's buffer table, arena binding, extern dispatch and output aliasing are
the code under test), plus the rule that the product itself never runs
anywhere but the GPU (``mlc/runtime/executor.py`` of the reference,
``tests/test_correctness.py:101-171``)."""

from __future__ import annotations

import subprocess
import sys

import pytest
import torch

import mlc
from mlc.config import Config
from mlc.runtime.executor import ExecutionError, select_backend
from models import all_models
from oracle import compile_reference

FULL = Config(cuda_graphs=False)


def _model(name):
    return next(t for t in all_models() if t[0] == name)


def test_wrong_input_shape_is_rejected():
    _, model, args = _model("two_input_chain")
    compiled = compile_reference(model, args, FULL)
    with pytest.raises(ExecutionError, match="compiled for"):
        compiled(torch.randn(5, 16), torch.randn(5, 16))


def test_outputs_alias_static_storage():
    _, model, args = _model("shared_producer")
    compiled = compile_reference(model, args, FULL)
    first = compiled(*args)
    kept = first.clone()
    second = compiled(args[0] * 2)
    assert second.data_ptr() == first.data_ptr()
    assert not torch.equal(first, kept), "the first result is overwritten by the next call"


def test_inputs_are_copied_not_aliased():
    _, model, args = _model("two_input_chain")
    compiled = compile_reference(model, args, FULL)
    x = args[0].clone()
    out = compiled(x, args[1]).clone()
    x.add_(100.0)
    again = compiled(args[0], args[1])
    torch.testing.assert_close(again, out, rtol=0, atol=0)


def test_arena_offsets_bind_buffers():
    _, model, args = _model("pre_norm_block")
    compiled = compile_reference(model, args, FULL)
    compiled(*args)
    arena = compiled._arena
    plan = compiled.schedule.plan
    assert arena.numel() == plan.arena_bytes
    for name, off in plan.offsets.items():
        t = compiled._resident.get(name)
        if t is not None:
            assert t.untyped_storage().data_ptr() == arena.untyped_storage().data_ptr()
            assert t.data_ptr() - arena.data_ptr() == off


def test_product_refuses_the_cpu():
    """No silent CPU fallback: mlc.compile on a CPU model raises."""
    _, model, args = _model("two_input_chain")
    with pytest.raises(ExecutionError, match="ROCm GPU"):
        mlc.compile(model, args, FULL)
    with pytest.raises(ExecutionError):
        select_backend(Config(backend="triton"), torch.device("cuda"))
    assert select_backend(Config(), torch.device("cuda")) == "hip"


def test_hip_runtime_refuses_a_cpu_device():
    from mlc.runtime.hip_runtime import HipRuntime
    from mlc.runtime.native import NativeError

    _, model, args = _model("two_input_chain")
    from mlc.api import build_pipeline
    from mlc.ir.capture import capture

    sched = build_pipeline(capture(model, args), FULL)
    with pytest.raises(NativeError, match="GPU"):
        HipRuntime(sched, FULL, torch.device("cpu"))


def test_bench_refuses_more_than_one_gpu():
    proc = subprocess.run([sys.executable, "bench.py", "--gpus", "2"], capture_output=True,
                          text=True, cwd=str(__import__("pathlib").Path(__file__).parents[1]))
    assert proc.returncode == 2
    assert "one GPU" in proc.stderr


def test_externs_without_tensor_inputs_run_once_into_their_own_memory():
    """``masked_fill`` with a float scalar exports ``aten.scalar_tensor``,
    which has no ``out=`` form and allocates. An extern that reads no tensor
    always gives the same result, so it runs once when the plan is built, into
    a buffer of its own (not an arena slice another buffer may reuse), and is
    never replayed: a captured forward then allocates nothing."""
    from mlc.kernels import ExternKernel

    class Fill(torch.nn.Module):
        def forward(self, x):
            return (x.masked_fill(x > 0.5, float("-inf")).softmax(-1) * 2.0).sum(-1)

    x = torch.randn(8, 64)
    compiled = compile_reference(Fill(), (x,), FULL)
    got = compiled(x).clone()
    assert [k.node.op for k in compiled.schedule.kernels if isinstance(k, ExternKernel)] == \
        ["aten.scalar_tensor.default"]
    kinds = [kind for kind, _ in compiled._plan]
    assert kinds.count("const") == 1 and "extern" not in kinds
    name = next(k for k in compiled.schedule.kernels if isinstance(k, ExternKernel)) \
        .outputs[0].buffer.name
    arena = compiled._arena
    t = compiled._resident[name]
    assert arena is None or not (arena.data_ptr() <= t.data_ptr() < arena.data_ptr() + arena.numel())
    torch.testing.assert_close(got, Fill()(x))
    torch.testing.assert_close(compiled(x * 3.0), Fill()(x * 3.0))


class _FlaggingRunner:
    """The oracle runner plus a CPU stand-in for the native embedding gather:
    an id outside the table yields a zero row and sets an error flag, which
    ``pending_error`` reports, the way the HIP runtime reports its device
    word's host mirror."""

    name = "torch"
    source = "# oracle"

    def __init__(self):
        from oracle import TorchReferenceRunner

        self._inner = TorchReferenceRunner()
        self.flag = 0
        self.fetches = 0

    def bind(self, k, buffers):
        return self._inner.bind(k, buffers)

    def launch(self, k, buffers):
        self._inner.launch(k, buffers)

    def bind_native_extern(self, k, buffers):
        if k.node.op != "aten.embedding.default":
            return None
        return ("gather", k, buffers)

    def run_bound(self, payload):
        if payload[0] != "gather":
            self._inner.run_bound(payload)
            return
        _, k, buffers = payload
        weight, ids = k.node.args[0], k.node.args[1]
        w = weight.layout.as_torch(buffers[weight.buffer.name])
        i = ids.layout.as_torch(buffers[ids.buffer.name]).reshape(-1)
        ok = (i >= 0) & (i < w.shape[0])
        rows = torch.where(ok[:, None], w[i.clamp(0, w.shape[0] - 1)], torch.zeros_like(w[:1]))
        out = k.node.outputs[0]
        out.layout.as_torch(buffers[out.buffer.name]).copy_(rows.reshape(out.shape))
        if not bool(ok.all()):
            self.flag = 1

    def fetch_errors(self):
        self.fetches += 1

    def pending_error(self):
        return "an embedding id was outside its table" if self.flag else None

    def clear_errors(self):
        self.flag = 0


class _Embed(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.emb = torch.nn.Embedding(10, 8)

    def forward(self, ids):
        return self.emb(ids) * 2.0


def test_invalid_embedding_id_raises_on_the_next_call():
    """The executor's side of the invalid-input word: a call whose embedding
    ids leave the table returns (its rows are zeros), the next call raises
    ``ExecutionError`` and clears the flag, and the call after that runs
    normally; ``check_errors`` raises at once. Every run fetches the word."""
    from mlc.api import build_pipeline
    from mlc.ir.capture import capture
    from mlc.runtime.executor import CompiledModel

    torch.manual_seed(0)
    model = _Embed()
    ids = torch.tensor([[1, 2, 3, 4]])
    graph = capture(model, (ids,))
    runner = _FlaggingRunner()
    compiled = CompiledModel(graph, build_pipeline(graph, FULL), FULL, torch.device("cpu"),
                             runner=runner)
    want = model(ids)
    torch.testing.assert_close(compiled(ids), want)
    bad = torch.tensor([[1, 12, 3, -1]])
    out = compiled(bad)
    assert torch.equal(out[0, 1], torch.zeros(8)) and torch.equal(out[0, 3], torch.zeros(8))
    with pytest.raises(ExecutionError, match="outside its table"):
        compiled(ids)
    torch.testing.assert_close(compiled(ids), want)
    compiled(bad)
    with pytest.raises(ExecutionError, match="outside its table"):
        compiled.check_errors()
    compiled.check_errors()
    assert runner.fetches >= 5
