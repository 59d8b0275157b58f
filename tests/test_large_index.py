"""Buffers of 2^31 elements or more: 64-bit offsets.

The generated kernels index with 32-bit offsets unless some operand's buffer
has at least 2^31 elements (``hip_backend.index_type``); then every offset,
row base and column term is 64-bit. The CPU tests check that choice in the
generated source for the three templates (pointwise, persistent reduction,
streamed reduction); the GPU tests run each at just over 2^31 fp32 elements
(8 GiB per buffer) and compare with PyTorch on the same device: bit-exact for
the pointwise chain, whose two operations round exactly as PyTorch's do, and
within fp32 rounding for the reductions. Element 2^31 and beyond is checked
like every other element.
"""

from __future__ import annotations

import pytest
import torch

from mlc.api import build_pipeline
from mlc.codegen.hip_backend import build_module
from mlc.config import Config
from mlc.ir.capture import capture

BIG = 2 ** 31


class AffineRelu(torch.nn.Module):
    def forward(self, x):
        return torch.relu(x * 2.0 + 1.0)


class Softmax(torch.nn.Module):
    def forward(self, x):
        return torch.softmax(x, dim=-1)


class RowSum(torch.nn.Module):
    def forward(self, x):
        return x.sum(dim=-1)


CASES = {
    # 2 x (2^30 + 512): the flat index passes 2^31 inside the second row
    "pointwise": (AffineRelu, (2, 2 ** 30 + 512), "pointwise"),
    # 2^21 + 3 rows of 1024, one wave per row
    "persistent": (Softmax, (2 ** 21 + 3, 1024), "persistent"),
    # rows of 32768 (> max_persistent_row): streamed
    "streamed": (RowSum, (2 ** 16 + 1, 2 ** 15), "streamed"),
}


def _module(name, device):
    cls, shape, _ = CASES[name]
    x = torch.empty(shape, device=device)
    model = cls()
    sched = build_pipeline(capture(model, (x,)), Config())
    return model, sched, build_module(sched, Config())


@pytest.mark.parametrize("name", sorted(CASES))
def test_large_buffers_get_64_bit_offsets(name):
    _, sched, mod = _module(name, "meta")
    assert len(sched.kernels) == 1
    spec = mod.launches[sched.kernels[0].name]
    assert spec.meta.get("mode", spec.meta["kind"]) == CASES[name][2]
    body = mod.functions[spec.symbol]
    assert "uint64_t" in body and "uint32_t" not in body


def test_small_buffers_keep_32_bit_offsets():
    x = torch.empty(4, 1024, device="meta")
    sched = build_pipeline(capture(Softmax(), (x,)), Config())
    mod = build_module(sched, Config())
    body = mod.functions[mod.launches[sched.kernels[0].name].symbol]
    assert "uint32_t" in body and "uint64_t" not in body


def _run(name):
    import mlc

    cls, shape, _ = CASES[name]
    g = torch.Generator(device="cuda").manual_seed(7)
    x = torch.randn(shape, device="cuda", generator=g)
    assert x.numel() >= BIG
    model = cls()
    print(name, list(shape), flush=True)
    compiled = mlc.compile(model, (x,), Config(cuda_graphs=False))
    got = compiled(x)
    torch.cuda.synchronize()
    return model, x, got


@pytest.mark.gpu
def test_pointwise_past_2_31_elements():
    model, x, got = _run("pointwise")
    want = model(x)
    assert torch.equal(got, want)
    del x, got, want
    torch.cuda.empty_cache()


@pytest.mark.gpu
def test_persistent_softmax_past_2_31_elements():
    model, x, got = _run("persistent")
    want = torch.softmax(x, dim=-1)
    err = (got - want).abs().max().item()
    print(f"  max abs diff vs torch softmax {err:.2e}")
    assert err <= 1e-6
    # every row sums to one, the last rows (past element 2^31) included
    assert (got[-4:].double().sum(dim=-1) - 1).abs().max().item() <= 1e-5
    del x, got, want
    torch.cuda.empty_cache()


@pytest.mark.gpu
def test_streamed_sum_past_2_31_elements():
    model, x, got = _run("streamed")
    exact = x.sum(dim=-1, dtype=torch.float64)
    # fp32 accumulation of 32768 N(0,1) terms in some order: within 1e-5 of
    # the row's absolute sum
    scale = x.abs().sum(dim=-1, dtype=torch.float64)
    rel = ((got.double() - exact).abs() / scale).max().item()
    print(f"  max error / row abs-sum {rel:.2e}")
    assert rel <= 1e-5
    del x, got, exact, scale
    torch.cuda.empty_cache()
