"""Pinning the CPU oracle before it is trusted as the parity checker.

* against eager PyTorch on every toy model under every pass configuration at
  the reference's bar (``tests/test_correctness.py:17-48`` of the reference);
* against the reference's OWN torch-backend outputs for the same seeded
  inputs (``tests/golden/reference_schedules.json``, written by the reference
  compiler), so the restatement is tied to the reference's arithmetic, not
  just to eager;
* numerical special cases the reference tests (two-pass variance against
  float64, large-mean layer norm, softmax on logits x100, streamed ==
  persistent, bit-identical exactness classes);
* planted mistakes in the oracle itself must be caught by these checks.
"""

from __future__ import annotations

import json
import pathlib

import pytest
import torch
import torch.nn as nn

import oracle.torch_reference as tr
from mlc.api import build_pipeline
from mlc.codegen.reduction_schedule import (detect_online_softmax, plan_passes, scalar_binds,
                                            varies_by_column)
from mlc.config import Config
from mlc.ir.capture import capture
from mlc.kernels import ReductionKernel
from models import all_models
from oracle import compile_reference

CONFIGS = {
    "no_fusion": Config(elementwise_fusion=False, recompute=False, reduction_fusion=False,
                        memory_planning=False, cuda_graphs=False),
    "elementwise": Config(reduction_fusion=False, recompute=False, memory_planning=False,
                          cuda_graphs=False),
    "elementwise_recompute": Config(reduction_fusion=False, memory_planning=False,
                                    cuda_graphs=False),
    "planned": Config(reduction_fusion=False, cuda_graphs=False),
    "all_passes": Config(cuda_graphs=False),
    "streamed": Config(cuda_graphs=False, max_persistent_row=4),
}
FULL = CONFIGS["all_passes"]
STREAMED = CONFIGS["streamed"]
GOLDEN = pathlib.Path(__file__).parent / "golden" / "reference_schedules.json"


def _model(name):
    return next(t for t in all_models() if t[0] == name)


@pytest.mark.parametrize("cname", list(CONFIGS))
@pytest.mark.parametrize("name", [m[0] for m in all_models()])
def test_oracle_matches_eager(name, cname):
    _, model, args = _model(name)
    with torch.no_grad():
        want = model(*args)
    got = compile_reference(model, args, CONFIGS[cname])(*args)
    torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-6)


@pytest.fixture(scope="module")
def golden():
    data = json.loads(GOLDEN.read_text())
    if data["torch"] != torch.__version__:
        pytest.skip(f"fixtures were written with torch {data['torch']}")
    return data["toy"]


@pytest.mark.parametrize("cname", ["no_fusion", "all_passes", "streamed"])
@pytest.mark.parametrize("name", [m[0] for m in all_models()])
def test_oracle_matches_reference_backend_outputs(golden, name, cname):
    """The reference's torch backend produced these numbers from the same
    seeded inputs; the restatement reproduces them to fp32 rounding."""
    _, model, args = _model(name)
    got = compile_reference(model, args, CONFIGS[cname])(*args)
    outs = got if isinstance(got, (list, tuple)) else [got]
    rec = golden[name][cname]
    for o, ref, shape in zip(outs, rec["outputs"], rec["output_shapes"]):
        assert list(o.shape) == shape
        want = torch.tensor(ref, dtype=torch.float64).reshape(shape)
        torch.testing.assert_close(o.double(), want, rtol=2e-6, atol=1e-7)


def test_oracle_matches_reference_backend_on_config1():
    """BASELINE config 1 (FFN block, fp32, seeded 0): the oracle against the
    reference torch backend's own output, written by the reference compiler
    on this image's CPU (``tests/golden/reference_config1_out.npy``). Both
    run the same torch CPU GEMMs and the same fp32 row statistics in the same
    order, so they agree bit for bit."""
    import numpy as np

    from mlc.bench.workloads import make

    meta = json.loads((GOLDEN.parent / "reference_config1.json").read_text())
    if meta["torch"] != torch.__version__:
        pytest.skip(f"fixture was written with torch {meta['torch']}")
    want = torch.from_numpy(np.load(GOLDEN.parent / "reference_config1_out.npy"))
    model, args = make("C1", "cpu")
    got = compile_reference(model, args)(*args)
    assert list(got.shape) == meta["output_shape"]
    torch.testing.assert_close(got.reshape(-1), want, rtol=0, atol=0)


@pytest.mark.parametrize("key", ["C2", "C3", "C4"])
def test_oracle_matches_reference_backend_on_fp16_models(key):
    """BASELINE configs 2-4 (BERT-base fp16 b1 and b32 pooled outputs, GPT-2
    small fp16 b1 logits): the oracle against the reference torch backend's
    own outputs, written by the reference compiler on this image's CPU
    (``tests/golden/reference_outputs_fp16.npz``: BERT in full; GPT-2 as every
    101st logit and each row's float64 sum and maximum). Bit for bit: both run
    the same torch CPU ops (fp16 storage, fp32 arithmetic) in the same order."""
    import numpy as np

    from mlc.bench.workloads import make

    ref = np.load(GOLDEN.parent / "reference_outputs_fp16.npz", allow_pickle=False)
    if str(ref["torch_version"]) != torch.__version__:
        pytest.skip(f"fixture was written with torch {ref['torch_version']}")
    model, args = make(key, "cpu")
    out = compile_reference(model, args)(*args)
    out = out if isinstance(out, torch.Tensor) else out[0]
    assert list(out.shape) == ref[f"{key}_shape"].tolist() and out.dtype == torch.float16
    if key == "C3":
        assert torch.equal(out.reshape(-1)[::101], torch.from_numpy(ref["C3_sample"]))
        rows = out.double().reshape(-1, out.shape[-1])
        assert np.array_equal(rows.sum(dim=1).numpy(), ref["C3_row_sum"])
        assert np.array_equal(rows.max(dim=1).values.numpy(), ref["C3_row_max"])
    else:
        assert torch.equal(out, torch.from_numpy(ref[f"{key}_out"]))


@pytest.mark.parametrize("name", [m[0] for m in all_models()])
def test_exactness_classes_are_bit_identical(name):
    """Configs without reduction fusion evaluate the same ops in the same
    order: results agree bit for bit (the reference's
    ``tests/test_correctness.py:51-74``)."""
    _, model, args = _model(name)
    base = compile_reference(model, args, CONFIGS["no_fusion"])(*args)
    for c in ("elementwise", "elementwise_recompute", "planned"):
        got = compile_reference(model, args, CONFIGS[c])(*args)
        torch.testing.assert_close(got, base, rtol=0, atol=0)


@pytest.mark.parametrize("name", [m[0] for m in all_models()])
def test_streaming_agrees_with_persistent(name):
    _, model, args = _model(name)
    persistent = compile_reference(model, args, FULL)(*args)
    streamed = compile_reference(model, args, STREAMED)(*args)
    torch.testing.assert_close(streamed, persistent, rtol=1e-5, atol=1e-6)


class _Softmax(nn.Module):
    def forward(self, x):
        return x.softmax(dim=-1)


class _Var(nn.Module):
    def forward(self, z):
        return z.var(dim=-1, unbiased=False)


class _MaskedSoftmax(nn.Module):
    """A causal ``masked_fill(-inf)`` softmax over ``x`` plus a padding mask
    that hides the first ``pad`` columns of row 0."""

    def __init__(self, pad: int):
        super().__init__()
        self.pad = pad

    def forward(self, x):
        t = x.shape[-1]
        causal = torch.ones(t, t, dtype=torch.bool, device=x.device).triu(1)[: x.shape[-2]]
        hidden = causal.clone()
        hidden[0, : self.pad] = True
        hidden[0, -1] = False
        return x.masked_fill(hidden, float("-inf")).softmax(dim=-1)


@pytest.mark.parametrize("rows,cols,pad", [(96, 128, 100), (4, 2100, 1500)])
def test_streamed_softmax_with_all_inf_prefix(rows, cols, pad):
    """Streamed online softmax where a row's first columns (and, for the
    wide rows, its whole first 1024-column chunk) are -inf: finite and equal
    to eager softmax, as the persistent form is."""
    torch.manual_seed(0)
    x = torch.randn(rows, cols)
    model = _MaskedSoftmax(pad)
    want = model(x)
    assert torch.isfinite(want).all()
    for cfg in (FULL, STREAMED):
        got = compile_reference(model, (x,), cfg)(x)
        torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-6)


def test_softmax_is_stable_on_large_logits():
    x = torch.randn(4, 64) * 100
    for cfg in (FULL, STREAMED):
        got = compile_reference(_Softmax(), (x,), cfg)(x)
        assert torch.isfinite(got).all()
        torch.testing.assert_close(got, x.softmax(dim=-1), rtol=1e-5, atol=1e-6)
        torch.testing.assert_close(got.sum(-1), torch.ones(4), rtol=1e-5, atol=1e-6)


def test_variance_two_pass_against_float64():
    torch.manual_seed(0)
    x = torch.randn(8, 128) + 1e4
    exact = x.double().var(dim=-1, unbiased=False)
    naive = (x.pow(2).mean(-1) - x.mean(-1).pow(2)).double()
    naive_err = (naive - exact).abs().max().item()
    for cfg in (FULL, STREAMED):
        got = compile_reference(_Var(), (x,), cfg)(x).double()
        err = (got - exact).abs().max().item()
        assert err < 1e-3 and err < naive_err / 100


def test_layernorm_on_a_large_mean_stays_accurate():
    torch.manual_seed(0)
    x = torch.randn(8, 128) + 1e4
    model = nn.LayerNorm(128).eval()
    with torch.no_grad():
        exact = torch.nn.functional.layer_norm(x.double(), (128,), model.weight.double(),
                                               model.bias.double(), model.eps)
    for cfg in (FULL, STREAMED):
        got = compile_reference(model, (x,), cfg)(x).double()
        assert (got - exact).abs().max().item() < 5e-3


def _reductions(sched):
    return [k for k in sched.kernels if isinstance(k, ReductionKernel)]


def test_online_softmax_detection_and_passes():
    _, model, args = _model("masked_softmax")
    k = _reductions(build_pipeline(capture(model, args), STREAMED))[0]
    assert detect_online_softmax(k) is not None
    passes = plan_passes(k)
    assert len(passes) == 2 and passes[0].online_softmax is not None
    _, model, args = _model("norm_affine")
    ln = _reductions(build_pipeline(capture(model, args), STREAMED))[0]
    assert detect_online_softmax(ln) is None
    vector, scalars = varies_by_column(ln), {b.name for b in scalar_binds(ln)}
    assert vector and scalars and not (vector & scalars)


# -- planted mistakes: each must be caught by the checks above ----------------

@pytest.mark.parametrize("fn,wrong", [("sub", torch.add), ("exp", torch.exp2),
                                      ("rsqrt", torch.sqrt)])
def test_planted_oracle_mistake_is_caught(monkeypatch, fn, wrong):
    monkeypatch.setitem(tr.TORCH_FN, fn, wrong)
    _, model, args = _model("pre_norm_block")
    with torch.no_grad():
        want = model(*args)
    got = compile_reference(model, args, FULL)(*args)
    assert not torch.allclose(got, want, rtol=1e-5, atol=1e-6)


def test_planted_reduce_identity_mistake_is_caught(monkeypatch):
    """A max that ignored part of the row (as a wrong identity would) fails."""
    monkeypatch.setitem(tr._REDUCE, "max", lambda v: v[:, : max(1, v.shape[1] // 2)]
                        .amax(dim=1, keepdim=True))

    class Amax(nn.Module):
        def forward(self, x):
            return x.amax(dim=-1) * 2.0

    torch.manual_seed(1)
    x = torch.randn(16, 64)
    got = compile_reference(Amax(), (x,), FULL)(x)
    assert not torch.allclose(got, x.amax(dim=-1) * 2.0)
