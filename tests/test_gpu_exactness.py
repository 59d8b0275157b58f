"""The reference's exactness classes, held on the HIP path.

The reference asserts two bit-for-bit equalities among its own pass
configurations (``tests/test_correctness.py:51-74`` and
``tests/test_memory_planning.py:63-73`` of the reference):

* ``no_fusion`` = ``elementwise`` = ``elementwise_recompute`` = ``planned``.
  None of these passes changes the order of a floating-point operation; they
  only change which kernel computes a value and where it waits. On the HIP
  path every generated kernel is compiled with contraction off
  (``-ffp-contract=off``), division by a constant is correctly rounded
  (``mlc::div_rcp``) and a fused chain keeps each intermediate in fp32, which
  for an fp32 model is exactly what a stored and reloaded intermediate holds,
  so fusing or recomputing a chain must not move a bit.
* planned = unplanned: the arena only moves buffers, so the results are
  bit-identical. Held here for the toy models under the reference's planned /
  unplanned pair and under all passes, and for BASELINE configs 2-4 (BERT-base
  fp16 b1 and b32, GPT-2 small fp16 b1).

Every comparison is at rtol = atol = 0.
"""

from __future__ import annotations

import pytest
import torch

import mlc
from gpu_util import flat_outputs
from mlc.bench.workloads import make
from mlc.config import Config
from models import all_models

pytestmark = pytest.mark.gpu

EXACT = {
    "no_fusion": Config(elementwise_fusion=False, recompute=False, reduction_fusion=False,
                        memory_planning=False, cuda_graphs=False),
    "elementwise": Config(reduction_fusion=False, recompute=False, memory_planning=False,
                          cuda_graphs=False),
    "elementwise_recompute": Config(reduction_fusion=False, memory_planning=False,
                                    cuda_graphs=False),
    "planned": Config(reduction_fusion=False, cuda_graphs=False),
}

#: (planned, unplanned) pairs: the reference's own pair, and the same with
#: reduction fusion on
PLANNING_PAIRS = {
    "no_reduction_fusion": (Config(reduction_fusion=False, cuda_graphs=False),
                            Config(reduction_fusion=False, cuda_graphs=False,
                                   memory_planning=False)),
    "all_passes": (Config(cuda_graphs=False), Config(cuda_graphs=False, memory_planning=False)),
}


def _run(model, args, cfg):
    out = mlc.compile(model, args, cfg)(*args)
    torch.cuda.synchronize()
    return [o.detach().cpu().clone() for o in flat_outputs(out)]


def _assert_bit_identical(got, base, what):
    assert len(got) == len(base)
    for g, b in zip(got, base):
        assert g.dtype == b.dtype and g.shape == b.shape, what
        # NaN-aware bitwise equality: compare the raw bit patterns
        if g.is_floating_point():
            same = torch.equal(g.view(torch.int32 if g.element_size() == 4 else torch.int16),
                               b.view(torch.int32 if b.element_size() == 4 else torch.int16))
        else:
            same = torch.equal(g, b)
        if not same:
            diff = (g.double() - b.double()).abs().max().item()
            raise AssertionError(f"{what}: not bit-identical (max abs diff {diff:.3e})")


def _cuda(name):
    _, model, args = next(t for t in all_models() if t[0] == name)
    return model.to("cuda"), tuple(a.to("cuda") for a in args)


@pytest.mark.parametrize("name", [m[0] for m in all_models()])
def test_reordering_free_passes_are_bit_identical_on_hip(name):
    model, args = _cuda(name)
    print(f"exactness classes: {name}", flush=True)
    base = _run(model, args, EXACT["no_fusion"])
    for cname in list(EXACT)[1:]:
        _assert_bit_identical(_run(model, args, EXACT[cname]), base,
                              f"{name}: {cname} vs no_fusion")
    model.to("cpu")


@pytest.mark.parametrize("pair", list(PLANNING_PAIRS))
@pytest.mark.parametrize("name", [m[0] for m in all_models()])
def test_planning_does_not_change_hip_results(name, pair):
    model, args = _cuda(name)
    print(f"planned vs unplanned: {name} ({pair})", flush=True)
    planned, unplanned = PLANNING_PAIRS[pair]
    _assert_bit_identical(_run(model, args, planned), _run(model, args, unplanned),
                          f"{name}: planned vs unplanned ({pair})")
    model.to("cpu")


@pytest.mark.parametrize("pair", list(PLANNING_PAIRS))
@pytest.mark.parametrize("key", ["C2", "C3", "C4"])
def test_planning_does_not_change_fp16_model_results(key, pair):
    """BASELINE configs 2-4 (BERT-base fp16 b1 and b32, GPT-2 small fp16
    b1): the arena moves buffers only, so the outputs are bit-identical with
    and without it."""
    model, args = make(key, "cuda")
    print(f"planned vs unplanned: {key} ({pair})", flush=True)
    planned, unplanned = PLANNING_PAIRS[pair]
    _assert_bit_identical(_run(model, args, planned), _run(model, args, unplanned),
                          f"{key}: planned vs unplanned ({pair})")


@pytest.mark.parametrize("key", ["C2", "C3", "C4"])
def test_graph_replay_equals_planned_run_fp16(key):
    """The captured hipGraph replays exactly the planned run, on every replay."""
    model, args = make(key, "cuda")
    print(f"graph replay vs planned run: {key}", flush=True)
    eager = _run(model, args, Config(cuda_graphs=False))
    compiled = mlc.compile(model, args, Config())
    for _ in range(3):
        got = [o.detach().cpu().clone() for o in flat_outputs(compiled(*args))]
        torch.cuda.synchronize()
        _assert_bit_identical(got, eager, f"{key}: graph replay vs planned run")
