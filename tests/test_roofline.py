"""The byte model the bandwidth rooflines are priced in, against the closed
forms derived from the model source (per kernel family) and the totals the
survey of the reference derives for each benchmark configuration."""

from __future__ import annotations

import pytest

from mlc.api import build_pipeline
from mlc.bench.roofline import algorithmic_bytes, extern_bytes, forward_bytes
from mlc.config import Config
from mlc.kernels import ExternKernel, PointwiseKernel, ReductionKernel
from workload_cache import graph_of

N, D, FF, H, T, E = 128, 768, 3072, 12, 128, 2  # BERT b1 s128, fp16


def _generated(sched):
    return [k for k in sched.kernels if not isinstance(k, ExternKernel)]


def test_bert_b1_family_closed_forms():
    sched = build_pipeline(graph_of("C2"), Config())
    got = {algorithmic_bytes(k) for k in _generated(sched)}
    assert (2 * N * D + D) * E in got                    # q/k/v bias-add
    assert (2 * H * T * T + T) * E in got                # softmax with the mask row
    assert (3 * N * D + 3 * D) * E in got                # LayerNorm + bias + residual
    assert (2 * N * FF + FF) * E in got                  # fc1 bias + GELU
    assert 2 * N * D * E in got                          # context copy


@pytest.mark.parametrize("key,n,mb", [("C2", 100, 62.4), ("C3", 73, 67.3), ("C4", 136, 2435.5),
                                      ("C5", 109, 13949.2)])
def test_generated_kernel_totals(key, n, mb):
    """Totals over every generated kernel: BERT fp16 b1 62.4 MB, b32 2.435 GB,
    GPT-2 fp16 b1 67.3 MB, b32 s512 13.95 GB."""
    gen = _generated(build_pipeline(graph_of(key), Config()))
    assert len(gen) == n
    assert all(isinstance(k, (PointwiseKernel, ReductionKernel)) for k in gen)
    assert round(sum(algorithmic_bytes(k) for k in gen) / 1e6, 1) == mb


def test_bert_b1_forward_floor():
    """The whole forward with its library GEMMs (weights read once): about
    296 MB for BERT fp16 b1, a 37 us floor at 8 TB/s."""
    sched = build_pipeline(graph_of("C2"), Config())
    b = forward_bytes(sched)
    assert 290e6 < b < 300e6
    mms = [k for k in sched.kernels if isinstance(k, ExternKernel)
           and k.node.op == "aten.mm.default" and k.outputs[0].shape == (N, FF)]
    assert extern_bytes(mms[0]) == (N * D + D * FF + N * FF) * E
