"""Algorithmic HBM bytes of a generated kernel, the unit the bandwidth
roofline is priced in.

    bytes(k) = sum over distinct (buffer, index map) inputs of
                   (distinct elements addressed) * itemsize
             + sum over outputs of (elements written) * itemsize

An index map's distinct elements are the product of the sizes of its
canonical terms (stride-0 dims are already dropped, so a broadcast operand
counts once). This equals the reference cost model's traffic
(``mlc/passes/cost.py:44-59``) when no operand is broadcast-expanded. A fused
attention kernel is priced the same way: q, k, v and the reduction's other
operands read once, the output written once (the scores and probabilities it
keeps on chip are not HBM traffic).
"""

from __future__ import annotations

import math

import torch

from ..codegen.index import IndexMap
from ..kernels import AttentionKernel, ExternKernel, PointwiseKernel, ReductionKernel

#: MI355X published peak HBM3E bandwidth, GB/s
HBM_PEAK_GBS = 8000.0


def _itemsize(dtype: torch.dtype) -> int:
    return torch.empty((), dtype=dtype).element_size()


def distinct_elements(imap: IndexMap) -> int:
    return math.prod(size for a in imap.axes for size, _, _ in a.terms)


def algorithmic_bytes(k) -> int:
    if isinstance(k, ExternKernel):
        if k.node.op == "aten.embedding.default":
            out = k.outputs[0]
            ids = k.node.args[1]
            return 2 * out.numel * _itemsize(out.dtype) + ids.numel * _itemsize(ids.dtype)
        raise TypeError(f"no byte model for extern {k.node.op}")
    if not isinstance(k, (PointwiseKernel, ReductionKernel, AttentionKernel)):
        raise TypeError(type(k).__name__)
    seen = set()
    total = 0
    for a in k.inputs:
        key = (a.value.buffer.name, a.index.render())
        if key in seen:
            continue
        seen.add(key)
        total += distinct_elements(a.index) * _itemsize(a.dtype)
    for a in k.outputs:
        total += distinct_elements(a.index) * _itemsize(a.dtype)
    return total


def extern_bytes(k: ExternKernel) -> int:
    """Algorithmic bytes of a library call: every distinct operand view read
    once (a GEMM's weights included) plus every output written once."""
    seen = set()
    total = 0
    for v in k.inputs:
        key = (v.buffer.name, v.layout)
        if key in seen:
            continue
        seen.add(key)
        total += v.numel * _itemsize(v.dtype)
    for v in k.outputs:
        total += v.numel * _itemsize(v.dtype)
    return total


def forward_bytes(schedule) -> int:
    """Algorithmic bytes of one whole forward: every kernel, generated or
    library, at its algorithmic traffic. Divided by the HBM peak it is the
    bytes-moved floor of the forward's latency."""
    total = 0
    for k in schedule.kernels:
        if isinstance(k, ExternKernel) and k.node.op != "aten.embedding.default":
            total += extern_bytes(k)
        else:
            total += algorithmic_bytes(k)
    return total
