"""Layout selection: an opt-in schedule change (``Config.layout_selection``).

A pointwise kernel whose only consumer is a copy that re-lays its output out
(BERT's q/k/v bias-adds at batch > 1, each followed by a ``clone`` into the
``[B, H, T, Dh]`` or ``[B, H, Dh, T]`` layout ``bmm`` needs) is merged with
that copy: the merged kernel iterates in the copy's order, reads the
producer's inputs through the composed index maps and writes the copy's
output directly, so the intermediate buffer and one launch disappear. This is
the first "next" row of the survey: deleting the transpose copies by writing
the producer's output in the consumer's layout.

Composition: the copy reads the producer's output ``O`` (written at
identity over the producer's space) through a strided view ``R``. For each
producer input read at map ``M`` the composed read ``M(R(c))`` must be affine
in the copy's index ``c``; the pass derives the affine form from the deltas
along each dimension and verifies it exactly over every index before it
rewrites anything. The merged kernel takes the producer's place in the
schedule (its inputs are ready there, and the producer's input -- a GEMM
output -- is still hot in cache).
"""

from __future__ import annotations

import functools
import math

import numpy as np

from ..codegen.index import IndexMap, flat_index
from ..ir.scalar import Load
from ..ir.types import Layout
from ..kernels import KernelArg, PointwiseKernel, Schedule

#: maps over more points than this are checked on a sample (plus all corners)
EXHAUSTIVE_LIMIT = 1 << 22


def _eval(imap: IndexMap, p: np.ndarray) -> np.ndarray:
    out = np.full(p.shape, imap.base, dtype=np.int64)
    for a in imap.axes:
        for size, os_, is_ in a.terms:
            out += ((p // os_) % size) * is_
    return out


def _affine(shape, strides, offset, sample) -> np.ndarray:
    """offset + sum_i c_i * strides[i] at every multi-index ``c`` of
    ``shape`` (by broadcast outer sums), or at the sampled flat indices."""
    if sample is None:
        acc = np.array(offset, dtype=np.int64)
        for n, st in zip(shape, strides):
            acc = acc[..., None] + np.arange(n, dtype=np.int64) * st
        return acc.reshape(-1)
    acc = np.full(sample.shape, offset, dtype=np.int64)
    rem = sample
    for n, st in zip(reversed(shape), reversed(strides)):
        acc += (rem % n) * st
        rem = rem // n
    return acc


def _sample(shape):
    n = math.prod(shape)
    if n <= EXHAUSTIVE_LIMIT:
        return None
    rng = np.random.default_rng(0)
    corners = [sum((shape[i] - 1) * math.prod(shape[i + 1:]) for i in range(len(shape))
                   if (bit >> i) & 1) for bit in range(1 << len(shape))]
    return np.concatenate([rng.integers(0, n, size=1 << 20, dtype=np.int64),
                           np.array(corners, dtype=np.int64)])


@functools.lru_cache(maxsize=4096)
def compose(view: Layout, imap: IndexMap) -> Layout | None:
    """The layout, over ``view``'s shape, of ``imap`` read at the offsets
    ``view`` addresses -- or None when that read is not affine. Memoised:
    every transformer layer asks the same question."""
    shape = view.shape
    base = int(_eval(imap, np.array([view.offset], dtype=np.int64))[0])
    deltas = []
    for n, st in zip(shape, view.strides):
        if n == 1:
            deltas.append(0)
            continue
        step = np.array([view.offset + st], dtype=np.int64)
        deltas.append(int(_eval(imap, step)[0]) - base)
    sample = _sample(shape)
    want = _eval(imap, _affine(shape, view.strides, view.offset, sample))
    got = _affine(shape, deltas, base, sample)
    if not np.array_equal(want, got) or base < 0 or any(d < 0 for d in deltas):
        return None
    return Layout(tuple(shape), tuple(deltas), base)


def is_pure_copy(k) -> bool:
    if not isinstance(k, PointwiseKernel) or len(k.inputs) != 1 or len(k.outputs) != 1:
        return False
    out = k.outputs[0]
    expr = k.out_expr.get(out.value.name)
    return (not k.body and isinstance(expr, Load) and expr.slot == 0
            and out.index.is_identity() and k.inputs[0].dtype == out.dtype)


def fold_relayout_copies(schedule: Schedule) -> int:
    """Merge pointwise producers into the copies that re-lay them out. When
    every reader of a producer's output is such a copy (GPT-2's fused qkv
    bias-add, read as three head-major slices), each copy gets its own merged
    kernel computing just the elements it reads. Returns the copies merged."""
    kernels = schedule.kernels
    graph_outputs = {v.buffer.name for v in schedule.graph.outputs}
    readers: dict[str, list[int]] = {}
    for i, k in enumerate(kernels):
        for name in {v.buffer.name for v in k.reads()}:
            readers.setdefault(name, []).append(i)
    replace: dict[int, list] = {}
    removed: set[int] = set()
    merged = 0
    for i, p in enumerate(kernels):
        if i in removed or not isinstance(p, PointwiseKernel) or len(p.outputs) != 1:
            continue
        out = p.outputs[0].value
        copies = readers.get(out.buffer.name, [])
        if (not copies or out.buffer.name in graph_outputs or not p.outputs[0].index.is_identity()
                or math.prod(p.space) != out.buffer.numel
                or not all(is_pure_copy(kernels[j]) for j in copies)):
            continue
        fused = []
        for j in copies:
            c = kernels[j]
            inputs = []
            for a in p.inputs:
                lay = compose(c.inputs[0].value.layout, a.index)
                if lay is None:
                    break
                inputs.append(KernelArg(a.value, flat_index(c.space, lay)))
            else:
                fused.append(PointwiseKernel(
                    name=c.name if len(copies) > 1 else p.name, space=c.space, inputs=inputs,
                    outputs=list(c.outputs), body=list(p.body),
                    out_expr={c.outputs[0].value.name: p.out_expr[out.name]},
                    nodes=list(p.nodes) + list(c.nodes)))
                continue
            break
        if len(fused) != len(copies):
            continue
        replace[i] = fused
        removed.update(copies)
        merged += len(copies)
    new: list = []
    for idx, k in enumerate(kernels):
        if idx in replace:
            new.extend(replace[idx])
        elif idx not in removed:
            new.append(k)
    schedule.kernels = new
    return merged
