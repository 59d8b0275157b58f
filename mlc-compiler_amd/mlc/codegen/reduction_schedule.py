"""Passes over the row of a reduction kernel.

A persistent kernel makes one pass (load the row, run every step, store). A
streamed kernel (row longer than ``max_persistent_row``) makes one pass per
reduction plus a final pass for the element-space stores, except that a max
followed by ``sum(exp(x - max))`` collapses into one online-softmax pass:

    m' = max(m, max(chunk));  l' = l * exp(m - m') + sum(exp(chunk - m'))

Reference behaviour followed: ``mlc/codegen/reduction_schedule.py:23-219``.
"""

from __future__ import annotations

from dataclasses import dataclass, field

from ..ir.scalar import Call, Expr, Load, Ref, refs, walk
from ..kernels import Bind, Reduce, ReductionKernel


@dataclass
class OnlineSoftmax:
    max_step: Reduce
    sum_step: Reduce
    #: the expression being maxed, whose shift the sum exponentiates
    value: Expr


@dataclass
class Pass:
    """One traversal of the row: column-varying binds to recompute, the
    accumulators updated, and the element outputs stored."""

    binds: list[Bind] = field(default_factory=list)
    reduces: list[Reduce] = field(default_factory=list)
    stores: list[str] = field(default_factory=list)
    online_softmax: OnlineSoftmax | None = None


def dependencies(steps: list) -> dict[str, set[str]]:
    """step name -> the steps it needs, not looking past a reduce (whose
    result is a scalar that survives between passes)."""
    by_name = {s.name: s for s in steps}
    memo: dict[str, set[str]] = {}

    def need(name: str) -> set[str]:
        if name in memo:
            return memo[name]
        memo[name] = set()
        found: set[str] = set()
        step = by_name.get(name)
        if step is not None:
            for r in refs(step.expr):
                found.add(r)
                if not isinstance(by_name.get(r), Reduce):
                    found |= need(r)
        memo[name] = found
        return found

    return {s.name: need(s.name) for s in steps}


def varies_by_column(kernel: ReductionKernel) -> set[str]:
    """Bind steps that are vectors over the column axis."""
    col_slots = {i for i, a in enumerate(kernel.inputs) if a.index.varies_along("col")}
    vec: set[str] = set()
    for s in kernel.steps:
        if isinstance(s, Reduce):
            continue
        slots = {x.slot for x in walk(s.expr) if isinstance(x, Load)}
        if slots & col_slots or refs(s.expr) & vec:
            vec.add(s.name)
    return vec


def detect_online_softmax(kernel: ReductionKernel) -> OnlineSoftmax | None:
    """Exactly two reduces: a max, then a sum of ``exp(x - max)`` of the same x."""
    reds = kernel.reduces
    if len(reds) != 2 or reds[0].kind != "max" or reds[1].kind != "sum":
        return None
    first, second = reds
    by_name = {s.name: s for s in kernel.steps}

    def through_binds(e: Expr) -> Expr:
        while isinstance(e, Ref) and isinstance(by_name.get(e.name), Bind):
            e = by_name[e.name].expr
        return e

    body = through_binds(second.expr)
    if not (isinstance(body, Call) and body.fn == "exp"):
        return None
    inner = through_binds(body.args[0])
    if not (isinstance(inner, Call) and inner.fn == "sub"):
        return None
    shifted, sub = through_binds(inner.args[0]), inner.args[1]
    if not (isinstance(sub, Ref) and sub.name == first.name):
        return None
    if shifted != through_binds(first.expr):
        return None
    return OnlineSoftmax(first, second, first.expr)


def _in_order(steps: list, names: set[str]) -> list[str]:
    return [s.name for s in steps if s.name in names]


def plan_passes(kernel: ReductionKernel) -> list[Pass]:
    element_stores = [a.value.name for a in kernel.outputs
                      if a.value.name not in kernel.row_outputs]
    if not kernel.two_pass:
        return [Pass(binds=[s for s in kernel.steps if isinstance(s, Bind)],
                     reduces=kernel.reduces, stores=element_stores)]

    deps = dependencies(kernel.steps)
    vector = varies_by_column(kernel)
    by_name = {s.name: s for s in kernel.steps}
    online = detect_online_softmax(kernel)

    def vector_binds(names: set[str]) -> list[Bind]:
        return [by_name[n] for n in _in_order(kernel.steps, names)
                if isinstance(by_name[n], Bind) and n in vector]

    passes: list[Pass] = []
    reds = kernel.reduces
    i = 0
    while i < len(reds):
        r = reds[i]
        if online is not None and r is online.max_step:
            # the subtract and exp between the two reduces are subsumed by the
            # recurrence; only what the maxed expression needs is recomputed
            passes.append(Pass(binds=vector_binds(deps[r.name]),
                               reduces=[online.max_step, online.sum_step],
                               online_softmax=online))
            i += 2
            continue
        passes.append(Pass(binds=vector_binds(deps[r.name] | {r.name}), reduces=[r]))
        i += 1

    if element_stores:
        needed: set[str] = set()
        for nm in element_stores:
            for ref in refs(kernel.out_expr[nm]):
                needed.add(ref)
                needed |= deps.get(ref, set())
        passes.append(Pass(binds=vector_binds(needed), stores=element_stores))
    return passes


def scalar_binds(kernel: ReductionKernel) -> list[Bind]:
    """Bind steps constant along the row (hoisted out of streaming loops)."""
    vector = varies_by_column(kernel)
    return [s for s in kernel.steps if isinstance(s, Bind) and s.name not in vector]
