"""Passes over the row: how a reduction kernel's steps are traversed.

A *persistent* kernel holds its row: one pass loads it, runs every step and
stores. A *streamed* kernel (rows longer than ``max_persistent_row``)
cannot, so each reduction gets a pass of its own over memory, in step order,
and a last pass computes and stores the element outputs. A pass re-evaluates
only the binds it needs that vary along the columns; binds that read only
row values (reduction results, per-row operands) are scalars computed once
(``scalar_binds``).

One pattern collapses two streamed passes into one: a max reduction followed
by a sum of ``exp(x - max)`` of the same ``x`` (softmax). The running
recurrence ``m' = max(m, x)``, ``l' = l * exp(m - m') + exp(x - m')`` yields
both in one pass, every exponent still non-positive
(:class:`OnlineSoftmax`). The HIP streamed template and the test oracle both
follow this partition (reference counterpart:
``mlc/codegen/reduction_schedule.py:119-219``).
"""

from __future__ import annotations

from dataclasses import dataclass, field

from ..ir.scalar import Call, Expr, Load, Ref, refs, walk
from ..kernels import Bind, Reduce, ReductionKernel


@dataclass
class OnlineSoftmax:
    max_step: Reduce
    sum_step: Reduce
    #: the expression maxed over (its shift is exponentiated and summed)
    value: Expr


@dataclass
class Pass:
    #: column-varying binds evaluated in this pass, in step order
    binds: list[Bind] = field(default_factory=list)
    #: reductions accumulated in this pass (two for an online softmax)
    reduces: list[Reduce] = field(default_factory=list)
    #: element outputs stored in this pass
    stores: list[str] = field(default_factory=list)
    online_softmax: OnlineSoftmax | None = None


def dependencies(steps: list) -> dict[str, set[str]]:
    """Step name -> every step it needs, through binds; a reduction it reads is
    included but not looked behind (its result outlives the pass that made
    it, so nothing feeding it is evaluated again)."""
    kind = {s.name: s for s in steps}
    needs: dict[str, set[str]] = {}
    for s in steps:  # steps only read earlier steps, so one forward sweep does
        found: set[str] = set()
        for r in refs(s.expr):
            found.add(r)
            if not isinstance(kind.get(r), Reduce):
                found |= needs.get(r, set())
        needs[s.name] = found
    return needs


def varies_by_column(kernel: ReductionKernel) -> set[str]:
    """Names of the binds whose value differs from column to column."""
    column_slots = {i for i, a in enumerate(kernel.inputs) if a.index.varies_along("col")}
    vector: set[str] = set()
    for s in kernel.steps:
        if isinstance(s, Bind):
            slots = {x.slot for x in walk(s.expr) if isinstance(x, Load)}
            if slots & column_slots or refs(s.expr) & vector:
                vector.add(s.name)
    return vector


def scalar_binds(kernel: ReductionKernel) -> list[Bind]:
    """Binds that are one value per row (hoisted out of any column loop)."""
    vector = varies_by_column(kernel)
    return [s for s in kernel.steps if isinstance(s, Bind) and s.name not in vector]


def detect_online_softmax(kernel: ReductionKernel) -> OnlineSoftmax | None:
    """The kernel's two reductions as a max and a sum of ``exp(x - max)``
    over the same ``x``, or None."""
    reduces = kernel.reduces
    if [r.kind for r in reduces] != ["max", "sum"]:
        return None
    peak, total = reduces
    binds = {s.name: s.expr for s in kernel.steps if isinstance(s, Bind)}

    def unfold(e: Expr) -> Expr:
        while isinstance(e, Ref) and e.name in binds:
            e = binds[e.name]
        return e

    def call_of(e: Expr, fn: str) -> Call | None:
        e = unfold(e)
        return e if isinstance(e, Call) and e.fn == fn else None

    exp = call_of(total.expr, "exp")
    shift = call_of(exp.args[0], "sub") if exp is not None else None
    if shift is None or shift.args[1] != Ref(peak.name):
        return None
    if unfold(shift.args[0]) != unfold(peak.expr):
        return None
    return OnlineSoftmax(peak, total, peak.expr)


def plan_passes(kernel: ReductionKernel) -> list[Pass]:
    """The passes over the row, in the order they run."""
    element_stores = [a.value.name for a in kernel.outputs if a.value.name not in kernel.row_outputs]
    if not kernel.two_pass:
        return [Pass(binds=[s for s in kernel.steps if isinstance(s, Bind)],
                     reduces=kernel.reduces, stores=element_stores)]

    needs = dependencies(kernel.steps)
    vector = varies_by_column(kernel)

    def vector_binds(names: set[str]) -> list[Bind]:
        return [s for s in kernel.steps
                if s.name in names and isinstance(s, Bind) and s.name in vector]

    online = detect_online_softmax(kernel)
    passes: list[Pass] = []
    for r in kernel.reduces:
        if online is not None and r is online.sum_step:
            continue  # accumulated with the max by the recurrence
        if online is not None and r is online.max_step:
            # only what the maxed value needs: the shift and exponential
            # between the two reductions are the recurrence's own work
            passes.append(Pass(binds=vector_binds(needs[r.name]), reduces=[r, online.sum_step],
                               online_softmax=online))
        else:
            passes.append(Pass(binds=vector_binds(needs[r.name] | {r.name}), reduces=[r]))
    if element_stores:
        wanted: set[str] = set()
        for name in element_stores:
            for ref in refs(kernel.out_expr[name]):
                wanted |= {ref} | needs.get(ref, set())
        passes.append(Pass(binds=vector_binds(wanted), stores=element_stores))
    return passes
