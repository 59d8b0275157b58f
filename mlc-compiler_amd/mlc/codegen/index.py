"""Affine index maps: a kernel's iteration variables -> an operand's offset.

A kernel walks named iteration variables (``idx`` for a pointwise kernel,
``row``/``col`` for a reduction). Each operand is a :class:`Layout` over its
buffer, so its element offset at a point is affine in the digits of those
variables:

    offset = base + sum over variables v, over terms (size, step, stride):
             ((v // step) % size) * stride

where ``step`` is the term's stride in the iteration space (row-major over
the variable's own dims) and ``stride`` its stride in the operand. The terms
of each variable are kept *canonical* -- size-1 dims dropped, neighbours that
are contiguous in both spaces coalesced, stride-0 (broadcast) dims dropped --
so that two operands with equal maps touch the same element at every point
(the test fusion uses to replace a load by a register), and so the rendered
text is short: a contiguous operand renders as ``idx``, a bias as
``(idx % 768)``.

The rendered strings are the kernel-IR contract of the reference
(``mlc/codegen/index.py:36-163``): the CPU oracle ``eval``s them and the
golden schedules hold them, so their format is kept character for character.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Sequence

from ..ir.types import Layout, contiguous_strides

#: (size, step in the iteration space, stride in the operand)
Term = tuple[int, int, int]


def _term_text(var: str, numel: int, term: Term) -> str:
    size, step, stride = term
    text = var if step == 1 else f"({var} // {step})"
    if size * step != numel:  # the term does not reach the variable's top
        text = f"({text} % {size})"
    return text if stride == 1 else f"{text} * {stride}"


def _sum_text(parts: list[str]) -> str:
    if len(parts) > 1:
        return "(" + " + ".join(parts) + ")"
    return parts[0] if parts else "0"


@dataclass(frozen=True)
class Axis:
    """One iteration variable's contribution to the offset."""

    var: str
    numel: int
    #: canonical terms, outermost first
    terms: tuple[Term, ...] = ()

    @property
    def is_constant(self) -> bool:
        """The operand is the same along this variable (a broadcast)."""
        return not self.terms

    @property
    def is_identity(self) -> bool:
        return self.terms == ((self.numel, 1, 1),)

    def render(self) -> list[str]:
        return [_term_text(self.var, self.numel, t) for t in self.terms]


@dataclass(frozen=True)
class IndexMap:
    axes: tuple[Axis, ...]
    base: int = 0

    def axis(self, var: str) -> Axis | None:
        found = [a for a in self.axes if a.var == var]
        return found[0] if found else None

    def varies_along(self, var: str) -> bool:
        a = self.axis(var)
        return bool(a and a.terms)

    def is_identity(self) -> bool:
        return not self.base and len(self.axes) == 1 and self.axes[0].is_identity

    def is_scalar(self) -> bool:
        """One element for every iteration point."""
        return not any(a.terms for a in self.axes)

    def _text(self, leave_out: str | None) -> str:
        parts = [p for a in self.axes if a.var != leave_out for p in a.render()]
        return _sum_text(parts + ([str(self.base)] if self.base else []))

    def render(self) -> str:
        return self._text(None)

    def render_without(self, var: str) -> str:
        """The offset without ``var``'s terms: what a reduction hoists as the
        row base before walking the columns."""
        return self._text(var)

    def evaluate(self, **point: int) -> int:
        """The offset at one iteration point (host-side checks)."""
        return self.base + sum(((point[a.var] // step) % size) * stride
                               for a in self.axes for size, step, stride in a.terms)


def _canonical_terms(space: Sequence[int], strides: Sequence[int]) -> tuple[Term, ...]:
    steps = contiguous_strides(space)
    merged: list[Term] = []
    for size, step, stride in zip(space, steps, strides):
        if size == 1:
            continue
        if merged:
            o_size, o_step, o_stride = merged[-1]
            # the outer term continues this one in both spaces: one term
            if o_step == step * size and o_stride == stride * size:
                merged[-1] = (o_size * size, step, stride)
                continue
        merged.append((size, step, stride))
    return tuple(t for t in merged if t[2])


def build_index(groups: Sequence[tuple[str, Sequence[int]]], layout: Layout) -> IndexMap:
    """The map of ``layout`` when the iteration is the concatenation of the
    named ``groups`` (e.g. ``[("row", rows), ("col", cols)]``). A layout of
    fewer or size-1 dims is broadcast to the full iteration shape first."""
    groups = [(var, tuple(int(d) for d in dims)) for var, dims in groups]
    full = tuple(d for _, dims in groups for d in dims)
    if layout.shape != full:
        layout = layout.expand(full)
    axes, start = [], 0
    for var, dims in groups:
        stop = start + len(dims)
        axes.append(Axis(var, math.prod(dims), _canonical_terms(dims, layout.strides[start:stop])))
        start = stop
    return IndexMap(tuple(axes), layout.offset)


def flat_index(space: Sequence[int], layout: Layout, var: str = "idx") -> IndexMap:
    """The one-variable map of a pointwise kernel."""
    return build_index([(var, space)], layout)
