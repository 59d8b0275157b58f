"""Affine index maps from a kernel's iteration variables to buffer offsets.

    offset = base + sum over axes, over kept dims:
             ((var // out_stride) % size) * in_stride

Each axis is canonicalised by dropping size-1 dims, merging runs contiguous
in both the iteration space and the operand, and dropping stride-0 dims.
Canonical maps compare equal exactly when two operands address the same
element at every iteration, which is how fusion decides a read can reuse a
register, and the rendered string is the same text the HIP backend emits and
the CPU oracle evaluates.

Reference behaviour followed: ``mlc/codegen/index.py:36-163`` (canonical form
and rendering rules: the rendered strings are part of the kernel-IR contract).
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Sequence

from ..ir.types import Layout, contiguous_strides

Term = tuple[int, int, int]  # (size, out_stride, in_stride)


@dataclass(frozen=True)
class Axis:
    var: str
    numel: int
    #: (size, out_stride, in_stride), outermost first
    terms: tuple[Term, ...] = ()

    @property
    def is_constant(self) -> bool:
        return len(self.terms) == 0

    @property
    def is_identity(self) -> bool:
        return self.terms == ((self.numel, 1, 1),)

    def render(self) -> list[str]:
        out: list[str] = []
        for size, ostride, istride in self.terms:
            s = self.var if ostride == 1 else f"({self.var} // {ostride})"
            if size * ostride != self.numel:
                s = f"({s} % {size})"
            if istride != 1:
                s = f"{s} * {istride}"
            out.append(s)
        return out


def _join(parts: list[str]) -> str:
    if not parts:
        return "0"
    if len(parts) == 1:
        return parts[0]
    return "(" + " + ".join(parts) + ")"


@dataclass(frozen=True)
class IndexMap:
    axes: tuple[Axis, ...]
    base: int = 0

    def axis(self, var: str) -> Axis | None:
        return next((a for a in self.axes if a.var == var), None)

    def varies_along(self, var: str) -> bool:
        a = self.axis(var)
        return a is not None and not a.is_constant

    def is_identity(self) -> bool:
        return self.base == 0 and len(self.axes) == 1 and self.axes[0].is_identity

    def is_scalar(self) -> bool:
        return all(a.is_constant for a in self.axes)

    def _parts(self, skip: str | None = None) -> list[str]:
        parts: list[str] = []
        for a in self.axes:
            if a.var != skip:
                parts.extend(a.render())
        if self.base:
            parts.append(str(self.base))
        return parts

    def render(self) -> str:
        return _join(self._parts())

    def render_without(self, var: str) -> str:
        """The offset with ``var``'s contribution left out (a row base)."""
        return _join(self._parts(skip=var))

    def evaluate(self, **values: int) -> int:
        """The offset at one concrete iteration point (host-side checks)."""
        total = self.base
        for a in self.axes:
            v = values[a.var]
            for size, ostride, istride in a.terms:
                total += ((v // ostride) % size) * istride
        return total


def _simplify(space: Sequence[int], strides: Sequence[int]) -> tuple[Term, ...]:
    ostrides = contiguous_strides(space)
    terms = [(space[d], ostrides[d], strides[d]) for d in range(len(space)) if space[d] != 1]
    merged = True
    while merged and len(terms) > 1:
        merged = False
        for d in range(len(terms) - 1):
            n0, o0, i0 = terms[d]
            n1, o1, i1 = terms[d + 1]
            if o0 == o1 * n1 and i0 == i1 * n1:
                terms[d:d + 2] = [(n0 * n1, o1, i1)]
                merged = True
                break
    return tuple(t for t in terms if t[2] != 0)


def build_index(groups: Sequence[tuple[str, Sequence[int]]], layout: Layout) -> IndexMap:
    """Index map of ``layout`` under an iteration split into named groups whose
    concatenated shapes equal the layout's shape (broadcast first if not)."""
    full = tuple(int(d) for _, shape in groups for d in shape)
    if layout.shape != full:
        layout = layout.expand(full)
    axes: list[Axis] = []
    pos = 0
    for var, shape in groups:
        shp = tuple(int(d) for d in shape)
        k = len(shp)
        axes.append(Axis(var, math.prod(shp) if shp else 1,
                         _simplify(shp, layout.strides[pos:pos + k])))
        pos += k
    return IndexMap(tuple(axes), layout.offset)


def flat_index(space: Sequence[int], layout: Layout, var: str = "idx") -> IndexMap:
    return build_index([(var, space)], layout)
