"""Kernel IR: what lowering hands to the HIP backend (and to the test oracle).

A :class:`Schedule` is the program: kernels in execution order. Every kernel
exposes the same two questions the memory planner asks -- which values it
reads (``reads``) and writes (``writes``) -- and, for the generated kinds, how
it addresses each operand (a :class:`KernelArg`: value + :class:`IndexMap`
over the kernel's iteration variables; pointers are buffer bases, view
offsets live in the map's ``base``).

Kinds:

* :class:`PointwiseKernel` -- one flat space ``idx``; ``body`` is a list of
  ``(temp, Expr)`` lines, ``out_expr`` names what each output stores.
* :class:`ReductionKernel` -- rows x columns; ``steps`` interleaves
  ``Bind`` (per-element or per-row values) and ``Reduce`` (a cross-column
  reduction) in evaluation order, so softmax is bind, reduce(max), bind,
  bind, reduce(sum), bind over one load of the row. ``row_outputs`` are
  stored once per row; ``two_pass`` marks rows streamed in chunks.
* :class:`AttentionKernel` -- bmm, the reduction over its scores and the
  bmm that consumes the probabilities, as one kernel (a schedule variant).
* :class:`ExternKernel` -- a library call (GEMMs, opaque ops).

Field names and the kinds' ``summary`` lines are the reference's kernel-IR
contract (``mlc/kernels.py:23-232``); the golden schedules record them.
"""

from __future__ import annotations

import math
from collections import Counter
from dataclasses import dataclass, field

import torch

from .codegen.index import IndexMap
from .ir.graph import Node, Value
from .ir.scalar import Expr


@dataclass
class KernelArg:
    value: Value
    index: IndexMap

    name = property(lambda self: self.value.name)
    buffer = property(lambda self: self.value.buffer)
    dtype = property(lambda self: self.value.dtype)


def _op_names(nodes: list[Node]) -> str:
    """``aten.add.Tensor`` -> ``add``, comma separated."""
    return ", ".join(n.op.rsplit(".", 2)[-2] for n in nodes)


@dataclass
class Kernel:
    name: str

    # generated kernels keep KernelArg operands; ExternKernel overrides both
    def reads(self) -> list[Value]:
        return [a.value for a in self.inputs]

    def writes(self) -> list[Value]:
        return [a.value for a in self.outputs]

    def summary(self) -> str:
        return self.name

    def _arity(self) -> str:
        return f"{len(self.inputs)}in {len(self.outputs)}out"


@dataclass
class PointwiseKernel(Kernel):
    space: tuple[int, ...]
    inputs: list[KernelArg]
    outputs: list[KernelArg]
    body: list[tuple[str, Expr]]
    out_expr: dict[str, Expr]
    nodes: list[Node] = field(default_factory=list)

    @property
    def numel(self) -> int:
        return math.prod(self.space)

    def summary(self) -> str:
        return f"{self.name}: pointwise{list(self.space)} {self._arity()} [{_op_names(self.nodes)}]"


@dataclass
class Bind:
    """A value computed in the kernel (per element, or per row when it reads
    only row values)."""

    name: str
    expr: Expr


@dataclass
class Reduce:
    """``kind`` (sum/max/min/prod) of ``expr`` across the row's columns."""

    name: str
    kind: str
    expr: Expr


Step = Bind | Reduce


@dataclass
class ReductionKernel(Kernel):
    row_space: tuple[int, ...]
    reduce_space: tuple[int, ...]
    inputs: list[KernelArg]
    outputs: list[KernelArg]
    steps: list[Step]
    out_expr: dict[str, Expr]
    row_outputs: set[str] = field(default_factory=set)
    nodes: list[Node] = field(default_factory=list)
    two_pass: bool = False

    n_rows = property(lambda self: math.prod(self.row_space))
    reduce_numel = property(lambda self: math.prod(self.reduce_space))

    @property
    def reduces(self) -> list[Reduce]:
        return [s for s in self.steps if type(s) is Reduce]

    def summary(self) -> str:
        kinds = "+".join(r.kind for r in self.reduces) or "none"
        how = "streamed" if self.two_pass else "persistent"
        return (f"{self.name}: reduction {self.n_rows}x{self.reduce_numel} {kinds} ({how}) "
                f"{self._arity()} [{_op_names(self.nodes)}]")


@dataclass
class AttentionKernel(Kernel):
    """``out = steps(q @ kt) @ v`` per batch-head, scores and probabilities
    kept in registers; their storage roundings are applied as the unfused
    schedule stores them (scores to ``score_dtype`` before the reduction's
    steps, probabilities to ``prob_dtype`` before the second product).

    ``inputs`` are q, kt, v, then the reduction's other operands (maps over
    its row/col frame); ``softmax`` is the reduction kernel it absorbed, whose
    slot ``score_slot`` read the scores."""

    q: Value
    kt: Value
    v: Value
    out: Value
    softmax: "ReductionKernel"
    score_slot: int
    score_dtype: torch.dtype
    prob_dtype: torch.dtype
    inputs: list[KernelArg]
    outputs: list[KernelArg]
    nodes: list[Node] = field(default_factory=list)

    def summary(self) -> str:
        bh, t, d = self.q.shape
        return (f"{self.name}: attention {bh}x[{t}x{d}]x[{self.kt.shape[2]}] "
                f"{len(self.inputs)}in 1out [{_op_names(self.nodes)}]")


@dataclass
class ExternKernel(Kernel):
    node: Node
    inputs: list[Value]
    outputs: list[Value]

    def reads(self) -> list[Value]:
        return list(self.inputs)

    def writes(self) -> list[Value]:
        return list(self.outputs)

    def summary(self) -> str:
        operands = "x".join(str(list(v.shape)) for v in self.inputs)
        return f"{self.name}: extern {self.node.op} {operands}"


@dataclass
class Schedule:
    graph: object
    kernels: list[Kernel] = field(default_factory=list)
    #: set by the planner
    arena_bytes: int = 0
    plan: object | None = None

    def __iter__(self):
        return iter(self.kernels)

    def __len__(self) -> int:
        return len(self.kernels)

    def counts(self) -> dict[str, int]:
        """Kernels per kind: ``{"pointwise": .., "reduction": .., ...}``."""
        return dict(Counter(type(k).__name__.removesuffix("Kernel").lower() for k in self.kernels))

    def format(self) -> str:
        lines = [f"schedule({len(self)} kernels, {self.counts()})"]
        lines += [f"  {k.summary()}" for k in self.kernels]
        if self.plan is not None:
            lines.append(f"  {self.plan.summary()}")
        return "\n".join(lines)

    def __repr__(self) -> str:  # pragma: no cover - debug aid
        return self.format()
