"""Kernel IR: the contract between the fusion passes and the backends.

A :class:`Schedule` is an ordered list of kernels. Each names the values it
reads and writes (so the planner can compute live ranges) and carries, per
operand, the index map it is read or written at. The HIP backend consumes
exactly this; the CPU oracle executes the same objects.

Reference behaviour followed: ``mlc/kernels.py:23-232``.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

from .codegen.index import IndexMap
from .ir.graph import Node, Value
from .ir.scalar import Expr


@dataclass
class KernelArg:
    """One operand and the index map it is accessed by. Kernels receive the
    buffer's base pointer; view offsets live in ``index.base``."""

    value: Value
    index: IndexMap

    @property
    def name(self) -> str:
        return self.value.name

    @property
    def buffer(self):
        return self.value.buffer

    @property
    def dtype(self) -> torch.dtype:
        return self.value.dtype


@dataclass
class Kernel:
    name: str

    def reads(self) -> list[Value]:
        raise NotImplementedError

    def writes(self) -> list[Value]:
        raise NotImplementedError

    def summary(self) -> str:
        return self.name


def _op_names(nodes) -> str:
    return ", ".join(n.op.split(".")[-2] for n in nodes)


@dataclass
class PointwiseKernel(Kernel):
    """``out_j[map_j(idx)] = body(in_k[map_k(idx)])`` for idx over ``space``."""

    space: tuple[int, ...]
    inputs: list[KernelArg]
    outputs: list[KernelArg]
    body: list[tuple[str, Expr]]
    out_expr: dict[str, Expr]
    nodes: list[Node] = field(default_factory=list)

    @property
    def numel(self) -> int:
        return math.prod(self.space) if self.space else 1

    def reads(self) -> list[Value]:
        return [a.value for a in self.inputs]

    def writes(self) -> list[Value]:
        return [a.value for a in self.outputs]

    def summary(self) -> str:
        return (f"{self.name}: pointwise{list(self.space)} "
                f"{len(self.inputs)}in {len(self.outputs)}out [{_op_names(self.nodes)}]")


@dataclass
class Bind:
    """A pointwise value computed inside a reduction kernel."""

    name: str
    expr: Expr


@dataclass
class Reduce:
    """A reduction over the column axis of the kernel's frame."""

    name: str
    kind: str  # "sum" | "max" | "min" | "prod"
    expr: Expr


Step = Bind | Reduce


@dataclass
class ReductionKernel(Kernel):
    """One row per program; ``steps`` interleave binds and reduces in order
    (softmax is bind, max, bind, bind, sum, bind)."""

    row_space: tuple[int, ...]
    reduce_space: tuple[int, ...]
    inputs: list[KernelArg]
    outputs: list[KernelArg]
    steps: list[Step]
    out_expr: dict[str, Expr]
    row_outputs: set[str] = field(default_factory=set)
    nodes: list[Node] = field(default_factory=list)
    #: the row is longer than the persistent limit and is streamed
    two_pass: bool = False

    @property
    def reduce_numel(self) -> int:
        return math.prod(self.reduce_space) if self.reduce_space else 1

    @property
    def n_rows(self) -> int:
        return math.prod(self.row_space) if self.row_space else 1

    @property
    def reduces(self) -> list[Reduce]:
        return [s for s in self.steps if isinstance(s, Reduce)]

    def reads(self) -> list[Value]:
        return [a.value for a in self.inputs]

    def writes(self) -> list[Value]:
        return [a.value for a in self.outputs]

    def summary(self) -> str:
        kinds = "+".join(r.kind for r in self.reduces) or "none"
        mode = "streamed" if self.two_pass else "persistent"
        return (f"{self.name}: reduction {self.n_rows}x{self.reduce_numel} {kinds} ({mode}) "
                f"{len(self.inputs)}in {len(self.outputs)}out [{_op_names(self.nodes)}]")


@dataclass
class AttentionKernel(Kernel):
    """``out = steps(q @ kt) @ v`` per batch-head: a batched GEMM, the row
    reduction that follows it and the batched GEMM that consumes that, as one
    kernel (a schedule variant; the reference schedule keeps three). The
    score and probability tensors are never stored, but their storage
    roundings are kept: scores are rounded to ``score_dtype`` before the
    reduction's steps and probabilities to ``prob_dtype`` before the second
    GEMM, as the unfused schedule does.

    ``inputs`` are q, kt, v, then the reduction's other inputs (index maps
    over its ``row``/``col`` frame); ``softmax`` is the original reduction
    kernel, whose slot ``score_slot`` read the scores."""

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

    def reads(self) -> list[Value]:
        return [a.value for a in self.inputs]

    def writes(self) -> list[Value]:
        return [a.value for a in self.outputs]

    def summary(self) -> str:
        bh, t, d = self.q.shape
        return (f"{self.name}: attention {bh}x[{t}x{d}]x[{self.kt.shape[2]}] "
                f"{len(self.inputs)}in 1out [{_op_names(self.nodes)}]")


@dataclass
class ExternKernel(Kernel):
    """A library call (matmul, embedding, anything opaque)."""

    node: Node
    inputs: list[Value]
    outputs: list[Value]

    def reads(self) -> list[Value]:
        return list(self.inputs)

    def writes(self) -> list[Value]:
        return list(self.outputs)

    def summary(self) -> str:
        shapes = "x".join(str(list(v.shape)) for v in self.inputs)
        return f"{self.name}: extern {self.node.op} {shapes}"


@dataclass
class Schedule:
    graph: object
    kernels: list[Kernel] = field(default_factory=list)
    arena_bytes: int = 0
    plan: object | None = None

    def __iter__(self):
        return iter(self.kernels)

    def __len__(self) -> int:
        return len(self.kernels)

    def counts(self) -> dict[str, int]:
        out: dict[str, int] = {}
        for k in self.kernels:
            key = type(k).__name__.replace("Kernel", "").lower()
            out[key] = out.get(key, 0) + 1
        return out

    def format(self) -> str:
        lines = [f"schedule({len(self.kernels)} kernels, {self.counts()})"]
        lines += ["  " + k.summary() for k in self.kernels]
        if self.plan is not None:
            lines.append("  " + self.plan.summary())
        return "\n".join(lines)

    def __repr__(self) -> str:  # pragma: no cover
        return self.format()
