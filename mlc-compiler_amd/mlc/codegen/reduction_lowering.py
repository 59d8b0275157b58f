"""A reduction group -> :class:`ReductionKernel`.

The group's frame puts kept dims on the row axis and reduced dims on the
column axis; every operand is read through a layout permuted into that order
(``passes/frames.frame_layout``), so a value that does not vary along the
columns simply has no ``col`` term in its map and is a scalar per row.

Steps are built with the shared :class:`KernelAssembler` plus value
numbering: an identical ``Bind`` expression or ``(kind, expr)`` reduction is
emitted once, so the mean a decomposed LayerNorm computes twice (once inside
``var``, once on its own) is one step. Temps share one counter across the
``t`` (bind) and ``r`` (reduce) prefixes.

Composite reductions expand here because the expansion needs the frame:
``mean`` is a sum over the columns divided by their count, and ``var`` is
the two-pass form over the resident row -- the mean, then the sum of squared
deviations from it, divided by ``n - correction`` -- never
``E[x^2] - E[x]^2``, which cancels catastrophically for the large-mean rows a
normalised activation has. The expansion and naming give the reference's
steps (``mlc/codegen/reduction_lowering.py:166-270``).
"""

from __future__ import annotations

from ..config import Config
from ..ir.graph import Graph, Node, Value
from ..ir.ops import OpClass, lookup, op_class
from ..ir.scalar import Const, Expr, Load, Ref, call, substitute
from ..ir.types import Layout
from ..kernels import Bind, KernelArg, Reduce, ReductionKernel
from ..lower import KernelAssembler
from ..passes.frames import (ROW, Frame, ReductionLoweringError, classify_value, frame_layout,
                             group_frame, held_index, reads_held_values, storable_value)
from .index import build_index

__all__ = ["ReductionLoweringError", "build_reduction", "reads_held_values"]

_PRIMITIVE = frozenset({"sum", "max", "min", "prod"})


class _ReductionAssembler(KernelAssembler):
    def __init__(self, frame: Frame) -> None:
        super().__init__()
        self.frame = frame
        self.steps: list[Bind | Reduce] = []
        self._numbered: dict[tuple, Ref] = {}

    def operand(self, v: Value, target) -> Expr:
        axes, lay = frame_layout(v, target, self.frame)
        return self.read(v, build_index(axes, lay))

    def _once(self, key: tuple, make) -> Ref:
        if key not in self._numbered:
            step = make()
            self.steps.append(step)
            self._numbered[key] = Ref(step.name)
        return self._numbered[key]

    def bind(self, expr: Expr) -> Expr:
        if isinstance(expr, (Load, Ref, Const)):
            return expr
        return self._once(("bind", expr), lambda: Bind(self.new_name("t"), expr))

    def reduce(self, kind: str, expr: Expr) -> Ref:
        return self._once(("reduce", kind, expr), lambda: Reduce(self.new_name("r"), kind, expr))


def _correction(node: Node) -> float:
    """Bessel-style correction of a var node (keyword, else the first plain
    number after the input, else 0)."""
    if "correction" in node.kwargs:
        return float(node.kwargs["correction"] or 0)
    numbers = [a for a in node.args[1:] if isinstance(a, (int, float)) and not isinstance(a, bool)]
    return float(numbers[0]) if numbers else 0.0


def _expand(asm: _ReductionAssembler, node: Node, kind: str, x: Expr) -> list[Expr]:
    """Steps of one reduction node; one expression per output."""
    if kind in _PRIMITIVE:
        return [asm.reduce(kind, x)]
    if kind not in ("mean", "var", "var_mean"):
        raise ReductionLoweringError(f"{node.op}: reduction kind {kind!r} has no expansion")
    n = float(asm.frame.n_cols)
    mean = asm.bind(call("div", asm.reduce("sum", x), Const(n)))
    if kind == "mean":
        return [mean]
    deviation = asm.bind(call("sub", x, mean))
    squares = asm.reduce("sum", asm.bind(call("mul", deviation, deviation)))
    divisor = n - _correction(node)
    if divisor <= 0:
        raise ReductionLoweringError(f"{node.op}: correction {_correction(node)} leaves no "
                                     f"degrees of freedom over {n:g} columns")
    var = asm.bind(call("div", squares, Const(divisor)))
    return [var, mean] if kind == "var_mean" else [var]


def _output_map(o: Value, frame: Frame):
    """(index map, is a row output) of a value the kernel stores."""
    if classify_value(o, frame) == ROW:
        return build_index([("row", frame.row)], Layout.contiguous(frame.row)), True
    axes, lay = frame_layout(o, tuple(o.shape), frame)
    return build_index(axes, lay), False


def build_reduction(graph: Graph, group, stores: set[int], name: str,
                    cfg: Config) -> ReductionKernel:
    frame = group_frame(group.nodes)
    if frame is None:
        raise ReductionLoweringError("the reductions of a group disagree on their frame: "
                                     + ", ".join(n.op for n in group.nodes))
    asm = _ReductionAssembler(frame)
    for node in group.nodes:
        cls = op_class(node.op)
        if cls is OpClass.REDUCTION:
            kind = lookup(node.op).reduce(list(node.args), dict(node.kwargs))[0]
            src = node.args[0]
            results = _expand(asm, node, kind, asm.operand(src, tuple(src.shape)))
            if len(results) < len(node.outputs):
                raise ReductionLoweringError(f"{node.op}: {len(node.outputs)} results, "
                                             f"{len(results)} expanded")
            for o, e in zip(node.outputs, results):
                asm.held[id(o)] = (e, held_index(o, frame))
        elif cls is OpClass.POINTWISE:
            out = node.outputs[0]
            target = tuple(out.shape)
            args = [asm.operand(a, target) if isinstance(a, Value) else asm.literal_or_passthrough(a)
                    for a in node.args]
            asm.held[id(out)] = (asm.bind(asm.lowered(node, args)), held_index(out, frame))
        else:
            raise ReductionLoweringError(f"{node.op} ({cls.value}) cannot run inside a "
                                         "reduction kernel")

    outputs, out_expr, row_outputs = [], {}, set()
    for node in group.nodes:
        if id(node) not in group.owned:
            continue
        for o in (o for o in node.outputs if id(o) in stores):
            if not storable_value(o, frame):
                raise ReductionLoweringError(f"{node.op}: {o.name}{list(o.shape)} is evaluated "
                                             "per column of its rows but escapes the kernel")
            imap, per_row = _output_map(o, frame)
            if per_row:
                row_outputs.add(o.name)
            outputs.append(KernelArg(o, imap))
            out_expr[o.name] = asm.held[id(o)][0]

    inputs, renumber = asm.compact([s.expr for s in asm.steps] + list(out_expr.values()))
    if renumber is not None:
        for s in asm.steps:
            s.expr = substitute(s.expr, renumber)
        out_expr = {k: substitute(e, renumber) for k, e in out_expr.items()}
    return ReductionKernel(name=name, row_space=frame.row, reduce_space=frame.col, inputs=inputs,
                           outputs=outputs, steps=list(asm.steps), out_expr=out_expr,
                           row_outputs=row_outputs, nodes=list(group.nodes),
                           two_pass=frame.n_cols > cfg.max_persistent_row)
