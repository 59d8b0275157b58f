"""Build a ReductionKernel from a fused reduction group.

Kept dims become the row axis and reduced dims the column axis; every
operand is permuted into that order and indexed over ``(row, col)``. A value
constant along ``col`` (a row statistic, a per-row bias) simply has no column
term and is a scalar per row in the kernel.

Composite reductions expand here: ``mean`` is a sum and a divide; ``var`` is
the two-pass form (mean, then the sum of squared deviations from it) over the
resident row, never ``E[x^2] - E[x]^2``. Bind steps are CSE'd, so the mean a
decomposed layer norm computes twice is bound once.

Reference behaviour followed: ``mlc/codegen/reduction_lowering.py:43-309``.
"""

from __future__ import annotations

from typing import Any

from ..config import Config
from ..ir.graph import Graph, Node, Value
from ..ir.ops import OpClass, _S, lookup, op_class
from ..ir.scalar import Const, Expr, Load, Ref, call
from ..ir.scalar import loads as expr_loads
from ..ir.scalar import substitute
from ..ir.types import Layout
from ..kernels import Bind, KernelArg, Reduce, ReductionKernel
from ..passes.reduction_fusion import (ROW, Frame, _broadcasts_to, _group_frame, classify_value,
                                       frame_axes, storable_value)
from ..passes.scheduler import source_value
from .index import IndexMap, build_index


class ReductionLoweringError(Exception):
    pass


def _row_constant_layout(v: Value, frame: Frame) -> Layout:
    """A row-shaped value with the reduced dims appended at stride 0.

    ``classify`` also places a row-major reshape of the row shape (same
    element count, e.g. ``[1, 100]`` against row ``(100,)`` when a size-1
    axis is reduced after a transpose) in the row; that value is read through
    the reshape. The reference's lowering expands it instead
    (``reduction_lowering.py:66-68``) and raises a ValueError there."""
    shape = tuple(v.shape)
    if shape == frame.row:
        lay = v.layout
    elif _broadcasts_to(shape, frame.row):
        lay = v.layout.expand(frame.row)
    else:
        lay = v.layout.reshape(frame.row)
        if lay is None:
            raise ReductionLoweringError(
                f"{v.name} {shape} is neither a broadcast nor a view of the row shape {frame.row}")
    return Layout(frame.row + frame.col, lay.strides + (0,) * len(frame.col), lay.offset)


def frame_layout(v: Value, target: tuple[int, ...], frame: Frame) -> tuple[list, Layout]:
    """Axis split and layout to read ``v`` by, for a consumer of shape ``target``."""
    target = tuple(target)
    split = [("row", frame.row), ("col", frame.col)]
    if _broadcasts_to(target, frame.element):
        lay = v.layout if tuple(v.shape) == frame.element else v.layout.expand(frame.element)
        return split, lay.permute(frame.order)
    axes = frame_axes(target, frame)
    if axes[0][1] != frame.row:
        # reshaped element shape, indexed in its own equivalent frame
        lay = v.layout if tuple(v.shape) == target else v.layout.expand(target)
        return axes, lay
    return split, _row_constant_layout(v, frame)


class _Builder:
    def __init__(self, frame: Frame) -> None:
        self.frame = frame
        self.inputs: list[KernelArg] = []
        self._slots: dict[tuple, int] = {}
        self.steps: list[Any] = []
        self.env: dict[int, tuple[Expr, IndexMap]] = {}
        self._n = 0
        self._reduces: dict[tuple, Expr] = {}
        self._binds: dict[Expr, Expr] = {}

    def fresh(self, prefix: str = "t") -> str:
        name = f"{prefix}{self._n}"
        self._n += 1
        return name

    def load(self, v: Value, imap: IndexMap) -> Expr:
        key = (id(v.buffer), v.dtype, imap)
        slot = self._slots.get(key)
        if slot is None:
            slot = self._slots[key] = len(self.inputs)
            self.inputs.append(KernelArg(v, imap))
        return Load(slot)

    def operand(self, v: Value, target: tuple[int, ...]) -> Expr:
        axes, lay = frame_layout(v, target, self.frame)
        imap = build_index(axes, lay)
        live = self.env.get(id(source_value(v)))
        if live is not None and live[1] == imap:
            return live[0]
        return self.load(v, imap)

    def bind(self, expr: Expr, prefix: str = "t") -> Expr:
        if isinstance(expr, (Load, Ref, Const)):
            return expr
        hit = self._binds.get(expr)
        if hit is not None:
            return hit
        name = self.fresh(prefix)
        self.steps.append(Bind(name, expr))
        ref = self._binds[expr] = Ref(name)
        return ref

    def reduce(self, kind: str, expr: Expr) -> Expr:
        key = (kind, expr)
        hit = self._reduces.get(key)
        if hit is not None:
            return hit
        name = self.fresh("r")
        self.steps.append(Reduce(name, kind, expr))
        ref = self._reduces[key] = Ref(name)
        return ref


def _correction(node: Node) -> float:
    kw = dict(node.kwargs)
    if "correction" in kw:
        return float(kw["correction"] or 0)
    for a in node.args[1:]:
        if isinstance(a, (int, float)) and not isinstance(a, bool):
            return float(a)
    return 0.0


def _expand_reduction(b: _Builder, node: Node, kind: str, src: Expr) -> list[Expr]:
    n = float(b.frame.n_cols)
    if kind in ("sum", "max", "min", "prod"):
        return [b.reduce(kind, src)]
    if kind == "mean":
        return [b.bind(call("div", b.reduce("sum", src), Const(n)))]
    if kind in ("var", "var_mean"):
        mean = b.bind(call("div", b.reduce("sum", src), Const(n)))
        dev = b.bind(call("sub", src, mean))
        ss = b.reduce("sum", b.bind(call("mul", dev, dev)))
        denom = n - _correction(node)
        if denom <= 0:
            raise ReductionLoweringError(f"{node.op}: correction {_correction(node)} >= n={n}")
        var = b.bind(call("div", ss, Const(denom)))
        return [var, mean] if kind == "var_mean" else [var]
    raise ReductionLoweringError(f"no lowering for reduction kind {kind!r}")


def _held_index(v: Value, frame: Frame) -> IndexMap:
    """Map a value produced in the kernel is held at (compared against later
    reads to decide register reuse)."""
    axes, lay = frame_layout(v, tuple(v.shape), frame)
    if classify_value(v, frame) == ROW and (tuple(v.shape) == frame.row
                                            or not _broadcasts_to(v.shape, frame.element)):
        lay = _row_constant_layout(v, frame)
        axes = [("row", frame.row), ("col", frame.col)]
    return build_index(axes, lay)


def reads_held_values(nodes, frame: Frame) -> bool:
    """True when every member that reads a value another member produces
    reads it at the index map the kernel holds it at, so ``_Builder.operand``
    takes it from registers. A read through another map (a permuted view of
    an in-kernel value, e.g. ``layer_norm(cos(x).transpose(2, 0))``) would
    become a load of a buffer that this kernel itself writes, or never writes.
    The reference's fusion groups such a producer and its kernel reads
    unwritten memory; the fusion pass asks this before merging instead."""
    produced = {id(o): o for n in nodes for o in n.outputs}
    for n in nodes:
        if op_class(n.op) is OpClass.REDUCTION:
            reads = [(n.args[0], tuple(n.args[0].shape))] if isinstance(n.args[0], Value) else []
        else:
            reads = [(a, tuple(n.outputs[0].shape)) for a in n.args if isinstance(a, Value)]
        for a, target in reads:
            src = source_value(a)
            if id(src) not in produced:
                continue
            try:
                axes, lay = frame_layout(a, target, frame)
                if build_index(axes, lay) != _held_index(src, frame):
                    return False
            except (ValueError, ReductionLoweringError):
                return False
    return True


def build_reduction(graph: Graph, group, stores: set[int], name: str, cfg: Config) -> ReductionKernel:
    frame = _group_frame(group.nodes)
    if frame is None:
        raise ReductionLoweringError("reduction group has no single frame: "
                                     + ", ".join(n.op for n in group.nodes))
    b = _Builder(frame)
    for node in group.nodes:
        cls = op_class(node.op)
        if cls is OpClass.REDUCTION:
            kind, _, _ = lookup(node.op).reduce(list(node.args), dict(node.kwargs))
            src_val = node.args[0]
            results = _expand_reduction(b, node, kind, b.operand(src_val, tuple(src_val.shape)))
            if len(results) < len(node.outputs):
                raise ReductionLoweringError(
                    f"{node.op} has {len(node.outputs)} outputs, lowering gave {len(results)}")
            for o, e in zip(node.outputs, results):
                b.env[id(o)] = (e, _held_index(o, frame))
            continue
        if cls is not OpClass.POINTWISE:
            raise ReductionLoweringError(f"{node.op} cannot live in a reduction kernel")
        out0 = node.outputs[0]
        target = tuple(out0.shape)
        exprs: list = []
        for a in node.args:
            if isinstance(a, Value):
                exprs.append(b.operand(a, target))
            elif isinstance(a, (bool, int, float)):
                exprs.append(_S(a))
            else:
                exprs.append(a)
        spec = lookup(node.op)
        if spec is None or spec.lower is None:
            raise ReductionLoweringError(f"no lowering rule for {node.op}")
        e = b.bind(spec.lower(list(node.args), exprs, dict(node.kwargs)))
        b.env[id(out0)] = (e, _held_index(out0, frame))

    outputs: list[KernelArg] = []
    out_expr: dict[str, Expr] = {}
    row_outputs: set[str] = set()
    for node in group.nodes:
        if id(node) not in group.owned:
            continue
        for o in node.outputs:
            if id(o) not in stores:
                continue
            if not storable_value(o, frame):
                raise ReductionLoweringError(
                    f"{node.op} result {o.name}{list(o.shape)} is broadcast inside its kernel "
                    "but escapes it; the fusion pass should not have grouped it")
            if classify_value(o, frame) == ROW:
                imap = build_index([("row", frame.row)], Layout.contiguous(frame.row))
                row_outputs.add(o.name)
            else:
                axes, lay = frame_layout(o, tuple(o.shape), frame)
                imap = build_index(axes, lay)
            outputs.append(KernelArg(o, imap))
            out_expr[o.name] = b.env[id(o)][0]

    inputs, steps = _prune(b.inputs, b.steps, out_expr)
    return ReductionKernel(name=name, row_space=frame.row, reduce_space=frame.col, inputs=inputs,
                           outputs=outputs, steps=steps, out_expr=out_expr,
                           row_outputs=row_outputs, nodes=list(group.nodes),
                           two_pass=frame.n_cols > cfg.max_persistent_row)


def _prune(inputs: list[KernelArg], steps: list, out_expr: dict[str, Expr]):
    used: set[int] = set()
    for s in steps:
        used |= expr_loads(s.expr)
    for e in out_expr.values():
        used |= expr_loads(e)
    if len(used) == len(inputs):
        return inputs, steps
    keep = sorted(used)
    mapping = {Load(old): Load(new) for new, old in enumerate(keep)}
    for s in steps:
        s.expr = substitute(s.expr, mapping)
    for k in list(out_expr):
        out_expr[k] = substitute(out_expr[k], mapping)
    return [inputs[i] for i in keep], list(steps)
