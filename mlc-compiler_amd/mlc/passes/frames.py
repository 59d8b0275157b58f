"""The (row, column) geometry of a reduction group.

A reduction kernel runs over a *frame*: the reduced dims of its reductions'
(common) input shape are the column axis, the kept dims the rows. Everything
a reduction group holds is placed in that frame:

* ``ELEMENT`` -- varies along the columns: a vector per row in the kernel;
* ``ROW`` -- constant along the columns (a reduction result, a per-row bias):
  one scalar per row;
* ``ILLEGAL`` -- no place in the frame; the value cannot join the group.

Placement follows the shape: a shape that broadcasts to the element shape is
a row value exactly when every reduced position is 1 after right-alignment
(``[B, T, 1]`` is, the weight ``[D]`` is not); a keepdim=False result has the
reduced dims removed and matches or broadcasts to the row shape. With the
reduced dims innermost, a row-major reshape of the element shape (the
``[B*T, D]`` residual add before a ``[B, T, D]`` LayerNorm) addresses the same
elements in the same order and is placed too. This is the reference's frame
classification (``mlc/passes/reduction_fusion.py:55-258``), with one
difference: a reduction's own keepdim=False result is a row value even when
its shape also right-aligns onto the element shape (``classify_value``; the
reference refuses every graph holding such a reduction, so nothing it
compiles changes).

The second half turns placements into operand layouts over ``(row, col)``
index maps, for the lowering and for the fusion check that a member reads
every in-kernel value at the index map it is held at.
"""

from __future__ import annotations

import math
from typing import Iterable

from ..codegen.index import IndexMap, build_index
from ..ir.graph import Node, Value
from ..ir.ops import OpClass, lookup, op_class
from ..ir.shapes import ShapeError, broadcast_shapes
from ..ir.types import Layout
from .grouping import source_value

ELEMENT, ROW, ILLEGAL = "element", "row", None


class ReductionLoweringError(Exception):
    pass


class Frame:
    __slots__ = ("element", "reduce_dims", "row", "col", "order")

    def __init__(self, element: tuple[int, ...], reduce_dims: Iterable[int]) -> None:
        self.element = tuple(element)
        rank = len(self.element)
        self.reduce_dims = tuple(sorted(d % rank for d in reduce_dims))
        kept = tuple(i for i in range(rank) if i not in self.reduce_dims)
        self.row = tuple(self.element[i] for i in kept)
        self.col = tuple(self.element[i] for i in self.reduce_dims)
        #: dims reordered rows first, columns last
        self.order = kept + self.reduce_dims

    n_rows = property(lambda self: math.prod(self.row))
    n_cols = property(lambda self: math.prod(self.col))

    @property
    def trailing(self) -> bool:
        """The reduced dims are the innermost ones."""
        rank = len(self.element)
        return self.reduce_dims == tuple(range(rank - len(self.col), rank))

    def split(self) -> list[tuple[str, tuple[int, ...]]]:
        return [("row", self.row), ("col", self.col)]

    def __eq__(self, other) -> bool:
        return (isinstance(other, Frame) and other.element == self.element
                and other.reduce_dims == self.reduce_dims)

    def __hash__(self) -> int:
        return hash((self.element, self.reduce_dims))

    def __repr__(self) -> str:  # pragma: no cover - debug aid
        return f"Frame({list(self.element)} reduce {list(self.reduce_dims)})"


def _reduce_spec(node: Node):
    spec = lookup(node.op)
    if spec is None or spec.reduce is None:
        return None
    return spec.reduce(list(node.args), dict(node.kwargs))


def frame_of(node: Node) -> Frame | None:
    """The frame a reduction node reduces in (None for anything else)."""
    spec = lookup(node.op)
    if spec is None or spec.reduce is None or not isinstance(node.args[0], Value):
        return None
    return Frame(node.args[0].shape, _reduce_spec(node)[1])


def reduce_kind(node: Node) -> str:
    return _reduce_spec(node)[0]


def group_frame(nodes: Iterable[Node]) -> Frame | None:
    """The one frame all reductions among ``nodes`` share, else None."""
    frames = {frame_of(n) for n in nodes if op_class(n.op) is OpClass.REDUCTION} - {None}
    return frames.pop() if len(frames) == 1 else None


def _broadcasts(shape, target) -> bool:
    try:
        return broadcast_shapes([tuple(shape), tuple(target)]) == tuple(target)
    except ShapeError:
        return False


def _reshaped_element(shape: tuple[int, ...], frame: Frame) -> bool:
    """``shape`` ends in the column dims and its leading dims hold exactly the
    frame's rows: a row-major reshape of the element shape."""
    k = len(frame.col)
    return (k > 0 and len(shape) > k and shape[-k:] == frame.col
            and math.prod(shape[:-k]) == frame.n_rows)


def classify(shape, frame: Frame) -> str | None:
    """Where a value of ``shape`` lives in ``frame``."""
    shape = tuple(shape)
    if _broadcasts(shape, frame.element):
        padded = (1,) * (len(frame.element) - len(shape)) + shape
        return ELEMENT if any(padded[d] != 1 for d in frame.reduce_dims) else ROW
    if shape == frame.row or (frame.row and _broadcasts(shape, frame.row)):
        return ROW
    if math.prod(shape) == 1:
        return ROW
    if frame.trailing:
        if _reshaped_element(shape, frame):
            return ELEMENT
        if math.prod(shape) == frame.n_rows:
            return ROW
    return ILLEGAL


def classify_value(v: Value, frame: Frame) -> str | None:
    """``classify`` for a graph value: a keepdim=False result of a reduction
    in this frame is a row value whatever else its shape matches."""
    p = v.producer
    if (p is not None and op_class(p.op) is OpClass.REDUCTION and tuple(v.shape) == frame.row
            and frame_of(p) == frame):
        return ROW
    return classify(v.shape, frame)


def frame_axes(shape, frame: Frame) -> list[tuple[str, tuple[int, ...]]]:
    """The ``(row, col)`` split to index a value of ``shape`` by: for a
    reshaped element shape its own leading dims are the row axis (the same
    elements in the same order), otherwise the frame's own split."""
    shape = tuple(shape)
    if frame.trailing and shape != frame.element and _reshaped_element(shape, frame):
        return [("row", shape[:-len(frame.col)]), ("col", frame.col)]
    return frame.split()


def _stored_once(where: str | None, shape, frame: Frame) -> bool:
    n = math.prod(tuple(shape))
    if where == ROW:
        return n == frame.n_rows
    return where == ELEMENT and n == frame.n_rows * frame.n_cols


def storable(shape, frame: Frame) -> bool:
    """Every point of ``shape`` is visited exactly once by the kernel, so a
    value of it can be stored (a broadcast one could not)."""
    return _stored_once(classify(shape, frame), shape, frame)


def storable_value(v: Value, frame: Frame) -> bool:
    where = classify_value(v, frame)
    return _stored_once(where, v.shape, frame) if where == ROW else storable(v.shape, frame)


# --------------------------------------------------------------------------
# layouts over (row, col)
# --------------------------------------------------------------------------

def _without_ones(shape) -> tuple[int, ...]:
    return tuple(d for d in shape if d != 1)


def row_constant_layout(v: Value, frame: Frame, target=None) -> Layout:
    """A row-shaped value spread over the columns with stride 0. A row-major
    reshape of the row shape (same count, e.g. ``[1, 100]`` against rows
    ``(100,)``) is read through the reshape. Read in a node whose output
    ``target`` is the row shape with size-1 dims added or dropped (a keepdim
    row value whose 1 a view moved: ``[3, 1, 4099]`` for rows ``(3, 4099)``),
    the operand broadcasts against ``target`` first, as torch aligns it."""
    shape = tuple(v.shape)
    lay = v.layout
    if target is not None:
        target = tuple(target)
        if (target != frame.row and _without_ones(target) == _without_ones(frame.row)
                and shape != target and _broadcasts(shape, target)):
            lay, shape = lay.expand(target), target
    # leading size-1 dims beyond the row's rank only align the operand with
    # a reshaped row shape (a [1, 1] scalar read at [1, R] for rows (R,));
    # broadcasting ignores them
    extra = len(shape) - len(frame.row)
    if extra > 0 and all(d == 1 for d in shape[:extra]):
        lay, shape = lay.squeeze(range(extra)), shape[extra:]
    if shape == frame.row:
        pass
    elif _broadcasts(shape, frame.row):
        lay = lay.expand(frame.row)
    else:
        lay = lay.reshape(frame.row)
        if lay is None:
            raise ReductionLoweringError(f"{v.name}{list(shape)} neither broadcasts to nor views "
                                         f"the row shape {list(frame.row)}")
    return Layout(frame.row + frame.col, lay.strides + (0,) * len(frame.col), lay.offset)


def frame_layout(v: Value, target, frame: Frame) -> tuple[list, Layout]:
    """Axis split and layout for reading ``v`` in a node whose output has
    shape ``target``."""
    target = tuple(target)
    if _broadcasts(target, frame.element):
        lay = v.layout if tuple(v.shape) == frame.element else v.layout.expand(frame.element)
        return frame.split(), lay.permute(frame.order)
    axes = frame_axes(target, frame)
    if axes[0][1] == frame.row:
        return frame.split(), row_constant_layout(v, frame, target)
    # a reshaped element shape, indexed in its own equivalent split
    return axes, v.layout if tuple(v.shape) == target else v.layout.expand(target)


def held_index(v: Value, frame: Frame) -> IndexMap:
    """The map a value computed in the kernel is held at; a later read at an
    equal map takes the register instead of loading."""
    axes, lay = frame_layout(v, v.shape, frame)
    row_value = classify_value(v, frame) == ROW
    if row_value and (tuple(v.shape) == frame.row or not _broadcasts(v.shape, frame.element)):
        axes, lay = frame.split(), row_constant_layout(v, frame)
    return build_index(axes, lay)


def _reads(node: Node) -> list[tuple[Value, tuple[int, ...]]]:
    """(operand, the shape it is read in) for each value operand."""
    if op_class(node.op) is OpClass.REDUCTION:
        src = node.args[0]
        return [(src, tuple(src.shape))] if isinstance(src, Value) else []
    target = tuple(node.outputs[0].shape)
    return [(a, target) for a in node.args if isinstance(a, Value)]


def reads_held_values(nodes, frame: Frame) -> bool:
    """Every read of a value another member computes uses the map the value
    is held at. A read through another map (a permuted view of an in-kernel
    value, ``layer_norm(cos(x).transpose(2, 0))``) would load a buffer this
    kernel writes, or never writes; the reference's fusion accepts such a
    group and its kernel reads memory it never wrote. Fusion checks this
    before merging."""
    made = {id(o) for n in nodes for o in n.outputs}
    for n in nodes:
        for a, target in _reads(n):
            src = source_value(a)
            if id(src) not in made:
                continue
            try:
                axes, lay = frame_layout(a, target, frame)
                if build_index(axes, lay) != held_index(src, frame):
                    return False
            except (ValueError, ReductionLoweringError):
                return False
    return True
