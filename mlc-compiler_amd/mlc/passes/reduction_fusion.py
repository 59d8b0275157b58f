"""Reduction fusion: keep a row resident and do everything to it there.

Producers are pulled into a reduction (the scale and mask before softmax),
consumers of its result are pulled in (layer norm's normalise and affine),
and sibling reductions over the same row share one load (mean and variance).
A group runs in one (row, column) frame: kept dims are rows, reduced dims the
column axis.

Reference behaviour followed: ``mlc/passes/reduction_fusion.py:55-379``:
frame classification, storability, the legality checks and the fixed-point
growth loop with its neighbour visiting order. Two changes, each only where
the reference fails: a merge is refused when a member would read another
member's value through an index map other than the one the kernel holds it at
(the reference groups such producers and its kernel reads memory it never
wrote); and a reduction's own result is classified by its producer, not by
its shape alone (``classify_value``; the reference refuses graphs where that
shape also right-aligns onto the element shape).
"""

from __future__ import annotations

import math
from typing import Iterable

from ..config import Config
from ..ir.graph import Graph, Node, Value
from ..ir.ops import REDUCE_KINDS, OpClass, lookup, op_class
from ..ir.shapes import ShapeError, broadcast_shapes
from . import cost as costmod
from .fusion import _saved_traffic
from .scheduler import GroupGraph, UseInfo


def _prod(shape) -> int:
    return math.prod(shape) if shape else 1


class Frame:
    """(row, column) iteration frame of a reduction group."""

    __slots__ = ("element", "reduce_dims", "row", "col", "order")

    def __init__(self, element: tuple[int, ...], reduce_dims: tuple[int, ...]) -> None:
        self.element = tuple(element)
        rank = len(self.element)
        self.reduce_dims = tuple(sorted(d % rank for d in reduce_dims))
        kept = [i for i in range(rank) if i not in self.reduce_dims]
        self.row = tuple(self.element[i] for i in kept)
        self.col = tuple(self.element[i] for i in self.reduce_dims)
        #: kept dims first, reduced dims last
        self.order = tuple(kept) + self.reduce_dims

    @property
    def n_rows(self) -> int:
        return _prod(self.row)

    @property
    def n_cols(self) -> int:
        return _prod(self.col)

    @property
    def trailing(self) -> bool:
        """The reduced dims are the innermost ones."""
        rank = len(self.element)
        return self.reduce_dims == tuple(range(rank - len(self.col), rank))

    def __eq__(self, other) -> bool:
        return (isinstance(other, Frame) and self.element == other.element
                and self.reduce_dims == other.reduce_dims)

    def __hash__(self) -> int:
        return hash((self.element, self.reduce_dims))

    def __repr__(self) -> str:  # pragma: no cover
        return f"Frame({list(self.element)} reduce {list(self.reduce_dims)})"


def frame_of(node: Node) -> Frame | None:
    spec = lookup(node.op)
    if spec is None or spec.reduce is None:
        return None
    src = node.args[0]
    if not isinstance(src, Value):
        return None
    _, dims, _ = spec.reduce(list(node.args), dict(node.kwargs))
    return Frame(src.shape, dims)


def reduce_kind(node: Node) -> str:
    kind, _, _ = lookup(node.op).reduce(list(node.args), dict(node.kwargs))
    return kind


COMPOSITE = {"mean", "var", "var_mean"}


def is_associative(kind: str) -> bool:
    if kind in COMPOSITE:
        return True
    spec = REDUCE_KINDS.get(kind)
    return spec is not None and spec.associative


ELEMENT, ROW, ILLEGAL = "element", "row", None


def _broadcasts_to(shape, target) -> bool:
    try:
        return broadcast_shapes([tuple(shape), tuple(target)]) == tuple(target)
    except ShapeError:
        return False


def classify(shape: tuple[int, ...], frame: Frame) -> str | None:
    """ROW: constant along every reduced axis (a scalar per program);
    ELEMENT: varies along the column axis; None: no place in the frame."""
    shape = tuple(shape)
    rank = len(frame.element)
    if _broadcasts_to(shape, frame.element):
        aligned = (1,) * (rank - len(shape)) + shape
        return ROW if all(aligned[d] == 1 for d in frame.reduce_dims) else ELEMENT
    if shape == frame.row:
        return ROW
    if frame.row and _broadcasts_to(shape, frame.row):
        return ROW
    if _prod(shape) == 1:
        return ROW
    if frame.trailing:
        # a row-major reshape of the element or row shape addresses the same
        # elements in the same order when the reduced axes are innermost
        k = len(frame.col)
        if k and len(shape) > k and shape[-k:] == frame.col and _prod(shape[:-k]) == frame.n_rows:
            return ELEMENT
        if _prod(shape) == frame.n_rows:
            return ROW
    return ILLEGAL


def frame_axes(shape: tuple[int, ...], frame: Frame) -> list[tuple[str, tuple[int, ...]]]:
    """The (row, col) split to index a value of ``shape``: the frame's own, or
    for a reshaped element shape its own leading dims as the row axis."""
    shape = tuple(shape)
    k = len(frame.col)
    if (frame.trailing and k and len(shape) > k and shape[-k:] == frame.col
            and _prod(shape[:-k]) == frame.n_rows and shape != frame.element):
        return [("row", shape[:-k]), ("col", frame.col)]
    return [("row", frame.row), ("col", frame.col)]


def classify_value(v: Value, frame: Frame) -> str | None:
    """``classify`` for a value of the graph. A reduction's own keepdim=False
    result is a row value even when its shape also right-aligns onto the
    element shape (``[1, 128]`` against ``[1, 128, 128]``: LayerNorm with
    batch 1 and rows as long as the sequence). The reference classifies by
    shape alone there, so its lowering refuses every graph holding such a
    reduction (``reduction_lowering.py:242``); nothing it compiles changes."""
    p = v.producer
    if (p is not None and op_class(p.op) is OpClass.REDUCTION and tuple(v.shape) == frame.row
            and frame_of(p) == frame):
        return ROW
    return classify(v.shape, frame)


def storable_value(v: Value, frame: Frame) -> bool:
    """``storable`` for a value of the graph (see ``classify_value``)."""
    if classify_value(v, frame) == ROW:
        return _prod(v.shape) == frame.n_rows
    return storable(v.shape, frame)


def storable(shape: tuple[int, ...], frame: Frame) -> bool:
    """True when every point of ``shape`` is visited exactly once."""
    where = classify(shape, frame)
    n = _prod(shape)
    if where == ROW:
        return n == frame.n_rows
    if where == ELEMENT:
        return n == frame.n_rows * frame.n_cols
    return False


def _group_frame(nodes: Iterable[Node]) -> Frame | None:
    frames = {frame_of(n) for n in nodes if op_class(n.op) is OpClass.REDUCTION}
    frames.discard(None)
    return next(iter(frames)) if len(frames) == 1 else None


def _members_fit(nodes: Iterable[Node], frame: Frame) -> bool:
    for n in nodes:
        cls = op_class(n.op)
        if cls is OpClass.REDUCTION:
            if frame_of(n) != frame or not is_associative(reduce_kind(n)):
                return False
            if any(classify_value(o, frame) != ROW for o in n.outputs):
                return False
            continue
        if cls is not OpClass.POINTWISE:
            return False
        if any(classify(o.shape, frame) is ILLEGAL for o in n.outputs):
            return False
    return True


def _escape_ok(nodes, frame: Frame, uses: UseInfo, member_ids: set[int]) -> bool:
    for n in nodes:
        for o in n.outputs:
            if storable_value(o, frame):
                continue
            if uses.escapes(o) or not uses.consumers(o) <= member_ids:
                return False
    return True


def _profitable(gg: GroupGraph, a: int, b: int, frame: Frame, uses: UseInfo,
                member_ids: set[int], cfg: Config) -> bool:
    left = gg.group_members(gg.find(a))
    right = gg.group_members(gg.find(b))
    stores, loads = _saved_traffic(left, right, uses, member_ids)
    if not loads:
        # siblings share the load of the row rather than an intermediate
        if sum(op_class(n.op) is OpClass.REDUCTION for n in left + right) < 2:
            return False
        shared = {id(v.buffer) for n in left for v in n.unique_tensor_args()}
        common = [v for n in right for v in n.unique_tensor_args() if id(v.buffer) in shared]
        if not common:
            return False
        loads = common[:1]
    return bool(costmod.evaluate_merge(cfg, saved_stores=stores, saved_loads=loads,
                                       extra_loads=[], extra_evaluations=0, expr_ops=0))


def fuse_reductions(graph: Graph, gg: GroupGraph, cfg: Config, uses: UseInfo) -> None:
    """Grow every reduction group over producers, siblings and consumers,
    to a fixed point."""
    if not cfg.reduction_fusion:
        return
    seeds = [n for n in gg.nodes if op_class(n.op) is OpClass.REDUCTION]
    if not seeds:
        return
    changed = True
    while changed:
        changed = False
        for seed in seeds:
            gi = gg.group_of(seed)
            if gi is None:
                continue
            frame = _group_frame(gg.group_members(gg.find(gi)))
            if frame is None:
                continue
            for gj in _neighbours(gg, gi):
                if gg.find(gj) == gg.find(gi) or not gg.can_merge(gi, gj):
                    continue
                merged = gg.group_members(gg.find(gi)) + gg.group_members(gg.find(gj))
                if _group_frame(merged) != frame or not _members_fit(merged, frame):
                    continue
                member_ids = {id(n) for n in merged}
                if not _escape_ok(merged, frame, uses, member_ids):
                    continue
                if not _reads_held_values(merged, frame):
                    continue
                if not _profitable(gg, gi, gj, frame, uses, member_ids, cfg):
                    continue
                gi = gg.merge(gi, gj)
                changed = True


def _reads_held_values(nodes, frame: Frame) -> bool:
    # (the lowering owns the frame-to-index-map rules this compares)
    from ..codegen.reduction_lowering import reads_held_values

    return reads_held_values(nodes, frame)


def _neighbours(gg: GroupGraph, gi: int) -> list[int]:
    """Groups joined to ``gi`` by an edge, then reduction groups reading a
    buffer ``gi`` reads (how siblings find each other)."""
    root = gg.find(gi)
    out: list[int] = []
    seen: set[int] = set()
    for i in range(len(gg.nodes)):
        if gg.find(i) != root:
            continue
        for j in gg.preds[i] | gg.succs[i]:
            r = gg.find(j)
            if r != root and r not in seen:
                seen.add(r)
                out.append(r)
    read = {id(v.buffer) for n in gg.group_members(root) for v in n.unique_tensor_args()}
    for i, node in enumerate(gg.nodes):
        r = gg.find(i)
        if r == root or r in seen or op_class(node.op) is not OpClass.REDUCTION:
            continue
        if any(id(v.buffer) in read for v in node.unique_tensor_args()):
            seen.add(r)
            out.append(r)
    return out
