"""Reduction fusion: do everything to a row while it is resident.

Each reduction group grows, to a fixed point, over three kinds of neighbour:

* producers -- the scale and mask in front of a softmax run on the loaded row;
* consumers -- what reads the reduction's result broadcast back over the row
  (LayerNorm's normalise and affine) runs on the same registers;
* siblings -- another reduction over the same row and buffers (LayerNorm's
  mean and variance) shares the one load.

A merge must keep one frame (``frames.group_frame``), place every member in
it (reductions as row values over an associative kind, pointwise nodes
anywhere legal), keep values that are broadcast inside the kernel away from
readers outside it, read every in-kernel value at the map it is held at
(``frames.reads_held_values``), and pay in bytes like an elementwise merge;
siblings, which hand each other nothing, are priced as one row load saved.

The visiting order -- seeds in program order, each seed's neighbours edges
first (in the order the partition's edge sets iterate), then reductions that
read a buffer the group reads -- reproduces the reference's
(``mlc/passes/reduction_fusion.py:312-379``), because it decides the
schedule.
"""

from __future__ import annotations

from ..config import Config
from ..ir.graph import Graph, Node
from ..ir.ops import REDUCE_KINDS, OpClass, op_class
from .frames import (ILLEGAL, ROW, Frame, classify, classify_value, frame_of, group_frame,
                     reads_held_values, reduce_kind, storable_value)
from .grouping import GroupGraph, UseInfo, evaluate_merge, saved_traffic

#: reductions that lowering expands into several primitive ones
COMPOSITE = frozenset({"mean", "var", "var_mean"})


def is_associative(kind: str) -> bool:
    """Whether partial results of ``kind`` may be combined in any order."""
    spec = REDUCE_KINDS.get(kind)
    return kind in COMPOSITE or (spec is not None and spec.associative)


def _member_placed(node: Node, frame: Frame) -> bool:
    cls = op_class(node.op)
    if cls is OpClass.REDUCTION:
        return (frame_of(node) == frame and is_associative(reduce_kind(node))
                and all(classify_value(o, frame) == ROW for o in node.outputs))
    return cls is OpClass.POINTWISE and all(classify(o.shape, frame) is not ILLEGAL
                                            for o in node.outputs)


def _inside_only(nodes, frame: Frame, uses: UseInfo, ids: set[int]) -> bool:
    """Values the kernel cannot store (broadcast in it) are read only inside."""
    return all(not uses.escapes(o) and uses.consumers(o) <= ids
               for n in nodes for o in n.outputs if not storable_value(o, frame))


class _Growth:
    def __init__(self, gg: GroupGraph, cfg: Config, uses: UseInfo) -> None:
        self.gg, self.cfg, self.uses = gg, cfg, uses

    def run(self) -> None:
        gg = self.gg
        seeds = [n for n in gg.nodes if op_class(n.op) is OpClass.REDUCTION]
        grew = bool(seeds)
        while grew:
            grew = False
            for seed in seeds:
                mine = gg.group_of(seed)
                frame = group_frame(gg.group_members(gg.find(mine)))
                if frame is None:
                    continue
                for other in self._neighbours(mine):
                    if self._accepts(mine, other, frame):
                        mine = gg.merge(mine, other)
                        grew = True

    def _neighbours(self, g: int) -> list[int]:
        gg = self.gg
        root = gg.find(g)
        found: dict[int, None] = {}  # insertion-ordered set
        for i in range(len(gg.nodes)):
            if gg.find(i) == root:
                for j in gg.preds[i] | gg.succs[i]:
                    found.setdefault(gg.find(j))
        found.pop(root, None)
        read = {id(v.buffer) for n in gg.group_members(root) for v in n.unique_tensor_args()}
        for i, node in enumerate(gg.nodes):
            r = gg.find(i)
            if r == root or r in found or op_class(node.op) is not OpClass.REDUCTION:
                continue
            if any(id(v.buffer) in read for v in node.unique_tensor_args()):
                found[r] = None
        return list(found)

    def _accepts(self, mine: int, other: int, frame: Frame) -> bool:
        gg = self.gg
        if gg.find(mine) == gg.find(other) or not gg.can_merge(mine, other):
            return False
        a, b = gg.group_members(gg.find(mine)), gg.group_members(gg.find(other))
        joined = a + b
        if group_frame(joined) != frame or not all(_member_placed(n, frame) for n in joined):
            return False
        ids = {id(n) for n in joined}
        if not _inside_only(joined, frame, self.uses, ids) or not reads_held_values(joined, frame):
            return False
        return self._pays(a, b, ids)

    def _pays(self, a: list[Node], b: list[Node], ids: set[int]) -> bool:
        stores, loads = saved_traffic(a, b, self.uses, ids)
        if not loads:
            # siblings: what is saved is one load of a buffer both read
            if sum(op_class(n.op) is OpClass.REDUCTION for n in a + b) < 2:
                return False
            read = {id(v.buffer) for n in a for v in n.unique_tensor_args()}
            shared = [v for n in b for v in n.unique_tensor_args() if id(v.buffer) in read]
            if not shared:
                return False
            loads = shared[:1]
        return bool(evaluate_merge(self.cfg, saved_stores=stores, saved_loads=loads,
                                   extra_loads=[], extra_evaluations=0, expr_ops=0))


def fuse_reductions(graph: Graph, gg: GroupGraph, cfg: Config, uses: UseInfo) -> None:
    """Grow every reduction group in ``gg`` (a no-op with the pass off)."""
    if cfg.reduction_fusion:
        _Growth(gg, cfg, uses).run()
