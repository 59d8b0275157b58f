"""Fusion planning: which nodes share a kernel.

Elementwise fusion grows maximal pointwise chains over one iteration space
(an output that broadcasts into the space, or has the same element count as
it, fits). A member whose output is smaller than the space is recomputed per
point and so may not be visible outside the kernel (the escape rule). The
cost model decides the rest. Reduction fusion then grows reduction groups,
and recompute finally duplicates cheap multi-consumer producers.

Reference behaviour followed: ``mlc/passes/fusion.py:32-381``, including the
visiting order of the greedy loops and the tie-break in ``group_space``
(first maximal output in the order the candidate list is given), since both
decide which schedule comes out.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

from ..config import Config
from ..ir.graph import Graph, Node, Value
from ..ir.ops import OpClass, is_pointwise, op_class
from ..ir.shapes import ShapeError, broadcast_shapes
from . import cost as costmod
from .scheduler import GroupGraph, UseInfo, defining_node


def _prod(shape) -> int:
    return math.prod(shape) if shape else 1


@dataclass
class KernelGroup:
    """Nodes destined for one kernel. ``owned`` are those this kernel stores;
    nodes duplicated in by recompute are evaluated but not owned."""

    nodes: list[Node]
    owned: set[int] = field(default_factory=set)

    def __post_init__(self) -> None:
        if not self.owned:
            self.owned = {id(n) for n in self.nodes}

    @property
    def kind(self) -> str:
        classes = {op_class(n.op) for n in self.nodes}
        if OpClass.REDUCTION in classes:
            return "reduction"
        if classes == {OpClass.POINTWISE}:
            return "pointwise"
        return "extern"

    def space(self) -> tuple[int, ...]:
        return group_space(self.nodes)


def group_space(nodes) -> tuple[int, ...]:
    """The largest output shape among ``nodes`` (first one wins a tie)."""
    best: tuple[int, ...] = ()
    best_n = -1
    for n in nodes:
        for o in n.outputs:
            if o.numel > best_n:
                best, best_n = o.shape, o.numel
    return best


def _fits_space(shape: tuple[int, ...], space: tuple[int, ...]) -> str | None:
    """'full' (same element count: a row-major reshape of the space),
    'broadcast' (broadcasts into it) or None."""
    ns, nsp = _prod(shape), _prod(space)
    if ns == nsp:
        return "full"
    if ns > nsp:
        return None
    try:
        return "broadcast" if broadcast_shapes([shape, space]) == space else None
    except ShapeError:
        return None


def _merged_space(nodes) -> tuple[int, ...] | None:
    space = group_space(nodes)
    for n in nodes:
        for o in n.outputs:
            if _fits_space(o.shape, space) is None:
                return None
    return space


def _escape_ok(nodes, space, uses: UseInfo, member_ids: set[int]) -> bool:
    for n in nodes:
        for o in n.outputs:
            if _fits_space(o.shape, space) != "broadcast":
                continue
            if uses.escapes(o) or not uses.consumers(o) <= member_ids:
                return False
    return True


_TRANSCENDENTAL = ("exp", "log", "erf", "tanh", "sigmoid", "pow", "sqrt", "rsqrt", "sin", "cos")


def _estimate_ops(node: Node) -> int:
    tail = node.op.split(".")[-2] if "." in node.op else node.op
    return 12 if tail in _TRANSCENDENTAL else 2


def _reads_are_local(nodes, space) -> bool:
    from ..lower import reads_are_local

    return reads_are_local(nodes, space)


def _saved_traffic(a: list[Node], b: list[Node], uses: UseInfo, member_ids: set[int]):
    """Values that stop round-tripping through memory if ``a`` and ``b`` merge."""
    stores: list[Value] = []
    loads: list[Value] = []
    for group, other in ((a, b), (b, a)):
        other_ids = {id(n) for n in other}
        for n in group:
            for o in n.outputs:
                readers = uses.consumers(o)
                if not (readers & other_ids):
                    continue
                loads.append(o)
                if not uses.escapes(o) and readers <= member_ids:
                    stores.append(o)
    return stores, loads


def _worth_merging(gg, gi, gj, space, uses, member_ids, cfg: Config) -> bool:
    a = gg.group_members(gg.find(gi))
    b = gg.group_members(gg.find(gj))
    n_space = _prod(space)
    stores, loads = _saved_traffic(a, b, uses, member_ids)
    extra_evals = 0
    expr_ops = 0
    for group in (a, b):
        n_group = _prod(group_space(group))
        if n_group < n_space:
            extra_evals += n_space - n_group
            expr_ops = max(expr_ops, sum(_estimate_ops(n) for n in group))
    return bool(costmod.evaluate_merge(cfg, saved_stores=stores, saved_loads=loads,
                                       extra_loads=[], extra_evaluations=extra_evals,
                                       expr_ops=expr_ops))


def fuse_elementwise(graph: Graph, gg: GroupGraph, cfg: Config, uses: UseInfo) -> None:
    """Greedy, in program order: pull each pointwise node's pointwise
    producers into its group when every legality rule and the cost model agree."""
    if not cfg.elementwise_fusion:
        return
    for node in gg.nodes:
        if not is_pointwise(node.op):
            continue
        gi = gg.group_of(node)
        for v in node.unique_tensor_args():
            producer = defining_node(v)
            if producer is None or not is_pointwise(producer.op):
                continue
            gj = gg.group_of(producer)
            if gj is None or gg.find(gj) == gg.find(gi) or not gg.can_merge(gi, gj):
                continue
            merged = gg.group_members(gg.find(gi)) + gg.group_members(gg.find(gj))
            space = _merged_space(merged)
            if space is None:
                continue
            member_ids = {id(n) for n in merged}
            if not _escape_ok(merged, space, uses, member_ids):
                continue
            if not _reads_are_local(merged, space):
                continue
            if not _worth_merging(gg, gi, gj, space, uses, member_ids, cfg):
                continue
            gi = gg.merge(gi, gj)


# --------------------------------------------------------------------------
# Recompute
# --------------------------------------------------------------------------

def apply_recompute(graph: Graph, groups: list[KernelGroup], cfg: Config,
                    uses: UseInfo) -> list[KernelGroup]:
    """Duplicate a cheap pointwise producer group into each of its (two or
    more) consumer groups when that beats storing and reloading it."""
    if not cfg.recompute:
        return groups
    while True:
        owner = {id(n): gi for gi, g in enumerate(groups) for n in g.nodes if id(n) in g.owned}
        fired = False
        for gi, g in enumerate(groups):
            if g.kind != "pointwise":
                continue
            produced = [o for n in g.nodes if id(n) in g.owned for o in n.outputs]
            if any(uses.escapes(o) for o in produced):
                continue
            targets: set[int] = set()
            for o in produced:
                for cid in uses.consumers(o):
                    cg = owner.get(cid)
                    if cg is not None and cg != gi:
                        targets.add(cg)
            if len(targets) < 2:
                continue
            if not _recompute_legal(g, [groups[c] for c in targets], uses):
                continue
            if not _recompute_profitable(graph, groups, gi, targets, produced, cfg):
                continue
            for c in targets:
                present = {id(x) for x in groups[c].nodes}
                extra = [n for n in g.nodes if id(n) not in present]
                groups[c].nodes = _sorted_nodes(graph, groups[c].nodes + extra)
            groups = groups[:gi] + groups[gi + 1:]
            fired = True
            break
        if not fired:
            return groups


def _recompute_legal(producer: KernelGroup, targets: list[KernelGroup], uses: UseInfo) -> bool:
    """The merge rules per target, with the escape check made against all
    targets together (after duplication each consumer holds its own copy)."""
    if producer.kind != "pointwise" or any(t.kind != "pointwise" for t in targets):
        return False
    everyone = {id(n) for t in targets for n in t.nodes} | {id(n) for n in producer.nodes}
    for t in targets:
        merged = t.nodes + [n for n in producer.nodes if n not in t.nodes]
        space = _merged_space(merged)
        if space is None or not _escape_ok(merged, space, uses, everyone):
            return False
        if not _reads_are_local(merged, space):
            return False
    return True


def _recompute_profitable(graph, groups, gi, targets, produced, cfg) -> bool:
    g = groups[gi]
    ops = sum(_estimate_ops(n) for n in g.nodes)
    extra_evals = sum(_prod(groups[c].space()) for c in targets) - _prod(g.space())
    already = {id(v.buffer) for c in targets for n in groups[c].nodes
               for v in n.unique_tensor_args()}
    extra_loads = [v for n in g.nodes for v in n.unique_tensor_args()
                   if id(v.buffer) not in already]
    return bool(costmod.evaluate_merge(cfg, saved_stores=produced,
                                       saved_loads=produced * len(targets),
                                       extra_loads=extra_loads, extra_evaluations=extra_evals,
                                       expr_ops=ops, saved_launches=1))


def _sorted_nodes(graph: Graph, nodes) -> list[Node]:
    position = {id(n): i for i, n in enumerate(graph.nodes)}
    out: list[Node] = []
    seen: set[int] = set()
    for n in sorted(nodes, key=lambda n: position[id(n)]):
        if id(n) not in seen:
            seen.add(id(n))
            out.append(n)
    return out


def plan(graph: Graph, cfg: Config) -> list[KernelGroup]:
    """Elementwise fusion, then reduction fusion on the same group graph, then
    recompute over the materialised groups; returns groups in schedule order."""
    from .reduction_fusion import fuse_reductions

    uses = UseInfo(graph)
    gg = GroupGraph(graph)
    fuse_elementwise(graph, gg, cfg, uses)
    fuse_reductions(graph, gg, cfg, uses)
    groups = [KernelGroup(_sorted_nodes(graph, gg.group_members(r))) for r in gg.roots_in_order()]
    groups = apply_recompute(graph, groups, cfg, uses)
    _validate(groups)
    return groups


def _validate(groups: list[KernelGroup]) -> None:
    for g in groups:
        if g.kind != "pointwise":
            continue
        desc = ", ".join(f"{n.op}{list(n.out.shape)}" for n in g.nodes)
        space = _merged_space(g.nodes)
        if space is None:
            raise AssertionError("fusion produced an incoherent group: " + desc)
        if not _reads_are_local(g.nodes, space):
            raise AssertionError("fusion produced a group where one member reads another "
                                 "at a different index: " + desc)
