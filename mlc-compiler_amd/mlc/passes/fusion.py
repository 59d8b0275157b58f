"""The fusion plan: which nodes share a kernel, in which order kernels run.

``plan`` runs three passes over one :class:`GroupGraph` partition:

1. **Elementwise** (``_Elementwise``): in program order, each pointwise node
   tries to join the group of each pointwise producer it reads. A set of
   nodes is *coherent* over the iteration space of its largest output when
   every output either has the space's element count (a row-major reshape:
   the flat index names the same element) or broadcasts into it. Outputs that
   broadcast are re-evaluated at every point, so nothing outside the group
   may need them (escape rule), and no member may read another's value at a
   different index than it is held at (``lower.reads_are_local``). The merge
   must then pay for itself in bytes (``grouping.evaluate_merge``): stores and
   loads saved plus a launch, against re-evaluating work a group does over a
   smaller space than the merged one.
2. **Reductions** (``reduction_fusion.fuse_reductions``) grow reduction groups
   over producers, siblings and consumers.
3. **Recompute** (``_Recompute``), on the materialised groups: a cheap
   pointwise group read by two or more other pointwise groups is copied into
   each of them when that beats storing it once and loading it in each.

The candidate orders, coherence and escape rules and prices reproduce the
reference's elementwise and recompute passes (``mlc/passes/fusion.py:32-381``),
because they decide the schedule, which is held bit-exact.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

from ..config import Config
from ..ir.graph import Graph, Node, Value
from ..ir.ops import OpClass, is_pointwise, op_class
from ..ir.shapes import ShapeError, broadcast_shapes
from .grouping import GroupGraph, UseInfo, defining_node, evaluate_merge, saved_traffic

#: relations of an output shape to an iteration space (``_fits_space``)
FULL, BROADCAST = "full", "broadcast"

#: ops charged as expensive in the arithmetic term of the price
_TRANSCENDENTAL = frozenset({"exp", "log", "erf", "tanh", "sigmoid", "pow", "sqrt", "rsqrt",
                             "sin", "cos"})


@dataclass
class KernelGroup:
    """Nodes of one kernel. ``owned`` holds the ids of the nodes whose results
    this kernel stores; a node copied in by recompute is evaluated for its
    value only."""

    nodes: list[Node]
    owned: set[int] = field(default_factory=set)

    def __post_init__(self) -> None:
        self.owned = self.owned or {id(n) for n in self.nodes}

    @property
    def kind(self) -> str:
        classes = {op_class(n.op) for n in self.nodes}
        if OpClass.REDUCTION in classes:
            return "reduction"
        return "pointwise" if classes == {OpClass.POINTWISE} else "extern"

    def space(self) -> tuple[int, ...]:
        return group_space(self.nodes)


def group_space(nodes) -> tuple[int, ...]:
    """The shape of the output with the most elements (the earliest, in the
    order given, among equals)."""
    outs = [o for n in nodes for o in n.outputs]
    if not outs:
        return ()
    most = max(o.numel for o in outs)
    return next(o.shape for o in outs if o.numel == most)


def _fits_space(shape: tuple[int, ...], space: tuple[int, ...]) -> str | None:
    """``FULL`` (same element count), ``BROADCAST`` (broadcasts into
    ``space``) or None (no place in it)."""
    have, want = math.prod(shape), math.prod(space)
    if have == want:
        return FULL
    if have < want:
        try:
            if broadcast_shapes([tuple(shape), tuple(space)]) == tuple(space):
                return BROADCAST
        except ShapeError:
            pass
    return None


def _coherent_space(nodes) -> tuple[int, ...] | None:
    """The iteration space of ``nodes`` if every output fits it, else None."""
    space = group_space(nodes)
    fits = all(_fits_space(o.shape, space) for n in nodes for o in n.outputs)
    return space if fits else None


def _no_broadcast_escapes(nodes, space, uses: UseInfo, allowed: set[int]) -> bool:
    """Outputs evaluated per point of a larger space are read only by the
    nodes in ``allowed`` and are not graph outputs."""
    return all(not uses.escapes(o) and uses.consumers(o) <= allowed
               for n in nodes for o in n.outputs if _fits_space(o.shape, space) == BROADCAST)


def _ops_estimate(node: Node) -> int:
    """Scalar operations of one node for the price: 12 for a transcendental,
    2 otherwise."""
    name = node.op.split(".")[-2] if "." in node.op else node.op
    return 12 if name in _TRANSCENDENTAL else 2


def _register_local(nodes, space) -> bool:
    from ..lower import reads_are_local

    return reads_are_local(nodes, space)


def _in_program_order(graph: Graph, nodes) -> list[Node]:
    position = {id(n): i for i, n in enumerate(graph.nodes)}
    unique = {id(n): n for n in nodes}
    return sorted(unique.values(), key=lambda n: position[id(n)])


# --------------------------------------------------------------------------
# elementwise
# --------------------------------------------------------------------------

class _Elementwise:
    def __init__(self, gg: GroupGraph, cfg: Config, uses: UseInfo) -> None:
        self.gg, self.cfg, self.uses = gg, cfg, uses

    def run(self) -> None:
        gg = self.gg
        for node in gg.nodes:
            if not is_pointwise(node.op):
                continue
            mine = gg.group_of(node)
            for v in node.unique_tensor_args():
                producer = defining_node(v)
                if producer is None or not is_pointwise(producer.op):
                    continue
                theirs = gg.group_of(producer)
                if theirs is not None and self._should_merge(mine, theirs):
                    mine = gg.merge(mine, theirs)

    def _should_merge(self, mine: int, theirs: int) -> bool:
        gg = self.gg
        if gg.find(mine) == gg.find(theirs) or not gg.can_merge(mine, theirs):
            return False
        a, b = gg.group_members(gg.find(mine)), gg.group_members(gg.find(theirs))
        joined = a + b
        space = _coherent_space(joined)
        if space is None:
            return False
        ids = {id(n) for n in joined}
        if not _no_broadcast_escapes(joined, space, self.uses, ids):
            return False
        return _register_local(joined, space) and self._pays(a, b, space, ids)

    def _pays(self, a: list[Node], b: list[Node], space, ids: set[int]) -> bool:
        stores, loads = saved_traffic(a, b, self.uses, ids)
        size = math.prod(space)
        repeats, ops = 0, 0
        for part in (a, b):
            own = math.prod(group_space(part))
            if own < size:  # this part's work now runs at every point of the space
                repeats += size - own
                ops = max(ops, sum(map(_ops_estimate, part)))
        return bool(evaluate_merge(self.cfg, saved_stores=stores, saved_loads=loads,
                                   extra_loads=[], extra_evaluations=repeats, expr_ops=ops))


# --------------------------------------------------------------------------
# recompute
# --------------------------------------------------------------------------

class _Recompute:
    """Copy a cheap pointwise group into each pointwise group reading it,
    one group per round, until no group qualifies."""

    def __init__(self, graph: Graph, cfg: Config, uses: UseInfo) -> None:
        self.graph, self.cfg, self.uses = graph, cfg, uses

    def run(self, groups: list[KernelGroup]) -> list[KernelGroup]:
        while True:
            owner = {id(n): gi for gi, g in enumerate(groups) for n in g.nodes if id(n) in g.owned}
            chosen = next((gi for gi in range(len(groups))
                           if self._inline_everywhere(groups, gi, owner)), None)
            if chosen is None:
                return groups
            groups = groups[:chosen] + groups[chosen + 1:]

    def _inline_everywhere(self, groups: list[KernelGroup], gi: int, owner: dict) -> bool:
        """Inline group ``gi`` into all its reader groups if legal and
        profitable; True when it did (the group is then dropped)."""
        g = groups[gi]
        if g.kind != "pointwise":
            return False
        produced = [o for n in g.nodes if id(n) in g.owned for o in n.outputs]
        if any(self.uses.escapes(o) for o in produced):
            return False
        readers = {owner[c] for o in produced for c in self.uses.consumers(o)
                   if owner.get(c, gi) != gi}
        if len(readers) < 2:  # one reader: ordinary merging already decided
            return False
        targets = [groups[r] for r in readers]
        if not self._legal(g, targets) or not self._pays(g, targets, produced):
            return False
        for t in targets:
            present = {id(n) for n in t.nodes}
            t.nodes = _in_program_order(self.graph, t.nodes + [n for n in g.nodes
                                                               if id(n) not in present])
        return True

    def _legal(self, producer: KernelGroup, targets: list[KernelGroup]) -> bool:
        # escape is judged against every copy at once: after inlining, a value
        # read by two targets is held by both and has escaped nothing
        if any(t.kind != "pointwise" for t in targets):
            return False
        everyone = {id(n) for g in (producer, *targets) for n in g.nodes}
        for t in targets:
            joined = t.nodes + [n for n in producer.nodes if n not in t.nodes]
            space = _coherent_space(joined)
            if space is None or not _no_broadcast_escapes(joined, space, self.uses, everyone):
                return False
            if not _register_local(joined, space):
                return False
        return True

    def _pays(self, g: KernelGroup, targets: list[KernelGroup], produced: list[Value]) -> bool:
        repeats = sum(math.prod(t.space()) for t in targets) - math.prod(g.space())
        read = {id(v.buffer) for t in targets for n in t.nodes for v in n.unique_tensor_args()}
        new_loads = [v for n in g.nodes for v in n.unique_tensor_args() if id(v.buffer) not in read]
        return bool(evaluate_merge(self.cfg, saved_stores=produced,
                                   saved_loads=produced * len(targets), extra_loads=new_loads,
                                   extra_evaluations=repeats,
                                   expr_ops=sum(map(_ops_estimate, g.nodes)), saved_launches=1))


# --------------------------------------------------------------------------
# the plan
# --------------------------------------------------------------------------

def plan(graph: Graph, cfg: Config) -> list[KernelGroup]:
    """Every fusion pass, then the kernel groups in execution order."""
    from .reduction_fusion import fuse_reductions

    uses = UseInfo(graph)
    gg = GroupGraph(graph)
    if cfg.elementwise_fusion:
        _Elementwise(gg, cfg, uses).run()
    fuse_reductions(graph, gg, cfg, uses)
    groups = [KernelGroup(_in_program_order(graph, gg.group_members(r)))
              for r in gg.roots_in_order()]
    if cfg.recompute:
        groups = _Recompute(graph, cfg, uses).run(groups)
    for g in groups:
        _check_pointwise_group(g)
    return groups


def _check_pointwise_group(g: KernelGroup) -> None:
    """A pointwise group the passes produced must be coherent and read its
    own values where they are held; anything else would miscompile."""
    if g.kind != "pointwise":
        return
    listing = ", ".join(f"{n.op}{list(n.out.shape)}" for n in g.nodes)
    space = _coherent_space(g.nodes)
    if space is None:
        raise AssertionError(f"fused group has no common iteration space: {listing}")
    if not _register_local(g.nodes, space):
        raise AssertionError("fused group reads one member's value at another member's index, "
                             f"which no pointwise kernel expresses: {listing}")
