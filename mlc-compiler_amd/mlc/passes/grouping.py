"""What every fusion pass builds on: a partition of the nodes, who reads what,
and the byte price of a merge.

**Partition.** Fusion decides which graph nodes share a kernel: a partition
of the non-view nodes (views never become kernels; whoever reads one reads
through it). A merge is legal unless a *third* group lies on a dependency
path between the two -- that group would have to run both before and after
the merged kernel. :class:`GroupGraph` keeps the partition as a union-find
and answers that question from the transitive closure of the quotient graph
(descendants and ancestors per group as bitsets), updated on each merge for
the merged pair's ancestors and descendants only. ``roots_in_order`` then
orders the groups topologically, breaking ties by each group's earliest node
in program order.

**Uses.** :class:`UseInfo` answers "which kernels read this value", with view
chains collapsed, and whether a value is a graph output (then it must be
stored whatever fusion does).

**Price.** Inference here is memory bound, so a merge is priced in bytes of
HBM traffic: the intermediates that stop round-tripping and the launch that
disappears (``Config.effective_launch_bytes``) against extra loads and extra
arithmetic (at ``Config.flops_per_byte``). ``merge_pays`` is that comparison.

The decisions these make must equal the reference's (its
``mlc/passes/scheduler.py`` and ``cost.py``), since the schedules are held
bit-exact; the closure is exact, so every legality query is answered as the
reference's answers it.
"""

from __future__ import annotations

import heapq
from dataclasses import dataclass
from typing import Iterable, Sequence

from ..config import Config
from ..ir.graph import Graph, Node, Value
from ..ir.ops import OpClass, op_class
from ..ir.types import itemsize_of


def _is_view(node: Node | None) -> bool:
    return node is not None and op_class(node.op) is OpClass.VIEW


def _through_views(v: Value) -> tuple[Value, Node | None]:
    """Follow ``v`` back through view nodes: the last value reached and its
    producer (the first node that is not a view, or a view whose source is
    not a value)."""
    while _is_view(v.producer):
        src = v.producer.args[0]
        if not isinstance(src, Value):
            break
        v = src
    return v, v.producer


def defining_node(v: Value) -> Node | None:
    """The node whose work ``v`` is, seen through any views."""
    return _through_views(v)[1]


def source_value(v: Value) -> Value:
    """The value that owns ``v``'s storage, seen through any views."""
    return _through_views(v)[0]


# --------------------------------------------------------------------------
# partition
# --------------------------------------------------------------------------

def _union(masks: Iterable[int]) -> int:
    out = 0
    for m in masks:
        out |= m
    return out


def _bits(mask: int) -> Iterable[int]:
    while mask:
        low = mask & -mask
        yield low.bit_length() - 1
        mask ^= low


class GroupGraph:
    def __init__(self, graph: Graph, nodes: Iterable[Node] | None = None) -> None:
        self.graph = graph
        self.nodes = [n for n in (graph.nodes if nodes is None else nodes) if not _is_view(n)]
        self.index = {id(n): i for i, n in enumerate(self.nodes)}
        count = len(self.nodes)
        self._parent = list(range(count))
        self._members: dict[int, list[int]] = {i: [i] for i in range(count)}
        # direct dependencies between nodes (through views), in node indices;
        # insertion order is kept: neighbour visits in reduction fusion
        # iterate these sets
        self.preds: list[set[int]] = [set() for _ in range(count)]
        self.succs: list[set[int]] = [set() for _ in range(count)]
        for i, node in enumerate(self.nodes):
            for v in node.unique_tensor_args():
                j = self.index.get(id(defining_node(v)), i)
                if j != i:
                    self.preds[i].add(j)
                    self.succs[j].add(i)
        # reachability between groups, as bitsets of group roots; exact for the
        # quotient graph at all times (see ``merge``)
        self._down: dict[int, int] = {}
        self._up: dict[int, int] = {}
        for i in range(count - 1, -1, -1):  # program order is topological
            self._down[i] = _union((1 << s) | self._down[s] for s in self.succs[i])
        for i in range(count):
            self._up[i] = _union((1 << p) | self._up[p] for p in self.preds[i])

    # -- union-find -----------------------------------------------------------
    def find(self, i: int) -> int:
        root = i
        while self._parent[root] != root:
            root = self._parent[root]
        while self._parent[i] != root:  # compress the path walked
            self._parent[i], i = root, self._parent[i]
        return root

    def group_of(self, node: Node) -> int | None:
        i = self.index.get(id(node))
        return None if i is None else self.find(i)

    def group_members(self, root: int) -> list[Node]:
        return [self.nodes[i] for i in sorted(self._members.get(root, ()))]

    def roots(self) -> list[int]:
        return sorted(self._members)

    # -- reachability -------------------------------------------------------------
    def _quotient_edges(self) -> dict[int, set[int]]:
        out: dict[int, set[int]] = {r: set() for r in self._members}
        for i, succ in enumerate(self.succs):
            gi = self.find(i)
            out[gi].update(g for g in map(self.find, succ) if g != gi)
        return out

    def can_merge(self, a: int, b: int) -> bool:
        """False when some third group depends on one of ``a``/``b`` and is
        depended on by the other."""
        a, b = self.find(a), self.find(b)
        if a == b:
            return True
        down, up = self._down, self._up
        between = (down[a] & up[b]) | (down[b] & up[a])
        return not (between & ~((1 << a) | (1 << b)))

    def merge(self, a: int, b: int) -> int:
        """Join the groups of ``a`` and ``b``; the surviving root is the lower
        index, so roots stay near program order. Returns it."""
        a, b = self.find(a), self.find(b)
        if a == b:
            return a
        if not self.can_merge(a, b):
            raise ValueError(f"joining groups {a} and {b} would make them depend on each other "
                             "through a third group")
        keep, gone = min(a, b), max(a, b)
        self._parent[gone] = keep
        self._members[keep] += self._members.pop(gone)
        # The merged group reaches what either half reached; every group that
        # reached a half now reaches the merged group and all it reaches, and
        # symmetrically upwards. No other group's reachability changes, and
        # a legal merge has no group both above and below it.
        pair = (1 << a) | (1 << b)
        below = (self._down.pop(gone) | self._down[keep]) & ~pair
        above = (self._up.pop(gone) | self._up[keep]) & ~pair
        self._down[keep], self._up[keep] = below, above
        me = 1 << keep
        for x in _bits(above):
            self._down[x] = (self._down[x] & ~pair) | me | below
        for y in _bits(below):
            self._up[y] = (self._up[y] & ~pair) | me | above
        return keep

    def roots_in_order(self) -> list[int]:
        """Group roots in an order that respects every dependency, the group
        holding the earliest node first among those that are ready."""
        edges = self._quotient_edges()
        waiting = {g: 0 for g in edges}
        for succ in edges.values():
            for s in succ:
                waiting[s] += 1
        first = {g: min(m) for g, m in self._members.items()}
        ready = [(first[g], g) for g, n in waiting.items() if n == 0]
        heapq.heapify(ready)
        order: list[int] = []
        while ready:
            _, g = heapq.heappop(ready)
            order.append(g)
            for s in edges[g]:
                waiting[s] -= 1
                if not waiting[s]:
                    heapq.heappush(ready, (first[s], s))
        if len(order) != len(edges):
            raise RuntimeError("the groups depend on each other in a cycle: a merge was "
                               "allowed that should not have been")
        return order


# --------------------------------------------------------------------------
# uses
# --------------------------------------------------------------------------

class UseInfo:
    def __init__(self, graph: Graph) -> None:
        self.graph = graph
        self._readers = graph.use_map()
        self._kernels: dict[int, frozenset[int]] = {}
        self.escaping_buffers = {id(v.buffer) for v in graph.outputs}

    def consumers(self, v: Value) -> frozenset[int]:
        """ids of the non-view nodes reading ``v``, directly or through views."""
        key = id(v)
        if key not in self._kernels:
            found: set[int] = set()
            todo = [v]
            while todo:
                for reader in self._readers.get(id(todo.pop()), ()):
                    if _is_view(reader):
                        todo.extend(reader.outputs)
                    else:
                        found.add(id(reader))
            self._kernels[key] = frozenset(found)
        return self._kernels[key]

    def escapes(self, v: Value) -> bool:
        """``v``'s buffer is a graph output, so it is stored regardless."""
        return id(v.buffer) in self.escaping_buffers

    def node_consumers(self, node: Node) -> frozenset[int]:
        return frozenset().union(*(self.consumers(o) for o in node.outputs))


# --------------------------------------------------------------------------
# price
# --------------------------------------------------------------------------

def value_bytes(v: Value) -> int:
    """Bytes a kernel moves reading or writing ``v`` (the view's elements, not
    the whole buffer: one slice of a fused qkv output is a third of it)."""
    return v.numel * itemsize_of(v.dtype)


def traffic(reads: Iterable[Value], writes: Iterable[Value]) -> int:
    """One kernel's bytes: each distinct buffer read once, every write."""
    by_buffer = {id(v.buffer): v for v in reversed(list(reads))}
    return sum(map(value_bytes, by_buffer.values())) + sum(map(value_bytes, writes))


@dataclass
class MergeDecision:
    merge: bool
    benefit: float
    cost: float
    reason: str

    def __bool__(self) -> bool:
        return self.merge


def evaluate_merge(cfg: Config, *, saved_stores: Sequence[Value], saved_loads: Sequence[Value],
                   extra_loads: Sequence[Value], extra_evaluations: int, expr_ops: int,
                   saved_launches: int = 1) -> MergeDecision:
    """Bytes saved (stores and loads that disappear, launches at their byte
    price) against bytes added (new loads, and work evaluated
    ``extra_evaluations`` more times at ``expr_ops`` operations each)."""
    saved = float(sum(map(value_bytes, saved_stores))) + float(sum(map(value_bytes, saved_loads)))
    saved += saved_launches * cfg.effective_launch_bytes
    spent = float(sum(map(value_bytes, extra_loads)))
    repeats = extra_evaluations > 0
    if repeats and expr_ops > 0:
        spent += extra_evaluations * expr_ops / max(cfg.flops_per_byte, 1e-6)
    if repeats and expr_ops > cfg.max_recompute_ops:
        return MergeDecision(False, saved, spent,
                             f"{expr_ops} operations is too much to evaluate again")
    pays = saved > spent
    return MergeDecision(pays, saved, spent, "pays" if pays else "does not pay")


def merge_pays(cfg: Config, saved_stores: Sequence[Value], saved_loads: Sequence[Value], *,
               extra_loads: Sequence[Value] = (), extra_evaluations: int = 0,
               expr_ops: int = 0) -> bool:
    return bool(evaluate_merge(cfg, saved_stores=saved_stores, saved_loads=saved_loads,
                               extra_loads=extra_loads, extra_evaluations=extra_evaluations,
                               expr_ops=expr_ops))


def saved_traffic(a: list[Node], b: list[Node], uses: UseInfo,
                  member_ids: set[int]) -> tuple[list[Value], list[Value]]:
    """What merging node groups ``a`` and ``b`` saves: every value one group
    hands the other is a load that disappears, and a store too when nothing
    outside the merged group needs it."""
    stores: list[Value] = []
    loads: list[Value] = []
    for mine, theirs in ((a, b), (b, a)):
        other = {id(n) for n in theirs}
        for v in (o for n in mine for o in n.outputs):
            readers = uses.consumers(v)
            if readers & other:
                loads.append(v)
                if readers <= member_ids and not uses.escapes(v):
                    stores.append(v)
    return stores, loads
