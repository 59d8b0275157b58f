"""Grouping machinery shared by the fusion passes.

:class:`GroupGraph` partitions the non-view nodes into kernel groups with a
union-find that refuses any merge creating a cycle between groups: two groups
may merge only if no third group lies on a path between them. Reachability
over the quotient DAG is kept exact as integer bitsets of ancestors and
descendants per group root.

Reference behaviour followed: ``mlc/passes/scheduler.py:21-229``. The
direct-edge sets are built in the same order as the reference's, because the
reduction pass visits neighbour groups in set-iteration order and that order
decides which merges happen first.
"""

from __future__ import annotations

import heapq
from typing import Iterable

from ..ir.graph import Graph, Node, Value
from ..ir.ops import OpClass, op_class


def _is_view(node: Node) -> bool:
    return op_class(node.op) is OpClass.VIEW


def defining_node(v: Value) -> Node | None:
    """The node that computes ``v``'s data, looking through view chains."""
    n = v.producer
    while n is not None and _is_view(n):
        src = n.args[0]
        if not isinstance(src, Value):
            return n
        n = src.producer
    return n


def source_value(v: Value) -> Value:
    """The value that owns ``v``'s buffer, looking through view chains."""
    n = v.producer
    while n is not None and _is_view(n):
        src = n.args[0]
        if not isinstance(src, Value):
            break
        v = src
        n = src.producer
    return v


class GroupGraph:
    """Cycle-safe union-find over the schedulable (non-view) nodes."""

    def __init__(self, graph: Graph, nodes: Iterable[Node] | None = None) -> None:
        self.graph = graph
        pool = graph.nodes if nodes is None else nodes
        self.nodes = [n for n in pool if not _is_view(n)]
        self.index = {id(n): i for i, n in enumerate(self.nodes)}
        count = len(self.nodes)
        self.parent = list(range(count))
        self.members: list[list[int]] = [[i] for i in range(count)]

        self.preds: list[set[int]] = [set() for _ in range(count)]
        self.succs: list[set[int]] = [set() for _ in range(count)]
        for i, node in enumerate(self.nodes):
            for v in node.unique_tensor_args():
                d = defining_node(v)
                if d is None:
                    continue
                j = self.index.get(id(d))
                if j is not None and j != i:
                    self.preds[i].add(j)
                    self.succs[j].add(i)

        # nodes are in topological order, so one sweep each way closes the sets
        self.anc = [0] * count
        self.desc = [0] * count
        for i in range(count):
            acc = 0
            for j in self.preds[i]:
                acc |= (1 << j) | self.anc[j]
            self.anc[i] = acc
        for i in reversed(range(count)):
            acc = 0
            for j in self.succs[i]:
                acc |= (1 << j) | self.desc[j]
            self.desc[i] = acc

    def find(self, i: int) -> int:
        root = i
        while self.parent[root] != root:
            root = self.parent[root]
        while self.parent[i] != root:  # path compression
            self.parent[i], i = root, self.parent[i]
        return root

    def group_of(self, node: Node) -> int | None:
        i = self.index.get(id(node))
        return None if i is None else self.find(i)

    def group_members(self, root: int) -> list[Node]:
        return [self.nodes[i] for i in sorted(self.members[root])]

    def can_merge(self, a: int, b: int) -> bool:
        a, b = self.find(a), self.find(b)
        if a == b:
            return True
        pair = (1 << a) | (1 << b)
        between = ((self.desc[a] & self.anc[b]) | (self.desc[b] & self.anc[a])) & ~pair
        return between == 0

    def merge(self, a: int, b: int) -> int:
        a, b = self.find(a), self.find(b)
        if a == b:
            return a
        if not self.can_merge(a, b):
            raise ValueError("merge would create a cycle")
        keep, gone = min(a, b), max(a, b)
        pair = (1 << a) | (1 << b)
        self.parent[gone] = keep
        self.members[keep].extend(self.members[gone])
        self.members[gone] = []

        up = (self.anc[a] | self.anc[b]) & ~pair
        down = (self.desc[a] | self.desc[b]) & ~pair
        kbit, gbit = 1 << keep, 1 << gone
        for i in range(len(self.nodes)):
            if self.anc[i] & gbit:
                self.anc[i] = (self.anc[i] & ~gbit) | kbit
            if self.desc[i] & gbit:
                self.desc[i] = (self.desc[i] & ~gbit) | kbit
        self.anc[keep], self.desc[keep] = up, down
        self.anc[gone] = self.desc[gone] = 0
        # paths through the merged group connect its ancestors to its descendants
        for i in range(len(self.nodes)):
            if self.find(i) != i:
                continue
            bit = 1 << i
            if down & bit:
                self.anc[i] |= up | kbit
            if up & bit:
                self.desc[i] |= down | kbit
        return keep

    def roots_in_order(self) -> list[int]:
        """Group roots in a topological order; ties go to the group whose
        earliest member comes first in program order."""
        roots = [i for i in range(len(self.nodes)) if self.find(i) == i and self.members[i]]
        earliest = {r: min(self.members[r]) for r in roots}
        indegree = {r: 0 for r in roots}
        edges: dict[int, set[int]] = {r: set() for r in roots}
        for i in range(len(self.nodes)):
            gi = self.find(i)
            for j in self.preds[i]:
                gj = self.find(j)
                if gi != gj and gi not in edges[gj]:
                    edges[gj].add(gi)
                    indegree[gi] += 1
        ready = [(earliest[r], r) for r in roots if indegree[r] == 0]
        heapq.heapify(ready)
        order: list[int] = []
        while ready:
            _, r = heapq.heappop(ready)
            order.append(r)
            for s in edges[r]:
                indegree[s] -= 1
                if indegree[s] == 0:
                    heapq.heappush(ready, (earliest[s], s))
        if len(order) != len(roots):
            raise RuntimeError("group graph has a cycle; a merge check is wrong")
        return order


class UseInfo:
    """Consumers of each value with view chains collapsed."""

    def __init__(self, graph: Graph) -> None:
        self.graph = graph
        self._users = graph.use_map()
        self._memo: dict[int, frozenset[int]] = {}
        self.escaping_buffers = {id(v.buffer) for v in graph.outputs}

    def consumers(self, v: Value) -> frozenset[int]:
        """ids of the non-view nodes reading ``v`` directly or through views."""
        key = id(v)
        hit = self._memo.get(key)
        if hit is not None:
            return hit
        self._memo[key] = frozenset()
        found: set[int] = set()
        for u in self._users.get(key, []):
            if _is_view(u):
                for o in u.outputs:
                    found |= self.consumers(o)
            else:
                found.add(id(u))
        result = frozenset(found)
        self._memo[key] = result
        return result

    def escapes(self, v: Value) -> bool:
        return id(v.buffer) in self.escaping_buffers

    def node_consumers(self, node: Node) -> frozenset[int]:
        found: set[int] = set()
        for o in node.outputs:
            found |= self.consumers(o)
        return frozenset(found)
