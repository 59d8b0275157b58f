"""Graph IR: SSA values, each a named view onto a buffer, in topological order.

Reference behaviour followed: ``mlc/ir/graph.py:14-213``.
"""

from __future__ import annotations

import itertools
from dataclasses import dataclass, field
from typing import Any, Iterator, Sequence

import torch

from .types import Buffer, Layout


@dataclass(eq=False)
class Value:
    """One SSA value: ``layout`` read through ``buffer``."""

    name: str
    buffer: Buffer
    layout: Layout
    producer: "Node | None" = None
    index: int = 0

    @property
    def dtype(self) -> torch.dtype:
        return self.buffer.dtype

    @property
    def shape(self) -> tuple[int, ...]:
        return self.layout.shape

    @property
    def rank(self) -> int:
        return self.layout.rank

    @property
    def numel(self) -> int:
        return self.layout.numel

    def is_view_of(self, other: "Value") -> bool:
        return self.buffer is other.buffer

    def __repr__(self) -> str:  # pragma: no cover - debug aid
        return f"%{self.name}:{list(self.shape)}:{str(self.dtype).replace('torch.', '')}"

    __hash__ = object.__hash__


def _flatten_values(items) -> Iterator[Value]:
    for a in items:
        if isinstance(a, Value):
            yield a
        elif isinstance(a, (list, tuple)):
            for x in a:
                if isinstance(x, Value):
                    yield x


@dataclass(eq=False)
class Node:
    """One operation; ``op`` is the qualified ATen/prims name (or ``mlc.copy``)."""

    op: str
    args: tuple = ()
    kwargs: dict = field(default_factory=dict)
    outputs: list[Value] = field(default_factory=list)
    meta: dict = field(default_factory=dict)

    @property
    def out(self) -> Value:
        if len(self.outputs) != 1:
            raise ValueError(f"{self.op} has {len(self.outputs)} outputs")
        return self.outputs[0]

    def tensor_args(self) -> list[Value]:
        """Value operands in argument order (positional, then keyword), with repeats."""
        return list(_flatten_values(itertools.chain(self.args, self.kwargs.values())))

    def unique_tensor_args(self) -> list[Value]:
        seen: set[int] = set()
        out: list[Value] = []
        for v in self.tensor_args():
            if id(v) not in seen:
                seen.add(id(v))
                out.append(v)
        return out

    def __repr__(self) -> str:  # pragma: no cover - debug aid
        outs = ", ".join(repr(o) for o in self.outputs)
        parts = [_fmt(a) for a in self.args]
        parts += [f"{k}={_fmt(v)}" for k, v in self.kwargs.items()]
        return f"{outs} = {self.op}({', '.join(parts)})"

    __hash__ = object.__hash__


def _fmt(a: Any) -> str:
    if isinstance(a, Value):
        return f"%{a.name}"
    if isinstance(a, (list, tuple)):
        return "[" + ", ".join(_fmt(x) for x in a) + "]"
    return repr(a)


class Graph:
    """Placeholders (resident ``params`` and per-call ``inputs``), an ordered
    node list and the output values."""

    def __init__(self, name: str = "graph") -> None:
        self.name = name
        self.nodes: list[Node] = []
        self.inputs: list[Value] = []
        self.params: list[Value] = []
        self.outputs: list[Value] = []
        #: placeholder value name -> the tensor it holds
        self.param_tensors: dict[str, torch.Tensor] = {}
        #: placeholder value name -> state-dict key
        self.param_origin: dict[str, str] = {}
        self._counter = itertools.count()
        self.meta: dict = {}

    def fresh_name(self, prefix: str = "t") -> str:
        taken = {v.name for v in self.values()}
        while True:
            candidate = f"{prefix}{next(self._counter)}"
            if candidate not in taken:
                return candidate

    def new_buffer(self, shape: Sequence[int], dtype: torch.dtype,
                   kind: str = "intermediate", name: str | None = None) -> Buffer:
        return Buffer(name or self.fresh_name("buf"), tuple(shape), dtype, kind)

    def add_node(self, node: Node, before: Node | None = None) -> Node:
        if before is None:
            self.nodes.append(node)
        else:
            self.nodes.insert(self.nodes.index(before), node)
        for i, o in enumerate(node.outputs):
            o.producer = node
            o.index = i
        return node

    def placeholders(self) -> list[Value]:
        return list(self.params) + list(self.inputs)

    def values(self) -> Iterator[Value]:
        yield from self.params
        yield from self.inputs
        for n in self.nodes:
            yield from n.outputs

    def buffers(self) -> list[Buffer]:
        by_id: dict[int, Buffer] = {}
        for v in self.values():
            by_id.setdefault(id(v.buffer), v.buffer)
        return list(by_id.values())

    def use_map(self) -> dict[int, list[Node]]:
        """id(value) -> the nodes reading it, in program order."""
        uses: dict[int, list[Node]] = {}
        for n in self.nodes:
            for v in n.unique_tensor_args():
                uses.setdefault(id(v), []).append(n)
        return uses

    def users_of(self, v: Value) -> list[Node]:
        return self.use_map().get(id(v), [])

    def index_of(self, node: Node) -> int:
        return self.nodes.index(node)

    def topo_check(self) -> None:
        defined = {id(v) for v in self.placeholders()}
        for n in self.nodes:
            for v in n.unique_tensor_args():
                if id(v) not in defined:
                    raise ValueError(f"{n} reads undefined value %{v.name}")
            for o in n.outputs:
                if id(o) in defined:
                    raise ValueError(f"{n} redefines %{o.name}")
                defined.add(id(o))
        for v in self.outputs:
            if id(v) not in defined:
                raise ValueError(f"graph output %{v.name} is undefined")

    def dead_code_eliminate(self) -> int:
        live = {id(v) for v in self.outputs}
        kept: list[Node] = []
        for n in reversed(self.nodes):
            if n.meta.get("pin") or any(id(o) in live for o in n.outputs):
                kept.append(n)
                live.update(id(v) for v in n.unique_tensor_args())
        removed = len(self.nodes) - len(kept)
        self.nodes = kept[::-1]
        return removed

    def __repr__(self) -> str:  # pragma: no cover - debug aid
        from .printer import format_graph

        return format_graph(self)
