"""The program graph: SSA values over buffers, nodes in execution order.

* :class:`Value` -- a named SSA value, which is a :class:`Layout` window over
  a :class:`Buffer` (several values may share one buffer: views).
* :class:`Node` -- one op (an ``aten.*``/``prims.*`` overload name, or
  ``mlc.copy``) with positional/keyword arguments that may hold values, and
  its output values.
* :class:`Graph` -- placeholders (``params`` resident for the program's life,
  ``inputs`` copied in per call), the node list in a valid execution order,
  and the output values.

Identity, not equality, relates values and nodes (both hash by ``id``), so
the passes key their tables by ``id(value)``.
"""

from __future__ import annotations

import itertools
from dataclasses import dataclass, field
from typing import Any, Iterator, Sequence

import torch

from .types import Buffer, Layout


@dataclass(eq=False)
class Value:
    name: str
    buffer: Buffer
    layout: Layout
    #: the node that defines it (None for a placeholder)
    producer: "Node | None" = None
    #: which output of ``producer`` it is
    index: int = 0

    dtype = property(lambda self: self.buffer.dtype)
    shape = property(lambda self: self.layout.shape)
    rank = property(lambda self: self.layout.rank)
    numel = property(lambda self: self.layout.numel)

    def is_view_of(self, other: "Value") -> bool:
        """Both values are windows over the same storage."""
        return self.buffer is other.buffer

    __hash__ = object.__hash__

    def __repr__(self) -> str:  # pragma: no cover - debug aid
        return f"%{self.name}:{list(self.shape)}:{str(self.dtype).removeprefix('torch.')}"


def _values_in(items) -> Iterator[Value]:
    """Values among ``items``, looking one level into lists and tuples."""
    for item in items:
        nested = item if isinstance(item, (list, tuple)) else (item,)
        yield from (x for x in nested if isinstance(x, Value))


@dataclass(eq=False)
class Node:
    op: str
    args: tuple = ()
    kwargs: dict = field(default_factory=dict)
    outputs: list[Value] = field(default_factory=list)
    meta: dict = field(default_factory=dict)

    @property
    def out(self) -> Value:
        """The single output (raises for a multi-output node)."""
        if len(self.outputs) == 1:
            return self.outputs[0]
        raise ValueError(f"{self.op} defines {len(self.outputs)} values, not one")

    def tensor_args(self) -> list[Value]:
        """Value operands: positional then keyword, repeats kept."""
        return list(_values_in(itertools.chain(self.args, self.kwargs.values())))

    def unique_tensor_args(self) -> list[Value]:
        """Value operands in first-use order, each once."""
        return list({id(v): v for v in self.tensor_args()}.values())

    __hash__ = object.__hash__

    def __repr__(self) -> str:  # pragma: no cover - debug aid
        def show(a: Any) -> str:
            if isinstance(a, Value):
                return "%" + a.name
            if isinstance(a, (list, tuple)):
                return "[" + ", ".join(map(show, a)) + "]"
            return repr(a)

        operands = [show(a) for a in self.args] + [f"{k}={show(v)}" for k, v in self.kwargs.items()]
        return f"{', '.join(map(repr, self.outputs))} = {self.op}({', '.join(operands)})"


class Graph:
    def __init__(self, name: str = "graph") -> None:
        self.name = name
        self.params: list[Value] = []
        self.inputs: list[Value] = []
        self.nodes: list[Node] = []
        self.outputs: list[Value] = []
        #: placeholder value name -> its weight tensor
        self.param_tensors: dict[str, torch.Tensor] = {}
        #: placeholder value name -> the state-dict key it was read from
        self.param_origin: dict[str, str] = {}
        self.meta: dict = {}
        # one sequence shared by every prefix, so fresh names never collide
        self._serial = itertools.count()

    # -- building -------------------------------------------------------------
    def fresh_name(self, prefix: str = "t") -> str:
        """``prefix`` + the next serial number that names no value yet."""
        taken = {v.name for v in self.values()}
        return next(n for n in (f"{prefix}{i}" for i in self._serial) if n not in taken)

    def new_buffer(self, shape: Sequence[int], dtype: torch.dtype, kind: str = "intermediate",
                   name: str | None = None) -> Buffer:
        return Buffer(name if name else self.fresh_name("buf"), tuple(shape), dtype, kind)

    def add_node(self, node: Node, before: Node | None = None) -> Node:
        """Append ``node`` (or insert it ahead of ``before``) and make it the
        producer of its outputs."""
        at = len(self.nodes) if before is None else self.nodes.index(before)
        self.nodes.insert(at, node)
        for i, v in enumerate(node.outputs):
            v.producer, v.index = node, i
        return node

    # -- reading --------------------------------------------------------------
    def placeholders(self) -> list[Value]:
        """Every placeholder, in the compiled callable's order: params, inputs."""
        return [*self.params, *self.inputs]

    def values(self) -> Iterator[Value]:
        yield from self.placeholders()
        for n in self.nodes:
            yield from n.outputs

    def buffers(self) -> list[Buffer]:
        """Every distinct buffer, in the order its first value appears."""
        return list({id(v.buffer): v.buffer for v in self.values()}.values())

    def use_map(self) -> dict[int, list[Node]]:
        """``id(value)`` -> the nodes reading it, in program order (built fresh
        on every call, so it cannot go stale across rewrites)."""
        readers: dict[int, list[Node]] = {}
        for n in self.nodes:
            for v in n.unique_tensor_args():
                readers.setdefault(id(v), []).append(n)
        return readers

    def users_of(self, v: Value) -> list[Node]:
        return self.use_map().get(id(v), [])

    def index_of(self, node: Node) -> int:
        return self.nodes.index(node)

    # -- checks and cleanup ---------------------------------------------------
    def topo_check(self) -> None:
        """Every value is defined once, before anything reads it."""
        seen = {id(v) for v in self.placeholders()}
        for n in self.nodes:
            missing = [v for v in n.unique_tensor_args() if id(v) not in seen]
            if missing:
                raise ValueError(f"{n} reads %{missing[0].name} before it is defined")
            for v in n.outputs:
                if id(v) in seen:
                    raise ValueError(f"{n} defines %{v.name} a second time")
                seen.add(id(v))
        undefined = [v.name for v in self.outputs if id(v) not in seen]
        if undefined:
            raise ValueError(f"graph output %{undefined[0]} is never defined")

    def dead_code_eliminate(self) -> int:
        """Drop nodes that nothing live reads (``meta['pin']`` keeps a node).
        Returns how many were dropped."""
        needed = {id(v) for v in self.outputs}
        kept = []
        for n in self.nodes[::-1]:
            if not (n.meta.get("pin") or any(id(v) in needed for v in n.outputs)):
                continue
            kept.append(n)
            needed.update(id(v) for v in n.unique_tensor_args())
        dropped = len(self.nodes) - len(kept)
        self.nodes = kept[::-1]
        return dropped

    def __repr__(self) -> str:  # pragma: no cover - debug aid
        from .printer import format_graph

        return format_graph(self)
