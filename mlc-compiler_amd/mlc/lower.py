"""Fusion groups -> kernel IR.

Each pointwise group becomes an iteration space, operands with index maps, a
body of scalar expressions and a store list. A read of a value produced in
the same kernel becomes a register reference exactly when its index map
equals the one the value was produced at (canonical maps make that an
equality test that sees through reshapes); otherwise it is a load.

Reference behaviour followed: ``mlc/lower.py:40-292``: store set, read/write
index maps, the register-reuse rule, operand slot order and input pruning,
all of which fix the operand lists and index strings the backends see.
"""

from __future__ import annotations

from .codegen.index import IndexMap, flat_index
from .config import Config
from .ir.graph import Graph, Node, Value
from .ir.ops import _S, lookup
from .ir.scalar import Const, Expr, Load, Ref
from .ir.scalar import loads as expr_loads
from .ir.scalar import substitute
from .kernels import ExternKernel, Kernel, KernelArg, PointwiseKernel, Schedule
from .passes.fusion import KernelGroup, _fits_space, group_space
from .passes.scheduler import UseInfo, source_value


class LoweringError(Exception):
    pass


def build_schedule(graph: Graph, groups: list[KernelGroup], cfg: Config) -> Schedule:
    uses = UseInfo(graph)
    stores = _store_set(graph, groups, uses)
    kernels: list[Kernel] = []
    for i, group in enumerate(groups):
        name = f"k{i}"
        kind = group.kind
        if kind == "pointwise":
            kernels.append(build_pointwise(graph, group, stores, name))
        elif kind == "reduction" and cfg.reduction_fusion:
            from .codegen.reduction_lowering import build_reduction

            kernels.append(build_reduction(graph, group, stores, name, cfg))
        else:
            if len(group.nodes) != 1:
                raise LoweringError(f"group of {len(group.nodes)} nodes has no kernel form: "
                                    f"{[n.op for n in group.nodes]}")
            node = group.nodes[0]
            kernels.append(ExternKernel(name, node, node.unique_tensor_args(), list(node.outputs)))
    return Schedule(graph, kernels)


def _store_set(graph: Graph, groups: list[KernelGroup], uses: UseInfo) -> set[int]:
    """ids of values that must reach memory: graph outputs, and values read by
    some kernel that does not compute them itself."""
    kernels_of: dict[int, set[int]] = {}
    for gi, g in enumerate(groups):
        for n in g.nodes:
            kernels_of.setdefault(id(n), set()).add(gi)
    need: set[int] = set()
    empty: set[int] = set()
    for g in groups:
        for n in g.nodes:
            mine = kernels_of.get(id(n), empty)
            for o in n.outputs:
                if uses.escapes(o):
                    need.add(id(o))
                    continue
                if any(not kernels_of.get(c, empty) <= mine for c in uses.consumers(o)):
                    need.add(id(o))
    return need


def read_index(value: Value, consumer_shape: tuple[int, ...], space: tuple[int, ...]) -> IndexMap:
    """Map at which a pointwise kernel reads ``value`` for a consumer whose
    output has ``consumer_shape``."""
    if _fits_space(consumer_shape, space) == "broadcast":
        return flat_index(space, value.layout.expand(consumer_shape).expand(space))
    frame = tuple(consumer_shape)
    lay = value.layout if tuple(value.shape) == frame else value.layout.expand(frame)
    return flat_index(frame, lay)


def write_index(value: Value, space: tuple[int, ...]) -> IndexMap:
    """Map at which ``value`` is held once computed in a kernel over ``space``."""
    if _fits_space(value.shape, space) == "full":
        return flat_index(value.shape, value.layout)
    return flat_index(space, value.layout.expand(space))


def reads_are_local(nodes, space: tuple[int, ...]) -> bool:
    """True when every read of an in-kernel value hits the same index it was
    produced at, so it can stay in the reading thread's registers."""
    produced: dict[int, IndexMap] = {}
    for n in nodes:
        for o in n.outputs:
            if _fits_space(o.shape, space) is None:
                return False
            produced[id(o)] = write_index(o, space)
    for n in nodes:
        shape = n.out.shape
        for a in n.args:
            if not isinstance(a, Value):
                continue
            at = produced.get(id(source_value(a)))
            if at is None:
                continue
            try:
                if read_index(a, shape, space) != at:
                    return False
            except ValueError:
                return False
    return True


def _prune_inputs(inputs: list[KernelArg], body, out_expr) -> list[KernelArg]:
    """Drop operands nothing reads and renumber the remaining slots."""
    used: set[int] = set()
    for _, e in body:
        used |= expr_loads(e)
    for e in out_expr.values():
        used |= expr_loads(e)
    if len(used) == len(inputs):
        return inputs
    keep = sorted(used)
    mapping = {Load(old): Load(new) for new, old in enumerate(keep)}
    for i, (nm, e) in enumerate(body):
        body[i] = (nm, substitute(e, mapping))
    for k in list(out_expr):
        out_expr[k] = substitute(out_expr[k], mapping)
    return [inputs[i] for i in keep]


class _BodyBuilder:
    def __init__(self, graph: Graph, nodes: list[Node]) -> None:
        self.graph = graph
        self.nodes = nodes
        self.inputs: list[KernelArg] = []
        self._slots: dict[tuple, int] = {}
        #: id(value) -> (expression holding it, index map it is held at)
        self.env: dict[int, tuple[Expr, IndexMap]] = {}
        self.body: list[tuple[str, Expr]] = []
        self._temps = 0

    def fresh(self) -> str:
        name = f"t{self._temps}"
        self._temps += 1
        return name

    def load(self, v: Value, imap: IndexMap) -> Expr:
        key = (id(v.buffer), v.dtype, imap)
        slot = self._slots.get(key)
        if slot is None:
            slot = self._slots[key] = len(self.inputs)
            self.inputs.append(KernelArg(v, imap))
        return Load(slot)

    def operand(self, v: Value, imap: IndexMap) -> Expr:
        live = self.env.get(id(source_value(v)))
        if live is not None and live[1] == imap:
            return live[0]
        return self.load(v, imap)

    def emit(self, node: Node, arg_exprs: list) -> Expr:
        """Lower one node; a bare load/ref/literal result gets no body line."""
        spec = lookup(node.op)
        if spec is None or spec.lower is None:
            raise LoweringError(f"no lowering rule for {node.op}")
        expr = spec.lower(list(node.args), arg_exprs, dict(node.kwargs))
        if isinstance(expr, (Load, Ref, Const)):
            return expr
        name = self.fresh()
        self.body.append((name, expr))
        return Ref(name)


def build_pointwise(graph: Graph, group: KernelGroup, stores: set[int], name: str) -> PointwiseKernel:
    nodes = group.nodes
    space = group_space(nodes)
    b = _BodyBuilder(graph, nodes)
    for node in nodes:
        out = node.out
        if _fits_space(out.shape, space) is None:
            raise LoweringError(f"{node.op} shape {out.shape} does not fit space {space}")
        exprs: list = []
        for a in node.args:
            if isinstance(a, Value):
                exprs.append(b.operand(a, read_index(a, out.shape, space)))
            elif isinstance(a, (bool, int, float)):
                exprs.append(_S(a))
            else:
                exprs.append(a)
        b.env[id(out)] = (b.emit(node, exprs), write_index(out, space))

    outputs: list[KernelArg] = []
    out_expr: dict[str, Expr] = {}
    for node in nodes:
        if id(node) not in group.owned:
            continue
        out = node.out
        if id(out) not in stores:
            continue
        if _fits_space(out.shape, space) != "full":
            raise LoweringError(f"{node.op} is broadcast inside its kernel but its result "
                                "escapes; the fusion pass should not have grouped it")
        outputs.append(KernelArg(out, flat_index(out.shape, out.layout)))
        out_expr[out.name] = b.env[id(out)][0]

    inputs = _prune_inputs(b.inputs, b.body, out_expr)
    return PointwiseKernel(name=name, space=tuple(space), inputs=inputs, outputs=outputs,
                           body=b.body, out_expr=out_expr, nodes=list(nodes))
