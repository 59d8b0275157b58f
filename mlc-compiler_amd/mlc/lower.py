"""Fusion groups -> kernel IR.

``build_schedule`` turns each group into one kernel: a pointwise group into a
:class:`PointwiseKernel`, a reduction group into a :class:`ReductionKernel`
(``codegen/reduction_lowering.py``), anything else -- matmuls, opaque ops,
reductions with the pass off -- into an :class:`ExternKernel` library call.

Both generated kinds are assembled the same way (:class:`KernelAssembler`):
walk the group's nodes in program order, lower each through the op
registry's rule, and resolve every tensor operand to an *index map* over the
kernel's iteration variables. An operand that an earlier member computed at
the same map is taken from that member's register; otherwise it becomes a
load slot (one slot per distinct buffer, dtype and map). Because index maps
are canonical, a ``[B*T, D]`` GEMM output and the ``[B, T, D]`` view the next
op reads are the same map, so the pair fuses without the value reaching
memory. At the end, slots nothing reads are dropped and the rest renumbered.

A value is stored when the graph returns it or some kernel that does not
compute it reads it (``_values_to_store``; after recompute a node can be in
several kernels, so this is decided over the whole schedule).

Temp naming, slot order and the pruning rule give the reference's kernel IR
for the same groups (``mlc/lower.py:40-292``), which the golden schedules
check.
"""

from __future__ import annotations

from .codegen.index import IndexMap, flat_index
from .config import Config
from .ir.graph import Graph, Node, Value
from .ir.ops import _literal, lookup
from .ir.scalar import Const, Expr, Load, Ref, loads, substitute
from .kernels import ExternKernel, KernelArg, PointwiseKernel, Schedule
from .passes.fusion import BROADCAST, FULL, KernelGroup, _fits_space, group_space
from .passes.grouping import UseInfo, source_value


class LoweringError(Exception):
    pass


def build_schedule(graph: Graph, groups: list[KernelGroup], cfg: Config) -> Schedule:
    stores = _values_to_store(groups, UseInfo(graph))
    kernels = []
    for i, group in enumerate(groups):
        name, kind = f"k{i}", group.kind
        if kind == "pointwise":
            kernels.append(build_pointwise(graph, group, stores, name))
        elif kind == "reduction" and cfg.reduction_fusion:
            from .codegen.reduction_lowering import build_reduction

            kernels.append(build_reduction(graph, group, stores, name, cfg))
        elif len(group.nodes) == 1:
            node = group.nodes[0]
            kernels.append(ExternKernel(name, node, node.unique_tensor_args(), list(node.outputs)))
        else:
            raise LoweringError(f"{len(group.nodes)} nodes grouped into one library call: "
                                f"{[n.op for n in group.nodes]}")
    return Schedule(graph, kernels)


def _values_to_store(groups: list[KernelGroup], uses: UseInfo) -> set[int]:
    """ids of values that reach memory: graph outputs, and values some node
    reads in a kernel that does not compute them."""
    homes: dict[int, set[int]] = {}
    for gi, g in enumerate(groups):
        for n in g.nodes:
            homes.setdefault(id(n), set()).add(gi)
    stored = set()
    for n in {id(n): n for g in groups for n in g.nodes}.values():
        here = homes[id(n)]
        for o in n.outputs:
            if uses.escapes(o) or any(not homes.get(c, set()) <= here for c in uses.consumers(o)):
                stored.add(id(o))
    return stored


# --------------------------------------------------------------------------
# index maps of a pointwise kernel
# --------------------------------------------------------------------------

def read_index(value: Value, consumer_shape, space) -> IndexMap:
    """The map a pointwise kernel over ``space`` reads ``value`` at, for a
    node whose output has ``consumer_shape``: the operand broadcasts into the
    node's shape, which broadcasts into (or reshapes to) the space."""
    consumer_shape = tuple(consumer_shape)
    if _fits_space(consumer_shape, space) == BROADCAST:
        return flat_index(space, value.layout.expand(consumer_shape).expand(space))
    if tuple(value.shape) == consumer_shape:
        return flat_index(consumer_shape, value.layout)
    return flat_index(consumer_shape, value.layout.expand(consumer_shape))


def write_index(value: Value, space) -> IndexMap:
    """The map ``value`` is held at once a kernel over ``space`` computed it."""
    if _fits_space(value.shape, space) == FULL:
        return flat_index(value.shape, value.layout)
    return flat_index(space, value.layout.expand(space))


def reads_are_local(nodes, space) -> bool:
    """Each member reads every value another member computes at the map that
    value is held at, so the read stays in the reading thread's registers.
    (A bias add over ``[B*T, D]`` and a clone of a transposed view of it have
    equal element counts, but iteration i would need iteration perm(i)'s
    value: such a pair cannot share a pointwise kernel.)"""
    held: dict[int, IndexMap] = {}
    for o in (o for n in nodes for o in n.outputs):
        if _fits_space(o.shape, space) is None:
            return False
        held[id(o)] = write_index(o, space)
    for n in nodes:
        for a in (a for a in n.args if isinstance(a, Value)):
            at = held.get(id(source_value(a)))
            if at is None:
                continue
            try:
                if read_index(a, n.out.shape, space) != at:
                    return False
            except ValueError:
                return False
    return True


# --------------------------------------------------------------------------
# assembling a kernel
# --------------------------------------------------------------------------

class KernelAssembler:
    """Operand slots, values held in registers and temp names of one kernel
    under construction (subclassed per kernel kind)."""

    def __init__(self) -> None:
        self.inputs: list[KernelArg] = []
        self._slot_of: dict[tuple, int] = {}
        #: id(value) -> (expression holding it, map it is held at)
        self.held: dict[int, tuple[Expr, IndexMap]] = {}
        self._serial = 0

    def new_name(self, prefix: str = "t") -> str:
        self._serial += 1
        return f"{prefix}{self._serial - 1}"

    def load(self, v: Value, imap: IndexMap) -> Expr:
        key = (id(v.buffer), v.dtype, imap)
        if key not in self._slot_of:
            self._slot_of[key] = len(self.inputs)
            self.inputs.append(KernelArg(v, imap))
        return Load(self._slot_of[key])

    def read(self, v: Value, imap: IndexMap) -> Expr:
        """The register holding ``v`` at ``imap`` if there is one, else a load."""
        held = self.held.get(id(source_value(v)))
        return held[0] if held is not None and held[1] == imap else self.load(v, imap)

    @staticmethod
    def lowered(node: Node, arg_exprs: list) -> Expr:
        spec = lookup(node.op)
        if spec is None or spec.lower is None:
            raise LoweringError(f"{node.op} has no scalar lowering rule")
        return spec.lower(list(node.args), arg_exprs, dict(node.kwargs))

    @staticmethod
    def literal_or_passthrough(a):
        """Non-tensor arguments: numbers become literals; dims, dtypes and the
        like pass through for the lowering rule to read."""
        return _literal(a) if isinstance(a, (bool, int, float)) else a

    def compact(self, exprs: list[Expr]) -> tuple[list[KernelArg], dict[Expr, Expr] | None]:
        """Drop slots none of ``exprs`` reads: the kept operands, and the
        renumbering to apply (None when every slot is read)."""
        used = set().union(*map(loads, exprs)) if exprs else set()
        if len(used) == len(self.inputs):
            return self.inputs, None
        kept = sorted(used)
        return [self.inputs[i] for i in kept], {Load(old): Load(new) for new, old in enumerate(kept)}


class _PointwiseAssembler(KernelAssembler):
    def __init__(self) -> None:
        super().__init__()
        self.body: list[tuple[str, Expr]] = []

    def bind(self, expr: Expr) -> Expr:
        """One body line per real operation: a lowering that is a bare load,
        register or literal (a clone, a no-op cast) binds nothing."""
        if isinstance(expr, (Load, Ref, Const)):
            return expr
        name = self.new_name()
        self.body.append((name, expr))
        return Ref(name)


def build_pointwise(graph: Graph, group: KernelGroup, stores: set[int], name: str) -> PointwiseKernel:
    nodes = group.nodes
    space = tuple(group_space(nodes))
    asm = _PointwiseAssembler()
    for node in nodes:
        out = node.out
        if _fits_space(out.shape, space) is None:
            raise LoweringError(f"{node.op}{list(out.shape)} has no place in the space {space}")
        args = [asm.read(a, read_index(a, out.shape, space)) if isinstance(a, Value)
                else asm.literal_or_passthrough(a) for a in node.args]
        asm.held[id(out)] = (asm.bind(asm.lowered(node, args)), write_index(out, space))

    outputs, out_expr = [], {}
    for node in nodes:
        out = node.out
        if id(node) not in group.owned or id(out) not in stores:
            continue
        if _fits_space(out.shape, space) != FULL:
            raise LoweringError(f"{node.op}: a value evaluated per point of a larger space "
                                "escapes its kernel")
        outputs.append(KernelArg(out, flat_index(out.shape, out.layout)))
        out_expr[out.name] = asm.held[id(out)][0]

    inputs, renumber = asm.compact([e for _, e in asm.body] + list(out_expr.values()))
    body = asm.body
    if renumber is not None:
        body = [(t, substitute(e, renumber)) for t, e in body]
        out_expr = {k: substitute(e, renumber) for k, e in out_expr.items()}
    return PointwiseKernel(name=name, space=space, inputs=inputs, outputs=outputs, body=body,
                           out_expr=out_expr, nodes=list(nodes))
