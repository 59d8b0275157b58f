"""Result types of graph nodes, derived by the compiler itself.

Capture builds every value's shape and dtype from the placeholders forward
with the rules here (``infer`` dispatches on the op's class; views go
through ``infer_view`` because they produce a layout over an existing
buffer rather than a new buffer). The exporter's own fake-tensor metadata is
kept only as a cross-check (``verify_against_export``), so a wrong rule is
reported by op name instead of surfacing as a miscompile.

dtype rule: torch's promotion over *tensor* operands. Python scalars are
weak in torch (``half * 2.0`` stays half), so they are left out, except that
a float scalar makes an integer or bool expression float32 -- the one
weak-scalar case these models hit (reference counterpart:
``mlc/ir/shapes.py:29-98``).
"""

from __future__ import annotations

import functools
import itertools
from typing import Sequence

import torch

from .graph import Value
from .ops import OpClass, lookup, op_class
from .types import Layout

Shape = tuple[int, ...]
_INTEGRAL = (torch.bool, torch.int32, torch.int64)


class ShapeError(Exception):
    pass


def _require(ok: bool, what: str) -> None:
    if not ok:
        raise ShapeError(what)


def promote(dtypes: Sequence[torch.dtype]) -> torch.dtype:
    """torch's promotion over ``dtypes``; float32 for none."""
    return functools.reduce(torch.promote_types, dtypes) if dtypes else torch.float32


def broadcast_shapes(shapes: Sequence[Shape]) -> Shape:
    """The common shape of right-aligned ``shapes`` (numpy rules)."""
    columns = itertools.zip_longest(*(tuple(s)[::-1] for s in shapes), fillvalue=1)
    out = []
    for pos, sizes in enumerate(columns):
        wide = {d for d in sizes if d != 1}
        _require(len(wide) <= 1, f"shapes {list(shapes)} do not broadcast: sizes "
                                 f"{sorted(wide)} meet {pos} dims from the right")
        out.append(wide.pop() if wide else 1)
    return tuple(out[::-1])


# --------------------------------------------------------------------------
# rules per op class
# --------------------------------------------------------------------------

def infer_pointwise(op: str, args: list, kwargs: dict) -> tuple[Shape, torch.dtype]:
    tensors = [a for a in args if isinstance(a, Value)]
    _require(bool(tensors), f"{op}: a pointwise op needs at least one tensor operand")
    shape = broadcast_shapes([t.shape for t in tensors])
    spec = lookup(op)
    forced = spec.dtype_rule(args, kwargs) if spec is not None and spec.dtype_rule else None
    if forced is not None:
        return shape, forced
    dtype = promote([t.dtype for t in tensors])
    if dtype in _INTEGRAL and any(isinstance(a, float) for a in args):
        dtype = torch.float32
    return shape, dtype


def infer_reduction(op: str, args: list, kwargs: dict) -> list[tuple[Shape, torch.dtype]]:
    spec = lookup(op)
    _require(spec is not None and spec.reduce is not None, f"{op} is not a reduction")
    src = args[0]
    kind, dims, keepdim = spec.reduce(args, kwargs)
    kept = tuple(1 if i in dims else d for i, d in enumerate(src.shape)
                 if keepdim or i not in dims)
    dtype = kwargs.get("dtype")
    if not dtype:
        averaging = kind in ("mean", "var", "var_mean")
        dtype = torch.float32 if averaging and src.dtype in _INTEGRAL else src.dtype
    return [(kept, dtype)] * spec.n_outputs


def _mm(a: Value, b: Value) -> tuple[Shape, list]:
    _require(a.shape[1] == b.shape[0], f"mm of {a.shape} and {b.shape}")
    return (a.shape[0], b.shape[1]), [a, b]


def _bmm(a: Value, b: Value) -> tuple[Shape, list]:
    _require(a.shape[0] == b.shape[0] and a.shape[2] == b.shape[1],
             f"bmm of {a.shape} and {b.shape}")
    return (a.shape[0], a.shape[1], b.shape[2]), [a, b]


def _addmm(bias: Value, a: Value, b: Value) -> tuple[Shape, list]:
    _require(a.shape[1] == b.shape[0], f"addmm of {a.shape} and {b.shape}")
    return (a.shape[0], b.shape[1]), [bias, a, b]


def _baddbmm(bias: Value, a: Value, b: Value) -> tuple[Shape, list]:
    return (a.shape[0], a.shape[1], b.shape[2]), [bias, a, b]


def _matmul(a: Value, b: Value) -> tuple[Shape, list]:
    if a.rank == 2 and b.rank == 2:
        return (a.shape[0], b.shape[1]), [a, b]
    return broadcast_shapes([a.shape[:-2], b.shape[:-2]]) + (a.shape[-2], b.shape[-1]), [a, b]


_MATMUL_RULES = {
    "aten.mm.default": _mm, "aten.bmm.default": _bmm, "aten.addmm.default": _addmm,
    "aten.baddbmm.default": _baddbmm, "aten.matmul.default": _matmul,
}


def infer_matmul(op: str, args: list, kwargs: dict) -> tuple[Shape, torch.dtype]:
    rule = _MATMUL_RULES.get(op)
    _require(rule is not None, f"{op}: no matmul shape rule")
    arity = rule.__code__.co_argcount
    shape, operands = rule(*args[:arity])
    return shape, promote([v.dtype for v in operands])


def infer_view(op: str, args: list, kwargs: dict) -> Layout:
    """The layout a view op gives its first operand."""
    spec = lookup(op)
    _require(spec is not None and spec.view is not None, f"{op} is not a view")
    return spec.view(args[0].layout, args, kwargs)


_BY_CLASS = {
    OpClass.POINTWISE: lambda op, a, kw: [infer_pointwise(op, a, kw)],
    OpClass.REDUCTION: infer_reduction,
    OpClass.MATMUL: lambda op, a, kw: [infer_matmul(op, a, kw)],
}


def infer(op: str, args: list, kwargs: dict) -> list[tuple[Shape, torch.dtype]]:
    """``(shape, dtype)`` of each result of ``op`` (not for views)."""
    cls = op_class(op)
    rule = _BY_CLASS.get(cls)
    _require(rule is not None, f"{op}: {cls.value} ops have no result-type rule")
    return rule(op, args, kwargs)


def verify_against_export(graph) -> list[str]:
    """Every node's derived types against the fake tensors torch.export
    recorded (``meta['export_val']``); one line per disagreement. Nodes whose
    types were taken from that metadata in the first place are skipped."""
    found: list[str] = []
    for n in graph.nodes:
        recorded = n.meta.get("export_val")
        if recorded is None or n.meta.get("types_from_export"):
            continue
        recorded = list(recorded) if isinstance(recorded, (list, tuple)) else [recorded]
        if len(recorded) != len(n.outputs):
            found.append(f"{n.op}: export recorded {len(recorded)} results, the graph has "
                         f"{len(n.outputs)}")
            continue
        for mine, theirs in zip(n.outputs, recorded):
            if theirs is None:
                continue
            if tuple(theirs.shape) != tuple(mine.shape):
                found.append(f"{n.op} %{mine.name}: shape {tuple(mine.shape)}, export "
                             f"{tuple(theirs.shape)}")
            if theirs.dtype != mine.dtype:
                found.append(f"{n.op} %{mine.name}: dtype {mine.dtype}, export {theirs.dtype}")
    return found
