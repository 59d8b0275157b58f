"""Shape and dtype propagation.

Every intermediate type is derived here from the placeholders forward; the
exporter's FakeTensor metadata is kept on each node only so tests can check
these rules against it (:func:`verify_against_export`).

Reference behaviour followed: ``mlc/ir/shapes.py:20-188``.
"""

from __future__ import annotations

from typing import Sequence

import torch

from .graph import Value
from .ops import OpClass, lookup, op_class
from .types import Layout


class ShapeError(Exception):
    pass


def promote(dtypes: Sequence[torch.dtype]) -> torch.dtype:
    """Promotion over tensor operands only (python scalars are weak and are
    left out by the caller, so ``half * 2.0`` stays half)."""
    if not dtypes:
        return torch.float32
    out = dtypes[0]
    for d in dtypes[1:]:
        out = torch.promote_types(out, d)
    return out


def broadcast_shapes(shapes: Sequence[tuple[int, ...]]) -> tuple[int, ...]:
    rank = max((len(s) for s in shapes), default=0)
    result: list[int] = []
    for pos in range(rank):
        size = 1
        for s in shapes:
            k = pos - (rank - len(s))
            d = s[k] if k >= 0 else 1
            if d == 1:
                continue
            if size != 1 and size != d:
                raise ShapeError(f"cannot broadcast {list(shapes)} at dim {pos}: {size} vs {d}")
            size = d
        result.append(size)
    return tuple(result)


def infer_pointwise(op: str, args: list, kwargs: dict) -> tuple[tuple[int, ...], torch.dtype]:
    tensors = [a for a in args if isinstance(a, Value)]
    if not tensors:
        raise ShapeError(f"{op} has no tensor operand")
    shape = broadcast_shapes([t.shape for t in tensors])
    spec = lookup(op)
    if spec is not None and spec.dtype_rule is not None:
        dt = spec.dtype_rule(args, kwargs)
        if dt is not None:
            return shape, dt
    dtype = promote([t.dtype for t in tensors])
    if dtype in (torch.int32, torch.int64, torch.bool) and any(isinstance(a, float) for a in args):
        # a float python scalar makes an integer expression float
        dtype = torch.float32
    return shape, dtype


def infer_reduction(op: str, args: list, kwargs: dict) -> list[tuple[tuple[int, ...], torch.dtype]]:
    spec = lookup(op)
    assert spec is not None and spec.reduce is not None
    src = args[0]
    kind, dims, keep = spec.reduce(args, kwargs)
    shape: list[int] = []
    for i, d in enumerate(src.shape):
        if i not in dims:
            shape.append(d)
        elif keep:
            shape.append(1)
    dtype = kwargs.get("dtype")
    if not dtype:
        integral = src.dtype in (torch.bool, torch.int32, torch.int64)
        dtype = torch.float32 if integral and kind in ("mean", "var", "var_mean") else src.dtype
    return [(tuple(shape), dtype)] * spec.n_outputs


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise ShapeError(msg)


def infer_matmul(op: str, args: list, kwargs: dict) -> tuple[tuple[int, ...], torch.dtype]:
    if op == "aten.mm.default":
        a, b = args[0], args[1]
        _require(a.shape[1] == b.shape[0], f"mm: {a.shape} x {b.shape}")
        return (a.shape[0], b.shape[1]), promote([a.dtype, b.dtype])
    if op == "aten.bmm.default":
        a, b = args[0], args[1]
        _require(a.shape[0] == b.shape[0] and a.shape[2] == b.shape[1],
                 f"bmm: {a.shape} x {b.shape}")
        return (a.shape[0], a.shape[1], b.shape[2]), promote([a.dtype, b.dtype])
    if op == "aten.addmm.default":
        bias, a, b = args[0], args[1], args[2]
        _require(a.shape[1] == b.shape[0], f"addmm: {a.shape} x {b.shape}")
        return (a.shape[0], b.shape[1]), promote([bias.dtype, a.dtype, b.dtype])
    if op == "aten.baddbmm.default":
        bias, a, b = args[0], args[1], args[2]
        return (a.shape[0], a.shape[1], b.shape[2]), promote([bias.dtype, a.dtype, b.dtype])
    if op == "aten.matmul.default":
        a, b = args[0], args[1]
        if a.rank == 2 and b.rank == 2:
            return (a.shape[0], b.shape[1]), promote([a.dtype, b.dtype])
        batch = broadcast_shapes([a.shape[:-2], b.shape[:-2]])
        return batch + (a.shape[-2], b.shape[-1]), promote([a.dtype, b.dtype])
    raise ShapeError(f"no matmul rule for {op}")


def infer_view(op: str, args: list, kwargs: dict) -> Layout:
    spec = lookup(op)
    assert spec is not None and spec.view is not None
    return spec.view(args[0].layout, args, kwargs)


def infer(op: str, args: list, kwargs: dict) -> list[tuple[tuple[int, ...], torch.dtype]]:
    cls = op_class(op)
    if cls is OpClass.POINTWISE:
        return [infer_pointwise(op, args, kwargs)]
    if cls is OpClass.REDUCTION:
        return infer_reduction(op, args, kwargs)
    if cls is OpClass.MATMUL:
        return [infer_matmul(op, args, kwargs)]
    raise ShapeError(f"no shape rule for {op} (class {cls.value})")


def verify_against_export(graph) -> list[str]:
    """Differences between propagated types and the exporter's metadata."""
    problems: list[str] = []
    for n in graph.nodes:
        ref = n.meta.get("export_val")
        if ref is None or n.meta.get("types_from_export"):
            continue
        refs = list(ref) if isinstance(ref, (list, tuple)) else [ref]
        if len(refs) != len(n.outputs):
            problems.append(f"{n.op}: {len(n.outputs)} outputs, export says {len(refs)}")
            continue
        for got, want in zip(n.outputs, refs):
            if want is None:
                continue
            if tuple(want.shape) != tuple(got.shape):
                problems.append(f"{n.op} %{got.name}: shape {tuple(got.shape)} != {tuple(want.shape)}")
            if want.dtype != got.dtype:
                problems.append(f"{n.op} %{got.name}: dtype {got.dtype} != {want.dtype}")
    return problems
