"""The tensor type of every scalar value as the reference's torch backend holds
it, so that the generated kernels round where that backend rounds.

The reference evaluates a kernel body with torch ops over whole tensors
(``mlc/codegen/torch_backend.py:20-118`` of the reference):

* an input read from a narrow-float buffer (fp16, bf16) is promoted to fp32
  on load (``:53-62``), so arithmetic on loaded values is fp32 and is rounded
  only by the store;
* a constant is a 0-dim tensor of its dtype, a boolean constant a tensor
  shaped like the operands (``:76-79``);
* a cast converts (``:80-81``), and every call then takes torch's result type
  of its operands (``:82-87``): an operand cast to fp16 or bf16 makes the
  arithmetic that follows narrow, and torch rounds each narrow result to its
  type;
* a row reduction keeps its operand's type (a sum of booleans or integers is
  int64), and the streamed form's online-softmax max and sum are fp32 tensors
  (``:204-215``).

``kernel_types`` types every temporary of a kernel that way; the HIP renderer
keeps fp32 registers throughout and rounds a narrow-typed result to its type
(one fp32 operation then one rounding, which is how torch's CPU kernels
evaluate fp16 and bf16 arithmetic; their add and sub convert a 0-dim
constant to the narrow type first, their mul and div use its fp32 value, and
the renderer does the same).
"""

from __future__ import annotations

from functools import lru_cache
from typing import Callable

import torch

from ..ir.scalar import Call, Cast, Const, Expr, Load, Ref
from ..kernels import Bind, PointwiseKernel, Reduce, ReductionKernel

#: torch type of a value and whether it has dimensions (a 0-dim constant
#: does not, and so does not decide the result type of a call against a
#: dimensioned operand of the same category)
VType = tuple[torch.dtype, bool]

#: the scalar functions as torch functions (the reference's table,
#: ``torch_backend.py:20-52``), used here on meta tensors for their result
#: types only
_TORCH_FN: dict[str, Callable] = {
    "neg": lambda a: -a, "abs": torch.abs, "reciprocal": torch.reciprocal,
    "exp": torch.exp, "log": torch.log, "sqrt": torch.sqrt, "rsqrt": torch.rsqrt,
    "sin": torch.sin, "cos": torch.cos, "tanh": torch.tanh, "erf": torch.erf,
    "sigmoid": torch.sigmoid, "floor": torch.floor, "logical_not": torch.logical_not,
    "add": torch.add, "sub": torch.sub, "mul": torch.mul, "div": torch.div,
    "pow": torch.pow, "maximum": torch.maximum, "minimum": torch.minimum,
    "gt": torch.gt, "lt": torch.lt, "ge": torch.ge, "le": torch.le, "eq": torch.eq,
    "ne": torch.ne, "logical_and": torch.logical_and, "logical_or": torch.logical_or,
    "where": torch.where,
}

_BUFFER = {torch.float16: torch.float32, torch.bfloat16: torch.float32}


def load_type(dtype: torch.dtype) -> VType:
    """The type of an element read from a buffer of ``dtype``."""
    return _BUFFER.get(dtype, dtype), True


@lru_cache(maxsize=None)
def call_type(fn: str, args: tuple[VType, ...]) -> VType:
    """Result type of scalar function ``fn`` over operands of these types. A
    combination torch itself refuses (the negation of a boolean, say) is
    typed fp32, which rounds nothing: the register code decides its value."""
    ts = [torch.empty((1,) if dim else (), dtype=dt, device="meta") for dt, dim in args]
    dims = any(dim for _, dim in args)
    try:
        return _TORCH_FN[fn](*ts).dtype, dims
    except (RuntimeError, TypeError, NotImplementedError):
        return torch.float32, dims


def expr_type(e: Expr, inputs: Callable[[int], VType], temps: Callable[[str], VType],
              memo: dict[int, VType] | None = None) -> VType:
    """Type of ``e`` given those of the inputs (by slot) and temporaries."""
    memo = {} if memo is None else memo
    got = memo.get(id(e))
    if got is not None:
        return got
    if isinstance(e, Load):
        t = inputs(e.slot)
    elif isinstance(e, Ref):
        t = temps(e.name)
    elif isinstance(e, Const):
        if isinstance(e.value, bool) or e.dtype == torch.bool:
            t = (torch.bool, True)
        elif e.dtype is not None:
            t = (e.dtype, False)
        else:
            t = (torch.int64 if isinstance(e.value, int) else torch.float32, False)
    elif isinstance(e, Cast):
        t = (e.dtype, expr_type(e.x, inputs, temps, memo)[1])
    elif isinstance(e, Call):
        t = call_type(e.fn, tuple(expr_type(a, inputs, temps, memo) for a in e.args))
    else:
        raise TypeError(f"cannot type {type(e).__name__}")
    memo[id(e)] = t
    return t


def reduce_type(kind: str, t: VType) -> VType:
    """Type of a row reduction (a ``[rows, 1]`` tensor) of values of type ``t``."""
    if kind in ("sum", "prod") and not t[0].is_floating_point:
        return torch.int64, True
    return t[0], True


def kernel_types(k, online: frozenset[str] = frozenset()) -> dict[str, VType]:
    """Type of every temporary of pointwise or reduction kernel ``k``;
    ``online`` names the reductions a streamed kernel computes with the
    online-softmax recurrence (fp32 in the reference)."""
    types: dict[str, VType] = {}

    def inputs(slot: int) -> VType:
        return load_type(k.inputs[slot].dtype)

    memo: dict[int, VType] = {}
    if isinstance(k, PointwiseKernel):
        for name, e in k.body:
            types[name] = expr_type(e, inputs, types.__getitem__, memo)
        return types
    assert isinstance(k, ReductionKernel)
    for s in k.steps:
        t = expr_type(s.expr, inputs, types.__getitem__, memo)
        if isinstance(s, Reduce):
            t = (torch.float32, True) if s.name in online else reduce_type(s.kind, t)
        else:
            assert isinstance(s, Bind)
        types[s.name] = t
    return types


#: the narrow types, each with the device function that rounds an fp32 value to it
ROUND = {torch.float16: "mlc::round_f16", torch.bfloat16: "mlc::round_bf16"}
