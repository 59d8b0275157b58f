"""Scalar expression IR: the per-element body of a fused kernel.

The HIP backend renders these expressions into device C++; the CPU oracle
evaluates the same expressions with torch ops. Expressions are immutable and
hashable so they double as keys for common-subexpression elimination.

Reference behaviour followed: ``mlc/ir/scalar.py:23-225`` (node kinds, the
function table with its arities, and the exact identities folded at build
time).
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Any

import torch


class Expr:
    __slots__ = ()


@dataclass(frozen=True)
class Load(Expr):
    """The kernel operand in input slot ``slot``, read at the current point."""

    slot: int


@dataclass(frozen=True)
class Ref(Expr):
    """A temporary bound earlier in the same kernel (a body line or a reduce)."""

    name: str


@dataclass(frozen=True)
class Const(Expr):
    value: Any
    dtype: torch.dtype | None = None


@dataclass(frozen=True)
class Call(Expr):
    fn: str
    args: tuple[Expr, ...]


@dataclass(frozen=True)
class Cast(Expr):
    x: Expr
    dtype: torch.dtype


def cast(x: Expr, dtype: torch.dtype) -> Expr:
    """Cast ``x``; a literal absorbs the dtype instead of getting a Cast node."""
    if isinstance(x, Const):
        return Const(x.value, dtype)
    return Cast(x, dtype)


@dataclass(frozen=True)
class FnSpec:
    arity: int
    bool_result: bool = False
    float_only: bool = False


def _table() -> dict[str, FnSpec]:
    t: dict[str, FnSpec] = {}
    for n in ("neg", "abs", "floor"):
        t[n] = FnSpec(1)
    for n in ("reciprocal", "exp", "log", "sqrt", "rsqrt", "sin", "cos", "tanh",
              "erf", "sigmoid"):
        t[n] = FnSpec(1, float_only=True)
    t["logical_not"] = FnSpec(1, bool_result=True)
    for n in ("add", "sub", "mul", "div", "pow", "maximum", "minimum"):
        t[n] = FnSpec(2)
    for n in ("gt", "lt", "ge", "le", "eq", "ne", "logical_and", "logical_or"):
        t[n] = FnSpec(2, bool_result=True)
    t["where"] = FnSpec(3)
    return t


#: every scalar function a kernel body may use
FUNCTIONS: dict[str, FnSpec] = _table()


def call(fn: str, *args: Expr) -> Expr:
    spec = FUNCTIONS.get(fn)
    if spec is None:
        raise KeyError(f"unknown scalar function {fn!r}")
    if len(args) != spec.arity:
        raise ValueError(f"{fn} takes {spec.arity} args, got {len(args)}")
    for a in args:
        if not isinstance(a, Expr):
            raise TypeError(f"{fn} arg is {type(a).__name__}, expected Expr")
    folded = _fold(fn, args)
    return folded if folded is not None else Call(fn, tuple(args))


def _is_literal(e: Expr, v) -> bool:
    return isinstance(e, Const) and not isinstance(e.value, bool) and e.value == v


def _fold(fn: str, args: tuple[Expr, ...]) -> Expr | None:
    """Identities exact for every float including NaN/inf (x*1, x/1, 1*x,
    x+0, x-0, 0+x) and folding of all-literal arithmetic."""
    if fn in ("mul", "div") and _is_literal(args[1], 1):
        return args[0]
    if fn == "mul" and _is_literal(args[0], 1):
        return args[1]
    if fn in ("add", "sub") and _is_literal(args[1], 0):
        return args[0]
    if fn == "add" and _is_literal(args[0], 0):
        return args[1]
    if all(isinstance(a, Const) for a in args):
        value = _fold_literals(fn, [a.value for a in args])
        if value is not None:
            return Const(value)
    return None


_LITERAL_OPS = {
    "add": lambda a, b: a + b,
    "sub": lambda a, b: a - b,
    "mul": lambda a, b: a * b,
    "div": lambda a, b: a / b,
    "neg": lambda a: -a,
    "sqrt": math.sqrt,
    "exp": math.exp,
}


def _fold_literals(fn: str, values: list):
    op = _LITERAL_OPS.get(fn)
    if op is None:
        return None
    try:
        return op(*values)
    except (ZeroDivisionError, ValueError, OverflowError):
        return None


def walk(e: Expr):
    """Every subexpression of ``e``, children first."""
    if isinstance(e, Call):
        for a in e.args:
            yield from walk(a)
    elif isinstance(e, Cast):
        yield from walk(e.x)
    yield e


def loads(e: Expr) -> set[int]:
    return {s.slot for s in walk(e) if isinstance(s, Load)}


def refs(e: Expr) -> set[str]:
    return {s.name for s in walk(e) if isinstance(s, Ref)}


def substitute(e: Expr, mapping: dict[Expr, Expr]) -> Expr:
    if e in mapping:
        return mapping[e]
    if isinstance(e, Call):
        return Call(e.fn, tuple(substitute(a, mapping) for a in e.args))
    if isinstance(e, Cast):
        return Cast(substitute(e.x, mapping), e.dtype)
    return e


def size(e: Expr) -> int:
    """Distinct nodes in the expression DAG."""
    return len(set(walk(e)))
