"""Per-element expressions: the body language of fused kernels.

A fused kernel's arithmetic is a DAG of five node kinds -- ``Load`` (an
input operand at the current point), ``Ref`` (a temporary bound earlier in
the kernel), ``Const``, ``Call`` (one function of :data:`FUNCTIONS`) and
``Cast``. The HIP emitter renders the DAG to device C++, the test oracle
evaluates it with torch ops; both read the same nodes. Nodes are frozen
dataclasses, so equal subexpressions hash equal and serve as CSE keys.

Construction goes through :func:`call`, which checks arity and applies the
rewrites that are exact for every float (``x*1``, ``x/1``, ``1*x``, ``x+0``,
``x-0``, ``0+x``) and folds literal arithmetic, as the reference's builder
does (``mlc/ir/scalar.py:130-191``): the kernels then never see the
``mm * 1 + bias * 1`` that decomposing ``addmm`` produces.
"""

from __future__ import annotations

import math
import operator
from dataclasses import dataclass
from typing import Any, Callable, Iterator

import torch


class Expr:
    __slots__ = ()


@dataclass(frozen=True)
class Load(Expr):
    slot: int


@dataclass(frozen=True)
class Ref(Expr):
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


# --------------------------------------------------------------------------
# the function table
# --------------------------------------------------------------------------

@dataclass(frozen=True)
class FnSpec:
    arity: int
    #: the result is torch.bool whatever the operands are
    bool_result: bool = False
    #: defined for floating-point operands only
    float_only: bool = False


def _spec_table() -> dict[str, FnSpec]:
    # name -> (arity, flags); "b" = bool result, "f" = float operands only
    rows = """
        neg 1 -     abs 1 -     floor 1 -    logical_not 1 b
        reciprocal 1 f  exp 1 f  log 1 f  sqrt 1 f  rsqrt 1 f
        sin 1 f  cos 1 f  tanh 1 f  erf 1 f  sigmoid 1 f
        add 2 -  sub 2 -  mul 2 -  div 2 -  pow 2 -  maximum 2 -  minimum 2 -
        gt 2 b  lt 2 b  ge 2 b  le 2 b  eq 2 b  ne 2 b  logical_and 2 b  logical_or 2 b
        where 3 -
    """.split()
    return {name: FnSpec(int(arity), bool_result=flag == "b", float_only=flag == "f")
            for name, arity, flag in zip(rows[0::3], rows[1::3], rows[2::3])}


#: every function a kernel body may call, with its arity and result kind
FUNCTIONS: dict[str, FnSpec] = _spec_table()


# --------------------------------------------------------------------------
# construction
# --------------------------------------------------------------------------

def cast(x: Expr, dtype: torch.dtype) -> Expr:
    """``x`` converted to ``dtype``; a literal takes the dtype itself."""
    return Const(x.value, dtype) if isinstance(x, Const) else Cast(x, dtype)


#: fn -> (identity on the left, identity on the right); None: no such side
_IDENTITIES: dict[str, tuple[Any, Any]] = {
    "mul": (1, 1), "div": (None, 1), "add": (0, 0), "sub": (None, 0),
}

#: literal arithmetic folded at build time (Python float semantics)
_LITERAL: dict[str, Callable] = {
    "add": operator.add, "sub": operator.sub, "mul": operator.mul,
    "div": operator.truediv, "neg": operator.neg, "sqrt": math.sqrt, "exp": math.exp,
}


def _literal_equals(e: Expr, v: Any) -> bool:
    # a bool literal is a mask value, never an arithmetic identity
    return isinstance(e, Const) and type(e.value) is not bool and e.value == v


def _simplified(fn: str, args: tuple[Expr, ...]) -> Expr | None:
    left, right = _IDENTITIES.get(fn, (None, None))
    if right is not None and _literal_equals(args[1], right):
        return args[0]
    if left is not None and _literal_equals(args[0], left):
        return args[1]
    op = _LITERAL.get(fn)
    if op is not None and all(isinstance(a, Const) for a in args):
        try:
            return Const(op(*(a.value for a in args)))
        except (ZeroDivisionError, ValueError, OverflowError):
            return None
    return None


def call(fn: str, *args: Expr) -> Expr:
    """``fn(*args)``, checked against :data:`FUNCTIONS` and simplified."""
    try:
        spec = FUNCTIONS[fn]
    except KeyError:
        raise KeyError(f"scalar function {fn!r} is not in the kernel function table") from None
    if len(args) != spec.arity:
        raise ValueError(f"scalar function {fn} expects {spec.arity} operand(s), got {len(args)}")
    bad = [type(a).__name__ for a in args if not isinstance(a, Expr)]
    if bad:
        raise TypeError(f"scalar function {fn}: operand of type {bad[0]} is not an Expr")
    return _simplified(fn, args) or Call(fn, tuple(args))


# --------------------------------------------------------------------------
# traversal
# --------------------------------------------------------------------------

def _children(e: Expr) -> tuple[Expr, ...]:
    if isinstance(e, Call):
        return e.args
    if isinstance(e, Cast):
        return (e.x,)
    return ()


def walk(e: Expr) -> Iterator[Expr]:
    """Every subexpression of ``e`` in post-order (operands left to right,
    then the node), shared subtrees once per use."""
    stack: list[tuple[Expr, bool]] = [(e, False)]
    while stack:
        node, expanded = stack.pop()
        if expanded:
            yield node
            continue
        stack.append((node, True))
        stack.extend((c, False) for c in reversed(_children(node)))


def loads(e: Expr) -> set[int]:
    """Input slots ``e`` reads."""
    return {x.slot for x in walk(e) if isinstance(x, Load)}


def refs(e: Expr) -> set[str]:
    """Temporaries ``e`` reads."""
    return {x.name for x in walk(e) if isinstance(x, Ref)}


def substitute(e: Expr, mapping: dict[Expr, Expr]) -> Expr:
    """``e`` with every subexpression that is a key of ``mapping`` replaced
    (outermost match wins; replacements are not rewritten again)."""
    hit = mapping.get(e)
    if hit is not None:
        return hit
    if isinstance(e, Call):
        return Call(e.fn, tuple(substitute(a, mapping) for a in e.args))
    if isinstance(e, Cast):
        return Cast(substitute(e.x, mapping), e.dtype)
    return e


def size(e: Expr) -> int:
    """Distinct nodes of the DAG rooted at ``e``."""
    return len(set(walk(e)))
