"""HIP source generation for gfx950: one ``extern "C" __global__`` function per
distinct fused kernel, instantiating the hand-written CDNA4 templates in
``templates/mlc_cdna4.h``.

This replaces the reference's Triton emitters
(``mlc/codegen/triton_backend.py:206-287``, ``triton_reduction.py:73-274``)
behind the same seam: it consumes the kernel IR (``PointwiseKernel`` /
``ReductionKernel``) and returns source plus a launch table. Semantics kept
from the reference: narrow floats load into fp32 registers, arithmetic is
fp32, stores round back to the buffer dtype (round-to-nearest-even); after an
explicit cast to fp16 or bf16 each result is rounded to that type, as the
reference's torch evaluation rounds it (``value_types``); reduce identities
neutralise masked lanes; row-constant operands are scalar loads.

The MI355X design:

* **pointwise**: one thread per V-element pack (V*itemsize = 16 bytes), so
  every contiguous operand moves with 128-bit loads/stores; an operand whose
  index is constant over a pack (a bias broadcast down rows, a row statistic)
  is one scalar load; anything else is gathered per element. 256-thread
  workgroups, grid = packs / 256.
* **persistent reduction**: each row is owned by G lanes (a power of two);
  lane ``l`` holds columns ``(k*G + l)*V .. +V`` for ``k < K`` in VGPRs, so a
  row is read once with coalesced 128-bit loads. Rows of <= 64 lanes reduce
  with DPP and v_permlane16/32_swap inside the wave and several rows share a
  workgroup; wider rows span whole waves and combine through LDS.
* **streamed reduction** (rows longer than ``max_persistent_row``): one row
  per 256-thread workgroup, one chunked pass over HBM per reduce (or one
  online-softmax pass for max+sum(exp)), then a store pass.

Identical kernel bodies (every transformer layer repeats the same ones) are
emitted once and shared by name.
"""

from __future__ import annotations

import hashlib
import math
import struct
from dataclasses import dataclass, field

import numpy as np
import torch

from ..config import Config
from ..ir.scalar import Call, Cast, Const, Expr, Load, Ref, loads as expr_loads, refs as expr_refs
from ..kernels import AttentionKernel, Bind, ExternKernel, PointwiseKernel, Reduce, ReductionKernel, Schedule
from ..ir.graph import Value
from .index import IndexMap, build_index
from .reduction_schedule import plan_passes, scalar_binds, varies_by_column
from .value_types import ROUND, VType, expr_type, kernel_types, load_type

WAVE = 64

#: storage type of each buffer dtype in device code
STORAGE = {
    torch.float32: "float",
    torch.float16: "mlc::f16",
    torch.bfloat16: "mlc::bf16",
    torch.float64: "double",
    torch.int64: "int64_t",
    torch.int32: "int32_t",
    torch.int16: "int16_t",
    torch.int8: "int8_t",
    torch.uint8: "uint8_t",
    torch.bool: "bool",
}

_RANK = {"bool": 0, "int64_t": 1, "float": 2, "double": 3}


def compute_type(dtype: torch.dtype) -> str:
    """Register type a loaded element of ``dtype`` is held in."""
    if dtype in (torch.float16, torch.bfloat16, torch.float32):
        return "float"
    if dtype == torch.float64:
        return "double"
    if dtype == torch.bool:
        return "bool"
    return "int64_t"


def itemsize(dtype: torch.dtype) -> int:
    return torch.empty((), dtype=dtype).element_size()


# --------------------------------------------------------------------------
# expressions
# --------------------------------------------------------------------------

def float_literal(v: float) -> str:
    """The fp32 value of ``v`` as an exact hexadecimal float literal (the
    oracle also holds literals as fp32 0-dim tensors)."""
    if v != v:
        return "__builtin_nanf(\"\")"
    if v == math.inf:
        return "__builtin_huge_valf()"
    if v == -math.inf:
        return "(-__builtin_huge_valf())"
    f32 = struct.unpack("<f", struct.pack("<f", float(v)))[0] if abs(v) < 3.5e38 else v
    if f32 in (math.inf, -math.inf):
        return "__builtin_huge_valf()" if f32 > 0 else "(-__builtin_huge_valf())"
    return f"{float(f32).hex()}f"


def _round_half(v: float, dtype: torch.dtype) -> float:
    return float(torch.tensor(v, dtype=dtype).float().item())


class Renderer:
    """Renders scalar expressions to C++ with their register types.

    ``operand(slot)`` and ``temp(name)`` give the C++ expression (and type)
    that reads an input or a temporary at the current element. ``half_slots``
    are the inputs stored as fp16 and ``defs`` the temporaries' defining
    expressions: with them, fp32 add/sub/mul with an operand just converted
    from fp16 render as the equal fma against an opaque constant (the
    hardware's mixed-precision fma reads the fp16 half directly), and
    ``X * 2^k + y`` with an fp16 ``X`` becomes one fma (``X * 2^k`` is exact
    for every fp16 X when |k| <= 100, so the fma rounds once where the two
    operations would round once too).
    """

    def __init__(self, operand, temp, half_slots=frozenset(), defs=None, to_fp16=frozenset(),
                 vtypes=None) -> None:
        self.operand = operand
        self.temp = temp
        self.half_slots = frozenset(half_slots)
        self.defs = defs if defs is not None else {}
        #: temporaries whose every use rounds them to fp16
        self.to_fp16 = frozenset(to_fp16)
        self._plain = False
        #: (input types by slot, temporary types by name) as the reference's
        #: torch evaluation holds them (``value_types``): a call whose result
        #: is typed fp16 or bf16 is rounded to that type
        self.vtypes = vtypes
        self._vmemo: dict[int, VType] = {}

    def bind(self, name: str, e: Expr) -> tuple[str, str]:
        """Render the defining expression of temporary ``name``. An add, sub
        or mul of two fp16 values whose result is only rounded to fp16 stays
        the plain operation: the compiler evaluates that in fp16 directly
        (exact, since fp32 holds more than twice fp16's precision) with packed
        half instructions, two elements per instruction."""
        return self.store(e, name in self.to_fp16)

    def store(self, e: Expr, to_fp16: bool) -> tuple[str, str]:
        """Render ``e`` for a value that is only rounded to fp16 when ``to_fp16``."""
        if (to_fp16 and isinstance(e, Call) and e.fn in ("add", "sub", "mul")
                and all(self.is_half(a) for a in e.args)):
            self._plain = True
        return self(e)

    def __call__(self, e: Expr) -> tuple[str, str]:
        if isinstance(e, Load):
            return self.operand(e.slot)
        if isinstance(e, Ref):
            return self.temp(e.name)
        if isinstance(e, Const):
            return self.const(e)
        if isinstance(e, Cast):
            code, _ = self(e.x)
            return cast_code(code, e.dtype)
        if isinstance(e, Call):
            return self.call(e)
        raise TypeError(f"cannot emit {type(e).__name__}")

    def is_half(self, e: Expr, depth: int = 0) -> bool:
        """Whether ``e`` is an fp32 register holding a value converted from
        fp16: an fp16 input, a rounding to fp16, or a temporary of either."""
        if isinstance(e, Load):
            return e.slot in self.half_slots
        if isinstance(e, Cast):
            return e.dtype == torch.float16 or (e.dtype == torch.float32 and self.is_half(e.x, depth))
        if isinstance(e, Ref) and depth < 8:
            d = self.defs.get(e.name)
            return d is not None and self.is_half(d, depth + 1)
        return False

    def exact_scale(self, e: Expr):
        """(X, c) when ``e`` is ``X * c`` or ``X / (1/c)`` with an fp16 ``X``
        and ``c = +-2^k``, |k| <= 100, directly or through one temporary."""
        if isinstance(e, Ref):
            e = self.defs.get(e.name, e)
        if not (isinstance(e, Call) and e.fn in ("mul", "div")):
            return None
        x, c = e.args
        if e.fn == "mul" and isinstance(x, Const):
            x, c = c, x
        if not isinstance(c, Const) or not self.is_half(x):
            return None
        fast = _const_divisor(c)
        if fast is None or not fast[2]:
            return None
        v = fast[0] if e.fn == "mul" else fast[1]
        if not (2.0 ** -100 <= abs(v) <= 2.0 ** 100):
            return None
        return x, v

    def mixed(self, e: Call, codes: list[str]) -> str | None:
        """The fma form of an fp32 add/sub/mul described above, or None."""
        x, y = e.args
        if e.fn in ("add", "sub"):
            sign = 1.0 if e.fn == "add" else -1.0
            sx = self.exact_scale(x)
            if sx is not None:  # X*c + y  or  X*c - y
                other = codes[1] if e.fn == "add" else f"(-{codes[1]})"
                return f"__builtin_fmaf({self(sx[0])[0]}, {float_literal(sx[1])}, {other})"
            sy = self.exact_scale(y)
            if sy is not None:  # x + Y*c  or  x - Y*c
                return f"__builtin_fmaf({self(sy[0])[0]}, {float_literal(sign * sy[1])}, {codes[0]})"
            if e.fn == "sub":
                if self.is_half(x) or self.is_half(y):
                    return f"__builtin_fmaf({codes[1]}, mlc::neg_one_(), {codes[0]})"
                return None
            if self.is_half(x):
                return f"__builtin_fmaf({codes[0]}, mlc::one_(), {codes[1]})"
            if self.is_half(y):
                return f"__builtin_fmaf({codes[1]}, mlc::one_(), {codes[0]})"
            return None
        if self.is_half(x):
            return f"__builtin_fmaf({codes[0]}, {codes[1]}, mlc::neg_zero_())"
        if self.is_half(y):
            return f"__builtin_fmaf({codes[1]}, {codes[0]}, mlc::neg_zero_())"
        return None

    @staticmethod
    def const(e: Const) -> tuple[str, str]:
        v, dt = e.value, e.dtype
        if isinstance(v, bool) or dt == torch.bool:
            return ("true" if v else "false"), "bool"
        if dt in (torch.float16, torch.bfloat16):
            return float_literal(_round_half(float(v), dt)), "float"
        if dt in (torch.int64, torch.int32, torch.int16, torch.int8, torch.uint8):
            return f"((int64_t){int(v)}LL)", "int64_t"
        if isinstance(v, int) and dt is None:
            return f"((int64_t){v}LL)", "int64_t"
        return float_literal(float(v)), "float"

    def value_type(self, e: Expr) -> VType | None:
        if self.vtypes is None:
            return None
        ins, temps = self.vtypes
        return expr_type(e, ins.__getitem__, lambda n: temps.get(n, (torch.float32, True)),
                         self._vmemo)

    def call(self, e: Call) -> tuple[str, str]:
        code, t = self._call(e)
        if t == "float":
            nt = self.value_type(e)
            if nt is not None and nt[0] in ROUND:
                code = f"{ROUND[nt[0]]}({code})"
        return code, t

    def _call(self, e: Call) -> tuple[str, str]:
        plain, self._plain = self._plain, False
        args = [self(a) for a in e.args]
        if e.fn in ("add", "sub"):
            nt = self.value_type(e)
            if nt is not None and nt[0] in ROUND:
                # torch's CPU add and sub of an fp16/bf16 tensor and a 0-dim
                # constant first convert the constant to that type (its mul
                # and div use the constant's fp32 value)
                args = [(float_literal(_round_half(float(x.value), nt[0])), "float")
                        if isinstance(x, Const) and not isinstance(x.value, bool) else arg
                        for x, arg in zip(e.args, args)]
        codes = [c for c, _ in args]
        types = [t for _, t in args]
        top = max(types, key=lambda t: _RANK[t]) if types else "float"
        fn = e.fn
        a = codes[0]
        if fn in ("add", "sub", "mul"):
            if types[0] == "float" and types[1] == "float" and not plain:
                m = self.mixed(e, codes)
                if m is not None:
                    return m, "float"
            op = {"add": "+", "sub": "-", "mul": "*"}[fn]
            t = "int64_t" if top == "bool" else top
            return f"({a} {op} {codes[1]})", t
        if fn == "div":
            if _RANK[top] <= _RANK["int64_t"]:
                return f"((float)({a}) / (float)({codes[1]}))", "float"
            if top == "float":
                fast = _const_divisor(e.args[1])
                if fast is not None:
                    c, y, exact_mul = fast
                    if exact_mul:
                        if self.is_half(e.args[0]):
                            return f"__builtin_fmaf({a}, {float_literal(y)}, mlc::neg_zero_())", "float"
                        return f"({a} * {float_literal(y)})", "float"
                    return f"mlc::div_rcp({a}, {float_literal(c)}, {float_literal(y)})", "float"
            return f"({a} / {codes[1]})", top
        if fn in ("gt", "lt", "ge", "le", "eq", "ne"):
            op = {"gt": ">", "lt": "<", "ge": ">=", "le": "<=", "eq": "==", "ne": "!="}[fn]
            return f"({a} {op} {codes[1]})", "bool"
        if fn == "logical_and":
            return f"((bool)({a}) && (bool)({codes[1]}))", "bool"
        if fn == "logical_or":
            return f"((bool)({a}) || (bool)({codes[1]}))", "bool"
        if fn == "logical_not":
            return f"(!({a}))", "bool"
        if fn == "where":
            t = max(types[1:], key=lambda x: _RANK[x])
            return f"(({a}) ? ({t})({codes[1]}) : ({t})({codes[2]}))", t
        if fn in ("maximum", "minimum"):
            helper = "max_" if fn == "maximum" else "min_"
            return f"mlc::{helper}<{top}>(({top})({a}), ({top})({codes[1]}))", top
        if fn == "pow":
            t = "double" if top == "double" else "float"
            return f"mlc::pow_(({t})({a}), ({t})({codes[1]}))", t
        if fn == "neg":
            if types[0] == "float":
                return f"mlc::neg_({a})", "float"
            return f"(-({a}))", "int64_t" if types[0] == "bool" else types[0]
        if fn == "abs":
            return f"mlc::abs_({a})", types[0]
        if fn == "floor":
            return f"mlc::floor_({a})", types[0]
        if fn == "reciprocal":
            if types[0] == "double":
                return f"(1.0 / ({a}))", "double"
            return f"(1.0f / (float)({a}))", "float"
        if fn in ("exp", "log", "sqrt", "rsqrt", "sin", "cos", "tanh", "erf", "sigmoid"):
            t = "double" if types[0] == "double" else "float"
            arg = a if types[0] in ("float", "double", "int64_t") else f"(float)({a})"
            return f"mlc::{fn}_({arg})", t
        raise KeyError(f"no HIP form for scalar function {fn!r}")


def half_inputs(k) -> frozenset[int]:
    """Input slots stored as fp16 (read into fp32 registers by conversion)."""
    return frozenset(i for i, a in enumerate(k.inputs) if a.dtype == torch.float16)


def value_types_of(k, online: frozenset[str] = frozenset()):
    """(input types, temporary types) of ``k`` for ``Renderer``."""
    return [load_type(a.dtype) for a in k.inputs], kernel_types(k, online)


def narrow_values(vt) -> frozenset[str]:
    """Temporaries typed fp16 or bf16: no fp32 shortcut may skip their rounding."""
    return frozenset(n for n, t in vt[1].items() if t[0] in ROUND)


def _reduced(step: Reduce, vt, code: str) -> str:
    """A row reduction's result, rounded to its type when that is fp16 or
    bf16 (torch reduces a narrow tensor in fp32 and rounds once)."""
    t = vt[1][step.name][0]
    return f"{ROUND[t]}({code})" if t in ROUND else code


def bind_defs(k: ReductionKernel) -> dict[str, Expr]:
    return {s.name: s.expr for s in k.steps if isinstance(s, Bind)}


HALF_STORAGE = (torch.float16, torch.bfloat16)


def rounded_only(name: str, exprs, stores, dtypes=HALF_STORAGE) -> bool:
    """Whether temporary ``name`` reaches nothing but a rounding to one of
    ``dtypes``: every use in ``exprs`` is a cast of it to such a type, and
    every store of it (``stores``: (expression, storage dtype) pairs) is into
    such a type. Its fp32 value is then never seen except through that
    rounding."""
    target = Ref(name)

    def bare_use(e) -> bool:
        if e == target:
            return True
        if isinstance(e, Cast):
            if e.x == target and e.dtype in dtypes:
                return False
            return bare_use(e.x)
        if isinstance(e, Call):
            return any(bare_use(a) for a in e.args)
        return False

    if any(bare_use(e) for e in exprs):
        return False
    for e, dt in stores:
        if e == target:
            if dt not in dtypes:
                return False
        elif bare_use(e):
            return False
    return True


def _uses(k):
    """(expressions, (stored expression, storage dtype) pairs) of a kernel."""
    if isinstance(k, ReductionKernel):
        exprs = [s.expr for s in k.steps]
    else:
        exprs = [e for _, e in k.body]
    return exprs, [(k.out_expr[a.value.name], a.dtype) for a in k.outputs]


def storage_rounded(k: ReductionKernel, name: str) -> bool:
    """``rounded_only`` for a temporary of ``k``, to fp16 or bf16."""
    return rounded_only(name, *_uses(k))


def fp16_rounded(k) -> frozenset[str]:
    """Temporaries of ``k`` that only reach a rounding to fp16."""
    exprs, stores = _uses(k)
    names = [s.name for s in k.steps if isinstance(s, Bind)] if isinstance(k, ReductionKernel) \
        else [n for n, _ in k.body]
    return frozenset(n for n in names if rounded_only(n, exprs, stores, (torch.float16,)))


def _fp32(v: float) -> float:
    return float(np.float32(v))


def _const_divisor(d: Expr):
    """(c, RN(1/c), whether x*RN(1/c) is exact) for a constant fp32 divisor
    in the normal range, else None. A power-of-two divisor has an exact
    reciprocal, so the division is a multiplication; any other one goes
    through ``mlc::div_rcp`` (Markstein), which returns the correctly rounded
    quotient."""
    if not isinstance(d, Const) or isinstance(d.value, bool) or d.dtype == torch.bool:
        return None
    if d.dtype in (torch.float16, torch.bfloat16):
        c = _round_half(float(d.value), d.dtype)
    elif d.dtype in (None, torch.float32) or (isinstance(d.value, int) and d.dtype is None):
        c = _fp32(float(d.value))
    else:
        return None
    if not math.isfinite(c) or c == 0.0 or not (2.0 ** -120 < abs(c) < 2.0 ** 120):
        return None
    y = float(np.float32(1.0) / np.float32(c))
    mant = math.frexp(abs(c))[0]
    return c, y, mant == 0.5


def _scalar_division(expr: Expr, scalars: set[str]):
    """(numerator, divisor name) when ``expr`` divides by a row-uniform fp32
    temporary (a reduce result or a row-scalar bind)."""
    if (isinstance(expr, Call) and expr.fn == "div" and isinstance(expr.args[1], Ref)
            and expr.args[1].name in scalars):
        return expr.args[0], expr.args[1].name
    return None


def cast_code(code: str, dtype: torch.dtype) -> tuple[str, str]:
    if dtype == torch.float32:
        return f"((float)({code}))", "float"
    if dtype == torch.float16:
        return f"mlc::round_f16((float)({code}))", "float"
    if dtype == torch.bfloat16:
        return f"mlc::round_bf16((float)({code}))", "float"
    if dtype == torch.float64:
        return f"((double)({code}))", "double"
    if dtype == torch.bool:
        return f"(({code}) != 0)", "bool"
    if dtype == torch.int32:
        return f"((int64_t)(int32_t)({code}))", "int64_t"
    return f"((int64_t)({code}))", "int64_t"


# --------------------------------------------------------------------------
# index arithmetic
# --------------------------------------------------------------------------

def axis_terms(imap: IndexMap, var: str):
    a = imap.axis(var)
    return a.terms if a is not None else ()


def axis_numel(imap: IndexMap, var: str) -> int:
    a = imap.axis(var)
    return a.numel if a is not None else 1


def render_terms(terms, numel: int, var: str, it: str) -> list[str]:
    parts = []
    for size, ostride, istride in terms:
        t = var if ostride == 1 else f"({var} / ({it}){ostride})"
        if size * ostride != numel:
            t = f"({t} % ({it}){size})"
        if istride != 1:
            t = f"{t} * ({it}){istride}"
        parts.append(t)
    return parts


def join_offset(parts: list[str], it: str) -> str:
    if not parts:
        return f"(({it})0)"
    return "(" + " + ".join(parts) + ")"


@dataclass
class Access:
    """How one operand is addressed over a V-element run of the fast axis."""

    mode: str  # "uniform" | "affine" | "gather"
    stride: int = 0
    aligned: bool = False


def classify_access(terms, numel: int, base_terms_is: list[int], base: int, V: int) -> Access:
    """Access mode of an axis whose packs start at multiples of V.

    ``terms`` are the axis's canonical terms; the run is affine when one term
    moves with unit iteration stride (and does not wrap inside a pack) and
    every other term is constant over the pack. ``aligned`` means the run
    starts on a V-element boundary for every pack, so 128-bit packs apply.
    """
    if V == 1:
        fast = [t for t in terms if t[1] == 1]
        if not fast:
            return Access("uniform")
        return Access("affine", stride=fast[0][2], aligned=False)
    fast = None
    for size, ostride, istride in terms:
        if ostride == 1:
            if size % V != 0 and size != numel:
                return Access("gather")
            fast = (size, ostride, istride)
        elif ostride % V != 0:
            return Access("gather")
    if fast is None:
        return Access("uniform")
    others = [t[2] for t in terms if t[1] != 1] + list(base_terms_is)
    aligned = fast[2] == 1 and base % V == 0 and all(s % V == 0 for s in others)
    return Access("affine", stride=fast[2], aligned=aligned)


def index_type(k) -> str:
    """32-bit offsets unless some operand's buffer is too large for them."""
    for a in list(k.inputs) + list(k.outputs):
        if a.value.buffer.numel >= 2 ** 31:
            return "uint64_t"
    return "uint32_t"


# --------------------------------------------------------------------------
# kernel sources
# --------------------------------------------------------------------------

@dataclass
class LaunchSpec:
    """Geometry for one kernel launch; ``symbol`` names the device function."""

    symbol: str
    grid: int
    block: int
    lds_bytes: int = 0
    meta: dict = field(default_factory=dict)


def _params(k) -> list[str]:
    ps = [f"const {STORAGE[a.dtype]}* __restrict__ in{i}" for i, a in enumerate(k.inputs)]
    ps += [f"{STORAGE[a.dtype]}* __restrict__ out{i}" for i, a in enumerate(k.outputs)]
    return ps


def _vec_width(dtypes) -> int:
    sizes = [itemsize(d) for d in dtypes]
    return max(1, 16 // min(sizes)) if sizes else 1


def emit_pointwise(k: PointwiseKernel, cfg: Config | None = None) -> tuple[str, LaunchSpec]:
    """Source (with the placeholder name ``KERNEL``) and launch spec."""
    N = k.numel
    it = index_type(k)
    V = _vec_width([a.dtype for a in k.inputs] + [a.dtype for a in k.outputs])
    while V > 1 and N < V:
        V //= 2

    accesses = []
    for a in k.inputs:
        terms = axis_terms(a.index, "idx")
        accesses.append(classify_access(terms, N, [], a.index.base, V))
    out_access = []
    for a in k.outputs:
        terms = axis_terms(a.index, "idx")
        out_access.append(classify_access(terms, N, [], a.index.base, V))

    def offset(a, var: str) -> str:
        parts = render_terms(axis_terms(a.index, "idx"), N, var, it)
        if a.index.base:
            parts.append(f"({it}){a.index.base}")
        return join_offset(parts, it)

    in_types = [compute_type(a.dtype) for a in k.inputs]
    temp_types: dict[str, str] = {}
    packs = -(-N // V)
    exact = N % V == 0
    B = pointwise_geometry(packs)
    L: list[str] = []
    L.append(f"extern \"C\" __global__ void __launch_bounds__({B}) "
             f"KERNEL({', '.join(_params(k))}) {{")
    L.append(f"  // pointwise over {list(k.space)} = {N} elements, one {V}-element pack "
             "per thread")
    L.append(f"  constexpr {it} N = ({it}){N};")
    L.append(f"  constexpr int V = {V};")
    L.append(f"  const {it} base = ({it})blockIdx.x * {B} + threadIdx.x;")

    half_slots = half_inputs(k)
    defs = dict(k.body)
    to_fp16 = fp16_rounded(k)
    vt = value_types_of(k)

    def body_lines(ref_in, indent: str) -> list[str]:
        lines = []
        r = Renderer(ref_in, lambda n: (n, temp_types[n]), half_slots, defs, to_fp16, vt)
        for name, expr in k.body:
            code, t = r.bind(name, expr)
            temp_types[name] = t
            lines.append(f"{indent}const {t} {name} = {code};")
        return lines, r

    # -- vector path: the pack's loads, then its arithmetic and stores --
    def pack_loads(e0: str) -> list[str]:
        out = []
        for i, (a, acc) in enumerate(zip(k.inputs, accesses)):
            ct, v = in_types[i], f"v{i}"
            if acc.mode == "uniform":
                out.append(f"    const {ct} {v} = mlc::ld(in{i} + {offset(a, e0)});")
            elif acc.mode == "affine" and acc.aligned:
                out.append(f"    {ct} {v}[V]; mlc::load_pack<V>({v}, in{i} + {offset(a, e0)});")
            elif acc.mode == "affine":
                out.append(f"    {ct} {v}[V];")
                out.append(f"    {{ const {it} o = {offset(a, e0)};")
                out.append("#pragma unroll")
                out.append(f"      for (int j = 0; j < V; ++j) {v}[j] = mlc::ld(in{i} + o + ({it})j * ({it}){acc.stride}); }}")
            else:
                out.append(f"    {ct} {v}[V];")
                out.append("#pragma unroll")
                out.append(f"    for (int j = 0; j < V; ++j) {v}[j] = mlc::ld(in{i} + {offset(a, '(' + e0 + ' + (' + it + ')j)')});")
        return out

    def pack_compute_store(e0: str) -> list[str]:
        def ref_vec(slot):
            mode = accesses[slot].mode
            return (f"v{slot}" if mode == "uniform" else f"v{slot}[j]"), in_types[slot]

        out = []
        for i, a in enumerate(k.outputs):
            out.append(f"    {compute_type_of_out(k, a)} o{i}[V];")
        out.append("#pragma unroll")
        out.append("    for (int j = 0; j < V; ++j) {")
        blines, r = body_lines(ref_vec, "      ")
        out += blines
        for i, a in enumerate(k.outputs):
            code, _ = r.store(k.out_expr[a.value.name], a.dtype == torch.float16)
            out.append(f"      o{i}[j] = {code};")
        out.append("    }")
        for i, (a, acc) in enumerate(zip(k.outputs, out_access)):
            if acc.mode == "affine" and acc.aligned:
                out.append(f"    mlc::store_pack<V>(out{i} + {offset(a, e0)}, o{i});")
            else:
                out.append("#pragma unroll")
                out.append(f"    for (int j = 0; j < V; ++j) mlc::st(out{i} + {offset(a, '(' + e0 + ' + (' + it + ')j)')}, o{i}[j]);")
        return out

    L.append(f"  const {it} e0 = base * V;")
    L.append("  if (e0 >= N) return;")
    vec = pack_loads("e0") + pack_compute_store("e0")

    if exact:
        L.append("  {")
        L += vec
        L.append("  }")
    else:
        L.append("  if (e0 + V <= N) {")
        L += vec
        L.append("  } else {")
        L.append(f"    for ({it} e = e0; e < N; ++e) {{")
        for i, a in enumerate(k.inputs):
            L.append(f"      const {in_types[i]} s{i} = mlc::ld(in{i} + {offset(a, 'e')});")
        temp_types.clear()
        blines, r = body_lines(lambda s: (f"s{s}", in_types[s]), "      ")
        L += blines
        for i, a in enumerate(k.outputs):
            code, _ = r.store(k.out_expr[a.value.name], a.dtype == torch.float16)
            L.append(f"      mlc::st(out{i} + {offset(a, 'e')}, {code});")
        L.append("    }")
        L.append("  }")
    L.append("}")

    grid = max(1, -(-packs // B))
    spec = LaunchSpec("", grid, B, 0,
                      {"kind": "pointwise", "vec": V, "numel": N,
                       "access": [a.mode + ("+aligned" if a.aligned else "") for a in accesses]})
    return "\n".join(L), spec


TRANSPOSE_TILE = 64
TRANSPOSE_BLOCK = 256


def transpose_pattern(k: PointwiseKernel):
    """The batched 2-D transpose a pointwise kernel performs, if any.

    Matches one contiguous output and one input (the *tiled* input) where the
    output's fastest dimension (``r``, size ``Rn``) is strided in the input
    (``Ri``), the input's unit-stride dimension (``c``, size ``Cn``) sits
    directly outside it in the output, and every other dimension is a whole
    ``Rn x Cn`` batch. Any other inputs must not vary along ``r`` (a bias
    indexed by ``c``, say): they are read once per output row. Returns
    (Rn, Cn, Ri, batches, tiled slot) or None.
    """
    if len(k.outputs) != 1:
        return None
    out = k.outputs[0]
    if not (out.index.base == 0 and axis_terms(out.index, "idx") == ((k.numel, 1, 1),)):
        return None
    if out.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        return None
    tiled = [i for i, a in enumerate(k.inputs)
             if any(t[1] == 1 for t in axis_terms(a.index, "idx"))]
    if len(tiled) != 1:
        return None
    slot = tiled[0]
    inp = k.inputs[slot]
    if inp.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        return None
    terms = axis_terms(inp.index, "idx")
    r = [t for t in terms if t[1] == 1]
    c = [t for t in terms if t[2] == 1]
    if len(r) != 1 or len(c) != 1 or r[0] is c[0] or r[0][2] == 1:
        return None
    Rn, _, Ri = r[0]
    Cn, Co, _ = c[0]
    if Co != Rn:
        return None
    plane = Rn * Cn
    if any(t[1] % plane for t in terms if t is not r[0] and t is not c[0]):
        return None
    T = TRANSPOSE_TILE
    if Rn % T or Cn % T:
        return None
    V = 16 // itemsize(inp.dtype)
    if 16 // itemsize(out.dtype) != V:
        return None
    others = [t[2] for t in terms if t is not r[0] and t is not c[0]]
    if inp.index.base % V or Ri % V or any(o % V for o in others):
        return None
    return Rn, Cn, Ri, k.numel // plane, slot


def emit_transpose(k: PointwiseKernel, cfg: Config | None = None) -> tuple[str, LaunchSpec] | None:
    """A batched transpose (with its elementwise body) staged through LDS in
    64x64 tiles: 128-bit loads along the tiled input's contiguous dimension,
    128-bit stores along the output's, so neither side gathers. Inputs that
    are constant along the output's fast dimension load once per output row."""
    pat = transpose_pattern(k)
    if pat is None:
        return None
    Rn, Cn, Ri, nb, slot = pat
    T, B = TRANSPOSE_TILE, TRANSPOSE_BLOCK
    inp, out = k.inputs[slot], k.outputs[0]
    S = STORAGE[inp.dtype]
    V = 16 // itemsize(inp.dtype)
    it = index_type(k)
    W = T + 2  # LDS row pitch: the transposed gather hits distinct banks
    per_thread = (T * T // V) // B

    def offset_at(a, var: str) -> str:
        parts = render_terms(axis_terms(a.index, "idx"), k.numel, var, it)
        if a.index.base:
            parts.append(f"({it}){a.index.base}")
        return join_offset(parts, it)

    in_types = [compute_type(a.dtype) for a in k.inputs]
    temp_types: dict[str, str] = {}

    def operand(s_: int):
        return ("x0" if s_ == slot else f"xr{s_}"), in_types[s_]

    r = Renderer(operand, lambda n: (n, temp_types[n]), vtypes=value_types_of(k))
    body = []
    for name, expr in k.body:
        code, t = r(expr)
        temp_types[name] = t
        body.append(f"      const {t} {name} = {code};")
    oc, _ = r(k.out_expr[out.value.name])
    rt_n, ct_n = Rn // T, Cn // T
    L = [f"extern \"C\" __global__ void __launch_bounds__({B}) "
         f"KERNEL({', '.join(_params(k))}) {{",
         f"  // transpose: {nb} x [{Rn} x {Cn}] (row stride {Ri}) -> [{Cn} x {Rn}], "
         f"{T}x{T} tiles through LDS",
         f"  constexpr int T = {T}, V = {V}, W = {W};",
         f"  __shared__ {S} tile[T * W];",
         f"  const {it} t = blockIdx.x;",
         f"  const {it} r0 = (t % ({it}){rt_n}) * T;",
         f"  const {it} c0 = ((t / ({it}){rt_n}) % ({it}){ct_n}) * T;",
         f"  const {it} b = t / ({it}){rt_n * ct_n};",
         f"  const {it} o0 = b * ({it}){Rn * Cn} + c0 * ({it}){Rn} + r0;",
         f"  const {it} i0 = {offset_at(inp, 'o0')};",
         "#pragma unroll",
         f"  for (int u = 0; u < {per_thread}; ++u) {{",
         f"    const int id = u * {B} + (int)threadIdx.x;",
         "    const int rr = id / (T / V), p = id % (T / V);",
         f"    const mlc::pack<{S}, V> w = *reinterpret_cast<const mlc::pack<{S}, V>*>("
         f"in{slot} + i0 + ({it})rr * ({it}){Ri} + ({it})(p * V));",
         "#pragma unroll",
         "    for (int j = 0; j < V; ++j) tile[rr * W + p * V + j] = w.x[j];",
         "  }",
         "  __syncthreads();",
         "#pragma unroll",
         f"  for (int u = 0; u < {per_thread}; ++u) {{",
         f"    const int id = u * {B} + (int)threadIdx.x;",
         "    const int cc = id / (T / V), q = id % (T / V);"]
    for s_, a in enumerate(k.inputs):
        if s_ != slot:
            L.append(f"    const {it} oc{s_} = o0 + ({it})cc * ({it}){Rn};")
            L.append(f"    const {in_types[s_]} xr{s_} = mlc::ld(in{s_} + {offset_at(a, f'oc{s_}')});")
    L += [f"    {compute_type_of_out(k, out)} o[V];",
          "#pragma unroll",
          "    for (int j = 0; j < V; ++j) {",
          "      const auto x0 = mlc::ld(&tile[(q * V + j) * W + cc]);"]
    L += body
    L += [f"      o[j] = {oc};",
          "    }",
          f"    mlc::store_pack<V>(out0 + o0 + ({it})cc * ({it}){Rn} + ({it})(q * V), o);",
          "  }",
          "}"]
    grid = nb * rt_n * ct_n
    spec = LaunchSpec("", grid, B, 0, {"kind": "transpose", "vec": V, "numel": k.numel,
                                       "tile": T, "rows": Rn, "cols": Cn, "batches": nb,
                                       "access": ["transpose"]})
    return "\n".join(L), spec


#: pointwise launch shape: threads per workgroup (one pack per thread: more
#: packs per thread, with every pack's loads issued first, measured slower at
#: every BERT b32 size, MALL-resident or cold)
POINTWISE_TUNING = {"block": 512}


def pointwise_geometry(packs: int) -> int:
    """Threads per workgroup of a pointwise launch over ``packs`` packs."""
    return POINTWISE_TUNING["block"]


def compute_type_of_out(k, a) -> str:
    """Register type of an output's stored expression."""
    e = k.out_expr[a.value.name]
    temp_types: dict[str, str] = {}
    if isinstance(k, PointwiseKernel):
        for name, expr in k.body:
            temp_types[name] = _type_only(expr, k, temp_types)
    else:
        for s in k.steps:
            temp_types[s.name] = _type_only(s.expr, k, temp_types)
    return _type_only(e, k, temp_types)


def _type_only(e: Expr, k, temp_types) -> str:
    r = Renderer(lambda s: ("x", compute_type(k.inputs[s].dtype)), lambda n: ("x", temp_types[n]))
    return r(e)[1]


# --------------------------------------------------------------------------
# persistent reductions
# --------------------------------------------------------------------------

_IDENTITY = {
    "sum": {"float": "0.0f", "double": "0.0", "int64_t": "((int64_t)0)"},
    "prod": {"float": "1.0f", "double": "1.0", "int64_t": "((int64_t)1)"},
    "max": {"float": "(-__builtin_huge_valf())", "double": "(-__builtin_huge_val())",
            "int64_t": "INT64_MIN"},
    "min": {"float": "__builtin_huge_valf()", "double": "__builtin_huge_val()",
            "int64_t": "INT64_MAX"},
}
_OP = {"sum": "mlc::OpSum", "prod": "mlc::OpProd", "max": "mlc::OpMax", "min": "mlc::OpMin"}


def _prev_pow2(n: int) -> int:
    return 1 << (max(1, n).bit_length() - 1)


#: persistent-reduction shape: packs each lane holds (the widest lane group
#: with ``min_packs <= K <= max_packs`` wins) and the workgroup size cap
#: ``few_rows``: at most this many rows (a batch-1 forward), a launch is latency-bound and
#: each lane's serial chain matters more than per-lane reuse: one pack per lane is allowed
REDUCTION_TUNING = {"min_packs": 2, "max_packs": 8, "block": 128, "few_rows": 4096}


def reduction_geometry(n_rows: int, n_cols: int, V: int) -> dict:
    """Lanes per row G, packs per lane K, rows per workgroup."""
    t = REDUCTION_TUNING
    nvec = -(-n_cols // V)
    min_packs = 1 if n_rows <= t["few_rows"] else t["min_packs"]
    G = None
    if nvec <= WAVE * t["max_packs"]:
        for g in (64, 32, 16, 8, 4, 2, 1):
            if g <= nvec and nvec % g == 0 and min_packs <= nvec // g <= t["max_packs"]:
                G = g
                break
        if G is None:
            for g in (64, 32, 16, 8, 4, 2, 1):
                if g <= nvec and nvec % g == 0 and nvec // g <= t["max_packs"]:
                    G = g
                    break
        if G is None:
            G = min(WAVE, _prev_pow2(nvec))
    else:
        G = 128
        while G < 1024 and -(-nvec // G) > t["max_packs"]:
            G *= 2
    # at least one pack: rows of zero columns (an empty reduced dim) keep
    # their one pack, every lane of it out of range, so each row reduces to
    # the identity and no column is loaded or stored
    K = max(1, -(-nvec // G))
    if G <= WAVE:
        cap = max(1, t["block"] // G)
        rows = max(WAVE // G, min(cap, max(1, -(-n_rows // 1024))))
        rows = 1 << (rows.bit_length() - 1) if rows & (rows - 1) else rows
    else:
        rows = 1
    return {"G": G, "K": K, "rows_per_wg": rows, "block": G * rows, "nvec": nvec}


def _row_col_access(k: ReductionKernel, a, V: int) -> Access:
    C = k.reduce_numel
    col = axis_terms(a.index, "col")
    row_is = [t[2] for t in axis_terms(a.index, "row")]
    return classify_access(col, C, row_is, a.index.base, V)


def _choose_reduction_vec(k: ReductionKernel) -> int:
    C = k.reduce_numel
    col_args = [a for a in k.inputs if a.index.varies_along("col")]
    col_args += [a for a in k.outputs if a.value.name not in k.row_outputs]
    V = _vec_width([a.dtype for a in col_args]) if col_args else 1
    while V > 1:
        if C % V == 0 and all(_row_col_access(k, a, V).mode != "gather" for a in col_args):
            break
        V //= 2
    return V


class _RowOffsets:
    def __init__(self, k: ReductionKernel, it: str) -> None:
        self.k = k
        self.it = it

    def row(self, a, var: str = "row") -> str:
        parts = render_terms(axis_terms(a.index, "row"), axis_numel(a.index, "row"), var, self.it)
        if a.index.base:
            parts.append(f"({self.it}){a.index.base}")
        return join_offset(parts, self.it)

    def col(self, a, var: str) -> str:
        return join_offset(render_terms(axis_terms(a.index, "col"), self.k.reduce_numel, var,
                                        self.it), self.it)


def emit_reduction(k: ReductionKernel, cfg: Config) -> tuple[str, LaunchSpec]:
    if k.two_pass:
        return emit_streamed(k, cfg)
    return emit_persistent(k, cfg)


def emit_persistent(k: ReductionKernel, cfg: Config) -> tuple[str, LaunchSpec]:
    R, C = k.n_rows, k.reduce_numel
    it = index_type(k)
    V = _choose_reduction_vec(k)
    geo = reduction_geometry(R, C, V)
    G, K, RPW, WG = geo["G"], geo["K"], geo["rows_per_wg"], geo["block"]
    exact = C == G * K * V
    offs = _RowOffsets(k, it)
    col_slots = [i for i, a in enumerate(k.inputs) if a.index.varies_along("col")]
    vector = varies_by_column(k)
    in_types = [compute_type(a.dtype) for a in k.inputs]
    temp_types: dict[str, str] = {}

    L: list[str] = []
    L.append(f"extern \"C\" __global__ void __launch_bounds__({WG}) "
             f"KERNEL({', '.join(_params(k))}) {{")
    L.append(f"  // persistent: {R} rows of {C}; {G} lanes x {K} packs x {V} per row, "
             f"{RPW} rows per workgroup")
    L.append(f"  constexpr {it} R = ({it}){R};")
    L.append(f"  constexpr {it} C = ({it}){C};")
    L.append(f"  constexpr int G = {G}, K = {K}, V = {V};")
    lds = 0
    if G > WAVE:
        for s in k.reduces:
            t = _type_only(s.expr, k, _step_types(k))
            L.append(f"  __shared__ {t} lds_{s.name}[G / 64];")
            lds += (G // WAVE) * {"float": 4, "double": 8, "int64_t": 8, "bool": 4}[t]
    L.append(f"  const {it} row = ({it})blockIdx.x * {RPW} + threadIdx.x / G;")
    L.append(f"  const {it} lane = threadIdx.x % G;")
    if R % RPW != 0:
        L.append("  if (row >= R) return;")
    if not exact:
        L.append("  bool valid[K];")
        L.append("#pragma unroll")
        L.append(f"  for (int p = 0; p < K; ++p) valid[p] = (({it})p * G + lane) * V < C;")

    # operands
    for i, a in enumerate(k.inputs):
        ct = in_types[i]
        if i not in col_slots:
            L.append(f"  const {ct} v{i} = mlc::ld(in{i} + {offs.row(a)});")
            continue
        acc = _row_col_access(k, a, V)
        L.append(f"  {ct} v{i}[K][V];")
        L.append(f"  {{ const {it} rb = {offs.row(a)};")
        L.append("#pragma unroll")
        L.append("    for (int p = 0; p < K; ++p) {")
        L.append(f"      const {it} c0 = (({it})p * G + lane) * V;")
        guard = "" if exact else "if (valid[p]) "
        if not exact:
            L.append("      if (!valid[p]) {")
            L.append("#pragma unroll")
            L.append(f"        for (int j = 0; j < V; ++j) v{i}[p][j] = ({ct})0;")
            L.append("        continue;")
            L.append("      }")
        if acc.mode == "affine" and acc.aligned:
            L.append(f"      mlc::load_pack<V>(v{i}[p], in{i} + rb + {offs.col(a, 'c0')});")
        elif acc.mode == "affine":
            L.append(f"      const {it} o = rb + {offs.col(a, 'c0')};")
            L.append("#pragma unroll")
            L.append(f"      for (int j = 0; j < V; ++j) v{i}[p][j] = mlc::ld(in{i} + o + ({it})j * ({it}){acc.stride});")
        else:
            L.append("#pragma unroll")
            L.append(f"      for (int j = 0; j < V; ++j) v{i}[p][j] = mlc::ld(in{i} + rb + {offs.col(a, '(c0 + (' + it + ')j)')});")
        L.append("    }")
        L.append("  }")
        del guard

    def ref_elem(slot):
        if slot in col_slots:
            return f"v{slot}[p][j]", in_types[slot]
        return f"v{slot}", in_types[slot]

    def ref_scalar(slot):
        if slot in col_slots:
            raise AssertionError("column operand read in a row-scalar expression")
        return f"v{slot}", in_types[slot]

    def temp_elem(name):
        return (f"{name}[p][j]" if name in vector else name), temp_types[name]

    def temp_scalar(name):
        if name in vector:
            raise AssertionError("vector temp read in a row-scalar expression")
        return name, temp_types[name]

    nonpos = nonpositive_args(k)
    half_slots, defs, to_fp16 = half_inputs(k), bind_defs(k), fp16_rounded(k)
    vt = value_types_of(k)
    narrow = narrow_values(vt)
    elem_r = _NonPosExpRenderer(ref_elem, temp_elem, nonpos, half_slots, defs, to_fp16,
                                fast_softmax_exps(k, nonpos) - narrow, vt)
    scal_r = Renderer(ref_scalar, temp_scalar, half_slots, defs, to_fp16, vt)
    rcp_for = _reciprocal_divisors(k, vector)

    def elem_loop(target: str, code: str) -> list[str]:
        return ["#pragma unroll", "  for (int p = 0; p < K; ++p)", "#pragma unroll",
                "    for (int j = 0; j < V; ++j)", f"      {target}[p][j] = {code};"]

    for s in k.steps:
        if isinstance(s, Bind):
            if s.name in vector:
                code, t = elem_r.bind(s.name, s.expr)
                temp_types[s.name] = t
                L.append(f"  {t} {s.name}[K][V];")
                sd = _scalar_division(s.expr, rcp_for) if s.name not in narrow else None
                if sd is not None and t == "float" and softmax_sum(k, sd[1], nonpos):
                    num, d = elem_r(sd[0])[0], sd[1]
                    L += elem_loop(s.name, _row_division(k, s.name, sd[0], num, d, nonpos))
                elif sd is not None and t == "float":
                    num, d = elem_r(sd[0])[0], sd[1]
                    L.append(f"  if (__all(ok_{d})) {{")
                    L += elem_loop(s.name, _row_division(k, s.name, sd[0], num, d, nonpos))
                    L.append("  } else {")
                    L += elem_loop(s.name, code)
                    L.append("  }")
                else:
                    L += elem_loop(s.name, code)
            else:
                code, t = scal_r.bind(s.name, s.expr)
                temp_types[s.name] = t
                L.append(f"  const {t} {s.name} = {code};")
                L += _reciprocal_lines(s.name, rcp_for)
            continue
        # Reduce
        code, t = elem_r(s.expr)
        if t == "bool":
            code, t = f"((int64_t)({code}))", "int64_t"
        temp_types[s.name] = t
        ident = _IDENTITY[s.kind][t]
        op = _OP[s.kind]
        varies = _expr_varies(s.expr, col_slots, vector)
        L.append(f"  {t} {s.name};")
        L.append("  {")
        if varies:
            L.append(f"    {t} acc = {ident};")
            L.append("#pragma unroll")
            L.append("    for (int p = 0; p < K; ++p) {")
            if not exact:
                L.append("      if (!valid[p]) continue;")
            L.append("#pragma unroll")
            L.append(f"      for (int j = 0; j < V; ++j) acc = {op}::f(acc, ({t})({code}));")
            L.append("    }")
        else:
            # constant along the row: every valid element contributes the same value
            scode, _ = scal_r(s.expr)
            L.append(f"    {t} acc = {ident};")
            L.append(f"    const {t} x = ({t})({scode});")
            L.append("#pragma unroll")
            L.append("    for (int p = 0; p < K; ++p) {")
            if not exact:
                L.append("      if (!valid[p]) continue;")
            L.append(f"      for (int j = 0; j < V; ++j) acc = {op}::f(acc, x);")
            L.append("    }")
        slot = f"lds_{s.name}" if G > WAVE else "nullptr"
        L.append(f"    {s.name} = {_reduced(s, vt, f'mlc::row_reduce<G, {op}>(acc, ({t}*){slot})')};")
        L.append("  }")
        L += _reciprocal_lines(s.name, rcp_for)

    # element stores
    for i, a in enumerate(k.outputs):
        nm = a.value.name
        if nm in k.row_outputs:
            continue
        e = k.out_expr[nm]
        acc = _row_col_access(k, a, V)
        ot = compute_type_of_out(k, a)
        L.append(f"  {{ // store out{i}")
        L.append(f"    const {it} rb = {offs.row(a)};")
        L.append("#pragma unroll")
        L.append("    for (int p = 0; p < K; ++p) {")
        if not exact:
            L.append("      if (!valid[p]) continue;")
        L.append(f"      const {it} c0 = (({it})p * G + lane) * V;")
        half_out = a.dtype == torch.float16
        if _expr_varies(e, col_slots, vector):
            code, _ = elem_r.store(e, half_out)
        else:
            code, _ = scal_r.store(e, half_out)
        L.append(f"      {ot} o[V];")
        L.append("#pragma unroll")
        L.append(f"      for (int j = 0; j < V; ++j) o[j] = {code};")
        if acc.mode == "affine" and acc.aligned:
            L.append(f"      mlc::store_pack<V>(out{i} + rb + {offs.col(a, 'c0')}, o);")
        else:
            L.append("#pragma unroll")
            L.append(f"      for (int j = 0; j < V; ++j) mlc::st(out{i} + rb + {offs.col(a, '(c0 + (' + it + ')j)')}, o[j]);")
        L.append("    }")
        L.append("  }")

    # row stores
    row_store = [(i, a) for i, a in enumerate(k.outputs) if a.value.name in k.row_outputs]
    if row_store:
        L.append("  if (lane == 0) {")
        for i, a in row_store:
            code, _ = scal_r.store(k.out_expr[a.value.name], a.dtype == torch.float16)
            L.append(f"    mlc::st(out{i} + {offs.row(a)}, {code});")
        L.append("  }")
    L.append("}")

    grid = -(-R // RPW)
    spec = LaunchSpec("", grid, WG, lds, {"kind": "reduction", "mode": "persistent", "vec": V,
                                          "lanes_per_row": G, "packs": K, "rows_per_wg": RPW,
                                          "rows": R, "cols": C})
    return "\n".join(L), spec


def nonpositive_args(k: ReductionKernel) -> set[Expr]:
    """Expressions that are ``x - rowmax(x)`` in ``k`` (a ``sub`` whose second
    operand is a max reduce of its first, and the binds holding one): never
    positive, so their ``exp`` needs no overflow path (``mlc::exp_nonpos``)."""
    maxes = {s.name: s.expr for s in k.steps if isinstance(s, Reduce) and s.kind == "max"}
    out: set[Expr] = set()

    def is_sub(e) -> bool:
        return (isinstance(e, Call) and e.fn == "sub" and isinstance(e.args[1], Ref)
                and maxes.get(e.args[1].name) == e.args[0])

    for s in k.steps:
        if isinstance(s, Bind) and is_sub(s.expr):
            out.add(s.expr)
            out.add(Ref(s.name))
    for s in k.steps:
        for e in _subexprs(s.expr):
            if is_sub(e):
                out.add(e)
    return out


def _subexprs(e):
    yield e
    if isinstance(e, Call):
        for a in e.args:
            yield from _subexprs(a)
    elif isinstance(e, Cast):
        yield from _subexprs(e.x)


def _bounded_exp(e: Expr, k: ReductionKernel, nonpos: set) -> bool:
    """``e`` is ``exp`` of a never-positive argument (or a bind holding one):
    at most 1, never infinite."""
    if isinstance(e, Ref):
        e = next((s.expr for s in k.steps if isinstance(s, Bind) and s.name == e.name), None)
    return isinstance(e, Call) and e.fn == "exp" and e.args[0] in nonpos


def softmax_sum(k: ReductionKernel, name: str, nonpos) -> bool:
    """Whether ``name`` is a row sum of ``exp(x - rowmax(x))`` (``nonpos``
    holds those arguments). The row's maximum element contributes exp(0) = 1
    and no term is negative, so the sum lies in [1, row length] or is NaN:
    always in the range where the hoisted reciprocal is exact enough, so its
    divisions need no range guard (a NaN sum gives NaN either way)."""
    step = next((s for s in k.steps if s.name == name), None)
    return (isinstance(step, Reduce) and step.kind == "sum"
            and _bounded_exp(step.expr, k, nonpos))


def _row_division(k: ReductionKernel, name: str, num_expr: Expr, num: str, d: str, nonpos) -> str:
    """Per-element ``num / d`` for a row-uniform divisor with ``rcp_d`` =
    RN(1/d) hoisted and d in the normal range (the caller's guard).

    A quotient that only reaches a rounding to fp16/bf16 is ``num * rcp_d``:
    at most 1.5 fp32 ulp from the quotient, 2^12 times below the half ulp of
    fp16 that the rounding then adds. The correctly rounded quotient and this
    product round to different fp16 values only when they straddle an fp16
    rounding boundary, and then by one fp16 ulp. Any other quotient is
    correctly rounded (``mlc::div_rcp``; ``div_rcp_finite`` when the numerator
    is a softmax's exp, never infinite)."""
    if storage_rounded(k, name):
        return f"({num} * rcp_{d})"
    div = "div_rcp_finite" if _bounded_exp(num_expr, k, nonpos) else "div_rcp"
    return f"mlc::{div}({num}, {d}, rcp_{d})"


def fast_softmax_exps(k: ReductionKernel, nonpos) -> frozenset[str]:
    """Binds ``e = exp(x - rowmax(x))`` of a softmax whose probabilities reach
    nothing but a rounding to fp16/bf16: ``e`` is read only by its row sum and
    by divisions ``e / sum``, the sum only by those divisions, and every
    quotient is storage-rounded (``storage_rounded``).

    Such an exp may be ``mlc::exp_fast_shift(x, rowmax)``, one fma and
    ``v_exp_f32``: the rounding of ``rowmax·log2 e`` is a common factor of the
    numerators and of their sum, so it cancels in the quotient, and what is
    left is the fma's one rounding of the exponent, about 1.2e-6 relative for
    exponents up to 20 in size, against fp16's half ulp of 4.9e-4 that the
    storage rounding adds (the attention kernels' softmax is written the same
    way, for the same reason)."""
    steps = {s.name: s for s in k.steps}
    found = set()
    for s in k.steps:
        if not (isinstance(s, Reduce) and isinstance(s.expr, Ref) and softmax_sum(k, s.name, nonpos)):
            continue
        e_name, total = s.expr.name, Ref(s.name)
        e_ref = Ref(e_name)
        bind = steps.get(e_name)
        if not (isinstance(bind, Bind) and isinstance(bind.expr, Call) and bind.expr.fn == "exp"):
            continue
        arg = bind.expr.args[0]
        arg = steps[arg.name].expr if isinstance(arg, Ref) and isinstance(steps.get(arg.name), Bind) else arg
        if not (isinstance(arg, Call) and arg.fn == "sub" and bind.expr.args[0] in nonpos):
            continue
        quotient = Call("div", (e_ref, total))
        ok = True
        divisions = []
        for st in k.steps:
            if st.name in (s.name, e_name):
                continue
            uses = set(_subexprs(st.expr))
            if total in uses or e_ref in uses:
                if isinstance(st, Bind) and st.expr == quotient and storage_rounded(k, st.name):
                    divisions.append(st.name)
                else:
                    ok = False
        for a in k.outputs:
            uses = set(_subexprs(k.out_expr[a.value.name]))
            if total in uses or e_ref in uses:
                ok = False
        if ok and divisions:
            found.add(e_name)
    return frozenset(found)


class _NonPosExpRenderer(Renderer):
    """``exp`` of an argument known to be at most 0 as ``mlc::exp_nonpos``;
    the binds of ``fast`` (``fast_softmax_exps``) as
    ``mlc::exp_fast_shift(x, rowmax)``."""

    def __init__(self, operand, temp, nonpos: set, half_slots=frozenset(), defs=None,
                 to_fp16=frozenset(), fast=frozenset(), vtypes=None) -> None:
        super().__init__(operand, temp, half_slots, defs, to_fp16, vtypes)
        self.nonpos = nonpos
        self.fast = frozenset(fast)

    def bind(self, name: str, e: Expr) -> tuple[str, str]:
        if name in self.fast:
            arg = e.args[0]
            if isinstance(arg, Ref):
                arg = self.defs[arg.name]
            (x, tx), (m, tm) = self(arg.args[0]), self(arg.args[1])
            if tx == "float" and tm == "float":
                return f"mlc::exp_fast_shift({x}, {m})", "float"
        return super().bind(name, e)

    def _call(self, e: Call) -> tuple[str, str]:
        if e.fn == "exp" and e.args[0] in self.nonpos:
            code, t = self(e.args[0])
            if t == "float":
                return f"mlc::exp_nonpos({code})", "float"
        return super()._call(e)


def _reciprocal_divisors(k: ReductionKernel, vector: set[str]) -> set[str]:
    """Row-uniform fp32 temporaries that some per-element bind divides by:
    each gets ``rcp_<name>`` = RN(1/name) once per row."""
    types = _step_types(k)
    scalars = {s.name for s in k.steps if isinstance(s, Reduce) or s.name not in vector}
    found = set()
    for s in k.steps:
        if isinstance(s, Bind) and s.name in vector and types[s.name] == "float":
            sd = _scalar_division(s.expr, scalars)
            if sd is not None and types.get(sd[1]) == "float":
                found.add(sd[1])
    return found


def _reciprocal_lines(name: str, rcp_for: set[str], indent: str = "  ") -> list[str]:
    if name not in rcp_for:
        return []
    return [f"{indent}const float rcp_{name} = 1.0f / {name};",
            f"{indent}const bool ok_{name} = mlc::rcp_ok({name});"]


def _step_types(k: ReductionKernel) -> dict[str, str]:
    types: dict[str, str] = {}
    for s in k.steps:
        t = _type_only(s.expr, k, types)
        if isinstance(s, Reduce) and t == "bool":
            t = "int64_t"
        types[s.name] = t
    return types


def _expr_varies(e: Expr, col_slots, vector) -> bool:
    return bool(expr_loads(e) & set(col_slots)) or bool(expr_refs(e) & set(vector))


# --------------------------------------------------------------------------
# streamed reductions
# --------------------------------------------------------------------------

STREAM_BLOCK = 256


def emit_streamed(k: ReductionKernel, cfg: Config) -> tuple[str, LaunchSpec]:
    """One row per workgroup; each pass of the reduction schedule streams the
    row from HBM in chunks of ``STREAM_BLOCK * V`` elements."""
    R, C = k.n_rows, k.reduce_numel
    it = index_type(k)
    V = _choose_reduction_vec(k)
    G = STREAM_BLOCK
    while G > WAVE and G * V > max(C, WAVE * V):
        G //= 2
    offs = _RowOffsets(k, it)
    col_slots = [i for i, a in enumerate(k.inputs) if a.index.varies_along("col")]
    vector = varies_by_column(k)
    scalars = {b.name for b in scalar_binds(k)}
    passes = plan_passes(k)
    in_types = [compute_type(a.dtype) for a in k.inputs]
    temp_types = _step_types(k)
    chunk_exact = C % (G * V) == 0

    L: list[str] = []
    L.append(f"extern \"C\" __global__ void __launch_bounds__({G}) "
             f"KERNEL({', '.join(_params(k))}) {{")
    L.append(f"  // streamed: {R} rows of {C}, {len(passes)} passes, chunks of {G} lanes x {V}")
    L.append(f"  constexpr {it} C = ({it}){C};")
    L.append(f"  constexpr int G = {G}, V = {V};")
    lds = 0
    need_lds = G > WAVE
    if need_lds:
        for p_i, p in enumerate(passes):
            for r in p.reduces:
                t = temp_types[r.name]
                L.append(f"  __shared__ {t} lds_{r.name}[G / 64];")
                lds += (G // WAVE) * (8 if t in ("double", "int64_t") else 4)
            if p.online_softmax is not None:
                L.append(f"  __shared__ float lds_w_{p.online_softmax.sum_step.name}[G / 64];")
                lds += (G // WAVE) * 4
    L.append(f"  const {it} row = ({it})blockIdx.x;")
    L.append(f"  const {it} lane = threadIdx.x;")
    for i, a in enumerate(k.inputs):
        if i not in col_slots:
            L.append(f"  const {in_types[i]} v{i} = mlc::ld(in{i} + {offs.row(a)});")

    def ref_elem(slot):
        if slot in col_slots:
            return f"v{slot}[j]", in_types[slot]
        return f"v{slot}", in_types[slot]

    def temp_elem(name):
        return (f"{name}[j]" if name in vector else name), temp_types[name]

    def temp_scalar(name):
        return name, temp_types[name]

    nonpos = nonpositive_args(k)
    half_slots, defs, to_fp16 = half_inputs(k), bind_defs(k), fp16_rounded(k)
    online_names = frozenset(n for p in passes if p.online_softmax is not None
                             for n in (p.online_softmax.max_step.name,
                                       p.online_softmax.sum_step.name))
    vt = value_types_of(k, online_names)
    narrow = narrow_values(vt)
    elem_r = _NonPosExpRenderer(ref_elem, temp_elem, nonpos, half_slots, defs, to_fp16, vtypes=vt)
    scal_r = Renderer(lambda s: (f"v{s}", in_types[s]), temp_scalar, half_slots, defs, to_fp16, vt)
    rcp_for = _reciprocal_divisors(k, vector)

    def slots_for(p) -> list[int]:
        used: set[int] = set()
        for b in p.binds:
            used |= expr_loads(b.expr)
        for r in p.reduces:
            used |= expr_loads(r.expr)
        if p.online_softmax is not None:
            used |= expr_loads(p.online_softmax.value)
        for nm in p.stores:
            used |= expr_loads(k.out_expr[nm])
        return sorted(used & set(col_slots))

    def emit_pass(p) -> list[str]:
        out: list[str] = []
        online = p.online_softmax
        if online is not None:
            out.append("  float m_run = (-__builtin_huge_valf()), l_run = 0.0f;")
        for r in p.reduces if online is None else []:
            t = temp_types[r.name]
            out.append(f"  {t} acc_{r.name} = {_IDENTITY[r.kind][t]};")
        out.append(f"  for ({it} base = 0; base < C; base += ({it})G * V) {{")
        out.append(f"    const {it} c0 = base + lane * V;")
        if not chunk_exact:
            out.append("    if (c0 >= C) continue;")
        for i in slots_for(p):
            a = k.inputs[i]
            acc = _row_col_access(k, a, V)
            ct = in_types[i]
            out.append(f"    {ct} v{i}[V];")
            if acc.mode == "affine" and acc.aligned:
                out.append(f"    mlc::load_pack<V>(v{i}, in{i} + {offs.row(a)} + {offs.col(a, 'c0')});")
            else:
                out.append("#pragma unroll")
                out.append(f"    for (int j = 0; j < V; ++j) v{i}[j] = mlc::ld(in{i} + {offs.row(a)} + {offs.col(a, '(c0 + (' + it + ')j)')});")
        for b in p.binds:
            code, t = elem_r.bind(b.name, b.expr)
            out.append(f"    {t} {b.name}[V];")
            sd = _scalar_division(b.expr, rcp_for) if b.name not in narrow else None
            if sd is not None and t == "float" and softmax_sum(k, sd[1], nonpos):
                num, d = elem_r(sd[0])[0], sd[1]
                out.append("#pragma unroll")
                out.append(f"    for (int j = 0; j < V; ++j) {b.name}[j] = "
                           f"{_row_division(k, b.name, sd[0], num, d, nonpos)};")
            elif sd is not None and t == "float":
                num, d = elem_r(sd[0])[0], sd[1]
                out.append(f"    if (__all(ok_{d})) {{")
                out.append("#pragma unroll")
                out.append(f"      for (int j = 0; j < V; ++j) {b.name}[j] = "
                           f"{_row_division(k, b.name, sd[0], num, d, nonpos)};")
                out.append("    } else {")
                out.append("#pragma unroll")
                out.append(f"      for (int j = 0; j < V; ++j) {b.name}[j] = {code};")
                out.append("    }")
            else:
                out.append("#pragma unroll")
                out.append(f"    for (int j = 0; j < V; ++j) {b.name}[j] = {code};")
        if online is not None:
            code, _ = elem_r(online.value)
            out.append("#pragma unroll")
            out.append("    for (int j = 0; j < V; ++j) {")
            out.append(f"      const float x = (float)({code});")
            out.append("      const float m_new = mlc::max_<float>(m_run, x);")
            # m_new is the max of m_run and x: both exponents are at most 0.
            # While every element this lane has seen is -inf, m_new is -inf
            # too; subtracting 0 then keeps exp(-inf - -inf) from being NaN.
            out.append("      const float m_sub = (m_new == (-__builtin_huge_valf())) ? 0.0f : m_new;")
            out.append("      const float alpha = (m_run == (-__builtin_huge_valf())) ? 0.0f : mlc::exp_nonpos(m_run - m_new);")
            out.append("      l_run = l_run * alpha + mlc::exp_nonpos(x - m_sub);")
            out.append("      m_run = m_new;")
            out.append("    }")
        else:
            for r in p.reduces:
                code, t = elem_r(r.expr)
                out.append("#pragma unroll")
                out.append(f"    for (int j = 0; j < V; ++j) acc_{r.name} = {_OP[r.kind]}::f(acc_{r.name}, ({t})({code}));")
        for nm in p.stores:
            i = next(ii for ii, a in enumerate(k.outputs) if a.value.name == nm)
            a = k.outputs[i]
            acc = _row_col_access(k, a, V)
            ot = compute_type_of_out(k, a)
            e = k.out_expr[nm]
            code, _ = (elem_r if _expr_varies(e, col_slots, vector) else scal_r).store(e, a.dtype == torch.float16)
            out.append(f"    {{ {ot} o[V];")
            out.append("#pragma unroll")
            out.append(f"      for (int j = 0; j < V; ++j) o[j] = {code};")
            if acc.mode == "affine" and acc.aligned:
                out.append(f"      mlc::store_pack<V>(out{i} + {offs.row(a)} + {offs.col(a, 'c0')}, o); }}")
            else:
                out.append("#pragma unroll")
                out.append(f"      for (int j = 0; j < V; ++j) mlc::st(out{i} + {offs.row(a)} + {offs.col(a, '(c0 + (' + it + ')j)')}, o[j]); }}")
        out.append("  }")
        if online is not None:
            mx, sm = online.max_step.name, online.sum_step.name
            slot = f"lds_{mx}" if need_lds else "nullptr"
            out.append(f"  const float {mx} = mlc::row_reduce<G, mlc::OpMax>(m_run, (float*){slot});")
            out.append(f"  const float w_{sm} = (m_run == (-__builtin_huge_valf())) ? 0.0f : mlc::exp_nonpos(m_run - {mx});")
            slot = f"lds_{sm}" if need_lds else "nullptr"
            out.append(f"  const float {sm} = mlc::row_reduce<G, mlc::OpSum>(l_run * w_{sm}, (float*){slot});")
            out += _reciprocal_lines(mx, rcp_for) + _reciprocal_lines(sm, rcp_for)
        else:
            for r in p.reduces:
                t = temp_types[r.name]
                slot = f"lds_{r.name}" if need_lds else "nullptr"
                out.append(f"  const {t} {r.name} = "
                           f"{_reduced(r, vt, f'mlc::row_reduce<G, {_OP[r.kind]}>(acc_{r.name}, ({t}*){slot})')};")
                out += _reciprocal_lines(r.name, rcp_for)
        return out

    owner = {r.name: p for p in passes for r in p.reduces}
    emitted: set[int] = set()
    for s in k.steps:
        if isinstance(s, Reduce):
            p = owner[s.name]
            if id(p) in emitted:
                continue
            emitted.add(id(p))
            L += emit_pass(p)
        elif s.name in scalars:
            code, t = scal_r.bind(s.name, s.expr)
            L.append(f"  const {t} {s.name} = {code};")
            L += _reciprocal_lines(s.name, rcp_for)
    for p in passes:
        if p.stores and not p.reduces:
            L += emit_pass(p)
    row_store = [(i, a) for i, a in enumerate(k.outputs) if a.value.name in k.row_outputs]
    if row_store:
        L.append("  if (lane == 0) {")
        for i, a in row_store:
            code, _ = scal_r.store(k.out_expr[a.value.name], a.dtype == torch.float16)
            L.append(f"    mlc::st(out{i} + {offs.row(a)}, {code});")
        L.append("  }")
    L.append("}")
    spec = LaunchSpec("", R, G, lds, {"kind": "reduction", "mode": "streamed", "vec": V,
                                      "lanes_per_row": G, "passes": len(passes),
                                      "rows": R, "cols": C})
    return "\n".join([x for x in L if x != ""]), spec


# --------------------------------------------------------------------------
# extern ops with a native template
# --------------------------------------------------------------------------

EMBED_BLOCK = 256


def emit_extern(k: ExternKernel, cfg: Config | None = None) -> tuple[str, LaunchSpec] | None:
    if k.node.op == "aten.embedding.default":
        return emit_embedding(k)
    return None


def emit_embedding(k: ExternKernel) -> tuple[str, LaunchSpec] | None:
    """``out[i, :] = weight[ids[i], :]`` -- the forward of ``aten.embedding``
    as a bit copy of 128-bit packs, one thread per pack. An id outside
    ``[0, rows of weight)`` yields a zero row and sets the error word (torch
    raises for such an id; the host reads the word back)."""
    node = k.node
    if len(node.args) < 2 or len(node.outputs) != 1:
        return None
    weight, ids = node.args[0], node.args[1]
    out = node.outputs[0]
    if not isinstance(weight, Value) or not isinstance(ids, Value) or len(weight.shape) != 2:
        return None
    if ids.dtype not in (torch.int64, torch.int32) or weight.dtype not in STORAGE:
        return None
    NV, D = weight.shape
    rows = math.prod(ids.shape) if ids.shape else 1
    if out.dtype != weight.dtype or tuple(out.shape) != tuple(ids.shape) + (D,):
        return None
    id_map = build_index([("row", ids.shape)], ids.layout)
    w_map = build_index([("vrow", (NV,)), ("col", (D,))], weight.layout)
    o_map = build_index([("row", ids.shape), ("col", (D,))], out.layout)
    big = max(weight.buffer.numel, out.buffer.numel, ids.buffer.numel) >= 2 ** 31
    it = "uint64_t" if big else "uint32_t"
    V = max(1, 16 // itemsize(weight.dtype))

    def unit_col(imap):
        return axis_terms(imap, "col") in (((D, 1, 1),), ()) if D > 1 else True

    def aligned(imap, var_row):
        others = [t[2] for t in axis_terms(imap, var_row)] + [imap.base]
        return all(o % V == 0 for o in others)

    while V > 1 and not (D % V == 0 and unit_col(w_map) and unit_col(o_map)
                         and aligned(w_map, "vrow") and aligned(o_map, "row")):
        V //= 2
    P = D // V if D % V == 0 else D
    if P * V != D:
        V, P = 1, D
    vrow_terms = axis_terms(w_map, "vrow")
    w_stride = vrow_terms[0][2] if vrow_terms else 0
    w_col = axis_terms(w_map, "col")
    w_cs = w_col[0][2] if w_col else 0
    o_col = axis_terms(o_map, "col")
    o_cs = o_col[0][2] if o_col else 0

    def row_off(imap) -> str:
        parts = render_terms(axis_terms(imap, "row"), rows, "row", it)
        if imap.base:
            parts.append(f"({it}){imap.base}")
        return join_offset(parts, it)

    S = STORAGE[weight.dtype]
    I = STORAGE[ids.dtype]
    L = [f"extern \"C\" __global__ void __launch_bounds__({EMBED_BLOCK}) "
         f"KERNEL(const {S}* __restrict__ in0, const {I}* __restrict__ in1, "
         f"{S}* __restrict__ out0, int* __restrict__ err) {{",
         f"  // embedding: {rows} ids into a [{NV}, {D}] table, {V}-element packs",
         f"  constexpr {it} P = ({it}){P};",
         f"  constexpr int V = {V};",
         f"  const {it} g = ({it})blockIdx.x * {EMBED_BLOCK} + threadIdx.x;",
         f"  if (g >= ({it}){rows} * P) return;",
         f"  const {it} row = g / P;",
         f"  const {it} col = (g % P) * V;",
         f"  const int64_t id = (int64_t)in1[{row_off(id_map)}];",
         f"  {S}* dst = out0 + {row_off(o_map)} + col * ({it}){o_cs};",
         f"  if (id < 0 || id >= (int64_t){NV}) {{",
         f"#pragma unroll",
         f"    for (int j = 0; j < V; ++j) dst[({it})j * ({it}){o_cs}] = mlc::cvt<{S}>(0.0f);",
         f"    *err = 1;",
         f"    return;",
         f"  }}",
         f"  const {S}* src = in0 + ({it}){w_map.base} + ({it})id * ({it}){w_stride} + col * ({it}){w_cs};"]
    if V > 1:
        L.append(f"  *reinterpret_cast<mlc::pack<{S}, V>*>(dst) = "
                 f"*reinterpret_cast<const mlc::pack<{S}, V>*>(src);")
    else:
        L.append("  *dst = *src;")
    L.append("}")
    total = rows * P
    spec = LaunchSpec("", max(1, -(-total // EMBED_BLOCK)), EMBED_BLOCK, 0,
                      {"kind": "embedding", "vec": V, "rows": rows, "cols": D, "table_rows": NV,
                       "buffers": [weight.buffer.name, ids.buffer.name, out.buffer.name],
                       "dtypes": [weight.dtype, ids.dtype, out.dtype],
                       "numels": [weight.buffer.numel, ids.buffer.numel, out.buffer.numel],
                       "error_word": True})
    return "\n".join(L), spec


# --------------------------------------------------------------------------
# module
# --------------------------------------------------------------------------

PRELUDE = """// Generated by mlc's HIP backend for gfx950. One function per distinct fused
// kernel; the launch table lives on the host side.
#include "mlc_cdna4.h"
"""


@dataclass
class Module:
    source: str
    launches: dict[str, LaunchSpec]
    #: symbol -> kernel body (for inspection)
    functions: dict[str, str]


def emit_kernel(k, cfg: Config) -> tuple[str, LaunchSpec] | None:
    """Source and launch spec of one kernel; ``None`` for an extern op that
    stays a library call."""
    if isinstance(k, PointwiseKernel):
        return emit_transpose(k, cfg) or emit_pointwise(k, cfg)
    if isinstance(k, ReductionKernel):
        return emit_reduction(k, cfg)
    if isinstance(k, ExternKernel):
        return emit_extern(k, cfg)
    if isinstance(k, AttentionKernel):
        from .hip_attention import emit_attention

        return emit_attention(k, cfg)
    raise TypeError(f"no HIP emitter for {type(k).__name__}")


def generate_module(schedule: Schedule, cfg: Config) -> str:
    """The HIP source of every generated kernel of ``schedule`` (and of every
    extern op with a native template), as one translation unit: the codegen
    seam of ``mlc/codegen/triton_backend.py:261-287``. The launch table of
    the same module is ``build_module(schedule, cfg).launches``."""
    return build_module(schedule, cfg).source


def build_module(schedule: Schedule, cfg: Config) -> Module:
    """Source, launch table and per-symbol bodies of ``schedule``'s module.
    Identical kernel bodies are emitted once, under a symbol named by the
    body's hash."""
    functions: dict[str, str] = {}
    launches: dict[str, LaunchSpec] = {}
    for k in schedule.kernels:
        emitted = emit_kernel(k, cfg)
        if emitted is None:
            continue
        body, spec = emitted
        digest = hashlib.sha256(body.encode()).hexdigest()[:16]
        symbol = f"mlc_{digest}"
        functions.setdefault(symbol, body.replace("KERNEL(", f"{symbol}(", 1))
        spec.symbol = symbol
        launches[k.name] = spec
    parts = [PRELUDE] + [functions[s] for s in sorted(functions)]
    return Module("\n\n".join(parts) + "\n", launches, functions)
