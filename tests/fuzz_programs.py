"""Seeded random programs for parity: independent chains of pointwise ops,
views (permute, transpose, strided slices, expand), broadcasting operands,
casts and reductions, all in one module so one compile covers them.

Each chain starts from its own input and draws its ops from what the lowering
registers (``mlc/ir/ops.py``), so every program compiles; the shapes are
small and ragged (sizes that 8-element packs do not divide, size-1 dims,
inner dims that are not the unit-stride one) to reach the kernels' tail,
strided and gather paths and the transpose template.
"""

from __future__ import annotations

import random

import torch
import torch.nn.functional as F

SIZES = (1, 2, 3, 5, 7, 8, 9, 16, 24, 33, 64, 100, 128)
DTYPES = (torch.float32, torch.float16, torch.bfloat16)

#: max |got - want| / max(|want|) between the HIP path and the oracle, by the
#: narrowest dtype a chain stores: a few units in the last place of the narrow
#: types (a transcendental or summation-order difference can flip one
#: rounding, which later ops carry), the fp32 bar otherwise
TOLERANCE = {torch.float32: 1e-5, torch.float16: 4e-3, torch.bfloat16: 3e-2}


#: row lengths beyond one wave's reach (multi-wave rows, long streamed rows)
WIDE = (700, 1000, 2049, 4099)


def _shape(rng: random.Random, wide: bool = False) -> list[int]:
    rank = rng.randint(1, 4 if not wide else 3)
    while True:
        s = [rng.choice(SIZES) for _ in range(rank)]
        if wide:
            s[rng.randrange(rank)] = rng.choice(WIDE)
        n = 1
        for d in s:
            n *= d
        if 16 <= n <= (40000 if not wide else 200000):
            return s


_UNARY = [
    ("exp", lambda t: torch.exp(torch.tanh(t))),
    ("tanh", torch.tanh),
    ("sigmoid", torch.sigmoid),
    ("relu", torch.relu),
    ("abs", torch.abs),
    ("neg", torch.neg),
    ("sin", torch.sin),
    ("cos", torch.cos),
    ("sqrt", lambda t: torch.sqrt(t.abs() + 1.0)),
    ("rsqrt", lambda t: torch.rsqrt(t.abs() + 0.5)),
    ("log", lambda t: torch.log(t.abs() + 1.0)),
    ("gelu", F.gelu),
    ("gelu_tanh", lambda t: F.gelu(t, approximate="tanh")),
    ("silu", F.silu),
    ("square", lambda t: torch.clamp(t, -8.0, 8.0) * torch.clamp(t, -8.0, 8.0)),
    ("cube", lambda t: torch.pow(torch.clamp(t, -2.0, 2.0), 3)),
    ("clamp", lambda t: torch.clamp(t, -0.5, 0.7)),
    ("affine", lambda t: t * 1.7 - 0.3),
    ("leaky", lambda t: torch.where(t > 0, t, t * 0.1)),
    ("recip", lambda t: 1.0 / (t.abs() + 1.0)),
]
# only as a chain's first op, on the inputs both sides read bit for bit: a
# floor or integer conversion of a computed value near an integer would turn
# one ulp into one unit
_FIRST = [("floor", lambda t: torch.floor(t * 4.0))]
_TO_INT = ("to_int", lambda t: (t * 4.0).to(torch.int64))
_INT_OPS = [
    ("int_affine", lambda t: t * 3 - 2),
    ("int_abs", torch.abs),
    ("int_neg", torch.neg),
    ("int_max", lambda t: torch.maximum(t, torch.zeros_like(t))),
    ("int_mask", lambda t: torch.where(t > 1, t, t - 5)),
    ("int_bool", lambda t: torch.logical_and(t > 0, t < 3)),
    ("int_to_float", lambda t: t.to(torch.float32) * 0.25),
]

_BINARY = [
    ("add", torch.add),
    ("sub", torch.sub),
    ("mul", lambda a, b: a * torch.tanh(b)),
    ("max", torch.maximum),
    ("min", torch.minimum),
    ("div", lambda a, b: a / (b.abs() + 1.0)),
    # continuous in its operands: a comparison whose branches differ would
    # turn a last-place rounding difference into a different value
    ("where", lambda a, b: torch.where(a > b, a, b)),
]


class Chain:
    """One chain: a start shape and dtype, its ops, and the shapes of the
    extra operands its binary ops read."""

    def __init__(self, rng: random.Random, wide: bool = False):
        self.shape = _shape(rng, wide)
        self.dtype = rng.choice(DTYPES)
        self.ops: list[tuple] = []
        self.extra: list[tuple[list[int], torch.dtype]] = []
        cur = list(self.shape)
        dtype = self.dtype
        #: every dtype a value of the chain is stored in
        self.dtypes = {dtype}
        reduced = False
        normalised = False
        int_prefix = False
        if rng.random() < 0.15:
            int_prefix = True
            # an integer prefix: int64 arithmetic, comparisons to bool, back to fp32
            self.ops.append(("unary",) + _TO_INT)
            for _ in range(rng.randint(1, 3)):
                name, fn = rng.choice(_INT_OPS[:5])
                self.ops.append(("unary", name, fn))
            name, fn = rng.choice(_INT_OPS[5:])
            self.ops.append(("unary", name, fn))
            if name == "int_bool":
                self.ops.append(("unary", "bool_to_float", lambda t: t.to(torch.float32) - 0.5))
            dtype = torch.float32
            self.dtypes.add(dtype)
        for step in range(rng.randint(2, 6)):
            kind = rng.random()
            if kind < 0.35:
                name, fn = rng.choice(_UNARY + (_FIRST if not self.ops else []))
                self.ops.append(("unary", name, fn))
            elif kind < 0.55:
                name, fn = rng.choice(_BINARY)
                # a broadcasting operand: some dims collapsed to 1, maybe fewer dims
                shp = [d if rng.random() < 0.6 else 1 for d in cur]
                while len(shp) > 1 and rng.random() < 0.3 and shp[0] == 1:
                    shp = shp[1:]
                self.extra.append((shp, dtype))
                self.ops.append(("binary", name, fn, len(self.extra) - 1))
            elif kind < 0.75 and len(cur) >= 2:
                v = rng.choice(["permute", "transpose", "slice", "expand"])
                if v == "permute":
                    dims = list(range(len(cur)))
                    rng.shuffle(dims)
                    self.ops.append(("view", "permute", dims))
                    cur = [cur[d] for d in dims]
                elif v == "transpose":
                    a, b = rng.sample(range(len(cur)), 2)
                    self.ops.append(("view", "transpose", (a, b)))
                    cur[a], cur[b] = cur[b], cur[a]
                elif v == "slice":
                    d = rng.randrange(len(cur))
                    if cur[d] >= 3:
                        start = rng.randint(0, 1)
                        stride = rng.choice([1, 2])
                        self.ops.append(("view", "slice", (d, start, stride)))
                        cur[d] = len(range(start, cur[d], stride))
                else:
                    ones = [i for i, n in enumerate(cur) if n == 1]
                    if ones:
                        d = rng.choice(ones)
                        cur[d] = rng.choice([3, 8])
                        self.ops.append(("view", "expand", list(cur)))
            elif kind < 0.83:
                to = rng.choice([t for t in DTYPES if t != dtype])
                self.ops.append(("cast", to))
                dtype = to
                self.dtypes.add(to)
            elif not reduced:
                d = rng.randrange(len(cur))
                r = rng.choice(["sum", "amax", "mean", "var", "softmax", "layer_norm"])
                if r == "layer_norm":
                    d = len(cur) - 1
                # a normalisation over a few near-equal values turns one ulp
                # into a unit: keep those rows wide
                if (r == "layer_norm" and cur[d] < 16) or (r == "var" and cur[d] < 4):
                    r = "sum"
                # a row of an integer prefix's few values may be one value
                # repeated, which a LayerNorm maps to 0 plus its mean's rounding
                # times 1/sqrt(eps); and a LayerNorm's row sums to 0 exactly,
                # so a later sum or mean is all cancellation. Both measure
                # rounding noise, not the kernels
                if r == "layer_norm" and int_prefix:
                    r = "softmax"
                if r in ("sum", "mean", "var") and normalised:
                    r = "amax"
                normalised |= r == "layer_norm"
                keep = rng.random() < 0.5
                self.ops.append(("reduce", r, d, keep))
                if r not in ("softmax", "layer_norm"):
                    reduced = True
                    if keep:
                        cur[d] = 1
                    elif len(cur) > 1:
                        cur.pop(d)
                    else:
                        cur = [1]
                        self.ops[-1] = ("reduce", r, d, True)
        if not self.ops or self.ops[-1][0] == "view":
            self.ops.append(("unary", "affine", _UNARY[17][1]))

    def run(self, x, extras):
        t = x
        for op in self.ops:
            kind = op[0]
            if kind == "unary":
                t = op[2](t)
            elif kind == "binary":
                t = op[2](t, extras[op[3]])
            elif kind == "view":
                if op[1] == "permute":
                    t = t.permute(*op[2])
                elif op[1] == "transpose":
                    t = t.transpose(*op[2])
                elif op[1] == "slice":
                    d, start, step = op[2]
                    t = t[(slice(None),) * d + (slice(start, None, step),)]
                else:
                    t = t.expand(*op[2])
            elif kind == "cast":
                t = t.to(op[1])
            else:
                _, r, d, keep = op
                if r == "sum":
                    t = t.sum(dim=d, keepdim=keep)
                elif r == "amax":
                    t = t.amax(dim=d, keepdim=keep)
                elif r == "mean":
                    t = t.mean(dim=d, keepdim=keep)
                elif r == "var":
                    t = t.var(dim=d, keepdim=keep, unbiased=False)
                elif r == "softmax":
                    t = t.softmax(dim=d)
                else:
                    t = F.layer_norm(t, (t.shape[-1],))
        return t


class Program(torch.nn.Module):
    """``n`` independent chains; forward takes every chain's inputs in order
    and returns one output per chain."""

    def __init__(self, seed: int, n: int, wide: bool = False):
        super().__init__()
        rng = random.Random(seed)
        self.chains = [Chain(rng, wide) for _ in range(n)]

    def forward(self, *args):
        outs = []
        i = 0
        for c in self.chains:
            x = args[i]
            extras = args[i + 1:i + 1 + len(c.extra)]
            i += 1 + len(c.extra)
            outs.append(c.run(x, extras))
        return tuple(outs)


def tolerance(chain: Chain) -> float:
    """The bar for ``chain`` against the oracle: set by the narrowest dtype
    any of its values is stored in."""
    return max(TOLERANCE[d] for d in chain.dtypes)


def program(seed: int, n: int = 24, wide: bool = False):
    """(model, example inputs) for ``seed``: values N(0, 1) from a generator
    seeded with ``seed``. ``wide`` gives every chain one dim of 700..4099."""
    model = Program(seed, n, wide)
    g = torch.Generator().manual_seed(seed)
    args = []
    for c in model.chains:
        args.append(torch.randn(c.shape, generator=g).to(c.dtype))
        for shp, dt in c.extra:
            args.append(torch.randn(shp, generator=g).to(dt))
    return model, tuple(args)


def max_rel_error(got: torch.Tensor, want: torch.Tensor) -> float:
    g, w = got.double(), want.double()
    if w.numel() == 0:
        return 0.0
    both_nan = torch.isnan(g) & torch.isnan(w)
    if not torch.equal(torch.isnan(g), torch.isnan(w)):
        return float("inf")
    g, w = g[~both_nan], w[~both_nan]
    inf = torch.isinf(w)
    if not torch.equal(g[inf], w[inf]):
        return float("inf")
    g, w = g[~inf], w[~inf]
    if w.numel() == 0:
        return 0.0
    scale = max(w.abs().max().item(), 1e-3)
    return (g - w).abs().max().item() / scale


def attention_case(seed: int, dtype=torch.float16):
    """A random attention problem for the fused kernels: (model, inputs,
    description). Queries in multiples of 16; up to 128 keys in multiples of
    32 (single pass) or 192..640 in multiples of 64 (key-blocked); head sizes
    32..128; one of five masks: padding at -10000 or -inf, causal (-inf, every
    row keeps its diagonal), a per-head additive bias, or zeros. Scaled by a
    division or a multiplication. ``dtype`` is fp16 or bf16."""
    import math

    rng = random.Random(1000 + seed)
    b, h = rng.choice([1, 2, 3]), rng.choice([1, 2, 4, 12])
    t = 16 * rng.randint(1, 16)
    tk = 32 * rng.randint(1, 4) if rng.random() < 0.5 else 64 * rng.randint(3, 10)
    d = rng.choice([32, 64, 96, 128])
    kind = rng.choice(["padding", "padding_inf", "causal", "bias", "zeros"])
    by_div = rng.random() < 0.5
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, h, t, d, generator=g).to(dtype)
    k = torch.randn(b, h, tk, d, generator=g).to(dtype)
    v = torch.randn(b, h, tk, d, generator=g).to(dtype)
    if kind in ("padding", "padding_inf"):
        keep = torch.rand(b, 1, 1, tk, generator=g) >= 0.2
        keep[..., 0] = True
        fill = -10000.0 if kind == "padding" else float("-inf")
        mask = torch.where(keep, 0.0, fill).to(dtype)
    elif kind == "causal":
        mask = torch.triu(torch.full((t, tk), float("-inf")), diagonal=1 + max(0, tk - t))
        mask = mask.to(dtype)[None, None]
    elif kind == "bias":
        mask = torch.randn(1, h, t, tk, generator=g).to(dtype)
    else:
        mask = torch.zeros(b, 1, 1, tk).to(dtype)

    class Attn(torch.nn.Module):
        def forward(self, q, k, v, mask):
            s = q @ k.transpose(-2, -1)
            s = s / math.sqrt(d) if by_div else s * (1.0 / math.sqrt(d))
            return (s + mask).softmax(dim=-1) @ v

    desc = (f"b{b} h{h} T{t} Tk{tk} d{d} {kind} {'div' if by_div else 'mul'}"
            + ("" if dtype == torch.float16 else f" {str(dtype)[6:]}"))
    return Attn(), (q, k, v, mask), desc


def block_case(seed: int):
    """A random transformer stack for the schedule variants: (model, inputs,
    description). BERT-style (post-norm, separate q/k/v projections, padding
    mask), GPT-style (pre-norm, one qkv projection split three ways, causal
    mask buffer) or unmasked; model width 64..256, head sizes 16..64 (16 and
    48 are refused by the attention fusion), 1-2 layers, GELU (erf or tanh)
    or ReLU, projections with or without bias; fp16 (or, one in four, fp32)
    weights N(0, 0.05)."""
    import math

    import torch.nn as nn

    rng = random.Random(2000 + seed)
    dh = rng.choice([16, 32, 48, 64, 64, 64])
    h = rng.choice([1, 2, 4])
    d = dh * h
    if d > 256:
        h, d = 256 // dh, dh * (256 // dh)
    t = rng.choice([16, 32, 48, 64, 96, 128, 128, 192, 256, 320])
    b = rng.choice([1, 2, 3])
    dtype = torch.float16 if rng.random() < 0.75 else torch.float32
    style = rng.choice(["bert", "gpt", "plain"])
    act = rng.choice(["gelu", "gelu_tanh", "relu"])
    bias = rng.random() < 0.8
    layers = rng.choice([1, 2])
    ff = 4 * d

    def activation(x):
        if act == "relu":
            return torch.relu(x)
        return F.gelu(x, approximate="tanh" if act == "gelu_tanh" else "none")

    class Layer(nn.Module):
        def __init__(self):
            super().__init__()
            if style == "gpt":
                self.qkv = nn.Linear(d, 3 * d, bias=bias)
            else:
                self.q = nn.Linear(d, d, bias=bias)
                self.k = nn.Linear(d, d, bias=bias)
                self.v = nn.Linear(d, d, bias=bias)
            self.o = nn.Linear(d, d, bias=bias)
            self.ln1 = nn.LayerNorm(d)
            self.ln2 = nn.LayerNorm(d)
            self.fc1 = nn.Linear(d, ff, bias=bias)
            self.fc2 = nn.Linear(ff, d, bias=bias)

        def attn(self, x, mask):
            bb, tt, _ = x.shape
            if style == "gpt":
                q, k, v = self.qkv(x).chunk(3, dim=-1)
            else:
                q, k, v = self.q(x), self.k(x), self.v(x)
            q, k, v = (y.view(bb, tt, h, dh).transpose(1, 2) for y in (q, k, v))
            s = (q @ k.transpose(-2, -1)) / math.sqrt(dh)
            if mask is not None:
                s = s + mask
            ctx = (s.softmax(dim=-1) @ v).transpose(1, 2).reshape(bb, tt, d)
            return self.o(ctx)

        def forward(self, x, mask):
            if style == "gpt":
                x = x + self.attn(self.ln1(x), mask)
                return x + self.fc2(activation(self.fc1(self.ln2(x))))
            x = self.ln1(x + self.attn(x, mask))
            return self.ln2(x + self.fc2(activation(self.fc1(x))))

    class Stack(nn.Module):
        def __init__(self):
            super().__init__()
            self.layers = nn.ModuleList(Layer() for _ in range(layers))
            tril = torch.tril(torch.ones(t, t))
            self.register_buffer("causal", ((1.0 - tril) * torch.finfo(torch.float32).min)
                                 .view(1, 1, t, t), persistent=False)

        def forward(self, x, keep):
            if style == "gpt":
                mask = self.causal
            elif style == "bert":
                mask = (1.0 - keep[:, None, None, :]) * torch.finfo(torch.float32).min
            else:
                mask = None
            for layer in self.layers:
                x = layer(x, mask)
            return x

    g = torch.Generator().manual_seed(seed)
    model = Stack()
    with torch.no_grad():
        for p_ in model.parameters():
            if p_.dim() > 1:
                p_.copy_(torch.randn(p_.shape, generator=g) * 0.05)
            elif p_ is not None:
                p_.copy_(torch.randn(p_.shape, generator=g) * 0.02)
    model = model.to(dtype)
    x = torch.randn(b, t, d, generator=g).to(dtype)
    keep = (torch.rand(b, t, generator=g) >= 0.15).to(dtype)
    keep[:, 0] = 1
    desc = (f"{style} b{b} T{t} d{d} h{h} {act} bias={bias} layers={layers} "
            f"{str(dtype).replace('torch.', '')}")
    return model, (x, keep), desc


def extern_case(seed: int):
    """Random chains through the extern ops (``mm``, ``bmm``, ``addmm``,
    ``matmul``, ``linear``) on transposed, sliced and expanded operands, with
    pointwise and reduction kernels around them: (model, inputs,
    description). Sizes 8..96; fp32 or fp16."""
    rng = random.Random(3000 + seed)
    dtype = rng.choice([torch.float32, torch.float16])
    m, k, n = (rng.choice([8, 16, 24, 33, 64, 96]) for _ in range(3))
    bt = rng.choice([1, 2, 3])
    kind = rng.choice(["mm_t", "mm_slice", "bmm_t", "addmm", "matmul_bcast", "linear"])
    g = torch.Generator().manual_seed(seed)

    def rn(*s):
        return (torch.randn(*s, generator=g) * 0.3).to(dtype)

    if kind == "mm_t":          # B given as [n, k], read transposed
        args = (rn(m, k), rn(n, k))
        fn = lambda a, b: torch.tanh(a * 1.5) @ b.t()
    elif kind == "mm_slice":    # every other column of A, a row slice of B
        args = (rn(m, 2 * k), rn(k + 3, n))
        fn = lambda a, b: torch.relu(a[:, ::2] @ b[1:k + 1]) + 0.5
    elif kind == "bmm_t":
        args = (rn(bt, m, k), rn(bt, n, k))
        fn = lambda a, b: (a @ b.transpose(1, 2)).softmax(dim=-1)
    elif kind == "addmm":
        args = (rn(m, k), rn(k, n), rn(n))
        fn = lambda a, b, c: torch.addmm(c, a, b) * 2.0
    elif kind == "matmul_bcast":  # a batch of A against one B
        args = (rn(bt, m, k), rn(k, n))
        fn = lambda a, b: F.layer_norm(torch.matmul(a, b), (n,)) if n > 1 else torch.matmul(a, b)
    else:
        args = (rn(bt, m, k), rn(n, k), rn(n))
        fn = lambda a, w, c: F.gelu(F.linear(a, w, c)).sum(dim=-1)

    class Ext(torch.nn.Module):
        def forward(self, *xs):
            return fn(*xs)

    return Ext(), args, f"{kind} m{m} k{k} n{n} b{bt} {str(dtype).replace('torch.', '')}"
