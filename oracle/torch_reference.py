"""CPU oracle: executes the kernel IR with torch ops in fp32.

TEST INFRASTRUCTURE ONLY. Nothing in the product (``mlc-compiler_amd/``)
imports this module; only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` do, as the checker / CPU baseline.

This restates the reference's torch backend
(``mlc/codegen/torch_backend.py:20-275``):

* narrow floats (fp16/bf16) are promoted to fp32 on load, all arithmetic is
  fp32, results are cast to the buffer dtype on store
  (``torch_backend.py:53-62``, ``:111-118``);
* every operand is gathered by ``eval``-ing the *rendered* index string
  against ``arange`` tensors, so index rendering is under test
  (``torch_backend.py:86-97``, ``:140-149``);
* reductions run row-vectorised: the persistent form walks the steps in order
  over the whole row (``:170-181``); the streamed form follows the pass
  partition chunk by chunk, including the online-softmax recurrence
  (``:182-233``).

Pinning (what fixes this oracle independently of itself):
* end-to-end equality with eager PyTorch on every toy model under every pass
  configuration at the reference's tolerances (rtol 1e-5 / atol 1e-6 fp32),
  and the reference's own torch-backend outputs for the same inputs
  (fixtures it wrote), ``tests/test_oracle.py``; for BASELINE configs 1-4
  (the fp32 FFN block, BERT-base fp16 b1 and b32, GPT-2 small fp16 b1) those
  outputs are reproduced bit for bit;
* seeded random programs (pointwise chains, views, casts, reductions, extern
  GEMMs, transformer stacks) against eager PyTorch, ``tests/test_fuzz.py``;
* the reference's index-rendering known answers (``tests/test_codegen.py``);
* numerical special cases from the reference's tests: two-pass variance
  against float64, large-mean layer norm, softmax on logits x100, and planted
  mistakes (a sign, exp2 for exp, a reduce identity) that must be caught
  (``tests/test_oracle.py``);
* streamed evaluation agrees with persistent evaluation.
Two deliberate differences from the reference's torch backend: a
reduction's row output is evaluated at one column, as the reference's Triton
kernels compute it (``run_reduction``; the torch backend fails on a row
output that reads a row-constant operand), and the streamed online-softmax
recurrence subtracts 0 instead of a running maximum that is still -inf (the
torch backend returns NaN for a row whose first chunk is all -inf, where
eager softmax is finite; pinned against eager in ``tests/test_oracle.py``).
Transcendentals (exp/erf/tanh/...) are torch's CPU implementations:
per-function parity against the reference's device libm is "parity
unpinned"; only the end-to-end tolerances pin them, as in the reference.
"""

from __future__ import annotations

import torch

from mlc.ir.scalar import Call, Cast, Const, Expr, Load, Ref
from mlc.kernels import AttentionKernel, Bind, ExternKernel, PointwiseKernel, Reduce, ReductionKernel

TORCH_FN = {
    "neg": torch.neg, "abs": torch.abs, "reciprocal": torch.reciprocal,
    "exp": torch.exp, "log": torch.log, "sqrt": torch.sqrt, "rsqrt": torch.rsqrt,
    "sin": torch.sin, "cos": torch.cos, "tanh": torch.tanh, "erf": torch.erf,
    "sigmoid": torch.sigmoid, "floor": torch.floor, "logical_not": torch.logical_not,
    "add": torch.add, "sub": torch.sub, "mul": torch.mul, "div": torch.div,
    "pow": torch.pow, "maximum": torch.maximum, "minimum": torch.minimum,
    "gt": torch.gt, "lt": torch.lt, "ge": torch.ge, "le": torch.le, "eq": torch.eq,
    "ne": torch.ne, "logical_and": torch.logical_and, "logical_or": torch.logical_or,
    "where": torch.where,
}

COMPUTE_DTYPE = torch.float32

_REDUCE = {
    "sum": lambda v: v.sum(dim=1, keepdim=True),
    "max": lambda v: v.amax(dim=1, keepdim=True),
    "min": lambda v: v.amin(dim=1, keepdim=True),
    "prod": lambda v: v.prod(dim=1, keepdim=True),
}

_COMBINE = {
    "sum": torch.add,
    "max": torch.maximum,
    "min": torch.minimum,
    "prod": torch.mul,
}


def _promote(t: torch.Tensor) -> torch.Tensor:
    return t.to(COMPUTE_DTYPE) if t.dtype in (torch.float16, torch.bfloat16) else t


def _offsets(src: str, env: dict, like: torch.Tensor) -> torch.Tensor:
    """Evaluate a rendered index expression over the iteration tensors."""
    out = eval(src, {"__builtins__": {}}, env)  # noqa: S307 - rendered by our own codegen
    if not torch.is_tensor(out):
        out = torch.zeros_like(like) + int(out)
    return out


def eval_expr(e: Expr, loads: list, refs: dict, like: torch.Tensor) -> torch.Tensor:
    if isinstance(e, Load):
        return loads[e.slot]
    if isinstance(e, Ref):
        return refs[e.name]
    if isinstance(e, Const):
        if isinstance(e.value, bool):
            return torch.full_like(like, float(e.value), dtype=torch.bool)
        return torch.as_tensor(e.value, dtype=e.dtype, device=like.device)
    if isinstance(e, Cast):
        return eval_expr(e.x, loads, refs, like).to(e.dtype)
    if isinstance(e, Call):
        fn = TORCH_FN.get(e.fn)
        if fn is None:
            raise KeyError(f"no torch equivalent for scalar function {e.fn!r}")
        return fn(*(eval_expr(a, loads, refs, like) for a in e.args))
    raise TypeError(f"cannot evaluate {type(e).__name__}")


def run_pointwise(k: PointwiseKernel, buffers: dict[str, torch.Tensor]) -> None:
    device = next(iter(buffers.values())).device if buffers else torch.device("cpu")
    idx = torch.arange(k.numel, device=device, dtype=torch.int64)
    env = {"idx": idx}
    loads = []
    for a in k.inputs:
        buf = buffers[a.value.buffer.name]
        src = a.index.render()
        if src == "idx" and buf.numel() == k.numel:
            loads.append(_promote(buf))
        else:
            loads.append(_promote(buf[_offsets(src, env, idx)]))
    like = loads[0] if loads else idx
    refs: dict[str, torch.Tensor] = {}
    for name, expr in k.body:
        refs[name] = eval_expr(expr, loads, refs, like)
    for a in k.outputs:
        val = eval_expr(k.out_expr[a.value.name], loads, refs, like)
        dest = buffers[a.value.buffer.name]
        where = _offsets(a.index.render(), env, idx)
        if not torch.is_tensor(val) or val.numel() == 1:
            val = torch.as_tensor(val, device=device).expand(k.numel)
        dest[where] = val.reshape(-1).to(dest.dtype)


def run_reduction(k: ReductionKernel, buffers: dict[str, torch.Tensor], chunk: int = 1024,
                  streamed: bool | None = None) -> None:
    """Row-vectorised evaluation. ``streamed`` defaults to the kernel's own
    mode; forcing ``False`` evaluates a streamed kernel persistently."""
    device = next(iter(buffers.values())).device if buffers else torch.device("cpu")
    n_rows, n_cols = k.n_rows, k.reduce_numel
    row = torch.arange(n_rows, device=device, dtype=torch.int64).unsqueeze(1)
    col0 = torch.zeros((1, 1), device=device, dtype=torch.int64)

    def gather(arg, col):
        buf = buffers[arg.value.buffer.name]
        off = _offsets(arg.index.render(), {"row": row, "col": col}, row)
        return _promote(buf[off.expand(n_rows, col.shape[1])])

    def load_all(col):
        return [gather(a, col) for a in k.inputs]

    def widen(expr, loads, refs, width):
        v = eval_expr(expr, loads, refs, loads[0] if loads else row)
        if not torch.is_tensor(v):
            v = torch.as_tensor(v, device=device)
        if v.dim() < 2 or v.shape[1] == 1:
            return v.expand(n_rows, width)
        return v

    def store(name, refs, loads, col):
        arg = next(a for a in k.outputs if a.value.name == name)
        val = eval_expr(k.out_expr[name], loads, refs, loads[0] if loads else row)
        dest = buffers[arg.value.buffer.name]
        off = _offsets(arg.index.render(), {"row": row, "col": col}, row)
        shape = (n_rows, col.shape[1])
        if not torch.is_tensor(val):
            val = torch.as_tensor(val, device=dest.device)
        dest[off.expand(shape).reshape(-1)] = val.expand(shape).reshape(-1).to(dest.dtype)

    element_stores = [a.value.name for a in k.outputs if a.value.name not in k.row_outputs]
    refs: dict[str, torch.Tensor] = {}
    use_streamed = k.two_pass if streamed is None else streamed

    if not use_streamed:
        col = torch.arange(n_cols, device=device, dtype=torch.int64).unsqueeze(0)
        loads = load_all(col)
        for step in k.steps:
            if isinstance(step, Reduce):
                refs[step.name] = _REDUCE[step.kind](widen(step.expr, loads, refs, n_cols))
            else:
                refs[step.name] = eval_expr(step.expr, loads, refs, loads[0] if loads else row)
        for name in element_stores:
            store(name, refs, loads, col)
        row_loads = loads
    else:
        from mlc.codegen.reduction_schedule import plan_passes, scalar_binds

        passes = plan_passes(_as_two_pass(k))
        owner = {r.name: p for p in passes for r in p.reduces}
        scalars = {b.name for b in scalar_binds(k)}
        row_loads = load_all(col0)
        width = max(1, min(n_cols, chunk))

        def run_pass(p):
            online = p.online_softmax
            accs: dict[str, torch.Tensor] = {}
            m = torch.full((n_rows, 1), -float("inf"), device=device)
            lsum = torch.zeros((n_rows, 1), device=device)
            for c0 in range(0, n_cols, width):
                c1 = min(c0 + width, n_cols)
                col = torch.arange(c0, c1, device=device, dtype=torch.int64).unsqueeze(0)
                loads = load_all(col)
                local = dict(refs)
                for b in p.binds:
                    local[b.name] = eval_expr(b.expr, loads, local, loads[0] if loads else row)
                if online is not None:
                    x = widen(online.value, loads, local, c1 - c0)
                    m_new = torch.maximum(m, x.amax(dim=1, keepdim=True))
                    # a row whose elements so far are all -inf has m_new = -inf;
                    # subtracting 0 there keeps exp(-inf - -inf) from being NaN
                    # (the reference's torch backend subtracts m_new as is,
                    # torch_backend.py:211-213, and returns NaN for such a
                    # row where eager softmax is finite)
                    inf = m_new == -float("inf")
                    alpha = torch.where(m == -float("inf"), 0.0, torch.exp(m - m_new))
                    m_sub = torch.where(inf, 0.0, m_new)
                    lsum = lsum * alpha + torch.exp(x - m_sub).sum(dim=1, keepdim=True)
                    m = m_new
                else:
                    for r in p.reduces:
                        part = _REDUCE[r.kind](widen(r.expr, loads, local, c1 - c0))
                        accs[r.name] = part if r.name not in accs else _COMBINE[r.kind](accs[r.name], part)
                for name in p.stores:
                    store(name, local, loads, col)
            if online is not None:
                refs[online.max_step.name] = m
                refs[online.sum_step.name] = lsum
            refs.update(accs)

        for step in k.steps:
            if isinstance(step, Reduce):
                if step.name not in refs:
                    run_pass(owner[step.name])
            elif step.name in scalars:
                refs[step.name] = eval_expr(step.expr, row_loads, refs,
                                            row_loads[0] if row_loads else row)
        for p in passes:
            if p.stores and not p.reduces:
                run_pass(p)

    for a in k.outputs:
        if a.value.name not in k.row_outputs:
            continue
        val = eval_expr(k.out_expr[a.value.name], row_loads, refs,
                        row_loads[0] if row_loads else row)
        if torch.is_tensor(val) and val.dim() == 2 and val.shape[1] > 1:
            # A row output does not vary along the row, so every column holds
            # its value; keep one. The reference's Triton kernels compute it
            # once per row from scalar loads (triton_reduction.py:94-111,
            # 268-270); its torch backend stores the full-row value here
            # (torch_backend.py:182,239-247) and fails with a shape error
            # when the row output reads a row-constant operand or a bind
            # evaluated over the row (``x.sum(0, keepdim=True) + y``).
            val = val[:, :1]
        dest = buffers[a.value.buffer.name]
        off = _offsets(a.index.render(), {"row": row, "col": col0}, row)
        if not torch.is_tensor(val):
            val = torch.as_tensor(val, device=device).expand(n_rows, 1)
        dest[off.reshape(-1)] = val.reshape(-1).to(dest.dtype)


def _as_two_pass(k: ReductionKernel) -> ReductionKernel:
    if k.two_pass:
        return k
    import copy

    twin = copy.copy(k)
    twin.two_pass = True
    return twin


def run_attention(k: AttentionKernel, buffers: dict[str, torch.Tensor]) -> None:
    """The three kernels the fused one replaces, in order: ``bmm`` (fp32
    products, rounded to the score dtype as the stored scores are), the
    reduction kernel over a private score buffer, and ``bmm`` with the
    values (reference: ``mlc/codegen/torch_backend.py:170-181`` for the
    reduction; the GEMMs are the extern ``aten.bmm`` calls they replace).
    The result is stored through the output's index map over its flat
    ``[BH, T, D]`` index, which also covers a folded permuting copy."""
    q, kt, v = (_promote(x.layout.as_torch(buffers[x.buffer.name])) for x in (k.q, k.kt, k.v))
    scores = torch.bmm(q, kt).to(k.score_dtype)
    sm = k.softmax
    score_buf = sm.inputs[k.score_slot].value.buffer
    prob = sm.outputs[0].value
    private = dict(buffers)
    private[score_buf.name] = scores.reshape(-1)
    private[prob.buffer.name] = torch.empty(prob.buffer.numel, dtype=prob.buffer.dtype,
                                            device=scores.device)
    run_reduction(sm, private, streamed=False)
    p = _promote(private[prob.buffer.name].view(scores.shape))
    o = torch.bmm(p, v).reshape(-1)
    arg = k.outputs[0]
    dest = buffers[arg.value.buffer.name]
    idx = torch.arange(o.numel(), device=o.device, dtype=torch.int64)
    dest[_offsets(arg.index.render(), {"idx": idx}, idx)] = o.to(dest.dtype)


def run_kernel(k, buffers: dict[str, torch.Tensor]) -> None:
    if isinstance(k, PointwiseKernel):
        run_pointwise(k, buffers)
    elif isinstance(k, ReductionKernel):
        run_reduction(k, buffers)
    elif isinstance(k, AttentionKernel):
        run_attention(k, buffers)
    else:
        raise TypeError(f"the oracle does not execute {type(k).__name__}")


class TorchReferenceRunner:
    """Kernel runner plugged into ``mlc.runtime.executor.CompiledModel`` by
    tests, so the product's executor logic (buffer table, arena binding,
    extern dispatch, output aliasing) runs on the CPU with this oracle
    executing the generated kernels."""

    name = "torch"
    source = "# torch reference oracle: no generated source"

    def bind(self, k, buffers):
        return (k, buffers)

    def run_bound(self, payload) -> None:
        run_kernel(*payload)

    def launch(self, k, buffers) -> None:
        run_kernel(k, buffers)
