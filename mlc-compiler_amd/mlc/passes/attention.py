"""Attention fusion: an opt-in schedule change (``Config.fused_attention``).

The reference schedule computes attention as three kernels: ``bmm`` for the
scores, a persistent row reduction (scale, mask, softmax), and ``bmm`` with
the values -- two launches more than needed and a round trip of the
``[BH, T, T]`` score and probability tensors through HBM. This pass replaces
that triple with one :class:`~mlc.kernels.AttentionKernel` that the HIP
backend emits as a single MFMA kernel per batch-head. The reduction's own
steps (whatever scale, mask and normalisation it holds) are kept and
rendered inside it.

Applies when the scores feed only the reduction, the reduction reads them at
identity over a ``[BH*T] x [Tk]`` frame and writes only the probabilities,
those feed only the second ``bmm`` as its first operand, scores,
probabilities and output are contiguous, T is a multiple of 16, the head size
a multiple of 32 up to 128, and the operands fp16 or bf16 (the 16-bit MFMAs
the kernel is built on). Up to 128 keys (a multiple of 32) every score of a row stays in
registers and the reduction's own steps are rendered, whatever they are.
Longer rows (a multiple of 64 keys) are streamed in key blocks with the
online-softmax recurrence, which needs the reduction to be exactly a softmax
(``exp(x - max) / sum``) of a per-element value ``x``.

When K or V is written by one of this compiler's pointwise kernels for the
attention alone, that kernel is re-derived to write K as ``[bh][key][d]``
and V as ``[bh][d][key]`` (the layouts the MFMA operands are read in), the
same index-map composition layout selection uses. A copy that only permutes
the fused kernel's output (BERT's context re-layout) is folded into the
kernel's stores.
"""

from __future__ import annotations

import math
from dataclasses import replace

import torch

from ..codegen.hip_attention import KEY_BLOCK, blocked_form
from ..codegen.index import flat_index
from ..ir.graph import Value
from ..ir.types import Layout
from ..kernels import (AttentionKernel, ExternKernel, KernelArg, PointwiseKernel,
                       ReductionKernel, Schedule)
from .layout import is_pure_copy, compose

#: keys held in registers by the single-pass kernel; longer rows are key-blocked
MAX_SEQ = 128
#: the key-blocked kernel's limit (keys are streamed; this bounds the row index math)
MAX_KEYS = 1 << 16
MAX_HEAD = 128


def _bmm(k) -> bool:
    return isinstance(k, ExternKernel) and k.node.op == "aten.bmm.default" and len(k.node.args) == 2


def fuse_attention(schedule: Schedule) -> int:
    """Replace every matching bmm -> reduction -> bmm triple; returns the
    number fused. The fused kernel takes the second ``bmm``'s place, where
    all of its inputs are ready (other kernels, such as a copy producing the
    values, may sit between the three)."""
    kernels = schedule.kernels
    graph_outputs = {v.buffer.name for v in schedule.graph.outputs}
    readers: dict[str, list[int]] = {}
    for i, k in enumerate(kernels):
        for name in {v.buffer.name for v in k.reads()}:
            readers.setdefault(name, []).append(i)
    replace: dict[int, AttentionKernel] = {}
    removed: set[int] = set()
    for i, k in enumerate(kernels):
        if i in removed or not _bmm(k):
            continue
        found = _match(kernels, i, readers, graph_outputs)
        if found is not None:
            j, m, att = found
            replace[m] = att
            removed.update((i, j))
    new = [replace.get(i, k) for i, k in enumerate(kernels) if i not in removed]
    new = _relayout_operands(new, graph_outputs)
    schedule.kernels = _fold_output_copies(new, graph_outputs)
    return len(replace)


def _output_copy(kernels, at: int, graph_outputs):
    """(copy index, output arg) when the fused kernel's output is read only by
    a copy that permutes it (BERT's context ``[BH, T, D] -> [B, T, H, D]``):
    the output arg writes the copy's buffer directly, indexed by the fused
    kernel's own flat output index. None when the permutation would break the
    kernel's 8-byte stores of four consecutive head-dim values."""
    k = kernels[at]
    buf = k.out.buffer
    readers = [i for i, x in enumerate(kernels) if any(v.buffer is buf for v in x.reads())]
    if buf.name in graph_outputs or len(readers) != 1:
        return None
    j = readers[0]
    c = kernels[j]
    if not is_pure_copy(c) or c.inputs[0].value.buffer is not buf:
        return None
    view = c.inputs[0].value.layout
    if view.offset != 0 or math.prod(view.shape) != buf.numel or c.numel != buf.numel:
        return None
    dest = Layout.contiguous(view.shape).strides
    dims = sorted(((st, n, o) for st, n, o in zip(view.strides, view.shape, dest) if n != 1),
                  key=lambda t: -t[0])
    expect = 1
    for st, n, _ in reversed(dims):  # a permutation of the contiguous output
        if st != expect:
            return None
        expect *= n
    shape = tuple(n for _, n, _ in dims)
    imap = flat_index(shape, Layout(shape, tuple(o for _, _, o in dims), 0))
    terms = imap.axes[0].terms if imap.axes else ()
    inner = [t for t in terms if t[1] == 1]
    if (imap.base % 4 or len(inner) != 1 or inner[0][2] != 1 or inner[0][0] % 4
            or any(t[2] % 4 for t in terms if t is not inner[0])):
        return None
    return j, KernelArg(c.outputs[0].value, imap)


def _fold_output_copies(kernels, graph_outputs):
    out = list(kernels)
    removed: set[int] = set()
    for at, k in enumerate(out):
        if not isinstance(k, AttentionKernel):
            continue
        found = _output_copy(out, at, graph_outputs)
        if found is None:
            continue
        j, arg = found
        out[at] = replace(k, out=arg.value, outputs=[arg], nodes=list(k.nodes) + list(out[j].nodes))
        removed.add(j)
    return [k for i, k in enumerate(out) if i not in removed]


def _operand_producer(kernels, at: int, value, graph_outputs):
    """Index of the pointwise kernel that writes ``value``'s whole buffer at
    identity and whose output only kernel ``at`` reads, else None."""
    buf = value.buffer
    if buf.name in graph_outputs or not (value.layout.is_contiguous() and value.layout.offset == 0):
        return None
    writers = [i for i, k in enumerate(kernels) if any(v.buffer is buf for v in k.writes())]
    readers = [i for i, k in enumerate(kernels) if any(v.buffer is buf for v in k.reads())]
    if len(writers) != 1 or readers != [at]:
        return None
    p = kernels[writers[0]]
    if (not isinstance(p, PointwiseKernel) or len(p.outputs) != 1 or p.numel != buf.numel
            or not p.outputs[0].index.is_identity()):
        return None
    return writers[0]


def _swap_walks(space, BH: int, minor):
    """Iteration shapes for the re-derived producer, minor dims swapped: the
    producer's own batch dims first (a head split into batch x heads stays
    affine there), then the operand's flat ``[BH, ...]`` view."""
    a, b = minor
    out = []
    if tuple(space[-2:]) == (a, b) and math.prod(space[:-2]) == BH:
        out.append(tuple(space[:-2]) + (b, a))
    out.append((BH, b, a))
    return out


def _relayout_operands(kernels, graph_outputs):
    """Let each fused kernel choose how K and V sit in HBM when its own
    pointwise producer writes them: K as ``[bh][key][d]`` and V as
    ``[bh][d][key]``, the layouts its MFMA operands are read in, so staging
    needs no transposing LDS stores. The producer is re-derived to iterate in
    the new order (inputs read through composed index maps, verified
    exactly); an operand whose composition is not affine keeps its layout."""
    out = list(kernels)
    for at, k in enumerate(out):
        if not isinstance(k, AttentionKernel):
            continue
        BH, D, Tk = k.kt.shape
        # (operand, its old minor dims, new view of the operand)
        wanted = (("kt", (D, Tk), (BH, D, Tk), (Tk * D, 1, D)),
                  ("v", (Tk, D), (BH, Tk, D), (Tk * D, 1, Tk)))
        for field, minor, shape, strides in wanted:
            val = getattr(k, field)
            if val.layout.strides == strides:
                continue
            i = _operand_producer(out, at, val, graph_outputs)
            if i is None:
                continue
            p = out[i]
            fused = None
            for space in _swap_walks(p.space, BH, minor):
                # new index (batch..., minor[1], minor[0]) -> old flat index
                old = Layout.contiguous(space[:-2] + (space[-1], space[-2]))
                walk = Layout(space, old.strides[:-2] + (old.strides[-1], old.strides[-2]), 0)
                inputs = []
                for a in p.inputs:
                    lay = compose(walk, a.index)
                    if lay is None:
                        break
                    inputs.append(KernelArg(a.value, flat_index(space, lay)))
                else:
                    o = p.outputs[0]
                    fused = PointwiseKernel(
                        name=p.name, space=space, inputs=inputs,
                        outputs=[KernelArg(o.value, flat_index(space, Layout.contiguous(space)))],
                        body=list(p.body), out_expr=dict(p.out_expr), nodes=list(p.nodes))
                    break
            if fused is None:
                continue
            out[i] = fused
            moved = Value(val.name, val.buffer, Layout(shape, strides, 0))
            k = replace(k, **{field: moved, "inputs": list(k.inputs)})
            k.inputs[1 if field == "kt" else 2] = KernelArg(moved, flat_index(shape, moved.layout))
            out[at] = k
    return out


def _only_reader(readers, value, graph_outputs) -> int | None:
    r = readers.get(value.buffer.name, [])
    if len(r) != 1 or value.buffer.name in graph_outputs:
        return None
    return r[0]


def _match(kernels, i, readers, graph_outputs):
    b1 = kernels[i]
    q, kt = b1.node.args
    s_val = b1.outputs[0]
    j = _only_reader(readers, s_val, graph_outputs)
    if j is None or j <= i:
        return None
    sm = kernels[j]
    if not isinstance(sm, ReductionKernel) or sm.two_pass or sm.row_outputs or len(sm.outputs) != 1:
        return None
    prob = sm.outputs[0].value
    m = _only_reader(readers, prob, graph_outputs)
    if m is None or m <= j or not _bmm(kernels[m]):
        return None
    b2 = kernels[m]
    p_val, v = b2.node.args
    o_val = b2.outputs[0]
    if p_val.buffer is not prob.buffer or len(q.shape) != 3 or len(kt.shape) != 3 or len(v.shape) != 3:
        return None
    BH, T, D = q.shape
    Tk = kt.shape[2]
    if kt.shape != (BH, D, Tk) or v.shape != (BH, Tk, D) or s_val.shape != (BH, T, Tk):
        return None
    if not (T % 16 == 0 and D % 32 == 0 and D <= MAX_HEAD):
        return None
    if Tk > MAX_SEQ:
        # the key-blocked kernel: whole key blocks, and a softmax it can
        # evaluate with the online recurrence
        if Tk % KEY_BLOCK or Tk > MAX_KEYS or blocked_form(kernels[j]) is None:
            return None
    elif Tk % 32:
        return None
    dt = q.dtype
    if dt not in (torch.float16, torch.bfloat16) or \
            any(x.dtype != dt for x in (kt, v, o_val, s_val, prob)):
        return None
    for x in (s_val, p_val, o_val):
        if not (x.layout.is_contiguous() and x.layout.offset == 0):
            return None
    # the reduction reads the scores once, at identity over its [BH*T, Tk] frame
    if sm.n_rows != BH * T or sm.reduce_numel != Tk:
        return None
    slots = [n for n, a in enumerate(sm.inputs) if a.value.buffer is s_val.buffer]
    ident = f"(row * {Tk} + col)"
    if len(slots) != 1 or sm.inputs[slots[0]].index.render() != ident:
        return None
    if sm.outputs[0].index.render() != ident:
        return None
    others = [a for n, a in enumerate(sm.inputs) if n != slots[0]]
    args = [KernelArg(x, flat_index(x.shape, x.layout)) for x in (q, kt, v)] + others
    att = AttentionKernel(
        name=b2.name, q=q, kt=kt, v=v, out=o_val, softmax=sm, score_slot=slots[0],
        score_dtype=s_val.dtype, prob_dtype=prob.dtype, inputs=args,
        outputs=[KernelArg(o_val, flat_index(o_val.shape, o_val.layout))],
        nodes=[b1.node] + list(sm.nodes) + [b2.node])
    return j, m, att
