"""GEMM bias epilogues: an opt-in schedule change (``Config.gemm_epilogue``).

Capture splits ``addmm`` into ``mm`` + ``add`` so the bias add can fuse with
the pointwise work after it (``mlc/ir/capture.py:294-319`` of the reference).
When nothing fuses with it -- BERT's q/k/v projections, where the add ends up
as a kernel of its own -- that split costs a launch and a round trip of the
GEMM output through HBM. This pass puts such an add back into the library
call: ``mm`` followed by a lone ``out = mm_out + bias`` kernel becomes one
``addmm(bias, a, b)`` extern (hipBLASLt applies the bias in its epilogue).

It runs after lowering and before planning, so the arena is planned for the
new schedule. Rounding differs from the split form (the GEMM result is not
rounded to the storage type before the bias is added), so the kernel
schedule and the numbers are those of this configuration, not the
reference's; the parity configuration leaves it off.
"""

from __future__ import annotations

import torch

from ..ir.graph import Node
from ..ir.scalar import Call, Load, Ref
from ..kernels import ExternKernel, PointwiseKernel, Schedule


def _lone_bias_add(k: PointwiseKernel):
    """(mm operand slot, bias slot) when ``k`` is exactly ``out = x + bias``
    over a contiguous [M, N] space with ``bias`` a length-N vector."""
    if len(k.nodes) != 1 or k.nodes[0].op != "aten.add.Tensor":
        return None
    if len(k.inputs) != 2 or len(k.outputs) != 1 or len(k.space) != 2 or len(k.body) > 1:
        return None
    M, N = k.space
    out = k.outputs[0]
    expr = k.out_expr.get(out.value.name)
    if k.body:
        name, value = k.body[0]
        if not (isinstance(expr, Ref) and expr.name == name):
            return None
        expr = value
    if not (isinstance(expr, Call) and expr.fn == "add" and len(expr.args) == 2
            and all(isinstance(a, Load) for a in expr.args)):
        return None
    if out.index.render() != "idx" or tuple(out.value.shape) != (M, N):
        return None
    for x, b in ((0, 1), (1, 0)):
        xa, ba = k.inputs[x], k.inputs[b]
        if xa.index.render() != "idx" or tuple(xa.value.shape) != (M, N):
            continue
        terms = ba.index.axis("idx").terms if ba.index.axis("idx") else ()
        if tuple(ba.value.shape) == (N,) and terms == ((N, 1, 1),) and ba.index.base == 0:
            if {a.slot for a in expr.args} == {x, b}:
                return x, b
    return None


def fold_bias_epilogues(schedule: Schedule) -> int:
    """Rewrite ``mm`` + lone bias-add pairs into ``addmm``; returns how many."""
    kernels = schedule.kernels
    graph = schedule.graph
    outputs = {v.buffer.name for v in graph.outputs}
    readers: dict[str, int] = {}
    for k in kernels:
        for v in {v.buffer.name for v in k.reads()}:
            readers[v] = readers.get(v, 0) + 1
    producer = {}
    for i, k in enumerate(kernels):
        if isinstance(k, ExternKernel) and k.node.op == "aten.mm.default":
            producer[k.outputs[0].buffer.name] = i
    removed: set[int] = set()
    folded = 0
    for i, k in enumerate(kernels):
        if not isinstance(k, PointwiseKernel):
            continue
        slots = _lone_bias_add(k)
        if slots is None:
            continue
        x, b = k.inputs[slots[0]].value, k.inputs[slots[1]].value
        j = producer.get(x.buffer.name)
        if j is None or readers.get(x.buffer.name) != 1 or x.buffer.name in outputs:
            continue
        mm = kernels[j]
        if mm.outputs[0].buffer is not x.buffer or x.dtype != b.dtype:
            continue
        a, w = mm.node.args[0], mm.node.args[1]
        out = k.outputs[0].value
        node = Node("aten.addmm.default", (b, a, w), {}, outputs=[out])
        node.meta["target"] = torch.ops.aten.addmm.default
        kernels[j] = ExternKernel(mm.name, node, node.unique_tensor_args(), [out])
        removed.add(i)
        folded += 1
    schedule.kernels = [k for i, k in enumerate(kernels) if i not in removed]
    return folded
