"""Parallel-GEMM merging: an opt-in graph rewrite (``Config.merge_parallel_gemms``).

BERT computes q, k and v with three ``addmm`` calls on the same activation.
At batch 1 each of those GEMMs is a few microseconds of launch-bound work, and
each bias add is another launch. This pass concatenates the weights (and
biases) of linear layers that read the same activation into one parameter,
so the graph does one ``mm`` and one bias ``add`` over ``[M, sum(O)]``, and
turns each original output into a column slice of the merged result -- the
layout GPT-2's checkpoints use for ``c_attn`` natively, which the rest of the
compiler already handles (slices, head-major copies, ``bmm`` on strided
views).

It runs on the captured graph, before fusion, so every later pass sees an
ordinary graph. Views downstream of a rewritten output are re-derived from
their sources with the same view rules capture uses; a group whose views
would no longer be expressible as a restride is left alone.
"""

from __future__ import annotations

import torch

from ..ir.graph import Graph, Node, Value
from ..ir.shapes import infer_view
from ..ir.types import Buffer, Layout


def _linear_candidates(graph: Graph):
    """(mm node, weight param, add node, bias param) for every split
    ``addmm`` whose weight is a transposed 2-D param and whose product feeds
    exactly one bias add of a 1-D param."""
    params = {id(v) for v in graph.params}
    uses = graph.use_map()
    producers = {id(o): n for n in graph.nodes for o in n.outputs}
    outputs = {id(v) for v in graph.outputs}
    found = []
    for n in graph.nodes:
        if n.op != "aten.mm.default" or len(n.args) != 2:
            continue
        a, wt = n.args
        pn = producers.get(id(wt))
        if (pn is None or pn.op != "aten.permute.default" or list(pn.args[1]) != [1, 0]
                or id(pn.args[0]) not in params or len(pn.args[0].shape) != 2):
            continue
        w = pn.args[0]
        mm_out = n.outputs[0]
        readers = uses.get(id(mm_out), [])
        if len(readers) != 1 or readers[0].op != "aten.add.Tensor" or id(mm_out) in outputs:
            continue
        add = readers[0]
        if len(add.args) != 2 or add.args[0] is not mm_out:
            continue
        bias = add.args[1]
        if (not isinstance(bias, Value) or id(bias) not in params or bias.shape != (w.shape[0],)
                or id(add.outputs[0]) in outputs):
            continue
        found.append((n, w, add, bias))
    return found


def merge_parallel_gemms(graph: Graph) -> int:
    """Merge linear layers that share their input; returns the number of
    GEMMs removed."""
    groups: dict[tuple, list] = {}
    for cand in _linear_candidates(graph):
        mm, w, add, bias = cand
        a = mm.args[0]
        key = (id(a.buffer), a.layout.shape, a.layout.strides, a.layout.offset, w.shape[1],
               w.dtype, bias.dtype)
        groups.setdefault(key, []).append(cand)
    removed = 0
    for members in groups.values():
        if len(members) >= 2 and _merge(graph, members):
            removed += len(members) - 1
    if removed:
        graph.dead_code_eliminate()
        used = {id(v) for n in graph.nodes for v in n.unique_tensor_args()}
        for v in list(graph.params):
            if id(v) not in used:
                graph.params.remove(v)
                graph.param_tensors.pop(v.name, None)
                graph.param_origin.pop(v.name, None)
    return removed


def _merge(graph: Graph, members) -> bool:
    first_mm = members[0][0]
    a = first_mm.args[0]
    widths = [m[1].shape[0] for m in members]
    total = sum(widths)
    w_cat = torch.cat([graph.param_tensors[m[1].name] for m in members], dim=0)
    b_cat = torch.cat([graph.param_tensors[m[3].name] for m in members], dim=0)
    dtype = members[0][1].dtype

    def param(prefix, tensor):
        name = graph.fresh_name(prefix)
        v = Value(name, Buffer(name, tuple(tensor.shape), dtype, "param"),
                  Layout.contiguous(tuple(tensor.shape)))
        graph.params.append(v)
        graph.param_tensors[name] = tensor
        graph.param_origin[name] = "+".join(graph.param_origin.get(m[1].name, m[1].name)
                                            for m in members)
        return v

    snapshot_nodes = list(graph.nodes)
    snapshot_params = list(graph.params)
    w_v = param("p_merged_weight_", w_cat)
    b_v = param("p_merged_bias_", b_cat)

    targets = {"aten.permute.default": torch.ops.aten.permute.default,
               "aten.mm.default": torch.ops.aten.mm.default,
               "aten.add.Tensor": torch.ops.aten.add.Tensor,
               "aten.slice.Tensor": torch.ops.aten.slice.Tensor}

    def node(op, args, out, view=False):
        nd = Node(op, tuple(args), {}, outputs=[out])
        nd.meta["target"] = targets[op]
        if view:
            nd.meta["is_view"] = True
        return nd

    M = a.shape[0]
    wt_name = graph.fresh_name("merged_wt")
    wt = Value(wt_name, w_v.buffer, infer_view("aten.permute.default", [w_v, [1, 0]], {}))
    mm_name = graph.fresh_name("merged_mm")
    mm_out = Value(mm_name, Buffer(mm_name, (M, total), dtype), Layout.contiguous((M, total)))
    sum_name = graph.fresh_name("merged_add")
    sum_out = Value(sum_name, Buffer(sum_name, (M, total), dtype), Layout.contiguous((M, total)))
    new_nodes = [node("aten.permute.default", (w_v, [1, 0]), wt, view=True),
                 node("aten.mm.default", (a, wt), mm_out),
                 node("aten.add.Tensor", (mm_out, b_v), sum_out)]

    # every original output becomes a column slice of the merged sum
    changed: list[tuple[Value, Buffer, Layout]] = []
    start = 0
    for (mm, _, add, _), width in zip(members, widths):
        o = add.outputs[0]
        changed.append((o, o.buffer, o.layout))
        args = (sum_out, 1, start, start + width, 1)
        o.buffer = sum_out.buffer
        o.layout = infer_view("aten.slice.Tensor", list(args), {})
        new_nodes.append(node("aten.slice.Tensor", args, o, view=True))
        start += width
    dropped = {id(m[0]) for m in members} | {id(m[2]) for m in members}
    at = graph.nodes.index(first_mm)
    graph.nodes = ([n for n in graph.nodes[:at] if id(n) not in dropped] + new_nodes
                   + [n for n in graph.nodes[at:] if id(n) not in dropped])
    for nd in new_nodes:
        for i, o in enumerate(nd.outputs):
            o.producer = nd
            o.index = i

    # re-derive the views downstream of the rewritten outputs
    moved = {id(c[0]) for c in changed}
    try:
        for nd in graph.nodes:
            if not nd.meta.get("is_view") or nd in new_nodes:
                continue
            src = nd.args[0]
            if id(src) not in moved:
                continue
            out = nd.outputs[0]
            lay = infer_view(nd.op, list(nd.args), nd.kwargs)
            if lay.max_offset() > src.buffer.numel:
                raise ValueError("view outside its buffer")
            changed.append((out, out.buffer, out.layout))
            out.buffer, out.layout = src.buffer, lay
            moved.add(id(out))
        graph.topo_check()
    except Exception:
        for v, buf, lay in reversed(changed):
            v.buffer, v.layout = buf, lay
        for m in members:
            for i, o in enumerate(m[2].outputs):
                o.producer, o.index = m[2], i
        graph.nodes = snapshot_nodes
        graph.params = snapshot_params
        for v in (w_v, b_v):
            graph.param_tensors.pop(v.name, None)
            graph.param_origin.pop(v.name, None)
        return False
    return True
