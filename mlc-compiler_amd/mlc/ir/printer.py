"""Readable graph dumps (the ``graph`` CLI view)."""

from __future__ import annotations

from .graph import Graph


def format_graph(g: Graph, show_buffers: bool = False) -> str:
    out = [f"graph {g.name}("]
    out += [f"    param {v!r}," for v in g.params]
    out += [f"    input {v!r}," for v in g.inputs]
    out.append(") {")
    for n in g.nodes:
        grp = n.meta.get("group")
        out.append(f"    {n!r}" + ("" if grp is None else f"    # group {grp}"))
    out.append(f"    return {', '.join(repr(v) for v in g.outputs)}")
    out.append("}")
    if show_buffers:
        out.append("buffers:")
        for b in g.buffers():
            at = "" if b.arena_offset is None else f" @{b.arena_offset}"
            out.append(f"    {b!r} {b.nbytes}B{at}")
    return "\n".join(out)
