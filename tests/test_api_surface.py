"""The reference's front-end helpers that the passes here do not call but a
user of the reference's API may: graph queries (``mlc/ir/graph.py``), the op
table's ``is_reduction`` (``mlc/ir/ops.py``), a layout's
``is_dense_from_zero`` (``mlc/ir/types.py``), the index map's
``is_constant`` / ``is_scalar`` (``mlc/codegen/index.py``) and the use
analysis's ``node_consumers`` (``mlc/passes/scheduler.py`` in the
reference). Each is checked against what the graph itself says."""

from __future__ import annotations

import torch

from mlc.codegen.index import build_index
from mlc.ir.capture import capture
from mlc.ir.ops import is_reduction, is_view
from mlc.ir.types import Layout
from mlc.passes.grouping import UseInfo
from models import all_models


def _graph(name):
    _, model, args = next(t for t in all_models() if t[0] == name)
    return capture(model, args)


def test_graph_queries_agree_with_the_node_list():
    g = _graph("masked_softmax")
    uses = g.use_map()
    for i, n in enumerate(g.nodes):
        assert g.index_of(n) == i
        for o in n.outputs:
            assert g.users_of(o) == uses.get(id(o), [])
            assert all(o in u.unique_tensor_args() for u in g.users_of(o))
            if is_view(n.op):
                assert o.is_view_of(n.args[0])
    b = g.new_buffer((3, 4), torch.float16)
    assert b.shape == (3, 4) and b.dtype == torch.float16 and b.kind == "intermediate"
    assert b.name != g.new_buffer((3, 4), torch.float16).name


def test_reductions_are_named_by_the_op_table():
    g = _graph("norm_affine")
    reds = [n.op for n in g.nodes if is_reduction(n.op)]
    assert reds and all(not is_reduction(n.op) for n in g.nodes if n.op.startswith("aten.add"))


def test_dense_from_zero_layouts():
    assert Layout((2, 3), (3, 1), 0).is_dense_from_zero()
    assert not Layout((2, 3), (3, 1), 1).is_dense_from_zero()     # starts later
    assert not Layout((2, 3), (1, 2), 0).is_dense_from_zero()     # transposed
    assert not Layout((2, 3), (0, 1), 0).is_dense_from_zero()     # broadcast


def test_constant_and_scalar_index_maps():
    bcast = build_index([("row", (4,)), ("col", (8,))], Layout((4, 8), (0, 1), 0))
    assert bcast.axes[0].is_constant and not bcast.axes[1].is_constant
    assert not bcast.is_scalar()
    one = build_index([("row", (4,)), ("col", (8,))], Layout((4, 8), (0, 0), 5))
    assert one.is_scalar() and all(a.is_constant for a in one.axes)


def test_node_consumers_are_the_readers_of_every_output():
    g = _graph("shared_producer")
    info = UseInfo(g)
    for n in g.nodes:
        want = frozenset().union(*(info.consumers(o) for o in n.outputs))
        assert info.node_consumers(n) == want
    producer = next(n for n in g.nodes if len(info.node_consumers(n)) >= 2)
    assert producer is not None
