"""Captured benchmark graphs, built once per test process.

Capturing BERT-base or GPT-2 takes seconds, and many tests start from the
same workload. ``graph_of(key)`` captures each workload once and hands every
caller its own deep copy (passes rewrite graphs in place); parameter tensors
and op handles are shared, never copied."""

from __future__ import annotations

import copy
import functools

from mlc.bench.workloads import make
from mlc.ir.capture import capture


@functools.lru_cache(maxsize=None)
def _captured(key: str):
    model, args = make(key)
    return model, args, capture(model, args)


def model_args(key: str):
    model, args, _ = _captured(key)
    return model, args


def graph_of(key: str):
    """A fresh copy of workload ``key``'s captured graph (seeded inputs)."""
    _, _, g = _captured(key)
    memo = {id(t): t for t in g.param_tensors.values()}
    for v in g.meta.values():
        memo[id(v)] = v
    for n in g.nodes:
        for v in n.meta.values():
            if not isinstance(v, (int, float, str, bool, type(None))):
                memo[id(v)] = v
    return copy.deepcopy(g, memo)
