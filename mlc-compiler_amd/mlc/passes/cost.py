"""Fusion cost model, in bytes of HBM traffic.

Arithmetic is converted at ``flops_per_byte`` and a saved launch is worth
``Config.effective_launch_bytes``. Reference behaviour followed:
``mlc/passes/cost.py:26-106`` (the same benefit/cost terms, so the same
groups form).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Iterable, Sequence

import torch

from ..config import Config
from ..ir.graph import Value
from ..ir.scalar import Expr, size as expr_size
from ..ir.types import itemsize_of


def itemsize(dtype: torch.dtype) -> int:
    return itemsize_of(dtype)


def value_bytes(v: Value) -> int:
    """Bytes of the view (not of the whole buffer)."""
    return v.numel * itemsize_of(v.dtype)


def traffic(reads: Iterable[Value], writes: Iterable[Value]) -> int:
    """HBM bytes of one kernel; each distinct buffer read counts once."""
    seen: set[int] = set()
    total = 0
    for v in reads:
        if id(v.buffer) not in seen:
            seen.add(id(v.buffer))
            total += value_bytes(v)
    return total + sum(value_bytes(v) for v in writes)


@dataclass
class MergeDecision:
    merge: bool
    benefit: float
    cost: float
    reason: str

    def __bool__(self) -> bool:
        return self.merge


def evaluate_merge(cfg: Config, *, saved_stores: Sequence[Value], saved_loads: Sequence[Value],
                   extra_loads: Sequence[Value], extra_evaluations: int, expr_ops: int,
                   saved_launches: int = 1) -> MergeDecision:
    benefit = float(sum(value_bytes(v) for v in saved_stores))
    benefit += float(sum(value_bytes(v) for v in saved_loads))
    benefit += saved_launches * cfg.effective_launch_bytes
    cost = float(sum(value_bytes(v) for v in extra_loads))
    if extra_evaluations > 0 and expr_ops > 0:
        cost += extra_evaluations * expr_ops / max(cfg.flops_per_byte, 1e-6)
    if expr_ops > cfg.max_recompute_ops and extra_evaluations > 0:
        return MergeDecision(False, benefit, cost, f"expression too large ({expr_ops} ops)")
    ok = benefit > cost
    return MergeDecision(ok, benefit, cost, "profitable" if ok else "not profitable")


def body_ops(body: Sequence[tuple[str, Expr]]) -> int:
    return sum(expr_size(e) for _, e in body)
