"""Storage and views.

A :class:`Buffer` is one contiguous allocation: the unit the planner places
in the arena and the unit a kernel stores into. A :class:`Layout` is a
``(shape, strides, offset)`` window onto a buffer. Every view op (permute,
expand, slice, reshape that needs no copy) only builds a new Layout, so views
never reach a kernel as work of their own.

Reference behaviour followed: ``mlc/ir/types.py:38-263``.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Iterable, Sequence

import torch

Shape = tuple[int, ...]
Strides = tuple[int, ...]


def contiguous_strides(shape: Sequence[int]) -> Strides:
    """Row-major strides for ``shape``."""
    out = []
    step = 1
    for d in reversed(tuple(shape)):
        out.append(step)
        step *= int(d)
    return tuple(reversed(out))


def _numel(shape: Sequence[int]) -> int:
    return math.prod(shape) if shape else 1


@dataclass(frozen=True)
class Layout:
    shape: Shape
    strides: Strides
    offset: int = 0

    def __post_init__(self) -> None:
        if len(self.shape) != len(self.strides):
            raise ValueError(f"rank mismatch: shape={self.shape} strides={self.strides}")
        for d in self.shape:
            if d < 0:
                raise ValueError(f"negative dim in {self.shape}")

    @staticmethod
    def contiguous(shape: Sequence[int], offset: int = 0) -> "Layout":
        shp = tuple(int(d) for d in shape)
        return Layout(shp, contiguous_strides(shp), offset)

    # -- queries ------------------------------------------------------------
    @property
    def rank(self) -> int:
        return len(self.shape)

    @property
    def numel(self) -> int:
        return _numel(self.shape)

    def is_contiguous(self) -> bool:
        return self.offset == 0 and self.strides == contiguous_strides(self.shape)

    def is_dense_from_zero(self) -> bool:
        return self.is_contiguous()

    def max_offset(self) -> int:
        """One past the highest element offset reachable through this view."""
        hi = self.offset
        for n, s in zip(self.shape, self.strides):
            if n > 0:
                hi += (n - 1) * s
        return hi + 1

    # -- view algebra -------------------------------------------------------
    def permute(self, dims: Sequence[int]) -> "Layout":
        r = self.rank
        order = [int(d) % r if r else 0 for d in dims]
        if sorted(order) != list(range(r)):
            raise ValueError(f"permute({list(dims)}) is not a permutation of rank {r}")
        return Layout(tuple(self.shape[d] for d in order),
                      tuple(self.strides[d] for d in order), self.offset)

    def expand(self, shape: Sequence[int]) -> "Layout":
        """Broadcast to ``shape`` (``-1`` keeps a size); new dims get stride 0."""
        want = [int(d) for d in shape]
        if len(want) < self.rank:
            raise ValueError(f"cannot expand rank {self.rank} to {len(want)} dims")
        lead = len(want) - self.rank
        have_shape = (1,) * lead + self.shape
        have_strides = (0,) * lead + self.strides
        shp: list[int] = []
        std: list[int] = []
        for i, w in enumerate(want):
            h = have_shape[i]
            if w == -1:
                w = h
            if w == h:
                shp.append(w)
                std.append(have_strides[i])
            elif h == 1:
                shp.append(w)
                std.append(0)
            else:
                raise ValueError(f"cannot expand dim {i} from {h} to {w}")
        return Layout(tuple(shp), tuple(std), self.offset)

    def unsqueeze(self, dim: int) -> "Layout":
        if dim < 0:
            dim += self.rank + 1
        s = self.strides[dim] * self.shape[dim] if dim < self.rank else 1
        return Layout(self.shape[:dim] + (1,) + self.shape[dim:],
                      self.strides[:dim] + (s,) + self.strides[dim:], self.offset)

    def squeeze(self, dims: Iterable[int] | None = None) -> "Layout":
        if dims is None:
            keep = [i for i, n in enumerate(self.shape) if n != 1]
        else:
            gone = {int(d) % self.rank for d in dims}
            keep = [i for i in range(self.rank)
                    if not (i in gone and self.shape[i] == 1)]
        return Layout(tuple(self.shape[i] for i in keep),
                      tuple(self.strides[i] for i in keep), self.offset)

    def slice(self, dim: int, start: int, end: int, step: int = 1) -> "Layout":
        dim %= self.rank
        n = self.shape[dim]
        lo = start + n if start < 0 else start
        lo = min(max(lo, 0), n)
        hi = end + n if end < 0 else end
        hi = min(max(hi, lo), n)
        length = (hi - lo + step - 1) // step
        shp = list(self.shape)
        std = list(self.strides)
        shp[dim] = length
        std[dim] = self.strides[dim] * step
        return Layout(tuple(shp), tuple(std), self.offset + lo * self.strides[dim])

    def reshape(self, shape: Sequence[int]) -> "Layout | None":
        """The same storage seen with ``shape``, or None when that needs a copy.

        A reshape is free when it only splits or joins dimensions inside runs
        that are contiguous in the existing layout (torch's ``view`` rule), so a
        strided slice can still have its last dimension split into heads.
        """
        shp = tuple(int(d) for d in shape)
        if _numel(shp) != self.numel:
            raise ValueError(f"reshape {self.shape} -> {shp} changes element count")
        if self.numel == 0:
            return Layout(shp, contiguous_strides(shp), self.offset)
        strides = view_strides(self.shape, self.strides, shp)
        if strides is None:
            return None
        return Layout(shp, strides, self.offset)

    def as_torch(self, storage: torch.Tensor) -> torch.Tensor:
        """This view over a flat 1-D ``storage`` tensor.

        ``as_strided`` offsets are relative to the underlying storage, so the
        flat tensor's own storage offset (non-zero for an arena slice) is added.
        """
        return storage.as_strided(self.shape, self.strides,
                                  self.offset + storage.storage_offset())

    def __repr__(self) -> str:  # pragma: no cover - debug aid
        if self.is_contiguous():
            return f"Layout{self.shape}"
        return f"Layout{self.shape} strides={self.strides} off={self.offset}"


def view_strides(old_shape: Shape, old_strides: Strides, new_shape: Shape) -> Strides | None:
    """Strides that view ``old`` storage as ``new_shape``, or None.

    Torch's stride computation for ``Tensor.view``: scan the old dims from the
    innermost outwards, close a chunk wherever the next-outer dim is not laid
    out directly after the current run, and require each chunk to be covered
    exactly by a run of new dims.
    """
    out = [0] * len(new_shape)
    vd = len(new_shape) - 1
    unit = old_strides[-1] if old_shape else 1
    chunk_elems = 1
    covered = 1
    for td in range(len(old_shape) - 1, -1, -1):
        chunk_elems *= old_shape[td]
        boundary = td == 0 or (old_shape[td - 1] != 1
                               and old_strides[td - 1] != chunk_elems * unit)
        if not boundary:
            continue
        while vd >= 0 and (covered < chunk_elems or new_shape[vd] == 1):
            out[vd] = covered * unit
            covered *= new_shape[vd]
            vd -= 1
        if covered != chunk_elems:
            return None
        if td > 0:
            unit = old_strides[td - 1]
            chunk_elems = 1
            covered = 1
    return tuple(out) if vd == -1 else None


# --------------------------------------------------------------------------
# Buffers
# --------------------------------------------------------------------------

#: buffer kinds the planner may place in the arena
PLANNABLE = ("intermediate",)

BUFFER_KINDS = ("input", "param", "intermediate", "output", "constant")

_ITEMSIZE: dict[torch.dtype, int] = {}


def itemsize_of(dtype: torch.dtype) -> int:
    n = _ITEMSIZE.get(dtype)
    if n is None:
        n = torch.empty((), dtype=dtype).element_size()
        _ITEMSIZE[dtype] = n
    return n


@dataclass(eq=False)
class Buffer:
    name: str
    shape: Shape
    dtype: torch.dtype
    kind: str = "intermediate"
    #: byte offset in the arena, set by the memory planner
    arena_offset: int | None = field(default=None, compare=False)

    def __post_init__(self) -> None:
        self.shape = tuple(int(d) for d in self.shape)
        if self.kind not in BUFFER_KINDS:
            raise ValueError(f"bad buffer kind {self.kind!r}")

    @property
    def numel(self) -> int:
        return _numel(self.shape)

    @property
    def itemsize(self) -> int:
        return itemsize_of(self.dtype)

    @property
    def nbytes(self) -> int:
        return self.numel * self.itemsize

    @property
    def plannable(self) -> bool:
        return self.kind in PLANNABLE

    def __repr__(self) -> str:  # pragma: no cover - debug aid
        dt = str(self.dtype).replace("torch.", "")
        return f"Buffer({self.name}, {self.shape}, {dt}, {self.kind})"
