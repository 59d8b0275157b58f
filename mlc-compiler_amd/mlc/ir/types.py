"""Storage and the views over it.

Two types carry every tensor in the IR:

* :class:`Buffer` -- one dense allocation (name, shape, dtype, kind). It is
  what the arena planner places and what a kernel stores into.
* :class:`Layout` -- an affine window ``(shape, strides, offset)`` in elements
  over some buffer. View ops only ever produce a new Layout, so a transpose,
  a slice or a broadcast costs nothing and later shows up in a kernel's index
  map instead of as a copy.

The one non-trivial view is ``reshape``: it is free exactly when every new
dimension falls inside one *chunk* of the old layout, a maximal group of
adjacent dims that step through memory as one dense run. That is the rule
``Tensor.view`` applies (reference counterpart: ``mlc/ir/types.py:148-218``);
it is implemented here chunk by chunk (``_chunks`` then ``_fit``), and the
resulting strides, size-1 dims included, are torch's.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Iterable, Sequence

import torch

Shape = tuple[int, ...]
Strides = tuple[int, ...]


def contiguous_strides(shape: Sequence[int]) -> Strides:
    """Row-major strides of ``shape`` (the last dim moves fastest)."""
    dims = [int(d) for d in shape]
    suffix = [math.prod(dims[i + 1:]) for i in range(len(dims))]
    return tuple(suffix)


def _chunks(shape: Shape, strides: Strides) -> list[tuple[int, int]]:
    """The old layout cut into dense runs, innermost first, as
    ``(elements, stride of the run's innermost dim)``. A dim continues the
    run inside it when it is size 1 or steps exactly over that run."""
    out: list[tuple[int, int]] = []
    count, base = 1, strides[-1]
    for d in range(len(shape) - 1, -1, -1):
        count *= shape[d]
        outer = d - 1
        if outer >= 0 and (shape[outer] == 1 or strides[outer] == count * base):
            continue
        out.append((count, base))
        if outer >= 0:
            count, base = 1, strides[outer]
    return out


def _fit(chunks: list[tuple[int, int]], new_shape: Shape) -> Strides | None:
    """Strides for ``new_shape`` such that every new dim lies in one chunk,
    or None. New dims are handed out innermost first; a chunk takes dims
    until it is covered, plus any size-1 dims that follow."""
    strides = [0] * len(new_shape)
    pos = len(new_shape) - 1
    for count, base in chunks:
        covered = 1
        while pos >= 0 and (covered < count or new_shape[pos] == 1):
            strides[pos] = covered * base
            covered *= new_shape[pos]
            pos -= 1
        if covered != count:
            return None
    return tuple(strides) if pos < 0 else None


@dataclass(frozen=True)
class Layout:
    """``element(i0, .., ik) = buffer[offset + sum(i_d * strides[d])]``."""

    shape: Shape
    strides: Strides
    offset: int = 0

    def __post_init__(self) -> None:
        if len(self.shape) != len(self.strides):
            raise ValueError(f"layout has {len(self.shape)} sizes but {len(self.strides)} "
                             f"strides ({self.shape} / {self.strides})")
        if min(self.shape, default=0) < 0:
            raise ValueError(f"layout size below zero: {self.shape}")

    @classmethod
    def contiguous(cls, shape: Sequence[int], offset: int = 0) -> "Layout":
        dims = tuple(int(d) for d in shape)
        return cls(dims, contiguous_strides(dims), offset)

    # -- properties -----------------------------------------------------------
    @property
    def rank(self) -> int:
        return len(self.shape)

    @property
    def numel(self) -> int:
        return math.prod(self.shape)

    def is_contiguous(self) -> bool:
        return self.offset == 0 and self.strides == contiguous_strides(self.shape)

    def is_dense_from_zero(self) -> bool:
        """Covers exactly elements ``[0, numel)`` of its buffer in order."""
        return self.is_contiguous()

    def max_offset(self) -> int:
        """One past the furthest element this window reaches."""
        reach = sum((d - 1) * s for d, s in zip(self.shape, self.strides) if d)
        return self.offset + reach + 1

    # -- views ----------------------------------------------------------------
    def _with(self, dims: Iterable[tuple[int, int]], offset: int | None = None) -> "Layout":
        pairs = list(dims)
        return Layout(tuple(p[0] for p in pairs), tuple(p[1] for p in pairs),
                      self.offset if offset is None else offset)

    def permute(self, dims: Sequence[int]) -> "Layout":
        order = [int(d) % max(self.rank, 1) for d in dims]
        if len(order) != self.rank or set(order) != set(range(self.rank)):
            raise ValueError(f"{list(dims)} does not reorder the {self.rank} dims of {self.shape}")
        pairs = list(zip(self.shape, self.strides))
        return self._with(pairs[d] for d in order)

    def expand(self, shape: Sequence[int]) -> "Layout":
        """Broadcast to ``shape`` (-1 keeps a size): size-1 dims, and dims
        added on the left, get stride 0."""
        want = [int(d) for d in shape]
        extra = len(want) - self.rank
        if extra < 0:
            raise ValueError(f"expand to {want} has fewer dims than {self.shape}")
        have = [(1, 0)] * extra + list(zip(self.shape, self.strides))
        out = []
        for i, ((size, stride), w) in enumerate(zip(have, want)):
            w = size if w == -1 else w
            if w == size:
                out.append((size, stride))
            elif size == 1:
                out.append((w, 0))
            else:
                raise ValueError(f"expand {self.shape} -> {tuple(want)}: dim {i} has size "
                                 f"{size}, not 1, and cannot become {w}")
        return self._with(out)

    def unsqueeze(self, dim: int) -> "Layout":
        at = dim + self.rank + 1 if dim < 0 else dim
        pairs = list(zip(self.shape, self.strides))
        stride = pairs[at][0] * pairs[at][1] if at < self.rank else 1
        pairs.insert(at, (1, stride))
        return self._with(pairs)

    def squeeze(self, dims: Iterable[int] | None = None) -> "Layout":
        if dims is None:
            gone = {i for i, d in enumerate(self.shape) if d == 1}
        else:
            gone = {d % self.rank for d in dims if self.shape[d % self.rank] == 1}
        return self._with(p for i, p in enumerate(zip(self.shape, self.strides))
                          if i not in gone)

    def slice(self, dim: int, start: int, end: int, step: int = 1) -> "Layout":
        d = dim % self.rank
        n = self.shape[d]

        def clamp(v: int, lo: int) -> int:
            return min(n, max(lo, v + n if v < 0 else v))

        lo = clamp(start, 0)
        hi = clamp(end, lo)
        pairs = list(zip(self.shape, self.strides))
        stride = pairs[d][1]
        pairs[d] = (-(-(hi - lo) // step), stride * step)
        return self._with(pairs, self.offset + lo * stride)

    def reshape(self, shape: Sequence[int]) -> "Layout | None":
        """The same elements under ``shape`` without copying, or None when
        some new dim would straddle two dense runs of this layout."""
        dims = tuple(int(d) for d in shape)
        if math.prod(dims) != self.numel:
            raise ValueError(f"reshape {self.shape} -> {dims}: {self.numel} elements vs "
                             f"{math.prod(dims)}")
        if self.numel == 0:
            return Layout(dims, contiguous_strides(dims), self.offset)
        if not self.shape:
            return Layout(dims, (), self.offset) if not dims else None
        strides = _fit(_chunks(self.shape, self.strides), dims)
        return None if strides is None else Layout(dims, strides, self.offset)

    def as_torch(self, storage: torch.Tensor) -> torch.Tensor:
        """This window over a flat 1-D ``storage`` tensor. ``as_strided``
        counts its offset from the start of the *storage*, so a storage that
        is itself a slice (an arena sub-range) adds its own offset."""
        return storage.as_strided(self.shape, self.strides,
                                  storage.storage_offset() + self.offset)

    def __repr__(self) -> str:  # pragma: no cover - debug aid
        if self.is_contiguous():
            return f"Layout{self.shape}"
        return f"Layout{self.shape} strides={self.strides} off={self.offset}"


# --------------------------------------------------------------------------
# buffers
# --------------------------------------------------------------------------

#: what a buffer holds; only intermediates are placed in the arena
BUFFER_KINDS = ("input", "param", "intermediate", "output", "constant")
PLANNABLE = ("intermediate",)

_ITEMSIZE: dict[torch.dtype, int] = {}


def itemsize_of(dtype: torch.dtype) -> int:
    """Bytes per element of ``dtype``."""
    size = _ITEMSIZE.get(dtype)
    if size is None:
        size = _ITEMSIZE[dtype] = torch.empty((), dtype=dtype).element_size()
    return size


@dataclass(eq=False)
class Buffer:
    name: str
    shape: Shape
    dtype: torch.dtype
    kind: str = "intermediate"
    #: byte offset in the arena, written by the planner (None: not placed)
    arena_offset: int | None = field(default=None, compare=False)

    def __post_init__(self) -> None:
        if self.kind not in BUFFER_KINDS:
            raise ValueError(f"buffer {self.name}: kind {self.kind!r} is not one of "
                             f"{BUFFER_KINDS}")
        self.shape = tuple(int(d) for d in self.shape)

    @property
    def numel(self) -> int:
        return math.prod(self.shape)

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
