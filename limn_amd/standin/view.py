"""View: a tensor's logical index as affine arithmetic over a flat buffer, plus a validity box.

Semantics follow reference `limn/view.py:20-143`:

- element (i0, i1, ...) lives at `offset + sum(i_d * strides[d])`;
- a size-1 dim always carries stride 0, so layouts compare on one footing;
- `mask` is a per-dim half-open [lo, hi) box; reads outside it are 0 (what `pad` produces);
- every movement (permute, expand, shrink, pad, reshape) maps a View to a View, so chains of
  movements collapse to one View and cost nothing until a kernel reads through it;
- `reshape` returns None when the layout cannot be re-expressed without a copy.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

Box = tuple[tuple[int, int], ...]


def canonical_strides(shape: tuple[int, ...]) -> tuple[int, ...]:
    """Row-major strides with size-1 dims at stride 0."""
    out = [0] * len(shape)
    step = 1
    for d in range(len(shape) - 1, -1, -1):
        out[d] = 0 if shape[d] == 1 else step
        step *= shape[d]
    return tuple(out)


def _box_or_none(shape: tuple[int, ...], box: Box) -> Box | None:
    full = all(lo == 0 and hi == size for (lo, hi), size in zip(box, shape))
    return None if full else box


@dataclass(frozen=True)
class View:
    shape: tuple[int, ...]
    strides: tuple[int, ...]
    offset: int
    mask: Box | None

    def __post_init__(self) -> None:
        fixed = tuple(0 if n == 1 else s for n, s in zip(self.shape, self.strides))
        if fixed != self.strides:
            object.__setattr__(self, "strides", fixed)

    @staticmethod
    def contiguous(shape: tuple[int, ...]) -> View:
        shape = tuple(shape)
        return View(shape, canonical_strides(shape), 0, None)

    @property
    def numel(self) -> int:
        return math.prod(self.shape)

    @property
    def is_dense(self) -> bool:
        """Unmasked and row-major (any offset): can be reshaped in place."""
        return self.mask is None and self.strides == canonical_strides(self.shape)

    @property
    def is_contiguous(self) -> bool:
        """Dense and starting at element 0."""
        return self.offset == 0 and self.is_dense

    def _box(self) -> Box:
        return self.mask if self.mask is not None else tuple((0, n) for n in self.shape)

    def permute(self, order: tuple[int, ...]) -> View:
        if sorted(order) != list(range(len(self.shape))):
            raise ValueError(f"permute order {order} is not a permutation of {len(self.shape)} dims")
        box = None if self.mask is None else tuple(self.mask[d] for d in order)
        return View(tuple(self.shape[d] for d in order), tuple(self.strides[d] for d in order), self.offset, box)

    def expand(self, shape: tuple[int, ...]) -> View:
        shape = tuple(shape)
        if len(shape) != len(self.shape) or any(old != new and old != 1 for old, new in zip(self.shape, shape)):
            raise ValueError(f"cannot expand {self.shape} to {shape}: only size-1 dims may grow")
        strides = tuple(0 if old != new else s for s, old, new in zip(self.strides, self.shape, shape))
        box = None
        if self.mask is not None:
            grown = []
            for (lo, hi), old, new in zip(self.mask, self.shape, shape):
                if old == new:
                    grown.append((lo, hi))
                else:  # the lone element is either in the box (every copy is) or not (none is)
                    grown.append((0, new) if (lo, hi) == (0, 1) else (0, 0))
            box = tuple(grown)
        return View(shape, strides, self.offset, box)

    def shrink(self, bounds: Box) -> View:
        bounds = tuple((int(lo), int(hi)) for lo, hi in bounds)
        if len(bounds) != len(self.shape) or not all(0 <= lo < hi <= n for (lo, hi), n in zip(bounds, self.shape)):
            raise ValueError(f"cannot shrink shape {self.shape} to bounds {bounds}")
        offset = self.offset + sum(lo * s for (lo, _), s in zip(bounds, self.strides))
        shape = tuple(hi - lo for lo, hi in bounds)
        box = None
        if self.mask is not None:
            moved = tuple((max(mlo - lo, 0), min(mhi - lo, hi - lo)) for (lo, hi), (mlo, mhi) in zip(bounds, self.mask))
            box = _box_or_none(shape, moved)
        return View(shape, self.strides, offset, box)

    def pad(self, padding: Box) -> View:
        padding = tuple((int(b), int(a)) for b, a in padding)
        if len(padding) != len(self.shape) or any(b < 0 or a < 0 for b, a in padding):
            raise ValueError(f"cannot pad shape {self.shape} with {padding}")
        offset = self.offset - sum(b * s for (b, _), s in zip(padding, self.strides))
        shape = tuple(n + b + a for n, (b, a) in zip(self.shape, padding))
        box = tuple((lo + b, hi + b) for (lo, hi), (b, _) in zip(self._box(), padding))
        return View(shape, self.strides, offset, _box_or_none(shape, box))

    def reshape(self, shape: tuple[int, ...]) -> View | None:
        shape = tuple(shape)
        if math.prod(shape) != self.numel:
            raise ValueError(f"cannot reshape {self.shape} to {shape}: element counts differ")
        if shape == self.shape:
            return self
        if self.is_dense:
            return View(shape, canonical_strides(shape), self.offset, None)
        # Otherwise only adding or dropping size-1 dims is free: the non-unit dims must survive
        # in order, and a dropped size-1 dim must not be masked away.
        box = self._box()
        real = [(s, m) for n, s, m in zip(self.shape, self.strides, box) if n != 1]
        if [n for n in self.shape if n != 1] != [n for n in shape if n != 1]:
            return None
        if any(m != (0, 1) for n, m in zip(self.shape, box) if n == 1):
            return None
        strides, masks = [], []
        it = iter(real)
        for n in shape:
            s, m = (0, (0, 1)) if n == 1 else next(it)
            strides.append(s)
            masks.append(m)
        return View(shape, tuple(strides), self.offset, _box_or_none(shape, tuple(masks)))
