"""Prefix-sliceable buffer structs (reference ``base/buffer.py:40-274``).

A ``SliceBuffer`` is a dataclass of tensors (and nested buffers) sharing a leading row dimension
described by its ``Layout``. ``buffers[:R]`` and ``buffers[:R, :T]`` return views of every member;
prefix slices (starting at row 0) are cached per instance so that repeated slicing returns the
same objects with the same data pointers, which is what a captured graph needs.
"""

from __future__ import annotations

import dataclasses

from dataclasses import dataclass
from itertools import product
from typing import Any, Dict, Tuple

from torch import Tensor

from sonic_sampler.base.tensor import PrefixContiguousTensor


GridKey = Tuple[int, int]


@dataclass(eq=False)
class Layout:

    # The batch size of the corresponding 1D / 2D grid.
    rows: int

    # The timesteps of the corresponding 2D grid.
    cols: int

    def __getitem__(self, indices) -> "Layout":

        if isinstance(indices, slice):

            return Layout(indices.indices(self.rows)[1], self.cols)

        if isinstance(indices, tuple) and len(indices) == 2 and all(isinstance(i, slice) for i in indices):

            return Layout(indices[0].indices(self.rows)[1], indices[1].indices(self.cols)[1])

        raise ValueError(f"unsupported slice indexing: {indices}")

    def __eq__(self, other) -> bool:

        return isinstance(other, Layout) and (self.rows, self.cols) == (other.rows, other.cols)

    def __hash__(self) -> int:

        return hash((self.rows, self.cols))


def validate(index: slice, bound: int) -> Tuple[int, int]:

    start, stop, step = index.indices(bound)

    if step != 1:

        raise ValueError("interval slicing is not supported")

    if not stop or start >= stop:

        raise ValueError("asked to slice an empty subset")

    return start, stop


@dataclass(eq=False, kw_only=True)
class SliceBuffer:

    # The associated layout of this buffer.
    layout: Layout

    def __post_init__(self) -> None:

        self._prefix_cache: Dict[GridKey, "SliceBuffer"] = {}

    def _slice_field(self, value: Any, indices) -> Any:

        if isinstance(value, (int, float, bool)) or value is None:

            return value

        if isinstance(indices, tuple):

            s, t = indices

            if isinstance(value, (PrefixContiguousTensor, Layout)):

                return value[s.start:s.stop, t.start:t.stop]

            return value[s.start:s.stop]

        return value[indices.start:indices.stop]

    def _make(self, indices) -> "SliceBuffer":

        kwargs = {
            f.name: self._slice_field(getattr(self, f.name), indices)
            for f in dataclasses.fields(self)
        }

        return self.__class__(**kwargs)

    def __getitem__(self, indices) -> "SliceBuffer":

        layout = self.layout

        if isinstance(indices, slice):

            start, stop = validate(indices, layout.rows)

            if start:

                return self._make(slice(start, stop))

            if stop == layout.rows:

                return self

            key = (stop, layout.cols)

        elif isinstance(indices, tuple) and len(indices) == 2 and all(isinstance(i, slice) for i in indices):

            rows, cols = indices
            col_start, col_stop = validate(cols, layout.cols)
            row_start, row_stop = validate(rows, layout.rows)

            if row_start or col_start:

                return self._make((slice(row_start, row_stop), slice(col_start, col_stop)))

            if col_stop == layout.cols:

                return self[slice(0, row_stop)]

            key = (row_stop, col_stop)
            indices = (slice(0, row_stop), slice(0, col_stop))

        else:

            raise ValueError("only 1d or 2d slicing are supported")

        if key not in self._prefix_cache:

            self._prefix_cache[key] = self._make(indices if isinstance(indices, tuple) else slice(0, key[0]))

        return self._prefix_cache[key]

    def bisect(self, pivot: int) -> Tuple["SliceBuffer", "SliceBuffer"]:

        if 0 < pivot < self.layout.rows:

            return self[:pivot], self[pivot:]

        raise ValueError("asked to bisect at boundaries resulting in an empty slice")

    def prepopulate(self, schedule) -> None:

        if (isinstance(schedule, (list, tuple)) and len(schedule) == 2
                and all(isinstance(x, (list, tuple)) for x in schedule)):

            for r, c in product(sorted(schedule[0]), sorted(schedule[1])):

                _ = self[:r, :c]

        elif isinstance(schedule, (list, tuple)) and schedule and isinstance(schedule[0], tuple):

            for r, c in sorted(schedule):

                _ = self[:r, :c]

        elif isinstance(schedule, (list, tuple)):

            for r in sorted(schedule):

                _ = self[:r]

        else:

            raise ValueError(f"unsupported schedule: {schedule}")

    def __tensors__(self):

        for f in dataclasses.fields(self):

            value = getattr(self, f.name)

            if isinstance(value, Tensor):

                yield value

            elif isinstance(value, SliceBuffer):

                yield from value.__tensors__()

    def __eq__(self, other) -> bool:

        return self is other

    def __hash__(self) -> int:

        return id(self)
