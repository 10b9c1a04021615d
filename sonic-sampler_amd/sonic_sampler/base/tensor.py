"""Tensor subclasses whose 2-D prefix slices are contiguous (reference ``base/tensor.py:24-87``).

``t[:b, :k]`` of a ``[R, T, ...]`` tensor returns the first ``b * k`` rows of the flattened
``[R * T, ...]`` view, reshaped to ``[b, k, ...]``: a contiguous block whose row stride is
``k * (...)``. Any other indexing behaves like ``torch.Tensor``.
"""

from __future__ import annotations

import weakref

from typing import Dict, Optional, Tuple

from torch import Tensor


class PrefixContiguousTensor(Tensor):

    def __slice__(self, rows: int, steps: int) -> Tensor:

        return Tensor.__getitem__(self.flatten(0, 1), slice(rows * steps)).unflatten(0, (rows, steps))

    def __can_slice__(self, s: slice, t: slice) -> Optional[Tuple[int, int]]:

        rows, steps = self.shape[0], self.shape[1]
        a, b, c = s.indices(rows)
        d, k, e = t.indices(steps)

        if a == 0 and c == 1 and d == 0 and e == 1 and b and k:

            return b, k

        return None

    def __getitem__(self, *args, **kwargs) -> Tensor:

        if len(args) == 1 and isinstance(args[0], tuple) and len(args[0]) == 2:

            s, t = args[0]

            if isinstance(s, slice) and isinstance(t, slice) and self.dim() >= 2:

                if (p := self.__can_slice__(s, t)) is not None:

                    return self.__slice__(*p)

        return super().__getitem__(*args, **kwargs)


class TimeDifferentiatedTensor(PrefixContiguousTensor):

    """A prefix-contiguous tensor stored time-major: ``[T, B, ...]`` indexed as ``[B, T, ...]``."""

    def __getitem__(self, *args, **kwargs) -> Tensor:

        final = args

        if len(args) == 1 and isinstance(args[0], tuple) and len(args[0]) >= 2:

            rows, steps, *rest = args[0]

            if isinstance(rows, slice) and isinstance(steps, slice):

                stop = steps.stop
                steps = slice(steps.start, stop and (stop - 1), steps.step)
                final = ((steps, rows, *rest),)

        elif len(args) == 1 and isinstance(args[0], slice):

            final = ((slice(None), args[0]),)

        return super().__getitem__(*final, **kwargs)


def prefix_contiguous(tensor: Tensor) -> PrefixContiguousTensor:

    return tensor.as_subclass(PrefixContiguousTensor)


# id(plane) -> (weak reference to the plane, {index: plain view})
_PLAIN_VIEWS: Dict[int, Tuple["weakref.ref[Tensor]", Dict[object, Tensor]]] = {}


def plain_view(plane: Tensor, column: Optional[int] = None) -> Tensor:
    """`plane`, or `plane[:, column]`, as a plain ``torch.Tensor`` view of the same memory, built
    once per plane object. Every operation on a tensor subclass (including reading a stride or a
    data pointer) dispatches through Python, a few microseconds each on the host; the entry points
    only pass the view's pointer and strides on. Entries whose plane has been freed are replaced
    (the weak reference tells a reused id apart)."""

    entry = _PLAIN_VIEWS.get(id(plane))

    if entry is None or entry[0]() is not plane:

        if len(_PLAIN_VIEWS) > 4096:

            for key in [k for k, (ref, _) in _PLAIN_VIEWS.items() if ref() is None]:

                del _PLAIN_VIEWS[key]

        entry = _PLAIN_VIEWS[id(plane)] = (weakref.ref(plane), {})

    views = entry[1]
    view = views.get(column)

    if view is None:

        base = plane.as_subclass(Tensor) if type(plane) is not Tensor else plane
        view = views[column] = base if column is None else base[:, column]

    return view
