"""Per-request control words (reference ``core/flags.py:42-574``).

``Indicator`` is a 12-bit flag word whose bits enable the logit processors and select the
sampling path; ``ScopedIndicators`` holds one word per request for the verifier (``target``) and
one for the drafter (``draft``); ``Flags`` packs both into a device tensor of shape ``[B, 2]`` and
stride ``[1, B]`` so that ``flags.target`` and ``flags.draft`` are contiguous ``[B]`` uint16
tensors, which is what the kernels read.
"""

from __future__ import annotations

import random as _random

from contextlib import nullcontext
from dataclasses import dataclass
from enum import Enum, IntFlag, unique
from itertools import compress, repeat
from typing import Callable, List, Optional

import torch

from torch import Tensor

from sonic_sampler.base import Layout, SliceBuffer
from sonic_sampler.base.tensor import plain_view
from sonic_sampler.ops import MAX_K


BOOL: torch.dtype = torch.bool
U16: torch.dtype = torch.uint16
I16: torch.dtype = torch.int16
I64: torch.dtype = torch.int64


@unique
class SamplingMode(str, Enum):

    # Assigns the indicator to the minimal greedy state, i.e. 0x40.
    MINIMAL = "minimal"

    # Removes the stochastic indicators and enables greedy.
    GREEDY = "greedy"

    # Enables everything but greedy, i.e. 0xFBF.
    MAXIMAL = "maximal"

    # Disables the grammar indicator.
    NON_GRAMMAR = "non_grammar"


@unique
class Indicator(IntFlag):

    GRAMMAR = 0x1
    MULTIPLICATIVE = 0x2
    FREQUENCY = 0x4
    PRESENCE = 0x8
    BIAS = 0x10
    TEMPERATURE = 0x20
    GREEDY = 0x40
    TOP_K = 0x80
    TOP_P = 0x100
    MIN_P = 0x200
    TOP_K_LOGPROBS = 0x400
    STOCHASTIC_VERIFY_GREEDY_DRAFT = 0x800

    @classmethod
    def all(cls) -> "Indicator":

        return cls((1 << len(cls.__members__)) - 1)

    @classmethod
    def stochastic(cls) -> "Indicator":

        return cls.TEMPERATURE | cls.TOP_K | cls.TOP_P | cls.MIN_P

    @classmethod
    def maximal(cls) -> "Indicator":

        return cls.all() ^ cls.GREEDY

    @classmethod
    def random(cls) -> "Indicator":

        indicator = cls(_random.randint(0, int(cls.all())))

        if indicator & cls.stochastic():

            indicator &= cls.maximal()

        return indicator

    @classmethod
    def default(cls) -> "Indicator":

        return cls(0)

    @classmethod
    def repetition(cls) -> "Indicator":

        return cls.MULTIPLICATIVE | cls.FREQUENCY | cls.PRESENCE

    @classmethod
    def indirection(cls) -> "Indicator":

        return cls.GRAMMAR | cls.repetition() | cls.BIAS

    @classmethod
    def cumulative(cls) -> "Indicator":

        return cls.TOP_K | cls.TOP_P | cls.MIN_P

    @classmethod
    def from_params(
        cls,
        grammar: bool = False,
        multiplicative: float = 1.0,
        frequency: float = 0.0,
        presence: float = 0.0,
        logit_bias: bool = False,
        temperature: float = 1.0,
        top_k: int = MAX_K,
        top_p: float = 1.0,
        min_p: float = 0.0,
        top_k_logprobs: int = 0,
        greedy_draft: bool = False,
    ) -> "Indicator":
        """Derives the bits from sampling parameters (reference ``core/flags.py:150-184``)."""

        greedy = top_k == 1

        bits = [
            grammar,
            multiplicative != 1.0,
            frequency != 0.0,
            presence != 0.0,
            logit_bias,
            temperature != 1.0,
            greedy,
            1 < top_k < MAX_K,
            not greedy and (0.0 < top_p < 1.0),
            not greedy and (0.0 < min_p < 1.0),
            not greedy and (0 < top_k_logprobs <= MAX_K),
            not greedy and greedy_draft,
        ]

        return cls(sum(int(bool(b)) << i for i, b in enumerate(bits)))

    def greedy(self) -> "Indicator":

        mask = (
            Indicator.all()
            ^ Indicator.stochastic()
            ^ Indicator.TOP_K_LOGPROBS
            ^ Indicator.STOCHASTIC_VERIFY_GREEDY_DRAFT
        )

        return (self & mask) | Indicator.GREEDY

    def disable(self, value: "Indicator") -> "Indicator":

        return self & (Indicator.all() ^ value)

    def resolve(self, mode: SamplingMode) -> "Indicator":

        if mode == SamplingMode.MINIMAL:

            return Indicator.GREEDY

        if mode == SamplingMode.MAXIMAL:

            return Indicator.maximal()

        if mode == SamplingMode.GREEDY:

            return self.greedy()

        if mode == SamplingMode.NON_GRAMMAR:

            return self.disable(Indicator.GRAMMAR)

        raise ValueError(f"unknown sampling mode {mode}")


def indexify(selectors: List[bool]) -> List[int]:

    return list(compress(range(len(selectors)), selectors))


def _host_kwargs(pinned: bool) -> dict:

    if pinned and torch.cuda.is_available():

        return dict(device="cpu", pin_memory=True)

    return dict(device="cpu")


@dataclass(eq=False, kw_only=True)
class ScopedIndicators(SliceBuffer):

    # The verifier's indicators, one per request.
    target: List[Indicator]

    # The drafter's indicators, one per request.
    draft: List[Indicator]

    @classmethod
    def shared(cls, size: int, timesteps: int, factory: Callable[[], Indicator]) -> "ScopedIndicators":

        target = [factory() for _ in range(size)]

        return cls(target=target, draft=target.copy(), layout=Layout(size, timesteps))

    @classmethod
    def random(cls, size: int, timesteps: int) -> "ScopedIndicators":

        return cls.shared(size=size, timesteps=timesteps, factory=Indicator.random)

    @classmethod
    def default(cls, size: int, timesteps: int) -> "ScopedIndicators":

        return cls.shared(size=size, timesteps=timesteps, factory=Indicator.default)

    @classmethod
    def from_pairs(cls, pairs, timesteps: int) -> "ScopedIndicators":

        target, draft = list(zip(*pairs))

        return cls(target=list(target), draft=list(draft), layout=Layout(len(target), timesteps))

    @classmethod
    def from_values(cls, size: int, timesteps: int, target, draft=None) -> "ScopedIndicators":

        layout = Layout(size, timesteps)

        if isinstance(target, list) and draft is None:

            return cls(target=target, draft=target.copy(), layout=layout)

        if isinstance(target, list) and isinstance(draft, list):

            return cls(target=target, draft=draft, layout=layout)

        if isinstance(target, Indicator) and draft is None:

            return cls(target=[target] * size, draft=[target] * size, layout=layout)

        if isinstance(target, Indicator) and isinstance(draft, Indicator):

            return cls(target=[target] * size, draft=[draft] * size, layout=layout)

        raise ValueError("unrecognized target or draft indicator(s)")

    @classmethod
    def from_params(
        cls,
        size: int,
        timesteps: int,
        multiplicative: Optional[List[float]] = None,
        frequency: Optional[List[float]] = None,
        presence: Optional[List[float]] = None,
        biases: Optional[List[Optional[dict]]] = None,
        temperature: Optional[List[float]] = None,
        top_k: Optional[List[int]] = None,
        top_p: Optional[List[float]] = None,
        min_p: Optional[List[float]] = None,
        top_logprobs: Optional[List[int]] = None,
        bitmasks: Optional[List[Optional[Tensor]]] = None,
        greedy_drafts=False,
    ) -> "ScopedIndicators":
        """Per-request indicators from parameter lists (reference ``core/flags.py:309-362``).

        As in the reference, an omitted ``temperature`` list defaults every entry to 0.0, which
        sets ``TEMPERATURE``; callers pass temperatures explicitly.
        """

        if top_k and any(k > MAX_K for k in top_k):

            raise ValueError(f"`top_k` greater than {MAX_K} is not supported")

        def fill(value):

            return repeat(value, size)

        drafter = greedy_drafts if isinstance(greedy_drafts, list) else list(fill(greedy_drafts))

        iterator = zip(
            (m is not None for m in bitmasks) if bitmasks else fill(False),
            multiplicative or fill(1.0),
            frequency or fill(0.0),
            presence or fill(0.0),
            (b is not None for b in biases) if biases else fill(False),
            temperature or fill(0.0),
            top_k or fill(MAX_K),
            top_p or fill(1.0),
            min_p or fill(0.0),
            top_logprobs or fill(0),
            drafter,
        )

        target = [Indicator.from_params(*args) for args in iterator]

        draft = [
            indicator.greedy() if greedy else indicator.disable(Indicator.TOP_K_LOGPROBS)
            for greedy, indicator in zip(drafter, target)
        ]

        return cls(target=target, draft=draft, layout=Layout(size, timesteps))

    @property
    def greedy_draft(self) -> bool:

        return all(Indicator.GREEDY in v for v in self.draft)

    @property
    def greedy_target(self) -> bool:

        return all(Indicator.GREEDY in v for v in self.target)

    @property
    def has_stochastic_draft(self) -> bool:

        return any(Indicator.GREEDY not in v for v in self.draft)

    @property
    def has_stochastic_target(self) -> bool:

        return any(Indicator.GREEDY not in v for v in self.target)

    @property
    def stochastic_selectors(self):

        return [
            (Indicator.GREEDY not in t, Indicator.GREEDY not in d)
            for t, d in zip(self.target, self.draft)
        ]

    def as_tensor(self, pinned: bool = False, host: bool = False) -> Tensor:

        values = [[int(v) for v in self.target], [int(v) for v in self.draft]]
        kwargs = _host_kwargs(True) if pinned else (dict(device="cpu") if host else {})

        return torch.tensor(values, dtype=torch.int32, **kwargs).to(U16)

    def subset(self, indices: List[int]) -> "ScopedIndicators":
        """The (target, draft) pairs of rows `indices`, in that order, as a new instance with the
        same timestep extent."""

        pairs = [(self.target[i], self.draft[i]) for i in indices]

        if not pairs:

            return ScopedIndicators(target=[], draft=[], layout=Layout(rows=0, cols=self.layout.cols))

        return ScopedIndicators.from_pairs(pairs, timesteps=self.layout.cols)

    def update(self, other: "ScopedIndicators", positions: Optional[List[int]] = None):
        """Row j of `other` replaces row positions[j]; without positions, row j replaces row j
        (`other` then covers the leading rows)."""

        rows = positions if positions else range(len(other.target))

        for row, target, draft in zip(rows, other.target, other.draft):

            self.target[row] = target
            self.draft[row] = draft

        return self


@dataclass(eq=False, kw_only=True)
class Flags(SliceBuffer):

    """The indicators of every request, packed as ``[B, 2]`` uint16 with stride ``[1, B]``."""

    # The readable indicators.
    indicators: ScopedIndicators

    # Host-side packed copy.
    pinned: Tensor

    # Device-side packed copy read by the kernels.
    packed: Tensor

    @classmethod
    def from_scoped(cls, indicators: ScopedIndicators, device: Optional[torch.device] = None) -> "Flags":

        layout = Layout(indicators.layout.rows, indicators.layout.cols)
        pinned = indicators.as_tensor(pinned=True)
        packed = pinned.to(device or torch.get_default_device())

        return cls(indicators=indicators, pinned=pinned.T, packed=packed.T, layout=layout)

    @classmethod
    def random(cls, size: int, timesteps: int, device=None) -> "Flags":

        return cls.from_scoped(ScopedIndicators.random(size=size, timesteps=timesteps), device)

    @classmethod
    def default(cls, size: int, timesteps: int, device=None) -> "Flags":

        return cls.from_scoped(ScopedIndicators.default(size=size, timesteps=timesteps), device)

    @classmethod
    def from_values(cls, size: int, timesteps: int, target, draft=None, device=None) -> "Flags":

        scoped = ScopedIndicators.from_values(size=size, timesteps=timesteps, target=target, draft=draft)

        return cls.from_scoped(scoped, device)

    @classmethod
    def resolve(cls, size: int, timesteps: int, target=None, draft=None, random: bool = False,
                device=None) -> "Flags":

        if target is None:

            return (cls.random if random else cls.default)(size, timesteps, device)

        return cls.from_values(size, timesteps, target, draft, device)

    @property
    def target(self) -> Tensor:

        return plain_view(self.packed, 0)

    @property
    def draft(self) -> Tensor:

        return plain_view(self.packed, 1)

    def subset(self, host_indices: List[int], device_indices: Tensor) -> "Flags":

        selector = torch.tensor(host_indices, device="cpu")
        pinned = self.pinned.to(torch.int32).index_select(0, selector).to(U16)
        packed = self.packed.to(torch.int32).index_select(0, device_indices).to(U16)

        # keep the [B, 2] / stride [1, B] layout
        packed = packed.T.contiguous().T

        return Flags(
            indicators=self.indicators.subset(host_indices),
            pinned=pinned.T.contiguous().T,
            packed=packed,
            layout=Layout(len(host_indices), self.layout.cols),
        )

    @property
    def all_greedy(self) -> bool:
        """Every request greedy in both scopes (reference ``core/flags.py:535-537``). Read from the
        host mirror that the constructors, `subset` and `update` keep equal to the readable lists:
        one vectorized test of bit 0x40 over the [B, 2] words instead of an enum test per word
        (about 7 µs against 500 at 512 slots, on every drafting call); a first target word without
        the bit answers at once, as the lists' own test does."""

        target = self.indicators.target

        if target and Indicator.GREEDY not in target[0]:

            return False

        if self.pinned.device.type != "cpu":

            return self.indicators.greedy_target and self.indicators.greedy_draft

        return bool((self.pinned.numpy() & int(Indicator.GREEDY)).all())

    def selectors(self, flag: Indicator) -> Tensor:

        return torch.tensor([(flag in v) for v in self.indicators.target], dtype=BOOL)

    def update(self, indicators: ScopedIndicators, positions: Optional[List[int]], stream=None) -> "Flags":
        """Installs `indicators` at rows `positions` (the leading rows when None): the readable
        lists, the pinned [B, 2] mirror, and an asynchronous copy of the mirror to the device words
        the kernels read (on `stream` when given): the leading rows, or for scattered positions the
        whole mirror in one copy (its other rows already equal their device words, so they are
        rewritten unchanged) instead of one copy per row."""

        self.indicators.update(indicators, positions)
        words = indicators.as_tensor(host=True).T  # [n, 2]: (target, draft) of each new row
        n = words.size(0)
        rows = list(positions) if positions else list(range(n))
        leading = rows == list(range(n))

        if leading:

            self.pinned[:n].copy_(words)

        else:

            index = torch.tensor(rows, dtype=I64)
            self.pinned.view(I16).index_copy_(0, index, words.view(I16))

        with (stream or nullcontext()):

            if leading:

                # one strided copy covers the leading rows of both columns
                self.packed[:n].copy_(self.pinned[:n], non_blocking=True)

            else:

                self.packed.copy_(self.pinned, non_blocking=True)

        return self
