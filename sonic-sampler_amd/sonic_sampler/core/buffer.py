"""Device-resident per-request sampling state (reference ``core/buffer.py:55-1352``).

Member names, shapes, dtypes and strides match the reference so that an engine built on it can
switch without changes:

======================================  ======================  ========
member                                  shape                   dtype
======================================  ======================  ========
``flags.packed``                        ``[B, 2]`` (stride 1,B) uint16
``temperature`` ``top_p`` ``min_p``     ``[B]``                 bfloat16
``top_k`` ``top_logprobs``              ``[B]``                 int32
``bias``                                ``[B, V]``              bfloat16
``repetition.{multiplicative,...}``     ``[B]``                 bfloat16
``repetition.counts.{context,decode}``  ``[B, V]``              int32
``grammar``                             ``[B, T, ceil(V/32)]``  uint32
``weights.gumbel.{target,draft}``       ``[B, T, V]``           bfloat16
``weights.uniform``                     ``[B, T]``              bfloat16
======================================  ======================  ========

``random`` fills every parameter whose indicator bit is off with its *neutral* value (temperature
1, top-k 128, top-p 1, min-p 0, zero penalties and bias, all-ones grammar), so that applying a
processor to a row that does not enable it is an exact no-op.
"""

from __future__ import annotations

import random as _random

from contextlib import nullcontext
from dataclasses import dataclass
from itertools import compress
from typing import List, Optional, Tuple

import torch

from torch import Generator, Tensor

from sonic_sampler.base import Layout, PrefixContiguousTensor, SliceBuffer, DEFAULT_TOP_LOGPROBS
from sonic_sampler.base.tensor import prefix_contiguous
from sonic_sampler.core.flags import Flags, Indicator, ScopedIndicators
from sonic_sampler.ops import MAX_K


__all__ = ["SamplingBuffers"]

I32 = torch.int32
I64 = torch.int64
U32 = torch.uint32
BOOL = torch.bool
BF16 = torch.bfloat16
TINY: float = torch.finfo(BF16).tiny


def cdiv(a: int, b: int) -> int:

    return -(-a // b)


def _pinned(shape, dtype) -> Tensor:

    return torch.empty(shape, dtype=dtype, device="cpu", pin_memory=torch.cuda.is_available())


def _device(device) -> torch.device:

    if device is not None:

        return torch.device(device)

    if torch.cuda.is_available():

        return torch.device(f"cuda:{torch.cuda.current_device()}")

    return torch.device("cpu")


@dataclass(eq=False, kw_only=True)
class GumbelNoise(SliceBuffer):

    # log(Exp(1)) noise for verification, [B, T, V].
    target: PrefixContiguousTensor

    # log(Exp(1)) noise for drafting, [B, T, V].
    draft: PrefixContiguousTensor

    @classmethod
    def empty(cls, size: int, timesteps: int, vocab_size: int) -> "GumbelNoise":

        pair = prefix_contiguous(torch.empty((2, size, timesteps, vocab_size), dtype=BF16))

        return cls(target=pair[0], draft=pair[1], layout=Layout(size, timesteps))

    @property
    def device(self) -> torch.device:

        return self.target.device

    @property
    def vocab_size(self) -> int:

        return self.target.size(-1)

    def subset(self, indices: Tensor) -> "GumbelNoise":

        return GumbelNoise(
            target=prefix_contiguous(self.target.index_select(0, indices)),
            draft=prefix_contiguous(self.draft.index_select(0, indices)),
            layout=Layout(indices.size(0), self.layout.cols),
        )

    def populate(self, row, generator: Optional[Generator], prefill: bool = False, draft: bool = False):

        if prefill:

            tensors = (self.target[row, 0], self.draft[row]) if draft else (self.target[row, 0],)

        else:

            tensors = ((self.draft if draft else self.target)[row],)

        for weight in tensors:

            weight.exponential_(1.0, generator=generator).log_()

        return self

    def update(self, targets: List[Optional[Tensor]], positions: Optional[List[int]] = None, stream=None):

        if any(selectors := [t is not None for t in targets]):

            iterator = zip(positions, targets) if positions else enumerate(targets)

            with (stream or nullcontext()):

                for i, target in compress(iterator, selectors):

                    self.target[i].copy_(target, non_blocking=True)

        return self

    def stage_weights(self, indices: Tensor, indicator: Tensor, stream=None):
        """Copies draft noise into target noise for the rows in ``indices`` whose draft indicator
        is stochastic, so verification sees the noise the drafter used (reference
        ``core/buffer.py:151-159``, ``ops/copy.py:21-127``)."""

        with (stream or nullcontext()):

            rows = indices.to(I64)
            stochastic = (indicator.to(I32).index_select(0, rows) & int(Indicator.GREEDY)) == 0
            keep = rows[stochastic]
            self.target.index_copy_(0, keep, self.draft.index_select(0, keep))

        return self


@dataclass(eq=False, kw_only=True)
class StochasticWeights(SliceBuffer):

    # U(0, 1] for the acceptance test, [B, T].
    uniform: PrefixContiguousTensor

    # Gumbel-max noise.
    gumbel: GumbelNoise

    @classmethod
    def empty(cls, size: int, timesteps: int, vocab_size: int) -> "StochasticWeights":

        uniform = prefix_contiguous(torch.empty((size, timesteps), dtype=BF16))

        return cls(uniform=uniform, gumbel=GumbelNoise.empty(size, timesteps, vocab_size),
                   layout=Layout(size, timesteps))

    @classmethod
    def random(cls, size: int, timesteps: int, vocab_size: int, generator=None) -> "StochasticWeights":

        weights = cls.empty(size, timesteps, vocab_size)

        weights.gumbel.target.exponential_(1.0, generator=generator).log_()
        weights.gumbel.draft.exponential_(1.0, generator=generator).log_()
        weights.uniform.uniform_(TINY, 1.0, generator=generator)

        return weights

    @property
    def device(self) -> torch.device:

        return self.gumbel.device

    def subset(self, indices: Tensor) -> "StochasticWeights":

        return StochasticWeights(
            uniform=prefix_contiguous(self.uniform.index_select(0, indices)),
            gumbel=self.gumbel.subset(indices),
            layout=Layout(indices.size(0), self.layout.cols),
        )

    def refresh(self, position, generator, prefill: bool, draft: bool) -> None:

        row = slice(None) if position is None else position

        self.gumbel.populate(row=row, generator=generator, prefill=prefill, draft=draft)

        if not prefill:

            self.uniform[row].uniform_(TINY, 1.0, generator=generator)


@dataclass(eq=False, kw_only=True)
class TokenCounts(SliceBuffer):

    # Prompt token histogram, [B, V].
    context: Tensor

    # Generated token histogram, [B, V]; updated by the kernels under `update_counts`.
    decode: Tensor

    # Host staging for context histograms.
    pinned: Tensor

    @classmethod
    def zeros(cls, size: int, timesteps: int, vocab_size: int) -> "TokenCounts":

        both = torch.zeros((2, size, vocab_size), dtype=I32)

        return cls(context=both[0], decode=both[1], pinned=_pinned((size, vocab_size), I32),
                   layout=Layout(size, timesteps))

    def subset(self, indices: Tensor) -> "TokenCounts":

        return TokenCounts(
            context=self.context.index_select(0, indices),
            decode=self.decode.index_select(0, indices),
            pinned=self.pinned.narrow(0, 0, indices.size(0)),
            layout=Layout(indices.size(0), self.layout.cols),
        )

    def update(self, counts: List[Tuple[Tensor, Tensor]], positions=None, stream=None):

        iterator = zip(positions, counts) if positions else enumerate(counts)

        with (stream or nullcontext()):

            for i, (context, decode) in iterator:

                self.context[i].copy_(context, non_blocking=True)
                self.decode[i].copy_(decode, non_blocking=True)

        return self

    def increment(self, tokens: Tensor) -> "TokenCounts":
        """Adds one count per token (testing helper; kernels update under `update_counts`)."""

        self.decode.scatter_add_(1, tokens.to(I64), torch.ones_like(tokens, dtype=I32))

        return self


@dataclass(eq=False, kw_only=True)
class RepetitionPenalties(SliceBuffer):

    counts: TokenCounts
    frequency: Tensor
    presence: Tensor
    multiplicative: Tensor
    pinned: Tensor

    @classmethod
    def default(cls, size: int, timesteps: int, vocab_size: int) -> "RepetitionPenalties":

        fp = torch.zeros((2, size), dtype=BF16)

        return cls(
            counts=TokenCounts.zeros(size, timesteps, vocab_size),
            frequency=fp[0],
            presence=fp[1],
            multiplicative=torch.ones(size, dtype=BF16),
            pinned=_pinned((3, size), BF16).T,
            layout=Layout(size, timesteps),
        )

    def subset(self, indices: Tensor) -> "RepetitionPenalties":

        return RepetitionPenalties(
            counts=self.counts.subset(indices),
            frequency=self.frequency.index_select(0, indices),
            presence=self.presence.index_select(0, indices),
            multiplicative=self.multiplicative.index_select(0, indices),
            pinned=self.pinned.narrow(0, 0, indices.size(0)),
            layout=Layout(indices.size(0), self.layout.cols),
        )


@dataclass(eq=False, kw_only=True)
class PinnedRelay(SliceBuffer):

    bias: Tensor
    float_values: Tensor
    int_values: Tensor

    @classmethod
    def default(cls, size: int, timesteps: int, vocab_size: int) -> "PinnedRelay":

        return cls(
            bias=_pinned((size, vocab_size), BF16),
            float_values=_pinned((3, size), BF16).T,
            int_values=_pinned((2, size), I32).T,
            layout=Layout(size, timesteps),
        )


def ensure_top_logprobs(indicators, maximum: int):

    if indicators and not maximum:

        if isinstance(indicators, list):

            return [j.disable(Indicator.TOP_K_LOGPROBS) for j in indicators]

        return indicators.disable(Indicator.TOP_K_LOGPROBS)

    return indicators


@dataclass(eq=False, kw_only=True)
class SamplingBuffers(SliceBuffer):

    grammar: PrefixContiguousTensor
    repetition: RepetitionPenalties
    bias: Tensor
    temperature: Tensor
    top_k: Tensor
    top_p: Tensor
    min_p: Tensor
    top_logprobs: Tensor
    pinned: PinnedRelay
    weights: StochasticWeights
    flags: Flags

    @classmethod
    def default(
        cls,
        size: int,
        timesteps: int,
        vocab_size: int,
        device: Optional[torch.device] = None,
        bounded: bool = True,
        noise: bool = True,
    ) -> "SamplingBuffers":
        """A neutral instance (reference ``core/buffer.py:938-986``).

        ``noise=False`` (an addition) leaves the Gumbel / uniform planes uninitialised instead of
        drawing them, for callers that populate them (or use Philox noise) anyway.
        """

        target = _device(device)

        with torch.device(target):

            grammar = torch.full((size, timesteps, cdiv(vocab_size, 32)), -1, dtype=I32).view(U32)

            return cls(
                grammar=prefix_contiguous(grammar),
                repetition=RepetitionPenalties.default(size, timesteps, vocab_size),
                bias=torch.zeros((size, vocab_size), dtype=BF16),
                temperature=torch.ones(size, dtype=BF16),
                top_k=torch.full((size,), MAX_K if bounded else vocab_size, dtype=I32),
                top_p=torch.ones(size, dtype=BF16),
                min_p=torch.zeros(size, dtype=BF16),
                top_logprobs=torch.zeros(size, dtype=I32),
                pinned=PinnedRelay.default(size, timesteps, vocab_size),
                weights=(StochasticWeights.random if noise else StochasticWeights.empty)(
                    size, timesteps, vocab_size),
                flags=Flags.default(size, timesteps, device=target),
                layout=Layout(size, timesteps),
            )

    @classmethod
    def random(
        cls,
        size: int,
        timesteps: int,
        vocab_size: int,
        indicators=None,
        device: Optional[torch.device] = None,
        seed: Optional[int] = None,
        bounded: bool = True,
        max_top_logprobs: int = DEFAULT_TOP_LOGPROBS,
    ) -> "SamplingBuffers":
        """A randomly populated instance for tests (reference ``core/buffer.py:819-936``).

        Values are drawn on the CPU from a generator seeded with ``seed`` and then moved to
        ``device``, so the same seed gives the same buffers on every host. Parameters whose
        indicator bit is off get their neutral value.
        """

        target = _device(device)
        gen = torch.Generator("cpu")

        if seed is not None:

            _random.seed(seed)
            gen.manual_seed(seed)

        indicators = ensure_top_logprobs(indicators, max_top_logprobs)
        flags = Flags.resolve(size, timesteps, target=indicators, random=True, device=target)
        on = lambda bit: flags.selectors(bit)  # noqa: E731

        def u(lo, hi, n=size):

            return torch.empty(n, dtype=torch.float32).uniform_(lo, hi, generator=gen).to(BF16)

        upper = MAX_K if bounded else vocab_size
        words = cdiv(vocab_size, 32)

        counts = torch.randint(0, 32, (2, size, vocab_size), dtype=I32, generator=gen)
        grammar = torch.randint(-(2 ** 31), 2 ** 31 - 1, (size, timesteps, words), dtype=I32, generator=gen)
        grammar.masked_fill_(~on(Indicator.GRAMMAR)[:, None, None], -1)

        frequency = u(-2, 2).masked_fill_(~on(Indicator.FREQUENCY), 0)
        presence = u(-2, 2).masked_fill_(~on(Indicator.PRESENCE), 0)
        multiplicative = u(0.5, 1.5).masked_fill_(~on(Indicator.MULTIPLICATIVE), 1)

        temperature = u(0.4, 1.25).masked_fill_(~on(Indicator.TEMPERATURE), 1)
        top_k = (
            torch.randint(2, upper, (size,), dtype=I32, generator=gen)
            .masked_fill_(on(Indicator.GREEDY), 1)
            .masked_fill_(~on(Indicator.TOP_K) & ~on(Indicator.GREEDY), upper)
        )
        top_p = u(0.5, 1.0).masked_fill_(~on(Indicator.TOP_P), 1)
        min_p = u(0.01, 0.5).masked_fill_(~on(Indicator.MIN_P), 0)

        bias = torch.empty((size, vocab_size), dtype=torch.float32).uniform_(-2.5, 2.5, generator=gen).to(BF16)
        drop = torch.randint(0, 2, (size, vocab_size), dtype=I32, generator=gen).bool()
        bias.masked_fill_(drop | ~on(Indicator.BIAS)[:, None], 0)

        if max_top_logprobs > 0:

            top_logprobs = (
                torch.randint(1, max_top_logprobs + 1, (size,), dtype=I32, generator=gen)
                .masked_fill_(~on(Indicator.TOP_K_LOGPROBS), 0)
            )

        else:

            top_logprobs = torch.zeros(size, dtype=I32)

        weights = StochasticWeights.empty(size, timesteps, vocab_size)
        weights.gumbel.target.exponential_(1.0, generator=gen).log_()
        weights.gumbel.draft.exponential_(1.0, generator=gen).log_()
        weights.uniform.uniform_(TINY, 1.0, generator=gen)

        move = lambda t: t.to(target)  # noqa: E731

        with torch.device(target):

            repetition = RepetitionPenalties(
                counts=TokenCounts(
                    context=move(counts[0]),
                    decode=move(counts[1]),
                    pinned=_pinned((size, vocab_size), I32),
                    layout=Layout(size, timesteps),
                ),
                frequency=move(frequency),
                presence=move(presence),
                multiplicative=move(multiplicative),
                pinned=_pinned((3, size), BF16).T,
                layout=Layout(size, timesteps),
            )

            pair = prefix_contiguous(
                torch.stack([weights.gumbel.target, weights.gumbel.draft]).to(target)
            )

            moved_weights = StochasticWeights(
                uniform=prefix_contiguous(move(weights.uniform)),
                gumbel=GumbelNoise(target=pair[0], draft=pair[1], layout=Layout(size, timesteps)),
                layout=Layout(size, timesteps),
            )

            return cls(
                grammar=prefix_contiguous(move(grammar).view(U32)),
                repetition=repetition,
                bias=move(bias),
                temperature=move(temperature),
                top_k=move(top_k),
                top_p=move(top_p),
                min_p=move(min_p),
                top_logprobs=move(top_logprobs),
                pinned=PinnedRelay.default(size, timesteps, vocab_size),
                weights=moved_weights,
                flags=flags,
                layout=Layout(size, timesteps),
            )

    @property
    def indicators(self) -> ScopedIndicators:

        return self.flags.indicators

    @property
    def device(self) -> torch.device:

        return self.weights.device

    @property
    def vocab_size(self) -> int:

        return self.weights.gumbel.vocab_size

    def subset(self, host_indices: List[int], device_indices: Tensor) -> "SamplingBuffers":
        """Gathers the rows ``host_indices`` into a new instance (reference ``:1003-1024``)."""

        return SamplingBuffers(
            grammar=prefix_contiguous(self.grammar.index_select(0, device_indices)),
            repetition=self.repetition.subset(device_indices),
            bias=self.bias.index_select(0, device_indices),
            temperature=self.temperature.index_select(0, device_indices),
            top_k=self.top_k.index_select(0, device_indices),
            top_p=self.top_p.index_select(0, device_indices),
            min_p=self.min_p.index_select(0, device_indices),
            top_logprobs=self.top_logprobs.index_select(0, device_indices),
            pinned=self.pinned[:device_indices.size(0)],
            weights=self.weights.subset(device_indices),
            flags=self.flags.subset(host_indices=host_indices, device_indices=device_indices),
            layout=Layout(len(host_indices), self.layout.cols),
        )

    def step_grammar(self, bitmasks, positions=None, timestep=None, stream=None, event=None):

        if bitmasks and any(selectors := [m is not None for m in bitmasks]):

            iterator = positions or range(len(bitmasks))

            with (stream or nullcontext()):

                for k, i in enumerate(iterator):

                    if selectors[k]:

                        target = self.grammar[i] if timestep is None else self.grammar[i, timestep]
                        target.copy_(bitmasks[k].view(target.dtype), non_blocking=True)

                if event:

                    event.record(stream)

        return self
