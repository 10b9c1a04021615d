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


def _rows(positions: Optional[List[int]], size: int) -> List[int]:
    """The rows an update touches: `positions`, or every row in order."""

    return list(positions) if positions else list(range(size))


def _present(items, positions: Optional[List[int]] = None):
    """(row, item) for every item that is not None: item j belongs to row positions[j], or to row
    j when no positions are given (the parallel-list convention of every population call)."""

    rows = positions if positions else range(len(items))

    return [(row, item) for row, item in zip(rows, items) if item is not None]


def _log_exponential_(plane: Tensor, generator: Optional[Generator]) -> None:
    """Fills `plane` with log(Exp(1)) draws, the Gumbel noise the kernels subtract."""

    plane.exponential_(1.0, generator=generator).log_()


def _send(device_rows: Tensor, host_rows: Tensor, positions: Optional[List[int]], stream=None) -> None:
    """Non-blocking host -> device copy of rows `positions` (all rows when None) on `stream`."""

    with (stream or nullcontext()):

        if positions:

            for i in positions:

                device_rows[i].copy_(host_rows[i], non_blocking=True)

        else:

            device_rows.copy_(host_rows, non_blocking=True)


def _stage(host_rows: Tensor, values: Tensor, positions: Optional[List[int]]) -> None:
    """Writes `values` ([n, ...], host) into the staging rows `positions` (all rows when None)."""

    if positions:

        host_rows.index_copy_(0, torch.tensor(positions, dtype=I64), values.to(host_rows.dtype))

    else:

        host_rows.copy_(values)


def initialize_generator(seed: Optional[int], device) -> Optional[Generator]:
    """A generator on `device` seeded with `seed` (which also seeds Python's `random`), or None
    (reference ``core/buffer.py:673-682``)."""

    if seed is None:

        return None

    _random.seed(seed)

    return torch.Generator(device).manual_seed(seed)


def resolve_updates(size: int, generator=None, selectors=None, positions=None, prefill=False):
    """The weight refreshes one update performs, as (row or None, generator, (target, draft),
    prefill) tuples (reference ``core/buffer.py:166-192``): one whole-batch refresh for a shared
    generator without positions or selectors, else one refresh per row of `positions` (or of the
    batch) with its own generator, selector pair and prefill flag when lists are given."""

    shared = generator is None or isinstance(generator, Generator)

    if shared and not positions and not selectors and not isinstance(prefill, list):

        return [(None, generator, (True, True), bool(prefill))]

    if shared and not positions and not selectors and isinstance(prefill, list) and not prefill:

        return [(None, generator, (True, True), False)]

    rows = _rows(positions, size)
    gens = generator if isinstance(generator, list) else [generator] * len(rows)
    pairs = selectors if selectors else [(True, True)] * len(rows)
    flags = prefill if isinstance(prefill, list) and prefill else [bool(prefill)] * len(rows)

    return list(zip(rows, gens, pairs, flags))


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

    def planes(self, row, prefill: bool, draft: bool) -> List[Tensor]:
        """The noise one refresh of `row` redraws. At prefill a single logit row is sampled, so
        the verifier needs timestep 0 only, and a stochastic drafter all of its timesteps. During
        decoding a stochastic drafter's noise is redrawn (the verifier's was staged from it by
        stage_weights just before); with a greedy drafter the verifier's own noise is."""

        if not prefill:

            return [self.draft[row] if draft else self.target[row]]

        return [self.target[row, 0], self.draft[row]] if draft else [self.target[row, 0]]

    def populate(self, row, generator: Optional[Generator], prefill: bool = False, draft: bool = False):

        for plane in self.planes(row, prefill, draft):

            _log_exponential_(plane, generator)

        return self

    def update(self, targets: List[Optional[Tensor]], positions: Optional[List[int]] = None, stream=None):
        """Carried-over drafter noise ([T, V] device tensors, None to leave a row alone) replaces
        the verifier's noise of its row (just-in-time batching, reference
        ``core/buffer.py:121-149``)."""

        moves = _present(targets, positions)

        if moves:

            with (stream or nullcontext()):

                for row, noise in moves:

                    self.target[row].copy_(noise, non_blocking=True)

        return self

    def stage_weights(self, indices: Tensor, indicator: Tensor, stream=None):
        """Copies draft noise into target noise for the rows in ``indices`` whose draft indicator
        is stochastic, so verification sees the noise the drafter used (reference
        ``core/buffer.py:151-159``, ``ops/copy.py:21-127``), with the library's
        ``ss_indexed_copy`` kernel. The planes must be device-resident: there is no host path."""

        if self.target.device.type != "cuda":

            raise RuntimeError("stage_weights copies with the ss_indexed_copy kernel: the noise planes "
                               f"must be on a GPU, not {self.target.device}")

        from sonic_sampler import _native

        with (stream or nullcontext()):

            _native.indexed_copy(self.draft, self.target, indices, indicator)

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
        """Redraws row `position` (every row when None): its Gumbel noise (GumbelNoise.planes),
        and outside prefill its acceptance uniforms on [TINY, 1), TINY keeping log(u) finite. A
        prefill row has nothing to verify yet."""

        rows = slice(None) if position is None else position
        self.gumbel.populate(row=rows, generator=generator, prefill=prefill, draft=draft)

        if prefill:

            return

        self.uniform[rows].uniform_(TINY, 1.0, generator=generator)

    def update(self, generator=None, selectors=None, targets=None, positions=None, prefill=False,
               stream=None, event=None) -> "StochasticWeights":
        """Redraws the noise between iterations (reference ``core/buffer.py:252-311``): every
        refresh of ``resolve_updates`` whose target selector is set redraws its row (prefill: the
        target noise of step 0, plus the draft noise when drafting is stochastic; decode: the
        selected plane and the uniforms), then ``targets`` (device noise rows from the drafter, at
        ``positions`` or in order) replace the target noise of every row that is not in prefill.
        The reference skips ``targets`` altogether whenever ``prefill`` is a non-empty list, which
        is how its just-in-time guide passes it; this follows the guide's per-request contract
        (docs/just-in-time.md:174-199)."""

        with (stream or nullcontext()):

            for row, rng, (target, draft), initial in resolve_updates(
                    self.layout.rows, generator, selectors, positions, prefill):

                if target:

                    self.refresh(position=row, generator=rng, prefill=initial, draft=draft)

            if targets:

                # carried noise replaces the verifier's on decode rows only (a prefill row has
                # nothing carried); `prefill` may be one flag or one per row
                initial = prefill if isinstance(prefill, list) and prefill else [bool(prefill)] * len(targets)
                decode = [None if first else noise for noise, first in zip(targets, initial)]
                # already on `stream`: a torch stream context cannot be entered twice
                self.gumbel.update(targets=decode, positions=positions)

            if event is not None:

                event.record(stream)

        return self

    def step(self, positions: List[int], scoped: ScopedIndicators, indicator: Tensor,
             indices: Optional[Tensor] = None, generator=None, stream=None, event=None) -> None:
        """After a decode iteration (reference ``core/buffer.py:313-344``): stage the draft noise
        of the device rows ``indices`` into the target noise when some drafting is stochastic,
        then redraw the noise of ``positions``."""

        if indices is not None and scoped.has_stochastic_draft:

            self.gumbel.stage_weights(indices=indices, indicator=indicator, stream=stream)

        self.update(generator=generator, selectors=scoped.stochastic_selectors, positions=positions,
                    stream=stream, event=event)


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

    @classmethod
    def random(cls, size: int, timesteps: int, vocab_size: int, generator=None) -> "TokenCounts":
        """Counts drawn uniformly from [0, 32) (reference ``core/buffer.py:359-375``)."""

        both = torch.randint(0, 32, (2, size, vocab_size), dtype=I32, generator=generator)

        return cls(context=both[0], decode=both[1], pinned=_pinned((size, vocab_size), I32),
                   layout=Layout(size, timesteps))

    def populate(self, encodings: List[Tensor], positions: List[int]) -> "TokenCounts":
        """Histograms each prompt (host int64 token ids) into the staging row of its position."""

        for i, tokens in zip(positions, encodings):

            row = self.pinned[i].zero_()
            row.scatter_add_(0, tokens.to(I64), torch.ones(tokens.numel(), dtype=I32))

        return self

    def allocate(self, encodings: List[Tensor], positions: List[int], stream=None) -> "TokenCounts":
        """Request admission (reference ``core/buffer.py:434-457``): the prompts' histograms,
        staged in pinned memory, become the context counts of `positions`, and the decode counts
        of those rows restart at zero (one fill over all of them)."""

        self.populate(encodings, positions)
        _send(self.context, self.pinned, positions, stream)

        with (stream or nullcontext()):

            rows = torch.tensor(positions, dtype=I64).to(self.decode.device, non_blocking=True)
            self.decode.index_fill_(0, rows, 0)

        return self

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

    @classmethod
    def random(cls, size: int, timesteps: int, vocab_size: int, generator=None,
               flags: Optional[Flags] = None) -> "RepetitionPenalties":
        """Random counts and penalties (reference ``core/buffer.py:493-532``); with `flags`, rows
        whose indicator leaves a penalty off get its neutral value."""

        freq_pres = torch.empty((2, size), dtype=BF16).uniform_(-2, 2, generator=generator)
        mult = torch.empty(size, dtype=BF16).uniform_(0.5, 1.5, generator=generator)

        if flags is not None:

            freq_pres[0].masked_fill_(~flags.selectors(Indicator.FREQUENCY), 0)
            freq_pres[1].masked_fill_(~flags.selectors(Indicator.PRESENCE), 0)
            mult.masked_fill_(~flags.selectors(Indicator.MULTIPLICATIVE), 1)

        return cls(counts=TokenCounts.random(size, timesteps, vocab_size, generator),
                   frequency=freq_pres[0], presence=freq_pres[1], multiplicative=mult,
                   pinned=_pinned((3, size), BF16).T, layout=Layout(size, timesteps))

    def populate(self, multiplicative: List[float], frequency: List[float], presence: List[float],
                 positions: Optional[List[int]] = None) -> "RepetitionPenalties":
        """Stages (multiplicative, frequency, presence) per row in the pinned relay."""

        values = torch.tensor([multiplicative, frequency, presence], dtype=BF16).T
        _stage(self.pinned, values, positions)

        return self

    def transfer(self, positions: Optional[List[int]], stream=None) -> "RepetitionPenalties":
        """Sends the staged penalties of `positions` (all rows when None) to the device."""

        for column, member in enumerate((self.multiplicative, self.frequency, self.presence)):

            _send(member, self.pinned[:, column], positions, stream)

        return self

    def update(self, counts: List[Tuple[Tensor, Tensor]], multiplicative: List[float],
               frequency: List[float], presence: List[float], positions: Optional[List[int]] = None,
               stream=None) -> "RepetitionPenalties":
        """Between iterations (reference ``core/buffer.py:606-637``): new penalties and the given
        (context, decode) count rows at `positions` (or in order)."""

        self.populate(multiplicative, frequency, presence, positions).transfer(positions, stream)
        self.counts.update(counts, positions, stream)

        return self

    def allocate(self, encodings: List[Tensor], multiplicative: List[float], frequency: List[float],
                 presence: List[float], positions: List[int], stream=None) -> "RepetitionPenalties":
        """Request admission (reference ``core/buffer.py:639-670``): penalties plus the prompts'
        context histograms at `positions`."""

        self.populate(multiplicative, frequency, presence, positions).transfer(positions, stream)
        self.counts.allocate(encodings, positions, stream)

        return self

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

    def update_bias(self, biases: List[Optional[dict]], positions: Optional[List[int]]) -> "PinnedRelay":
        """Rebuilds the staged bias row of every position with a bias map ({token: bias}): the row
        is cleared, then the map's entries are written (rows without a map are left alone)."""

        for i, mapping in zip(_rows(positions, len(biases)), biases):

            if mapping:

                row = self.bias[i].zero_()
                row.index_copy_(0, torch.tensor(list(mapping.keys()), dtype=I64),
                                torch.tensor(list(mapping.values()), dtype=BF16))

        return self

    def populate(self, biases: List[Optional[dict]], temperature: List[float], top_k: List[int],
                 top_p: List[float], min_p: List[float], top_logprobs: List[int],
                 positions: Optional[List[int]] = None) -> "PinnedRelay":
        """Stages (temperature, top_p, min_p), (top_k, top_logprobs) and the bias maps of the
        given rows (reference ``core/buffer.py:738-764``)."""

        _stage(self.float_values, torch.tensor([temperature, top_p, min_p], dtype=BF16).T, positions)
        _stage(self.int_values, torch.tensor([top_k, top_logprobs], dtype=I32).T, positions)

        return self.update_bias(biases, positions) if any(biases) else self


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
        """Writes grammar bitmasks (host int32 words, pinned for an asynchronous copy): bitmasks[j]
        goes to row positions[j] (row j without positions) at `timestep`, or at every timestep when
        `timestep` is None; None entries leave their rows alone (reference
        ``core/buffer.py:1026-1052``, whose positional form reads bitmasks[positions[j]] and so
        needs a full-batch list; this one follows the parallel lists its callers pass). Nothing
        is issued, and `event` is not recorded, when every entry is None."""

        moves = _present(bitmasks or [], positions)

        if not moves:

            return self

        with (stream or nullcontext()):

            for row, words in moves:

                target = self.grammar[row] if timestep is None else self.grammar[row, timestep]
                target.copy_(words.view(target.dtype), non_blocking=True)

            if event:

                event.record(stream)

        return self

    def step_weights(self, positions: List[int], indices: Optional[Tensor] = None, generator=None,
                     stream=None, event=None) -> "SamplingBuffers":
        """After each decode iteration (reference ``core/buffer.py:1054-1096``): when some of
        `positions` samples stochastically, stage the drafter's noise of the device rows `indices`
        into the verifier's and redraw the noise of `positions`; a no-op for greedy targets."""

        scoped = self.flags.indicators.subset(positions)

        if scoped.has_stochastic_target:

            self.weights.step(positions=positions, scoped=scoped, indicator=self.flags.draft,
                              indices=indices, generator=generator, stream=stream, event=event)

        return self

    def transfer(self, positions: Optional[List[int]], stream=None, event=None) -> "SamplingBuffers":
        """Sends the staged bias rows, (temperature, top_p, min_p) and (top_k, top_logprobs) of
        `positions` (all rows when None) to the device, then records `event`."""

        relay = self.pinned
        _send(self.bias, relay.bias, positions, stream)

        for column, member in enumerate((self.temperature, self.top_p, self.min_p)):

            _send(member, relay.float_values[:, column], positions, stream)

        for column, member in enumerate((self.top_k, self.top_logprobs)):

            _send(member, relay.int_values[:, column], positions, stream)

        if event is not None:

            event.record(stream)

        return self

    def _admit(self, scoped: ScopedIndicators, positions, stream, biases, temperature, top_k, top_p,
               min_p, top_logprobs) -> None:
        """Indicators and the non-repetition parameters of `positions` into the relays."""

        self.flags.update(indicators=scoped, positions=positions, stream=stream)
        self.pinned.populate(biases=biases, temperature=temperature, top_k=top_k, top_p=top_p,
                             min_p=min_p, top_logprobs=top_logprobs, positions=positions)

    def update(self, counts: List[Tuple[Tensor, Tensor]], target_gumbel: List[Optional[Tensor]],
               multiplicative: List[float], frequency: List[float], presence: List[float],
               biases: List[Optional[dict]], temperature: List[float], top_k: List[int],
               top_p: List[float], min_p: List[float], top_logprobs: List[int],
               positions: Optional[List[int]] = None, indicators=None, greedy_drafts=False,
               prefill=False, bitmasks: Optional[List[Optional[Tensor]]] = None, stream=None,
               generator=None):
        """Refreshes every parameter of `positions` (or of the first len(counts) rows) between
        iterations (reference ``core/buffer.py:1139-1237``), for engines that compose the batch
        anew each step: grammar, indicators (from the parameters unless given as (target, draft)
        pairs), biases, sampling parameters, penalties with their counts and, for stochastic
        targets, fresh noise (``target_gumbel`` rows replace the verifier's noise). With a
        `stream` the copies run on it and the returned event marks their end."""

        event = torch.cuda.Event() if stream is not None else None
        self.step_grammar(bitmasks, positions, stream=stream)

        if indicators is None:

            scoped = ScopedIndicators.from_params(
                size=len(counts), timesteps=self.layout.cols, multiplicative=multiplicative,
                frequency=frequency, presence=presence, biases=biases, temperature=temperature,
                top_k=top_k, top_p=top_p, min_p=min_p, top_logprobs=top_logprobs, bitmasks=bitmasks,
                greedy_drafts=greedy_drafts)

        else:

            scoped = ScopedIndicators.from_pairs(indicators, timesteps=self.layout.cols)

        self._admit(scoped, positions, stream, biases, temperature, top_k, top_p, min_p, top_logprobs)
        self.repetition.update(counts=counts, multiplicative=multiplicative, frequency=frequency,
                               presence=presence, positions=positions, stream=stream)

        if scoped.has_stochastic_target:

            self.weights.update(generator=generator, selectors=scoped.stochastic_selectors,
                                targets=target_gumbel, positions=positions, prefill=prefill, stream=stream)

        self.transfer(positions, stream=stream, event=event)

        return event

    def allocate(self, encodings: List[Tensor], multiplicative: List[float], frequency: List[float],
                 presence: List[float], biases: List[Optional[dict]], temperature: List[float],
                 top_k: List[int], top_p: List[float], min_p: List[float], top_logprobs: List[int],
                 positions: List[int], indicators: Optional[ScopedIndicators] = None,
                 greedy_drafts=False, bitmasks: Optional[List[Optional[Tensor]]] = None, stream=None,
                 generator=None):
        """Admits requests into the slots `positions` (reference ``core/buffer.py:1239-1352``), all
        inputs host-resident: the prompts' token histograms (`encodings`, int64 ids) become the
        context counts and the decode counts restart at zero, step 0 of the grammar takes
        `bitmasks`, the indicators follow from the parameters (unless given), and stochastic
        targets get their prefill noise. With a `stream` the copies run on it and the returned
        event marks their end."""

        event = torch.cuda.Event() if stream is not None else None
        self.step_grammar(bitmasks, positions, timestep=0, stream=stream)

        scoped = indicators if indicators is not None else ScopedIndicators.from_params(
            size=len(encodings), timesteps=self.layout.cols, multiplicative=multiplicative,
            frequency=frequency, presence=presence, biases=biases, temperature=temperature,
            top_k=top_k, top_p=top_p, min_p=min_p, top_logprobs=top_logprobs, bitmasks=bitmasks,
            greedy_drafts=greedy_drafts)

        self._admit(scoped, positions, stream, biases, temperature, top_k, top_p, min_p, top_logprobs)
        self.repetition.allocate(encodings=encodings, multiplicative=multiplicative, frequency=frequency,
                                 presence=presence, positions=positions, stream=stream)

        if scoped.has_stochastic_target:

            self.weights.update(generator=generator, selectors=scoped.stochastic_selectors,
                                positions=positions, prefill=True, stream=stream)

        self.transfer(positions, stream=stream, event=event)

        return event
