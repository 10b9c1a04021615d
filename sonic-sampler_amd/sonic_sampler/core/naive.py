"""Pure-torch sampling and verification over a ``SamplingBuffers`` (reference
``core/naive.py:53-708``).

This is the reference's validation API: the same processors, truncations, Gumbel-max selection
and chain verification written as whole-batch torch operations, runnable on any device. As in the
reference, a processor runs for the whole batch when any row's indicator enables it (buffers hold
neutral values for rows that do not), and the bounded path keeps the top-128 of each row. The
bounded top-128 is taken with a stable descending sort, so equal values keep the lowest index
first (the reference's ``topk`` leaves the order of ties unspecified on the CPU).
"""

from __future__ import annotations

from dataclasses import dataclass
from math import inf
from typing import Optional, Tuple

import torch

from torch import Tensor

from sonic_sampler.base import (
    DEFAULT_TOP_LOGPROBS,
    LogProbabilities,
    Selection,
    TopTargets,
    Verification,
)
from sonic_sampler.core.buffer import SamplingBuffers
from sonic_sampler.core.flags import Indicator
from sonic_sampler.ops import MAX_K


F32 = torch.float32
I32 = torch.int32
I64 = torch.int64
BF16 = torch.bfloat16

ValueIndices = Tuple[Tensor, Tensor]


def softmax(values: Tensor) -> Tuple[Tensor, Tensor]:
    """(fp32 probabilities, bf16 log-probabilities) via fp32 log_softmax."""

    logprobs = torch.log_softmax(values, dim=-1, dtype=F32)

    return logprobs.exp(), logprobs.to(BF16)


def subset_select(values: Tensor, mapping: Optional[Tensor], dim: int = -1) -> Tensor:

    return values if mapping is None else values.index_select(dim, mapping)


def remap(indices: Tensor, mapping: Optional[Tensor]) -> Tensor:

    if mapping is None:

        return indices

    return mapping.gather(0, indices.flatten().to(I64)).reshape_as(indices)


@dataclass(eq=False)
class NaiveSampler:

    buffers: SamplingBuffers
    bounded: bool = True
    max_top_logprobs: int = DEFAULT_TOP_LOGPROBS

    def is_enabled(self, flag: Indicator) -> bool:

        return any(flag & value for value in self.buffers.indicators.target)

    @property
    def is_greedy(self) -> bool:

        return self.buffers.flags.all_greedy

    @property
    def has_ordering(self) -> bool:

        return self.is_enabled(Indicator.cumulative())

    @property
    def return_top_logprobs(self) -> bool:

        return self.max_top_logprobs > 0 and self.is_enabled(Indicator.TOP_K_LOGPROBS)

    def grammar(self, logits: Tensor, bitmask: Tensor, mapping: Optional[Tensor] = None) -> Tensor:

        if self.is_enabled(Indicator.GRAMMAR):

            shifts = torch.arange(32, dtype=I32, device=logits.device)
            bits = (bitmask.view(I32)[..., None] >> shifts).flatten(-2)[..., : self.buffers.vocab_size]
            denied = (subset_select(bits, mapping) & 1) == 0
            logits.masked_fill_(denied, -inf)

        return logits

    def repetition(self, logits: Tensor, timestep: Optional[int] = None,
                   tokens: Optional[Tensor] = None, mapping: Optional[Tensor] = None) -> Tensor:

        if not self.is_enabled(Indicator.repetition()):

            return logits

        counts = self.buffers.repetition.counts
        context, decode = counts.context, counts.decode
        original = decode[..., 0].clone()
        row_dims = (None,) * (logits.dim() - 1)

        if tokens is not None:

            size, steps = tokens.shape
            history = tokens[:, None].expand(-1, steps, steps).tril(diagonal=-1).to(I64)

            if timestep is None:

                decode = decode[:, None].expand(size, steps, -1).scatter_add(
                    -1, history, torch.ones_like(history, dtype=I32))
                context = context[:, None]

            else:

                decode = decode.scatter_add(-1, history[:, timestep], torch.ones_like(tokens, dtype=I32))

            decode[..., 0].copy_(original[(slice(None),) + (None,) * (decode.dim() - 2)].expand_as(decode[..., 0]))

        decode = subset_select(decode, mapping)
        penalties = self.buffers.repetition

        if self.is_enabled(Indicator.MULTIPLICATIVE):

            total = subset_select(context, mapping) + decode
            scales = (
                penalties.multiplicative[(slice(None), *row_dims)]
                .expand_as(logits)
                .masked_fill(total <= 0, 1.0)
            )
            logits = torch.where(logits < 0, logits * scales, logits / scales)

        if self.is_enabled(Indicator.FREQUENCY):

            logits.addcmul_(decode, penalties.frequency[(slice(None), *row_dims)], value=-1)

        if self.is_enabled(Indicator.PRESENCE):

            logits.addcmul_(decode > 0, penalties.presence[(slice(None), *row_dims)], value=-1)

        return logits

    def bias(self, logits: Tensor, mapping: Optional[Tensor] = None) -> Tensor:

        if self.is_enabled(Indicator.BIAS):

            extra = (None,) * (logits.dim() - 2)
            logits.add_(subset_select(self.buffers.bias, mapping)[(slice(None), *extra)])

        return logits

    def temperature(self, logits: Tensor) -> Tensor:

        if self.is_enabled(Indicator.TEMPERATURE):

            logits.div_(self.buffers.temperature[(slice(None),) + (None,) * (logits.dim() - 1)])

        return logits

    def top_k(self, values: Tensor) -> Tensor:

        if self.is_enabled(Indicator.TOP_K):

            width = values.size(-1)
            mask = torch.arange(width, dtype=I32, device=values.device)[None] >= self.buffers.top_k[:, None]
            values.masked_fill_(mask[(slice(None),) + (None,) * (values.dim() - 2)], -inf)

        return values

    def top_p(self, values: Tensor) -> Tensor:

        if self.is_enabled(Indicator.TOP_P):

            upper = self.buffers.top_p[(slice(None),) + (None,) * (values.dim() - 1)]
            mask = values.softmax(dim=-1, dtype=F32).cumsum_(dim=-1).gt(upper)
            mask[..., 0] = False
            values.masked_fill_(mask, -inf)

        return values

    def min_p(self, values: Tensor) -> Tensor:

        if self.is_enabled(Indicator.MIN_P):

            scores = values.softmax(dim=-1)
            lower = self.buffers.min_p[(slice(None),) + (None,) * (values.dim() - 1)].mul(scores[..., :1])
            values.masked_fill_(scores < lower, -inf)

        return values

    def cumulative(self, logits: Tensor) -> Optional[ValueIndices]:

        if self.is_greedy:

            return None

        if self.bounded or self.has_ordering:

            values, indices = logits.sort(dim=-1, stable=True, descending=True)

            if self.bounded:

                values, indices = values[..., :MAX_K].contiguous(), indices[..., :MAX_K]

            values = self.min_p(self.top_p(self.top_k(values)))

            return values, indices.to(I32)

        return None

    def probabilities(self, values: Tensor, indices: Optional[Tensor] = None,
                      mapping: Optional[Tensor] = None) -> Tensor:

        base = torch.zeros_like(self.buffers.weights.gumbel.target[:, 0])

        if indices is None:

            return values if mapping is None else base.index_copy_(-1, mapping, values)

        return base.scatter_(-1, remap(indices, mapping).to(I64), values)

    def selection(self, logits: Tensor, weights: Tensor, pair: Optional[ValueIndices] = None,
                  mapping: Optional[Tensor] = None, logprobs: bool = False,
                  probs: bool = False) -> Selection:

        log_probs = top = probabilities = None

        if self.is_greedy:

            tokens = remap(logits.argmax(dim=-1, keepdim=True), mapping).to(I32)

            if logprobs:

                log_probs = LogProbabilities(selected=logits.new_zeros(tokens.shape))

            if probs:

                probabilities = self.probabilities(logits.new_ones(tokens.shape), indices=tokens)

        elif pair is None:

            targets = (logits - subset_select(weights, mapping)).argmax(dim=-1, keepdim=True)
            tokens = remap(targets, mapping).to(I32)

            if probs:

                scores, log_scores = softmax(logits)

                if logprobs:

                    selected = log_scores.gather(-1, targets)

                    if self.return_top_logprobs:

                        v, i = log_scores.topk(k=self.max_top_logprobs, dim=-1)
                        top = TopTargets(tokens=remap(i, mapping).to(I32), logprobs=v)

                    log_probs = LogProbabilities(selected=selected, top_k=top)

                probabilities = self.probabilities(scores, mapping=mapping)

            elif logprobs:

                lse = logits.logsumexp(dim=-1, keepdim=True)
                selected = logits.gather(-1, targets).sub_(lse)

                if self.return_top_logprobs:

                    v, i = logits.topk(k=self.max_top_logprobs, dim=-1)
                    top = TopTargets(tokens=remap(i, mapping).to(I32), logprobs=v.sub_(lse))

                log_probs = LogProbabilities(selected=selected, top_k=top)

        else:

            values, indices = pair
            indices = remap(indices, mapping)
            targets = (values - weights.gather(-1, indices.to(I64))).argmax(dim=-1, keepdim=True)
            tokens = indices.gather(-1, targets).to(I32)
            z = self.max_top_logprobs

            if probs:

                scores, log_scores = softmax(values)

                if logprobs:

                    selected = log_scores.gather(-1, targets)

                    if self.return_top_logprobs:

                        top = TopTargets(tokens=indices[:, :z].to(I32), logprobs=log_scores[:, :z])

                    log_probs = LogProbabilities(selected=selected, top_k=top)

                probabilities = self.probabilities(scores.to(BF16), indices=indices)

            elif logprobs:

                lse = values.to(F32).logsumexp(dim=-1, keepdim=True)
                selected = values.gather(-1, targets).sub_(lse)

                if self.return_top_logprobs:

                    top = TopTargets(tokens=indices[:, :z].to(I32), logprobs=values[:, :z].sub_(lse))

                log_probs = LogProbabilities(selected=selected, top_k=top)

        return Selection(tokens=tokens, probabilities=probabilities, logprobs=log_probs)

    def verification(self, logits: Tensor, weights: Tensor, tokens: Tensor, probs: Tensor,
                     pair: Optional[ValueIndices] = None, logprobs: bool = False) -> Verification:

        log_probs = top = None
        tokens64 = tokens.to(I64)

        if self.is_greedy:

            selections = logits.argmax(dim=-1).to(tokens.dtype)
            acceptances = selections == tokens
            acceptances[:, -1] = False
            offsets = acceptances.int().argmin(dim=-1, keepdim=True)

            if logprobs:

                log_probs = LogProbabilities(selected=logits.new_zeros(tokens.shape))

        elif pair is None:

            scores, log_scores = softmax(logits)
            drafted = tokens64[..., None]
            acceptances = (
                probs.gather(-1, drafted)
                .mul_(self.buffers.weights.uniform[..., None])
                .le(scores.gather(-1, drafted))
                .squeeze(-1)
            )
            acceptances[:, -1] = False
            offsets = acceptances.int().argmin(dim=-1, keepdim=True)
            rejected = offsets[..., None].expand(-1, 1, logits.size(-1)).to(I64)
            sampled = (
                scores.gather(1, rejected).sub_(probs.gather(1, rejected)).squeeze_(1)
                .clamp_min_(0).log_().sub_(weights.gather(1, rejected).squeeze_(1))
                .argmax(dim=-1, keepdim=True)
            )
            selections = tokens.scatter(-1, offsets.to(I64), sampled.to(tokens.dtype))

            if logprobs:

                selected = log_scores.gather(-1, selections.to(I64)[..., None]).squeeze_(-1)

                if self.return_top_logprobs:

                    v, i = log_scores.topk(k=self.max_top_logprobs, dim=-1)
                    top = TopTargets(tokens=i.to(I32), logprobs=v)

                log_probs = LogProbabilities(selected=selected, top_k=top)

        else:

            values, indices = pair
            scores, log_scores = softmax(values)
            drafted = tokens64[..., None]
            matches = indices.to(I64) == drafted
            positions = matches.int().argmax(dim=-1, keepdim=True)
            targets = scores.gather(-1, positions).squeeze(-1).masked_fill_(~matches.any(dim=-1), 0)
            acceptances = (
                probs.gather(-1, drafted).squeeze(-1)
                .mul_(self.buffers.weights.uniform)
                .le(targets)
            )
            acceptances[:, -1] = False
            offsets = acceptances.int().argmin(dim=-1, keepdim=True)
            rejected = offsets[..., None].expand(-1, 1, MAX_K).to(I64)
            candidates = indices.gather(1, rejected).squeeze_(1).to(I64)
            nested = offsets.to(I64) * probs.size(-1) + candidates
            marginals = probs.flatten(1, 2).gather(-1, nested)
            sampled = (
                scores.gather(1, rejected).squeeze_(1).sub_(marginals).clamp_min_(0).log_()
                .sub_(weights.flatten(1, 2).gather(-1, nested))
                .argmax(dim=-1, keepdim=True)
            )
            chosen = candidates.gather(-1, sampled).to(tokens.dtype)
            selections = tokens.scatter(-1, offsets.to(I64), chosen)

            if logprobs:

                positions = positions.squeeze(-1).scatter(-1, offsets.to(I64), sampled).unsqueeze(-1)
                selected = log_scores.gather(-1, positions).squeeze_(-1)

                if self.return_top_logprobs:

                    z = self.max_top_logprobs
                    top = TopTargets(tokens=indices[..., :z].to(I32), logprobs=log_scores[..., :z])

                log_probs = LogProbabilities(selected=selected, top_k=top)

        return Verification(tokens=selections, offsets=offsets.to(I32), logprobs=log_probs)

    def preamble(self, logits: Tensor, tokens: Optional[Tensor] = None,
                 timestep: Optional[int] = None, mapping: Optional[Tensor] = None):

        grammar = self.buffers.grammar if timestep is None else self.buffers.grammar[:, timestep]
        drafted = None if timestep == 0 else tokens

        masked = self.grammar(logits, grammar, mapping)
        penalized = self.repetition(masked, timestep=timestep, tokens=drafted, mapping=mapping)

        return self.cumulative(self.temperature(self.bias(penalized, mapping)))

    def singular(self, logits: Tensor, tokens: Optional[Tensor], timestep: int, *,
                 mapping: Optional[Tensor] = None, prefill: bool = False, logprobs: bool = False,
                 probs: bool = False) -> Selection:

        pair = self.preamble(logits, tokens=tokens, timestep=timestep, mapping=mapping)
        noise = self.buffers.weights.gumbel.target if prefill else self.buffers.weights.gumbel.draft

        return self.selection(logits, noise[:, timestep], pair, mapping, logprobs, probs)

    def multistep(self, logits: Tensor, tokens: Tensor, probs: Tensor, *,
                  logprobs: bool = False):

        pair = self.preamble(logits, tokens=tokens)
        verification = self.verification(logits, self.buffers.weights.gumbel.target, tokens,
                                         probs, pair, logprobs)

        return verification, pair
