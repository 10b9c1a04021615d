"""Pure-PyTorch sampler over a ``SamplingBuffers``: the public ``sonic_sampler.core.NaiveSampler``
(the reference exports a class of this name from ``core/naive.py:53-708`` for validation).

The computation is written as three batch stages that any torch device runs:

* ``process`` -- grammar mask, repetition / frequency / presence penalties over the decode counts
  (plus the drafted history), logit bias and temperature, each rounded to bf16 where the
  reference's PyTorch path rounds, and each applied only to the rows whose indicator word enables
  it (the reference enables a processor for the whole batch when any row asks for it, which gives
  the same result when disabled rows hold neutral parameters);
* ``candidates`` -- each row's 128 largest values by a stable descending sort (equal values keep
  the lowest index first), then top-k, top-p and min-p in that order, each on the values the
  previous one left;
* ``select`` (one step: Gumbel-max over ``bf16(v - w)``, greedy rows by argmax) and ``verify``
  (chain verification: accept draft i while ``bf16(u_i q_i(d_i)) <= p_i(d_i)``, resample the first
  rejection from ``max(p - q, 0)``, or emit the bonus token after the last step).

Where the reference disagrees with itself, this class follows the semantics of the fused kernels:
greedy rows take the argmax of the processed logits, ``prefill=False`` reads the draft scope (the
draft indicators and noise, as ``UnshardedFusedSingular.drafting`` does), and the top-128 ties go to
the lowest index.
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


def _gate(bits: Tensor, flag: int, ndim: int) -> Tensor:
    """Rows whose indicator word holds `flag`, shaped to broadcast over `ndim` dimensions."""

    return ((bits & int(flag)) != 0).reshape(-1, *([1] * (ndim - 1)))


def _through(values: Tensor, mapping: Optional[Tensor]) -> Tensor:
    """Target-vocabulary state seen through a draft -> target map (identity without one)."""

    return values if mapping is None else values.index_select(-1, mapping)


def _log_softmax(values: Tensor) -> Tuple[Tensor, Tensor]:
    """fp32 (probabilities, log-probabilities) of bf16 values."""

    logp = torch.log_softmax(values, dim=-1, dtype=F32)

    return logp.exp(), logp


@dataclass
class NaiveSampler:

    # The buffers every call reads: indicators, processor parameters, counts and noise.
    buffers: SamplingBuffers

    # Keep each row's top-128 (True) or its full sorted row (False) as the candidate set.
    bounded: bool = True

    # Top-k log-probabilities returned per row (Z).
    max_top_logprobs: int = DEFAULT_TOP_LOGPROBS

    # ---- indicator words ---------------------------------------------------------------------

    def _bits(self, scope: str, rows: int, device) -> Tensor:

        words = getattr(self.buffers.flags.indicators, scope)

        return torch.tensor([int(w) for w in words[:rows]], dtype=I64, device=device)

    # ---- stage 1: logit processors --------------------------------------------------------------

    def process(self, logits: Tensor, bits: Tensor, *, step: Optional[int] = None,
                history: Optional[Tensor] = None, mapping: Optional[Tensor] = None) -> Tensor:
        """Processed bf16 logits of [B, V] (one step, grammar row `step`) or [B, T, V] (chain,
        grammar rows 0..T-1). `history` is [B, H] drafted tokens: a one-step call counts all of
        them, a chain counts tokens[:, :i] at step i; token 0 never counts."""

        b = self.buffers
        x = logits.to(BF16).clone()
        chain = x.dim() == 3
        nd = x.dim()
        vocab = x.size(-1)

        if bool((bits & Indicator.GRAMMAR).any()):

            words = b.grammar.view(I32)
            words = words[:, :x.size(1)] if chain else words[:, step or 0]
            allowed = (words[..., None].bitwise_right_shift(torch.arange(32, device=x.device, dtype=I32)) & 1)
            allowed = _through(allowed.flatten(-2)[..., :b.repetition.counts.decode.size(-1)], mapping)[..., :vocab]
            x = x.masked_fill(_gate(bits, Indicator.GRAMMAR, nd) & (allowed == 0), -inf)

        penalties = Indicator.MULTIPLICATIVE | Indicator.FREQUENCY | Indicator.PRESENCE

        if bool((bits & penalties).any()):

            rep = b.repetition
            decode = rep.counts.decode[:x.size(0)]
            own = decode[:, :1].clone()

            if history is not None and history.numel():

                ones = torch.ones_like(history, dtype=decode.dtype)

                if chain:

                    # step i adds the drafts of steps < i (zero padding lands on token 0)
                    steps = x.size(1)
                    mask = torch.ones(steps, history.size(1), dtype=torch.bool, device=x.device).tril(-1)
                    earlier = history[:, None, :].expand(-1, steps, -1).masked_fill(~mask, 0).to(I64)
                    decode = decode[:, None].expand(-1, steps, -1).scatter_add(-1, earlier, ones[:, None].expand_as(earlier))

                else:

                    decode = decode.scatter_add(-1, history.to(I64), ones)

                decode[..., :1] = own[:, None] if chain else own

            elif chain:

                decode = decode[:, None].expand(-1, x.size(1), -1)

            decode = _through(decode, mapping)[..., :vocab]
            per_row = lambda t: t[:x.size(0)].reshape(-1, *([1] * (nd - 1)))  # noqa: E731

            if bool((bits & Indicator.MULTIPLICATIVE).any()):

                context = rep.counts.context[:x.size(0)]
                context = _through(context[:, None] if chain else context, mapping)[..., :vocab]
                seen = (context + decode) > 0
                factor = per_row(rep.multiplicative).expand_as(x).masked_fill(~seen, 1.0)
                scaled = torch.where(x < 0, x * factor, x / factor)
                x = torch.where(_gate(bits, Indicator.MULTIPLICATIVE, nd), scaled, x)

            if bool((bits & Indicator.FREQUENCY).any()):

                x = torch.where(_gate(bits, Indicator.FREQUENCY, nd),
                                x.addcmul(decode, per_row(rep.frequency), value=-1), x)

            if bool((bits & Indicator.PRESENCE).any()):

                x = torch.where(_gate(bits, Indicator.PRESENCE, nd),
                                x.addcmul(decode > 0, per_row(rep.presence), value=-1), x)

        if bool((bits & Indicator.BIAS).any()):

            bias = _through(b.bias[:x.size(0)], mapping)[..., :vocab]
            x = torch.where(_gate(bits, Indicator.BIAS, nd), x + (bias[:, None] if chain else bias), x)

        if bool((bits & Indicator.TEMPERATURE).any()):

            t = b.temperature[:x.size(0)].reshape(-1, *([1] * (nd - 1)))
            x = torch.where(_gate(bits, Indicator.TEMPERATURE, nd), x / t, x)

        return x

    # ---- stage 2: candidates and truncation -----------------------------------------------------

    def candidates(self, x: Tensor, bits: Tensor) -> ValueIndices:
        """Each row's candidates (values desc, ties to the lowest index) truncated by top-k, then
        top-p (fp32 softmax, cumulative sum > p masked, position 0 kept), then min-p (bf16
        softmax below bf16(min_p * max) masked)."""

        b = self.buffers
        nd = x.dim()
        values, indices = x.sort(dim=-1, stable=True, descending=True)

        if self.bounded:

            values, indices = values[..., :MAX_K].contiguous(), indices[..., :MAX_K]

        per_row = lambda t: t[:x.size(0)].reshape(-1, *([1] * (nd - 1)))  # noqa: E731
        position = torch.arange(values.size(-1), device=x.device, dtype=I32)
        values = values.masked_fill(_gate(bits, Indicator.TOP_K, nd) & (position >= per_row(b.top_k)), -inf)

        if bool((bits & Indicator.TOP_P).any()):

            over = values.softmax(dim=-1, dtype=F32).cumsum(dim=-1) > per_row(b.top_p)
            over[..., 0] = False
            values = values.masked_fill(_gate(bits, Indicator.TOP_P, nd) & over, -inf)

        if bool((bits & Indicator.MIN_P).any()):

            scores = values.softmax(dim=-1)
            floor = per_row(b.min_p) * scores[..., :1]
            values = values.masked_fill(_gate(bits, Indicator.MIN_P, nd) & (scores < floor), -inf)

        return values, indices.to(I32)

    # ---- stage 3a: one-step selection ----------------------------------------------------------

    def select(self, x: Tensor, bits: Tensor, noise: Tensor, cand: ValueIndices,
               mapping: Optional[Tensor], logprobs: bool, probs: bool) -> Selection:
        """Gumbel-max over bf16(v - w) on the candidates (first position on ties); greedy rows
        take the processed argmax. Noise and probabilities live in the target vocabulary."""

        values, indices = cand
        rows = x.size(0)
        greedy = (bits & Indicator.GREEDY) != 0
        targets = indices.to(I64) if mapping is None else mapping.to(I64)[indices.to(I64)]

        pick = (values - noise.gather(-1, targets)).argmax(dim=-1, keepdim=True)
        argmax = x.argmax(dim=-1, keepdim=True)
        argmax = argmax if mapping is None else mapping.to(I64)[argmax]
        tokens = torch.where(greedy[:, None], argmax, targets.gather(-1, pick)).to(I32)

        scores, logp = _log_softmax(values)
        probabilities = None

        if probs:

            probabilities = torch.zeros_like(self.buffers.weights.gumbel.target[:rows, 0])
            stochastic = ~greedy
            probabilities[stochastic] = probabilities[stochastic].scatter(
                -1, targets[stochastic], scores[stochastic].to(BF16))
            probabilities[greedy, argmax[greedy, 0]] = 1.0

        log_probs = None

        if logprobs:

            # with probabilities: log_softmax; without: v - logsumexp(v) (two fp32 roundings apart)
            shifted = logp if probs else values.to(F32) - values.to(F32).logsumexp(dim=-1, keepdim=True)
            selected = torch.where(greedy[:, None], 0.0, shifted.gather(-1, pick))
            top = None

            if self.max_top_logprobs > 0 and bool(((bits & Indicator.TOP_K_LOGPROBS) != 0).any()):

                z = self.max_top_logprobs
                top = TopTargets(tokens=targets[:, :z].to(I32), logprobs=shifted[:, :z].to(BF16))

            log_probs = LogProbabilities(selected=selected.to(BF16), top_k=top)

        return Selection(tokens=tokens, probabilities=probabilities, logprobs=log_probs)

    # ---- stage 3b: chain verification ----------------------------------------------------------

    def verify(self, x: Tensor, bits: Tensor, tokens: Tensor, q: Tensor, cand: ValueIndices,
               logprobs: bool) -> Verification:
        """Greedy rows: accept while the processed argmax equals the draft. Stochastic rows:
        accept step i while bf16(u_i q_i(d_i)) <= p_i(d_i) (p over the candidates, 0 outside),
        resample the first rejection j from argmax log(max(p_j - q_j, 0)) - w_j, or after the last
        draft take argmax log p - w at the bonus step. Returns the drafts with the correction or
        bonus written at `offsets`."""

        b = self.buffers
        values, indices = cand
        batch, steps = tokens.shape
        drafts = tokens.to(I64)
        last = torch.arange(steps, device=x.device) == steps - 1
        greedy = (bits & Indicator.GREEDY) != 0

        # greedy chains
        argmax = x.argmax(dim=-1)
        g_accept = (argmax == drafts) & ~last

        # stochastic chains
        scores, logp = _log_softmax(values)
        hit = indices.to(I64) == drafts[..., None]
        where = hit.int().argmax(dim=-1, keepdim=True)
        p_draft = scores.gather(-1, where)[..., 0].masked_fill(~hit.any(dim=-1), 0.0)
        q_draft = (q.gather(-1, drafts[..., None])[..., 0] * b.weights.uniform[:batch, :steps])
        s_accept = (q_draft <= p_draft) & ~last

        accept = torch.where(greedy[:, None], g_accept, s_accept)
        offsets = accept.int().argmin(dim=-1, keepdim=True)                       # first rejection
        j = offsets[:, 0]
        rows = torch.arange(batch, device=x.device)

        cand_j = indices[rows, j].to(I64)                                          # [B, 128]
        residual = (scores[rows, j] - q[rows, j].gather(-1, cand_j).to(F32)).clamp_min(0)
        noise = b.weights.gumbel.target[:batch].to(x.device)[rows, j].gather(-1, cand_j)
        pick = (residual.log() - noise.to(F32)).argmax(dim=-1)
        resampled = cand_j.gather(-1, pick[:, None])[:, 0]
        correction = torch.where(greedy, argmax[rows, j], resampled)

        out = tokens.clone()
        out[rows, j] = correction.to(out.dtype)
        log_probs = None

        if logprobs:

            position = where[..., 0].clone()
            position[rows, j] = pick
            selected = logp.gather(-1, position[..., None])[..., 0]
            selected = torch.where(greedy[:, None], 0.0, selected)
            top = None

            if self.max_top_logprobs > 0 and bool(((bits & Indicator.TOP_K_LOGPROBS) != 0).any()):

                z = self.max_top_logprobs
                top = TopTargets(tokens=indices[..., :z], logprobs=logp[..., :z].to(BF16))

            log_probs = LogProbabilities(selected=selected.to(BF16), top_k=top)

        return Verification(tokens=out, offsets=offsets.to(I32), logprobs=log_probs)

    # ---- entry points (reference signatures) ----------------------------------------------------

    def singular(self, logits: Tensor, tokens: Optional[Tensor], timestep: int, *,
                 mapping: Optional[Tensor] = None, prefill: bool = False, logprobs: bool = False,
                 probs: bool = False) -> Selection:
        """One step over [B, V] logits: the target scope and noise with ``prefill``, otherwise the
        draft scope with ``tokens[:, :timestep]`` as extra history and the draft noise of
        ``timestep``; ``mapping`` is the draft -> target (d2t) map."""

        scope = "target" if prefill else "draft"
        bits = self._bits(scope, logits.size(0), logits.device)
        history = None if (tokens is None or timestep == 0) else tokens[:, :timestep]
        x = self.process(logits, bits, step=timestep, history=history, mapping=mapping)
        noise = getattr(self.buffers.weights.gumbel, scope)[:logits.size(0), timestep]
        cand = self.candidates(x, bits)

        return self.select(x, bits, noise.to(BF16), cand, mapping, logprobs, probs)

    def multistep(self, logits: Tensor, tokens: Tensor, probs: Tensor, *,
                  logprobs: bool = False) -> Tuple[Verification, Optional[ValueIndices]]:
        """Chain verification of [B, gamma + 1, V] logits against [B, gamma + 1] drafts with draft
        probabilities [B, gamma (+ 1), V]; returns the verification and each row's candidates."""

        bits = self._bits("target", logits.size(0), logits.device)
        x = self.process(logits, bits, history=tokens)
        cand = self.candidates(x, bits)
        steps = tokens.size(1)

        if probs.size(1) < steps:

            pad = probs.new_zeros(probs.size(0), steps - probs.size(1), probs.size(2))
            probs = torch.cat([probs, pad], dim=1)

        return self.verify(x, bits, tokens, probs, cand, logprobs), cand
