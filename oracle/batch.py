"""Batched CPU restatement of the reference's PyTorch single-step path -- TEST INFRASTRUCTURE ONLY.

The reference's ``NaiveSampler`` runs one autoregressive step as a handful of torch operations
over the whole ``[B, V]`` batch (``core/naive.py:131-268`` processors, ``:270-348`` bounded top-128
and truncation, ``:377-495`` selection). This module states that same batch formulation, with the
same operations, dtypes and rounding points as the per-row restatement in ``oracle.sampler``, and
gates every processor per row with a mask (hazard H5: the reference gates batch-wide, which equals
per-row gating under neutral buffer fills). It is the CPU baseline that ``bench.py`` times (one
call over the batch, as the reference's PyTorch path runs) and ``tests/test_oracle.py`` checks it
row for row against ``oracle.sampler.singular``.
"""

from __future__ import annotations

from dataclasses import dataclass
from math import inf
from typing import Optional

import torch

from torch import Tensor

from oracle.sampler import (BF16, BIAS, F32, FREQ, GRAMMAR, GREEDY, I32, I64, MAX_K, MIN_P, MULT,
                            PRES, TEMP, TOP_K, TOP_K_LOGPROBS, TOP_P, State)


@dataclass
class BatchResult:
    tokens: Tensor          # [B] int64
    logprobs: Tensor        # [B] fp32 (0 for greedy rows)
    top_tokens: Tensor      # [B, Z] int64 (rows without 0x400 or a smaller limit: -1 past it)
    top_logprobs: Tensor    # [B, Z] fp32 (-inf past the row's limit)


def _rows(bits: Tensor, flag: int) -> Tensor:
    """[B, 1] mask of the rows whose indicator word holds `flag`."""

    return ((bits & flag) != 0)[:, None]


def process(logits: Tensor, st: State, bits: Tensor, step: int = 0) -> Tensor:
    """Grammar -> penalties -> bias -> temperature over the batch (reference core/naive.py:131-268);
    row b reads the state of slot b."""

    B, V = logits.shape
    x = logits.to(BF16).clone()

    if bool((bits & GRAMMAR).any()):

        words = st.grammar[:B, step].to(I32)
        allowed = (words[..., None].bitwise_right_shift(torch.arange(32, dtype=I32)) & 1).flatten(1)[:, :V]
        x.masked_fill_(_rows(bits, GRAMMAR) & (allowed == 0), -inf)

    decode = st.decode[:B, :V]

    if bool((bits & MULT).any()):

        total = st.context[:B, :V] + decode
        scales = st.multiplicative[:B, None].expand_as(x).masked_fill(total <= 0, 1.0)
        x = torch.where(_rows(bits, MULT), torch.where(x < 0, x * scales, x / scales), x)

    if bool((bits & FREQ).any()):

        x = torch.where(_rows(bits, FREQ), x.addcmul(decode, st.frequency[:B, None], value=-1), x)

    if bool((bits & PRES).any()):

        x = torch.where(_rows(bits, PRES), x.addcmul(decode > 0, st.presence[:B, None], value=-1), x)

    if bool((bits & BIAS).any()):

        x = torch.where(_rows(bits, BIAS), x + st.bias[:B, :V], x)

    if bool((bits & TEMP).any()):

        x = torch.where(_rows(bits, TEMP), x / st.temperature[:B, None], x)

    return x


def truncate(values: Tensor, st: State, bits: Tensor) -> Tensor:
    """top-k -> top-p -> min-p on [B, 128] sorted bf16 values (reference core/naive.py:270-328)."""

    B = values.size(0)
    position = torch.arange(values.size(-1), dtype=I32)[None]
    values.masked_fill_(_rows(bits, TOP_K) & position.ge(st.top_k[:B, None]), -inf)

    beyond = values.softmax(dim=-1, dtype=F32).cumsum_(dim=-1).gt(st.top_p[:B, None])
    beyond[:, 0] = False
    values.masked_fill_(_rows(bits, TOP_P) & beyond, -inf)

    scores = values.softmax(dim=-1)
    lower = st.min_p[:B, None].mul(scores[:, :1])
    values.masked_fill_(_rows(bits, MIN_P) & (scores < lower), -inf)

    return values


def singular(logits: Tensor, st: State, *, noise: Optional[Tensor] = None,
             max_top_logprobs: int = 5, bounded: str = "sort") -> BatchResult:
    """One autoregressive step over the batch (target indicators, row b at slot b, timestep 0),
    with logprobs and top-Z logprobs; ``noise`` is the [B, V] Gumbel plane (default: the state's
    target plane at timestep 0).

    ``bounded`` picks the bounded top-128: ``"sort"`` (the default) is a stable descending sort,
    ties to the lowest index as the parity contract requires (hazard H1); ``"topk"`` is the
    reference's own ``logits.topk(k=128)`` (``core/naive.py:336``), whose order among equal values
    torch leaves unspecified. Both select the same 128 values; ``"topk"`` is the formulation whose
    CPU time ``bench.py`` reports as the reference's."""

    B = logits.size(0)
    bits = torch.tensor(st.target[:B], dtype=I64)
    x = process(logits, st, bits)
    plane = (noise if noise is not None else st.gumbel_target[:B, 0]).to(BF16)

    if bounded == "topk":

        top, indices = x.topk(k=MAX_K, dim=-1)
        values = truncate(top, st, bits)

    elif bounded == "sort":

        # bounded top-128 as a stable descending sort (ties to the lowest index, hazard H1)
        ordered, order = x.sort(dim=-1, stable=True, descending=True)
        values = truncate(ordered[:, :MAX_K].contiguous(), st, bits)
        indices = order[:, :MAX_K]

    else:

        raise ValueError(f"unknown bounded top-128 formulation {bounded!r}")

    pick = (values - plane.gather(-1, indices)).argmax(dim=-1, keepdim=True)
    lse = values.to(F32).logsumexp(dim=-1, keepdim=True)
    shifted = values.to(F32) - lse

    greedy = (bits & GREEDY) != 0
    tokens = torch.where(greedy, indices[:, 0], indices.gather(-1, pick)[:, 0])
    logprobs = torch.where(greedy, torch.zeros(B), shifted.gather(-1, pick)[:, 0])

    limit = torch.where((bits & TOP_K_LOGPROBS) != 0, st.top_logprobs[:B].to(I64).clamp(max=max_top_logprobs), 0)
    limit = torch.where(greedy, 0, limit)
    keep = torch.arange(max_top_logprobs)[None] < limit[:, None]
    top_tokens = indices[:, :max_top_logprobs].masked_fill(~keep, -1)
    top_logprobs = shifted[:, :max_top_logprobs].masked_fill(~keep, -inf)

    return BatchResult(tokens=tokens, logprobs=logprobs, top_tokens=top_tokens, top_logprobs=top_logprobs)
