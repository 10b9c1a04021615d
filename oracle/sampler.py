"""Per-request CPU restatement of the reference's PyTorch sampling path -- TEST INFRASTRUCTURE ONLY.

Every arithmetic step uses the same torch CPU operation, dtype and rounding point as the
reference's ``NaiveSampler`` (``src/sonic_sampler/core/naive.py``), applied to one logit row (a
``[1, V]`` tensor) at a time, with the row's own indicator word deciding which processors run.
Under the neutral buffer fills of ``SamplingBuffers.random`` this equals the reference's batch-wide
gating (hazard H5). Composition rules the reference's PyTorch path lacks are taken from its
kernels: row -> slot indirection (``ops/prologue.py:265-267``, ``ops/singular.py:213-217``,
``ops/verify.py:47-49``), variable lookahead (``ops/verify.py:37-40``), decode-count updates
(``ops/singular.py:134-151``, ``ops/verify.py:75-91``) and the 0x800 masked residual
(``ops/verify.py:205-214``, equal to the reference's residual with a one-hot draft distribution).

Threshold decisions (top-p cumulative sum vs p, min-p, acceptance ``bf16(u q) <= p``, residual
argmax) depend on fp32 exp/log results that differ between implementations in the last bits.
Each record therefore carries ``knife``: True when a float64 recomputation puts a decision within
a relative 1e-5 of its threshold, where a different but correct fp32 evaluation may decide
differently. Parity tests allow a mismatch only on such rows. The fp32 ``exp`` / ``log`` inside
truncation and log-probabilities are the platform's and no check pins their last ulp: parity
unpinned there, which the tolerance on log-probabilities and the knife-edge rule absorb.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from math import inf
from typing import Dict, List, Optional, Sequence, Tuple

import torch

from torch import Tensor

F32 = torch.float32
F64 = torch.float64
I32 = torch.int32
I64 = torch.int64
BF16 = torch.bfloat16

MAX_K = 128

GRAMMAR, MULT, FREQ, PRES, BIAS, TEMP = 0x1, 0x2, 0x4, 0x8, 0x10, 0x20
GREEDY, TOP_K, TOP_P, MIN_P, TOP_K_LOGPROBS, SVGD = 0x40, 0x80, 0x100, 0x200, 0x400, 0x800

REL = 1e-5  # knife-edge band, relative


@dataclass
class State:
    """CPU copies of the members of a ``SamplingBuffers`` the path reads (reference
    ``core/buffer.py:784-817`` layouts)."""

    target: List[int]
    draft: List[int]
    grammar: Tensor          # [B, T, W] int32
    context: Tensor          # [B, V] int32
    decode: Tensor           # [B, V] int32
    bias: Tensor             # [B, V] bf16
    multiplicative: Tensor   # [B] bf16
    frequency: Tensor
    presence: Tensor
    temperature: Tensor
    top_p: Tensor
    min_p: Tensor
    top_k: Tensor            # [B] int32
    top_logprobs: Tensor     # [B] int32
    gumbel_target: Tensor    # [B, T, V] bf16
    gumbel_draft: Tensor     # [B, T, V] bf16
    uniform: Tensor          # [B, T] bf16

    @classmethod
    def from_buffers(cls, b) -> "State":

        cpu = lambda t: t.detach().to("cpu").clone()  # noqa: E731
        rep = b.repetition

        return cls(
            target=[int(v) for v in b.flags.indicators.target],
            draft=[int(v) for v in b.flags.indicators.draft],
            grammar=cpu(b.grammar.view(I32)).as_subclass(Tensor),
            context=cpu(rep.counts.context),
            decode=cpu(rep.counts.decode),
            bias=cpu(b.bias),
            multiplicative=cpu(rep.multiplicative),
            frequency=cpu(rep.frequency),
            presence=cpu(rep.presence),
            temperature=cpu(b.temperature),
            top_p=cpu(b.top_p),
            min_p=cpu(b.min_p),
            top_k=cpu(b.top_k),
            top_logprobs=cpu(b.top_logprobs),
            gumbel_target=cpu(b.weights.gumbel.target).as_subclass(Tensor),
            gumbel_draft=cpu(b.weights.gumbel.draft).as_subclass(Tensor),
            uniform=cpu(b.weights.uniform).as_subclass(Tensor),
        )


# ------------------------------------------------------------------------------------------------
# Prologue: grammar -> repetition -> bias -> temperature (reference core/naive.py:131-268, 648-673)
# ------------------------------------------------------------------------------------------------

def process_row(logits: Tensor, st: State, slot: int, ind: int, grammar_row: Optional[Tensor],
                history: Sequence[int], d2t: Optional[Tensor]) -> Tensor:
    """One bf16 logit row through the enabled processors; returns a bf16 [V] tensor."""

    x = logits.detach().to("cpu", BF16).clone()[None]
    mapping = None if d2t is None else d2t.to(I64)

    def sub(t: Tensor) -> Tensor:

        return t if mapping is None else t.index_select(-1, mapping)

    if ind & GRAMMAR and grammar_row is not None:

        # core/naive.py:138-159
        shifts = torch.arange(32, dtype=I32)
        bits = (grammar_row.to(I32)[:, None].bitwise_right_shift(shifts)).flatten()
        bits = sub(bits[: st.decode.size(-1)])[: x.size(-1)]
        x.masked_fill_(((bits & 1) ^ 1).bool()[None], -inf)

    if ind & (MULT | FREQ | PRES):

        # core/naive.py:171-236; the history is added to the slot's decode counts, token 0 never
        # counts (the reference pads with 0 and restores decode[..., 0]).
        decode = st.decode[slot].clone()
        original = decode[0].clone()

        if len(history):

            decode.scatter_add_(0, torch.tensor(list(history), dtype=I64),
                                torch.ones(len(history), dtype=I32))
            decode[0] = original

        decode = sub(decode)[None]

        if ind & MULT:

            total = sub(st.context[slot])[None] + decode
            scales = st.multiplicative[slot:slot + 1][:, None].expand_as(x).masked_fill(total <= 0, 1.0)
            x = torch.where(x < 0, x * scales, x / scales)

        if ind & FREQ:

            x.addcmul_(decode, st.frequency[slot:slot + 1][:, None], value=-1)

        if ind & PRES:

            x.addcmul_(decode > 0, st.presence[slot:slot + 1][:, None], value=-1)

    if ind & BIAS:

        x.add_(sub(st.bias[slot])[None])  # core/naive.py:240-253

    if ind & TEMP:

        x.div_(st.temperature[slot:slot + 1][:, None])  # core/naive.py:255-268

    return x[0]


# ------------------------------------------------------------------------------------------------
# Bounded top-128 and truncation (reference core/naive.py:270-348)
# ------------------------------------------------------------------------------------------------

def bounded(x: Tensor) -> Tuple[Tensor, Tensor]:
    """Top-128 as a stable descending sort: ties keep the lowest index (hazard H1)."""

    values, indices = x.sort(dim=-1, stable=True, descending=True)

    return values[..., :MAX_K].contiguous(), indices[..., :MAX_K].to(I32)


def _bf16_unstable(x64: Tensor) -> Tensor:
    """True where a relative 1e-5 perturbation changes the bf16 rounding of x."""

    lo = (x64 * (1 - REL)).to(F32).to(BF16)
    hi = (x64 * (1 + REL)).to(F32).to(BF16)

    return lo != hi


def truncate(values: Tensor, ind: int, st: State, slot: int) -> Tuple[Tensor, bool]:
    """top-k -> top-p -> min-p on [1, 128] bf16 values, each on the previous output."""

    knife = False

    if ind & TOP_K:

        mask = torch.arange(values.size(-1), dtype=I32)[None] >= st.top_k[slot]
        values.masked_fill_(mask, -inf)

    if ind & TOP_P:

        upper = st.top_p[slot:slot + 1][:, None]
        mask = values.softmax(dim=-1, dtype=F32).cumsum_(dim=-1).gt(upper)
        mask[..., 0] = False

        cum64 = values.to(F64).softmax(dim=-1).cumsum(dim=-1)
        p = float(upper)
        live = torch.isfinite(values)
        live[..., 0] = False
        knife |= bool(((cum64 - p).abs() <= REL * p)[live].any())

        values.masked_fill_(mask, -inf)

    if ind & MIN_P:

        scores = values.softmax(dim=-1)
        lower = st.min_p[slot:slot + 1][:, None].mul(scores[..., :1])

        s64 = values.to(F64).softmax(dim=-1)
        near = (scores.to(F64) - lower.to(F64)).abs() <= 2 * (lower.to(F64).abs() * 2.0 ** -7 + 1e-30)
        knife |= bool(_bf16_unstable(s64[..., :1]).any()) or bool((_bf16_unstable(s64) & near).any())

        values.masked_fill_(scores < lower, -inf)

    return values, knife


def log_softmax_pair(values: Tensor) -> Tuple[Tensor, Tensor]:
    """(fp32 probabilities, fp32 log-probabilities); the bf16 output is their rounding
    (reference ``softmax``, core/naive.py:53-58)."""

    logprobs = torch.log_softmax(values, dim=-1, dtype=F32)

    return logprobs.exp(), logprobs


# ------------------------------------------------------------------------------------------------
# Single step (reference core/naive.py:377-495 `selection`, :675-692 `singular`)
# ------------------------------------------------------------------------------------------------

@dataclass
class RowResult:
    token: int
    greedy: bool
    knife: bool = False
    logprob: Optional[float] = None             # fp32 value before the bf16 output rounding
    top_tokens: List[int] = field(default_factory=list)
    top_logprobs: List[float] = field(default_factory=list)   # fp32, before rounding
    probs: Optional[Dict[int, float]] = None    # target id -> fp32 probability before rounding
    values: Optional[Tensor] = None             # bf16 [128] truncated values (stochastic rows)
    indices: Optional[Tensor] = None            # int32 [128] (draft vocabulary ids)


def singular(
    logits: Tensor,
    st: State,
    *,
    scope: str = "target",
    timestep: int = 0,
    slot_mapping: Optional[Sequence[int]] = None,
    d2t: Optional[Tensor] = None,
    drafted: Optional[Tensor] = None,
    history: Optional[int] = None,
    noise: Optional[Tensor] = None,
    logprobs: bool = False,
    probs: bool = False,
    max_top_logprobs: int = 5,
) -> List[RowResult]:
    """Expected outputs of one single-step call, one record per logit row.

    ``scope`` selects the indicator list ("target": autoregressive, "draft": drafting);
    ``noise`` is the [slots, V_t] Gumbel plane (defaults to the scope's plane at ``timestep``);
    ``drafted`` / ``history``: row r sees ``drafted[r, :history]`` as extra decode history.
    """

    logits = logits.detach().to("cpu")
    rows = logits.size(0)
    indicators = st.target if scope == "target" else st.draft
    plane = noise if noise is not None else (st.gumbel_target if scope == "target" else st.gumbel_draft)[:, timestep]
    plane = plane.to("cpu")
    d2t_cpu = None if d2t is None else d2t.to("cpu").to(I64)
    out: List[RowResult] = []

    for r in range(rows):

        slot = int(slot_mapping[r]) if slot_mapping is not None else r
        ind = indicators[slot]
        grammar_row = st.grammar[slot, timestep]
        hist = [] if drafted is None or not history else [int(t) for t in drafted[r, :history]]
        x = process_row(logits[r], st, slot, ind, grammar_row, hist, d2t_cpu)

        if ind & GREEDY:

            index = int(x.argmax())
            token = int(d2t_cpu[index]) if d2t_cpu is not None else index
            out.append(RowResult(token=token, greedy=True, logprob=0.0 if logprobs else None))
            continue

        values, indices = bounded(x[None])
        values, knife = truncate(values, ind, st, slot)
        target_ids = indices.to(I64) if d2t_cpu is None else d2t_cpu[indices.to(I64)]

        weights = plane[slot].gather(-1, target_ids[0])[None]
        pos = int((values - weights).argmax(dim=-1))
        token = int(target_ids[0, pos])
        rec = RowResult(token=token, greedy=False, knife=knife, values=values[0].clone(),
                        indices=indices[0].clone())

        z_allowed = max_top_logprobs if (ind & TOP_K_LOGPROBS) else 0
        z_allowed = min(z_allowed, int(st.top_logprobs[slot]))

        if probs:

            scores, logp = log_softmax_pair(values)
            rec.probs = {int(t): float(s) for t, s in zip(target_ids[0], scores[0])}

            if logprobs:

                rec.logprob = float(logp[0, pos])
                rec.top_tokens = [int(t) for t in target_ids[0, :z_allowed]]
                rec.top_logprobs = [float(v) for v in logp[0, :z_allowed]]

        elif logprobs:

            lse = values.to(F32).logsumexp(dim=-1, keepdim=True)
            shifted = values.to(F32) - lse
            rec.logprob = float(shifted[0, pos])
            rec.top_tokens = [int(t) for t in target_ids[0, :z_allowed]]
            rec.top_logprobs = [float(v) for v in shifted[0, :z_allowed]]

        out.append(rec)

    return out


def apply_singular_counts(decode: Tensor, results: List[RowResult],
                          slot_mapping: Optional[Sequence[int]], prefill: bool) -> Tensor:
    """Decode counts after the call's update (reference ``ops/singular.py:134-151``)."""

    decode = decode.clone()

    for r, rec in enumerate(results):

        slot = int(slot_mapping[r]) if slot_mapping is not None else r

        if prefill:

            decode[slot, rec.token] = 1

        else:

            decode[slot, rec.token] += 1

    return decode


# ------------------------------------------------------------------------------------------------
# Chain verification (reference core/naive.py:497-646 `verification`, :694-708 `multistep`)
# ------------------------------------------------------------------------------------------------

@dataclass
class RequestResult:
    offset: int
    tokens: List[int]                      # emitted tokens, offset + 1 of them
    greedy: bool
    knife: bool = False
    logprobs: List[float] = field(default_factory=list)        # fp32 before rounding, per emitted
    top_tokens: List[List[int]] = field(default_factory=list)  # per emitted position
    top_logprobs: List[List[float]] = field(default_factory=list)
    row_values: List[Tensor] = field(default_factory=list)     # truncated bf16 values per row
    row_indices: List[Tensor] = field(default_factory=list)


def multistep(
    logits: Tensor,
    st: State,
    drafted: Tensor,
    cu_seqlens: Sequence[int],
    *,
    slot_mapping: Optional[Sequence[int]] = None,
    probabilities: Optional[Tensor] = None,
    noise: Optional[Tensor] = None,
    logprobs: bool = False,
    max_top_logprobs: int = 5,
) -> List[RequestResult]:
    """Expected outputs of one verification call, one record per request.

    ``logits`` is the flat [rows, V] bf16 layout, ``drafted`` the flat [rows] drafts and
    ``cu_seqlens`` the request boundaries (fixed lookahead: multiples of gamma + 1).
    ``probabilities`` is the [slots, gamma, V] draft distribution (None: point masses on the
    drafts, the 0x800 regime); ``noise`` the [slots, T, V] Gumbel planes (default target noise).
    """

    logits = logits.detach().to("cpu")
    drafted = drafted.detach().to("cpu").to(I64)
    planes = (noise if noise is not None else st.gumbel_target).to("cpu")
    q_all = None if probabilities is None else probabilities.detach().to("cpu")
    out: List[RequestResult] = []

    for b in range(len(cu_seqlens) - 1):

        margin, n = int(cu_seqlens[b]), int(cu_seqlens[b + 1]) - int(cu_seqlens[b])
        slot = int(slot_mapping[b]) if slot_mapping is not None else b
        ind = st.target[slot]
        drafts = [int(t) for t in drafted[margin:margin + n]]

        rows = [
            process_row(logits[margin + i], st, slot, ind, st.grammar[slot, i], drafts[:i], None)
            for i in range(n)
        ]

        if ind & GREEDY:

            selections = [int(x.argmax()) for x in rows]
            j = next((i for i in range(n - 1) if selections[i] != drafts[i]), n - 1)
            tokens = drafts[:j] + [selections[j]]
            out.append(RequestResult(offset=j, tokens=tokens, greedy=True,
                                     logprobs=[0.0] * (j + 1) if logprobs else []))
            continue

        knife = False
        values_rows, index_rows = [], []

        for x in rows:

            v, idx = bounded(x[None])
            v, k = truncate(v, ind, st, slot)
            knife |= k
            values_rows.append(v[0])
            index_rows.append(idx[0])

        values = torch.stack(values_rows)[None]          # [1, n, 128]
        indices = torch.stack(index_rows)[None]
        scores, logp = log_softmax_pair(values)          # fp32
        scores64 = values.to(F64).softmax(dim=-1)

        svgd = bool(ind & SVGD) or q_all is None
        q = torch.zeros(1, n, logits.size(-1), dtype=BF16)

        for i in range(n - 1):

            if svgd:

                q[0, i, drafts[i]] = 1.0

            else:

                q[0, i] = q_all[slot, i]

        u = st.uniform[slot, :n][None].clone()
        tok = torch.tensor(drafts, dtype=I64)[None]

        matches = indices.to(I64) == tok[..., None]
        positions = matches.int().argmax(dim=-1, keepdim=True)
        targets = scores.gather(-1, positions).squeeze(-1).masked_fill_(~matches.any(dim=-1), 0)
        lhs = q.gather(-1, tok[..., None]).squeeze(-1).mul_(u)                       # bf16
        acceptances = lhs.le(targets)
        acceptances[:, -1] = False
        j = int(acceptances.int().argmin(dim=-1))

        t64 = scores64.gather(-1, positions).squeeze(-1).masked_fill(~matches.any(dim=-1), 0)

        for i in range(min(j + 1, n - 1)):

            knife |= abs(float(lhs[0, i]) - float(t64[0, i])) <= REL * max(float(t64[0, i]), 1e-30)

        candidates = indices[0, j].to(I64)
        marginals = q[0, j].gather(-1, candidates)
        weights = planes[slot, j].gather(-1, candidates)
        z = scores[0, j].sub(marginals).clamp_min_(0).log_().sub_(weights)
        sampled = int(z.argmax())

        z64 = (scores64[0, j] - marginals.to(F64)).clamp_min(0).log() - weights.to(F64)
        finite = z64[torch.isfinite(z64)]

        if finite.numel() >= 2:

            top2 = finite.topk(2).values
            knife |= float(top2[0] - top2[1]) <= REL * max(abs(float(top2[0])), 1.0)

        emitted = drafts[:j] + [int(candidates[sampled])]
        rec = RequestResult(offset=j, tokens=emitted, greedy=False, knife=knife,
                            row_values=values_rows, row_indices=index_rows)

        if logprobs:

            pos = positions[0, :, 0].clone()
            pos[j] = sampled
            rec.logprobs = [float(logp[0, i, pos[i]]) for i in range(j + 1)]

            z_allowed = max_top_logprobs if (ind & TOP_K_LOGPROBS) else 0
            z_allowed = min(z_allowed, int(st.top_logprobs[slot]))

            for i in range(j + 1):

                rec.top_tokens.append([int(t) for t in indices[0, i, :z_allowed]])
                rec.top_logprobs.append([float(v) for v in logp[0, i, :z_allowed]])

        out.append(rec)

    return out


def apply_multistep_counts(decode: Tensor, results: List[RequestResult],
                           slot_mapping: Optional[Sequence[int]]) -> Tensor:
    """Decode counts after the verifier's update: +1 per emitted token (``ops/verify.py:425-429``)."""

    decode = decode.clone()

    for b, rec in enumerate(results):

        slot = int(slot_mapping[b]) if slot_mapping is not None else b

        for t in rec.tokens:

            decode[slot, t] += 1

    return decode


# ------------------------------------------------------------------------------------------------
# Output tolerance
# ------------------------------------------------------------------------------------------------

def bf16_within(actual: float, expected_fp32: float, rel: float = REL, floor: float = 0.0) -> bool:
    """True when the bf16 output equals the bf16 rounding of some value within `rel` (relative) of
    the fp32 reference value, or within the absolute `floor`; -inf must match exactly.

    Log-probabilities pass ``floor=LOGPROB_FLOOR``: an fp32 log-softmax ``(v - m) - log(s)`` with
    ``s = sum(exp(v - m))`` carries an absolute error of a few ulp of ``s`` (near 1) whatever the
    result's size, so close to 0 no fp32 evaluation -- the reference's included -- is relatively
    accurate to 1e-5 (e.g. log(1.0017) = 0.0017 with one ulp of s worth 7e-5 of it)."""

    if expected_fp32 == float("-inf") or actual == float("-inf"):

        return actual == expected_fp32

    band = max(abs(expected_fp32) * rel, floor) + 1e-30
    r = lambda v: float(torch.tensor(v, dtype=F32).to(BF16))  # noqa: E731

    return r(expected_fp32 - band) <= actual <= r(expected_fp32 + band)


# Absolute tolerance of fp32 log-probabilities: 4 ulp of 1.0 (see bf16_within).
LOGPROB_FLOOR = 2.0 ** -21
