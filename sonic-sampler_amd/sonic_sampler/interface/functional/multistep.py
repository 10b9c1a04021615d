"""Functional chain speculative verification (reference
``interface/functional/multistep.py:50-461``).

``fused_multistep`` keeps the reference's keyword set and layouts (fixed-gamma ``[B, gamma + 1, V]``
logits, or varlen ``[sum_i (gamma_i + 1), V]`` logits with ``cu_seqlens``) and calls
``ss_fused_multistep``, which launches the tile stage (prologue + tile top-128), the row stage
(merge, truncation, softmax) and the request stage (chain verification) back to back.

Additions to the reference's keywords (all optional): ``philox_seed`` / ``philox_offset`` (Gumbel
noise from the Philox stream instead of ``gumbel_noise``; a fresh seed is drawn when neither is
given); ``tile_events`` (a pair of timing ``torch.cuda.Event`` recorded by the tile kernel's own
dispatch at its start and end).

``values`` receives the truncated fp32 log-probabilities of each row's top-128 (the reference
stores their exponentials); ``indices`` the matching token ids.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from torch import Tensor

from sonic_sampler import _native
from sonic_sampler.base.sampler import Verification, DEFAULT_TOP_LOGPROBS
from sonic_sampler.interface.base import TopKStrategy
from sonic_sampler.interface.dispatch import ThreeStageWarpConfig
from sonic_sampler.interface.functional.base import (
    BF16,
    I32,
    collapse_2d,
    fresh_seed,
    require_cover,
    resolve_scratchpad,
    unit_stride,
    validate_block,
    validate_count_update,
)
from sonic_sampler.ops.base import MAX_K


FP32 = torch.float32
TINY: float = torch.finfo(BF16).tiny

MULTISTEP_ARGS = _native.Packer(_native.MultistepArgs)


def resolve_batch_vocab(logits: Tensor, cu_seqlens: Optional[Tensor], lookahead: Optional[int]):
    """(varlen, batch, gamma, vocab) from the logits layout (reference ``:50-106``)."""

    varlen = cu_seqlens is not None

    if logits.ndim == 2:

        n_rows, vocab_size = logits.shape

        if varlen:

            if not lookahead:

                raise ValueError("maximum lookahead must be defined for varlen logits")

            return varlen, cu_seqlens.size(0) - 1, lookahead, vocab_size

        if not lookahead:

            raise ValueError("found 2-D logits with zero lookahead")

        batch_size, margin = divmod(n_rows, lookahead + 1)

        if margin:

            raise ValueError("not varlen but total rows not a multiple of lookahead + 1")

        return varlen, batch_size, lookahead, vocab_size

    if logits.ndim == 3:

        if varlen:

            raise ValueError("expected varlen but logits has a fixed timestep dimension")

        batch_size, timesteps, vocab_size = logits.shape

        return varlen, batch_size, timesteps - 1, vocab_size

    raise ValueError(f"unsupported logits shape: {tuple(logits.shape)}")


def resolve_unpack_buffers(logits: Tensor, values: Optional[Tensor], indices: Optional[Tensor]):

    n_rows = collapse_2d(logits).size(0)

    values = values if values is not None else logits.new_empty((n_rows, MAX_K), dtype=FP32)
    indices = indices if indices is not None else logits.new_empty((n_rows, MAX_K), dtype=I32)

    if values.dtype != FP32 or indices.dtype != I32 or values.size(0) < n_rows or indices.size(0) < n_rows:

        raise ValueError("values / indices must be float32 / int32 buffers of >= rows x 128")

    if not (values.is_contiguous() and indices.is_contiguous()):

        raise ValueError("values / indices buffers must be contiguous")

    return values, indices


def resolve_uniform(noise: Optional[Tensor], logits: Tensor, batch_size: int, lookahead: int) -> Tensor:

    if noise is None:

        return logits.new_empty((batch_size, max(lookahead, 1))).uniform_(TINY, 1)

    return noise


def resolve_tokens(drafted: Tensor, output: Optional[Tensor]) -> Tensor:
    """The output token buffer: the caller's, or a new one. The reference clones the drafts here
    (``:163-165``); the request stage writes every row itself (the drafts, each request's emitted
    token at its offset), so a new buffer holds the same tokens without a copy launch ahead of the
    tile stage."""

    return output if output is not None else torch.empty_like(drafted, memory_format=torch.contiguous_format)


def fused_multistep(
    # Required.
    logits: Tensor,
    indicators: Tensor,
    drafted_tokens: Tensor,
    # Model & Engine Specific(s).
    local_vocab: Optional[int] = None,
    shard_size: Optional[int] = None,
    world_size: int = 1,
    local_rank: int = 0,
    lookahead: Optional[int] = None,
    max_top_logprobs: int = DEFAULT_TOP_LOGPROBS,
    # Conditional(s).
    enable_pdl: bool = True,
    update_counts: bool = False,
    return_logprobs: bool = False,
    # Kernel Specific(s).
    block_n: int = 4_096,
    # Buffer(s).
    scratchpad: Optional[Tensor] = None,
    values: Optional[Tensor] = None,
    indices: Optional[Tensor] = None,
    # Support(s).
    draft_probabilities: Optional[Tensor] = None,
    # Logit Manipulator(s).
    slot_mapping: Optional[Tensor] = None,
    cu_seqlens: Optional[Tensor] = None,
    grammar: Optional[Tensor] = None,
    context_counts: Optional[Tensor] = None,
    decode_counts: Optional[Tensor] = None,
    repetition_penalties: Optional[Tensor] = None,
    frequency_penalties: Optional[Tensor] = None,
    presence_penalties: Optional[Tensor] = None,
    logit_bias: Optional[Tensor] = None,
    temperature: Optional[Tensor] = None,
    top_k: Optional[Tensor] = None,
    top_p: Optional[Tensor] = None,
    min_p: Optional[Tensor] = None,
    # Selection Parameter(s).
    top_k_logprobs: Optional[Tensor] = None,
    gumbel_noise: Optional[Tensor] = None,
    uniform_noise: Optional[Tensor] = None,
    # Output Buffer(s).
    output_tokens: Optional[Tensor] = None,
    # Top-K Strategy & Tuning Configuration.
    topk_strategy: Optional[TopKStrategy] = None,
    warp_config: Optional[ThreeStageWarpConfig] = None,
    # Additions.
    philox_seed: Optional[int] = None,
    philox_offset: int = 0,
    tile_events: Optional[Tuple[torch.cuda.Event, torch.cuda.Event]] = None,
    all_greedy: bool = False,
) -> Verification:

    validate_count_update(update_counts, decode_counts)
    validate_block(block_n)

    if world_size != 1 or local_rank != 0:

        raise ValueError("sharded-vocabulary scratchpads are not supported by the gfx950 path "
                         "(gather the logits first)")

    varlen, batch_size, gamma, vocab_size = resolve_batch_vocab(logits, cu_seqlens, lookahead)

    if logits.dtype != BF16:

        raise ValueError(f"logits must be bfloat16, got {logits.dtype}")

    if gamma > 63:

        raise ValueError(f"lookahead above 63 is not supported, got {gamma}")

    if not 0 <= max_top_logprobs <= MAX_K:

        raise ValueError(f"top logprobs must be within the interval [0, {MAX_K}]")

    vocab_size = min(vocab_size, local_vocab or vocab_size)

    flat_logits = collapse_2d(logits)

    for name, t in (("logits", flat_logits), ("grammar", grammar), ("context_counts", context_counts),
                    ("decode_counts", decode_counts), ("logit_bias", logit_bias),
                    ("gumbel_noise", gumbel_noise), ("draft_probabilities", draft_probabilities),
                    ("indicators", indicators)):

        unit_stride(name, t)

    if not drafted_tokens.is_contiguous():

        raise ValueError("drafted_tokens must be contiguous")

    _native.require_device(logits, indicators, drafted_tokens)

    rows = flat_logits.size(0)
    # draft probabilities are read at [slot, step, token]: every slot of the buffers with a slot
    # mapping, every step of the lookahead
    require_cover("draft_probabilities", draft_probabilities,
                  indicators.size(0) if slot_mapping is not None else batch_size, vocab_size, steps=max(gamma, 1))

    _, _, bitpacked, vocab_blocks = resolve_scratchpad(flat_logits, block_n, scratchpad)
    values_buffer, indices_buffer = resolve_unpack_buffers(flat_logits, values, indices)

    uniform_weights = resolve_uniform(uniform_noise, logits, batch_size, gamma)

    if gumbel_noise is None and philox_seed is None:

        philox_seed = fresh_seed()

    tokens = resolve_tokens(drafted_tokens, output_tokens)

    if not tokens.is_contiguous():

        raise ValueError("output tokens must be contiguous")

    verification = Verification.from_tokens(
        tokens=tokens,
        batch_size=batch_size,
        timesteps=gamma + 1,
        logprobs=return_logprobs,
        varlen=varlen,
        top_logprobs=max_top_logprobs,
    )

    token_logprobs = top_values = top_tokens = None

    if verification.logprobs is not None:

        token_logprobs = verification.logprobs.selected

        if verification.logprobs.top_k is not None:

            top_values = collapse_2d(verification.logprobs.top_k.logprobs)
            top_tokens = collapse_2d(verification.logprobs.top_k.tokens)

    a = _native.addr
    s = _native.stride0

    def step_stride(t: Optional[Tensor]) -> int:

        return 0 if t is None else (t.stride(1) if t.dim() >= 3 else 0)

    philox_on = philox_seed is not None
    tile_start, tile_end = _native.event_pair(tile_events)

    # ss_multistep_args, field by field in declaration order (MULTISTEP_ARGS.fields names them).
    # all_greedy: the caller vouches that every row is greedy, so each request's argmax is taken in
    # the request stage and the row launch is skipped. A hint, never inferred here: a captured graph
    # replays whatever was decided at capture while the indicators may change in place between
    # replays.
    packed = MULTISTEP_ARGS.pack(
        a(flat_logits), flat_logits.stride(0), rows, batch_size, vocab_size, block_n, gamma,
        max_top_logprobs if top_values is not None else 0, int(update_counts), int(token_logprobs is not None),
        a(cu_seqlens), a(indicators), a(slot_mapping), a(drafted_tokens),
        a(grammar), s(grammar), step_stride(grammar),
        a(context_counts), s(context_counts), a(decode_counts), s(decode_counts),
        a(repetition_penalties), a(frequency_penalties), a(presence_penalties), a(logit_bias), s(logit_bias),
        a(temperature), a(top_k), a(top_p), a(min_p), a(top_k_logprobs),
        a(draft_probabilities), s(draft_probabilities), step_stride(draft_probabilities),
        a(uniform_weights), s(uniform_weights),
        0 if philox_on else a(gumbel_noise), 0 if philox_on else s(gumbel_noise),
        0 if philox_on else step_stride(gumbel_noise),
        philox_seed & 0xFFFFFFFFFFFFFFFF if philox_on else 0, philox_offset & 0xFFFFFFFF if philox_on else 0,
        int(philox_on),
        a(tokens), a(verification.offsets), a(token_logprobs), a(top_values), a(top_tokens), s(top_values),
        a(values_buffer), a(indices_buffer), a(bitpacked), bitpacked.stride(0), _native.stream_of(logits),
        tile_start or 0, tile_end or 0, int(bool(all_greedy)),
    )

    _native.check(_native.packed_entry("ss_fused_multistep")(packed), "ss_fused_multistep")

    return verification
