"""Functional single-step sampling (reference ``interface/functional/singular.py:38-322``).

``fused_singular`` keeps the reference's keyword set and buffer semantics and calls
``ss_fused_singular``, which launches the tile stage (prologue + tile top-128 per (row, tile)
workgroup) and the row stage (merge + selection per row) back to back.

Additions to the reference's keywords (all optional):

* ``timestep`` -- number of leading ``drafted_tokens`` columns that count as decode history. The
  modular ``drafting`` passes its timestep ``t`` (the reference's PyTorch semantics,
  ``core/naive.py:199-203``); when omitted, ``min(lookahead, drafted_tokens.size(1))`` columns are
  used, as the reference kernel does.
* ``philox_seed`` / ``philox_offset`` / ``philox_step`` -- draw the Gumbel noise from the
  counter-based Philox stream instead of ``gumbel_noise``. With neither given, a fresh seed is drawn
  from torch's default generator, replacing the reference's fresh ``exponential_().log_()`` plane.
* ``tile_events`` -- a pair of timing ``torch.cuda.Event`` recorded by the tile kernel's own
  dispatch at its start and end (per-kernel timing without extra stream packets).
* ``stage`` -- ``"tiles"`` launches only the tile stage (with ``world_size > 1``: this shard's
  candidate lists into slice ``local_rank`` of every scratchpad row), ``"rows"`` only the row stage
  (merge of all ``world_size`` slices and selection); ``None`` both. A tensor-parallel engine runs
  ``"tiles"``, all-gathers the scratchpad slices, then ``"rows"``.
* ``kernel_layout`` -- ``"tiles"`` (tile grid + row merge, two launches) or ``"rowwise"`` (one
  workgroup per row, one launch, rows of at most 16 tiles); ``None`` lets the library choose
  (currently the tile grid).
* ``static_scratch`` -- keep the tiles' candidate lists in the library's static device array
  (``ss_fused_singular_noalloc``) instead of a scratchpad: no scratchpad is allocated or passed,
  for callers that cannot allocate. Calls of this kind on one device share the array, so they must
  not overlap (one stream, one thread at a time); a call that needs more than
  ``SS_STATIC_SCRATCH_BYTES`` (8 MiB: rows x tiles x 512 B) raises ``RuntimeError``.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from torch import Tensor

from sonic_sampler import _native
from sonic_sampler.base.sampler import Selection, DEFAULT_TOP_LOGPROBS
from sonic_sampler.interface.base import TopKStrategy
from sonic_sampler.interface.dispatch import TwoStageWarpConfig
from sonic_sampler.interface.functional.base import (
    BF16,
    I32,
    fresh_seed,
    require_cover,
    unit_stride,
    validate_block,
    validate_count_update,
)
from sonic_sampler.ops.base import MAX_K


KERNEL_LAYOUTS = {None: _native.STRATEGY_AUTO, "tiles": _native.STRATEGY_TILES,
                  "rowwise": _native.STRATEGY_ROWWISE}

STAGES = {None: 0, "tiles": _native.STAGE_TILES, "rows": _native.STAGE_ROWS}

SINGULAR_ARGS = _native.Packer(_native.SingularArgs)


def resolve_tokens(buffer: Optional[Tensor], batch_size: int, source: Tensor) -> Tensor:

    return buffer if buffer is not None else source.new_empty(batch_size, 1, dtype=I32)


def resolve_probabilities(precondition: bool, source: Tensor, batch_size: int,
                          vocab_size: Optional[int] = None, buffer: Optional[Tensor] = None):

    if buffer is None and precondition:

        return source.new_zeros((batch_size, vocab_size or source.size(1)))

    return buffer


def fused_singular(
    # Required.
    logits: Tensor,
    indicators: Tensor,
    # Model & Engine Specific(s).
    local_vocab: Optional[int] = None,
    shard_size: Optional[int] = None,
    world_size: int = 1,
    local_rank: int = 0,
    lookahead: int = 0,
    target_vocab: Optional[int] = None,
    max_top_logprobs: int = DEFAULT_TOP_LOGPROBS,
    # Conditional(s).
    enable_pdl: bool = True,
    is_prefill: bool = False,
    update_counts: bool = False,
    return_logprobs: bool = False,
    return_probabilities: bool = False,
    # Kernel Specific(s).
    block_n: int = 4_096,
    # Buffer(s).
    scratchpad: Optional[Tensor] = None,
    # Logit Manipulator(s).
    slot_mapping: Optional[Tensor] = None,
    d2t_mapping: Optional[Tensor] = None,
    grammar: Optional[Tensor] = None,
    context_counts: Optional[Tensor] = None,
    decode_counts: Optional[Tensor] = None,
    drafted_tokens: Optional[Tensor] = None,
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
    # Output Buffer(s).
    output_tokens: Optional[Tensor] = None,
    draft_probabilities: Optional[Tensor] = None,
    # Top-K Strategy & Tuning Configuration.
    topk_strategy: Optional[TopKStrategy] = None,
    warp_config: Optional[TwoStageWarpConfig] = None,
    # Additions.
    timestep: Optional[int] = None,
    philox_seed: Optional[int] = None,
    philox_offset: int = 0,
    philox_step: int = 0,
    tile_events: Optional[Tuple[torch.cuda.Event, torch.cuda.Event]] = None,
    kernel_layout: Optional[str] = None,
    static_scratch: bool = False,
    stage: Optional[str] = None,
) -> Selection:

    validate_count_update(update_counts, decode_counts)
    validate_block(block_n)

    if kernel_layout not in KERNEL_LAYOUTS:

        raise ValueError(f"kernel_layout must be one of {sorted(k for k in KERNEL_LAYOUTS if k)} or None")

    if world_size < 1 or not 0 <= local_rank < world_size:

        raise ValueError(f"local rank {local_rank} outside a world of {world_size} shards")

    if stage not in STAGES:

        raise ValueError(f"stage must be one of {sorted(k for k in STAGES if k)} or None")

    if logits.dim() == 2 and (shard_size or 0) and shard_size < min(logits.size(1), local_vocab or logits.size(1)):

        raise ValueError(f"shard size {shard_size} is smaller than the local vocabulary")

    if logits.dtype != BF16 or logits.dim() != 2:

        raise ValueError(f"logits must be a 2-D bfloat16 tensor, got {logits.dtype} {tuple(logits.shape)}")

    if not 0 <= max_top_logprobs <= MAX_K:

        raise ValueError(f"top logprobs must be within the interval [0, {MAX_K}]")

    for name, t in (("logits", logits), ("grammar", grammar), ("context_counts", context_counts),
                    ("decode_counts", decode_counts), ("logit_bias", logit_bias),
                    ("gumbel_noise", gumbel_noise), ("draft_probabilities", draft_probabilities),
                    ("indicators", indicators), ("drafted_tokens", drafted_tokens)):

        unit_stride(name, t)

    _native.require_device(logits, indicators)

    batch_size, vocab_size = logits.shape
    vocab_size = min(vocab_size, local_vocab or vocab_size)
    shard_size = shard_size or vocab_size

    vocab_blocks = -(-vocab_size // block_n)

    if vocab_blocks <= 1:

        raise ValueError(f"total vocab blocks must be greater than 1, got {vocab_blocks} instead")

    if static_scratch:

        bitpacked = None

    elif scratchpad is None:

        bitpacked = logits.new_empty(batch_size, world_size * vocab_blocks * MAX_K, dtype=I32).view(torch.uint32)

    else:

        bitpacked = scratchpad

        if (bitpacked.size(0) < batch_size or bitpacked.stride(-1) != 1
                or bitpacked.stride(0) < world_size * vocab_blocks * MAX_K):

            raise ValueError("scratchpad too small for the given logits, block_n and world size")

    final_tokens = resolve_tokens(output_tokens, batch_size, logits)
    # the width of the probability rows and of the processors' per-slot planes
    target_width = target_vocab or (logit_bias.size(-1) if logit_bias is not None else world_size * shard_size)

    if return_probabilities:

        # the selection scatters at [slot, target id]: every slot of the buffers with a slot mapping
        require_cover("draft_probabilities", draft_probabilities,
                      indicators.size(0) if slot_mapping is not None else batch_size, target_width)

    probabilities = resolve_probabilities(
        precondition=return_probabilities,
        source=logits,
        batch_size=indicators.size(0),
        vocab_size=target_vocab,
        buffer=draft_probabilities,
    )

    selection = Selection.from_buffers(
        tokens=final_tokens,
        probabilities=probabilities,
        logprobs=return_logprobs,
        top_logprobs=max_top_logprobs,
    )

    token_logprobs = top_values = top_tokens = None

    if selection.logprobs is not None:

        token_logprobs = selection.logprobs.selected

        if selection.logprobs.top_k is not None:

            top_values = selection.logprobs.top_k.logprobs
            top_tokens = selection.logprobs.top_k.tokens

    if gumbel_noise is None and philox_seed is None:

        philox_seed = fresh_seed()

    history = 0

    if drafted_tokens is not None:

        history = timestep if timestep is not None else min(lookahead, drafted_tokens.size(1))
        history = max(0, min(history, drafted_tokens.size(1)))

    a = _native.addr
    s = _native.stride0
    philox_on = philox_seed is not None
    tile_start, tile_end = _native.event_pair(tile_events)

    # ss_singular_args, field by field in declaration order (SINGULAR_ARGS.fields names them)
    packed = SINGULAR_ARGS.pack(
        a(logits), logits.stride(0), batch_size, vocab_size,
        target_width, block_n, lookahead, history, max_top_logprobs if top_values is not None else 0,
        int(is_prefill), int(update_counts), int(token_logprobs is not None), int(probabilities is not None),
        KERNEL_LAYOUTS[kernel_layout],
        a(indicators), a(slot_mapping), a(d2t_mapping),
        a(grammar), s(grammar), a(context_counts), s(context_counts), a(decode_counts), s(decode_counts),
        a(drafted_tokens) if history else 0, s(drafted_tokens),
        a(repetition_penalties), a(frequency_penalties), a(presence_penalties),
        a(logit_bias), s(logit_bias),
        a(temperature), a(top_k), a(top_p), a(min_p), a(top_k_logprobs),
        0 if philox_on else a(gumbel_noise), 0 if philox_on else s(gumbel_noise),
        philox_seed & 0xFFFFFFFFFFFFFFFF if philox_on else 0, philox_offset & 0xFFFFFFFF if philox_on else 0,
        int(philox_on), philox_step, STAGES[stage],
        a(final_tokens), final_tokens.stride(0), a(token_logprobs), s(token_logprobs),
        a(top_values), a(top_tokens), s(top_values), a(probabilities), s(probabilities),
        a(bitpacked), s(bitpacked), _native.stream_of(logits),
        tile_start or 0, tile_end or 0, world_size, local_rank, shard_size, 0,
    )

    entry = "ss_fused_singular_noalloc" if static_scratch else "ss_fused_singular"
    _native.check(_native.packed_entry(entry)(packed), entry)

    return selection
