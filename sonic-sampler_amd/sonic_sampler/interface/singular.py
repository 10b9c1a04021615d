"""Modular single-step sampler (reference ``interface/singular.py:41-194``)."""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

from torch import Tensor

from sonic_sampler.base.sampler import Selection, DEFAULT_TOP_LOGPROBS
from sonic_sampler.base.tensor import plain_view
from sonic_sampler.core.buffer import SamplingBuffers
from sonic_sampler.interface.base import TwoStageTiling, TopKStrategy
from sonic_sampler.interface.dispatch import TwoStageWarpConfig
from sonic_sampler.interface.functional.singular import fused_singular
from sonic_sampler.ops.base import MAX_K


def resolve_tokens(tokens: Optional[Tensor], timestep: int, in_place: bool):

    output = drafted = None

    if tokens is not None:

        if in_place:

            output = tokens[:, timestep, None]

        if timestep:

            drafted = tokens

    return output, drafted


@dataclass(eq=False, kw_only=True)
class UnshardedFusedSingular(TwoStageTiling):

    # The speculation lookahead, gamma.
    lookahead: int

    # The width Z of the top-k logprob block.
    max_top_logprobs: int

    @classmethod
    def initialize(
        cls,
        vocab_size: int,
        batch_size: int = 32,
        lookahead: int = 0,
        pdl: bool = True,
        block_size: Optional[int] = None,
        arch=None,
        max_top_logprobs: int = DEFAULT_TOP_LOGPROBS,
        device=None,
    ) -> "UnshardedFusedSingular":

        factory, _, _ = cls.factory(
            vocab_size=vocab_size,
            batch_size=batch_size,
            lookahead=lookahead,
            k=MAX_K,
            top_logprobs=max_top_logprobs,
            block_size=block_size,
            arch=arch,
            enable_pdl=pdl,
            ensure_multiblock=True,
            unpacked_buffers=False,
            device=device,
            kinds=(None, "drafting"),
        )

        return cls(
            pdl=factory.pdl,
            block_n=factory.block_n,
            lookahead=lookahead,
            max_top_logprobs=max_top_logprobs,
            vocabulary=factory.vocabulary,
            scratchpad=factory.scratchpad,
            dispatch=factory.dispatch,
            kind_dispatch=factory.kind_dispatch,
        )

    def autoregressive(
        self,
        logits: Tensor,
        buffers: SamplingBuffers,
        prefill: bool = False,
        update_counts: bool = False,
        logprobs: bool = False,
        slot_mapping: Optional[Tensor] = None,
        strategy: Optional[TopKStrategy] = None,
        tuning: Optional[TwoStageWarpConfig] = None,
        philox_seed: Optional[int] = None,
        philox_offset: int = 0,
        tile_events=None,
        kernel_layout: Optional[str] = None,
    ) -> Selection:
        """One decode step over `buffers.flags.target` with `gumbel.target[:, 0]` noise.

        ``philox_seed`` switches the noise to the counter-based Philox stream (slot, timestep 0);
        ``kernel_layout`` ("tiles" / "rowwise") overrides the library's choice of kernel layout.
        """

        penalties = buffers.repetition
        counts = penalties.counts
        config, k_strategy, block_n = self.tuning(logits.size(0), strategy, tuning)

        return fused_singular(
            logits=logits,
            indicators=buffers.flags.target,
            max_top_logprobs=self.max_top_logprobs,
            enable_pdl=self.pdl,
            is_prefill=prefill,
            update_counts=update_counts,
            return_logprobs=logprobs,
            block_n=block_n,
            scratchpad=self.scratchpad,
            slot_mapping=slot_mapping,
            grammar=plain_view(buffers.grammar, 0),
            context_counts=counts.context,
            decode_counts=counts.decode,
            repetition_penalties=penalties.multiplicative,
            frequency_penalties=penalties.frequency,
            presence_penalties=penalties.presence,
            logit_bias=buffers.bias,
            temperature=buffers.temperature,
            top_k=buffers.top_k,
            top_p=buffers.top_p,
            min_p=buffers.min_p,
            top_k_logprobs=buffers.top_logprobs,
            gumbel_noise=None if philox_seed is not None else plain_view(buffers.weights.gumbel.target, 0),
            topk_strategy=k_strategy,
            warp_config=config,
            philox_seed=philox_seed,
            philox_offset=philox_offset,
            tile_events=tile_events,
            philox_step=0,
            kernel_layout=kernel_layout,
        )

    def drafting(
        self,
        logits: Tensor,
        buffers: SamplingBuffers,
        timestep: int = 0,
        tokens: Optional[Tensor] = None,
        probabilities: Optional[Tensor] = None,
        slot_mapping: Optional[Tensor] = None,
        d2t_mapping: Optional[Tensor] = None,
        target_vocab: Optional[int] = None,
        in_place: bool = False,
        strategy: Optional[TopKStrategy] = None,
        tuning: Optional[TwoStageWarpConfig] = None,
        philox_seed: Optional[int] = None,
        philox_offset: int = 0,
        tile_events=None,
        kernel_layout: Optional[str] = None,
    ) -> Selection:
        """One draft step over `buffers.flags.draft` with `gumbel.draft[:, timestep]` noise.

        For ``timestep > 0`` the first ``timestep`` columns of ``tokens`` count as decode history;
        ``kernel_layout`` ("tiles" / "rowwise") overrides the library's choice of kernel layout.
        """

        penalties = buffers.repetition
        counts = penalties.counts
        config, k_strategy, block_n = self.tuning(logits.size(0), strategy, tuning, kind="drafting")

        output_tokens, drafted_tokens = resolve_tokens(tokens, timestep, in_place)

        return fused_singular(
            logits=logits,
            indicators=buffers.flags.draft,
            lookahead=self.lookahead,
            target_vocab=target_vocab,
            max_top_logprobs=self.max_top_logprobs,
            enable_pdl=self.pdl,
            return_probabilities=not buffers.flags.all_greedy,
            block_n=block_n,
            scratchpad=self.scratchpad,
            slot_mapping=slot_mapping,
            d2t_mapping=d2t_mapping,
            grammar=plain_view(buffers.grammar, timestep),
            context_counts=counts.context,
            decode_counts=counts.decode,
            drafted_tokens=drafted_tokens,
            repetition_penalties=penalties.multiplicative,
            frequency_penalties=penalties.frequency,
            presence_penalties=penalties.presence,
            logit_bias=buffers.bias,
            temperature=buffers.temperature,
            top_k=buffers.top_k,
            top_p=buffers.top_p,
            min_p=buffers.min_p,
            top_k_logprobs=buffers.top_logprobs,
            gumbel_noise=None if philox_seed is not None else plain_view(buffers.weights.gumbel.draft, timestep),
            output_tokens=output_tokens,
            draft_probabilities=probabilities,
            topk_strategy=k_strategy,
            warp_config=config,
            timestep=timestep,
            philox_seed=philox_seed,
            philox_offset=philox_offset,
            tile_events=tile_events,
            philox_step=timestep,
            kernel_layout=kernel_layout,
        )
