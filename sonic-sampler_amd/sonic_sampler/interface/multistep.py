"""Modular chain speculative verifier (reference ``interface/multistep.py:43-161``)."""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

from torch import Tensor

from sonic_sampler.base.sampler import Verification, DEFAULT_TOP_LOGPROBS
from sonic_sampler.base.tensor import plain_view
from sonic_sampler.core.buffer import SamplingBuffers
from sonic_sampler.interface.base import TwoStageTiling, TopKStrategy
from sonic_sampler.interface.dispatch import ThreeStageWarpConfig
from sonic_sampler.interface.functional.base import collapse_2d
from sonic_sampler.interface.functional.multistep import fused_multistep
from sonic_sampler.ops.base import MAX_K


@dataclass(eq=False, kw_only=True)
class UnshardedFusedMultistep(TwoStageTiling):

    # The maximum speculation lookahead, gamma.
    lookahead: int

    # The width Z of the top-k logprob block.
    max_top_logprobs: int

    # fp32 truncated log-probabilities of each row's top-128, [B * (gamma + 1), 128].
    values: Tensor

    # int32 token ids of each row's top-128, [B * (gamma + 1), 128].
    indices: Tensor

    @classmethod
    def initialize(
        cls,
        vocab_size: int,
        lookahead: int,
        batch_size: int = 32,
        pdl: bool = True,
        block_size: Optional[int] = None,
        arch=None,
        max_top_logprobs: int = DEFAULT_TOP_LOGPROBS,
        device=None,
    ) -> "UnshardedFusedMultistep":

        factory, values, indices = cls.factory(
            vocab_size=vocab_size,
            batch_size=batch_size,
            lookahead=lookahead,
            k=MAX_K,
            top_logprobs=max_top_logprobs,
            block_size=block_size,
            arch=arch,
            enable_pdl=pdl,
            ensure_multiblock=True,
            unpacked_buffers=True,
            device=device,
            kinds=("multistep",),
        )

        return cls(
            pdl=factory.pdl,
            block_n=factory.block_n,
            lookahead=lookahead,
            max_top_logprobs=max_top_logprobs,
            vocabulary=factory.vocabulary,
            scratchpad=factory.scratchpad,
            values=values,
            indices=indices,
            dispatch=factory.dispatch,
        )

    def tuning(self, size: int, strategy=None, tuning: Optional[ThreeStageWarpConfig] = None):

        base = super().tuning(size, strategy, tuning and tuning.two_stage)

        if strategy is None and tuning is None:

            # the base lookup is kept per instance; so is the three-stage config built from it
            cache = self.__dict__.setdefault("_three_stage_cache", {})
            hit = cache.get(size)

            if hit is None or hit[0] is not base:

                hit = cache[size] = (base, self._three_stage(base, None))

            return hit[1]

        return self._three_stage(base, tuning)

    def _three_stage(self, base, tuning):

        config, k_strategy, block_n = base
        config = ThreeStageWarpConfig.from_config(
            config=config, third=tuning and tuning.third, gamma=self.lookahead
        )

        return config, k_strategy, block_n

    def __call__(
        self,
        logits: Tensor,
        tokens: Tensor,
        buffers: SamplingBuffers,
        probabilities: Optional[Tensor] = None,
        slot_mapping: Optional[Tensor] = None,
        update_counts: bool = False,
        logprobs: bool = False,
        in_place: bool = False,
        strategy: Optional[TopKStrategy] = None,
        tuning: Optional[ThreeStageWarpConfig] = None,
        cu_seqlens: Optional[Tensor] = None,
        philox_seed: Optional[int] = None,
        philox_offset: int = 0,
        tile_events=None,
        all_greedy: bool = False,
    ) -> Verification:
        """Verifies the drafts in `tokens` against target `logits`.

        ``cu_seqlens`` (an addition) selects the variable-lookahead layout: ``logits`` is
        ``[sum_i (gamma_i + 1), V]`` and ``tokens`` the matching flat ``[sum_i (gamma_i + 1)]``.
        ``all_greedy`` (an addition) tells the library that every row of `buffers.flags.target` is
        greedy, which saves a launch; a request that is not greedy is then not served, and its
        ``offsets`` entry reads -1.
        """

        penalties = buffers.repetition
        counts = penalties.counts
        config, k_strategy, block_n = self.tuning(collapse_2d(logits).size(0), strategy, tuning)
        weights = buffers.weights

        return fused_multistep(
            logits=logits,
            indicators=buffers.flags.target,
            drafted_tokens=tokens,
            lookahead=self.lookahead,
            max_top_logprobs=self.max_top_logprobs,
            enable_pdl=self.pdl,
            update_counts=update_counts,
            return_logprobs=logprobs,
            # the batch-tuned tile width, as the single-step API uses (the reference passes the
            # factory's width here); the scratchpad is sized for the narrowest width of the table
            block_n=block_n,
            scratchpad=self.scratchpad,
            values=self.values,
            indices=self.indices,
            draft_probabilities=probabilities,
            slot_mapping=slot_mapping,
            cu_seqlens=cu_seqlens,
            grammar=plain_view(buffers.grammar),
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
            gumbel_noise=None if philox_seed is not None else plain_view(weights.gumbel.target),
            uniform_noise=plain_view(weights.uniform),
            output_tokens=tokens if in_place else None,
            topk_strategy=k_strategy,
            warp_config=config,
            philox_seed=philox_seed,
            philox_offset=philox_offset,
            tile_events=tile_events,
            all_greedy=all_greedy,
        )
