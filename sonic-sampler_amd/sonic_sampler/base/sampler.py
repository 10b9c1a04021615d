"""Output containers of the sampling and verification calls.

Shapes and dtypes follow the reference (``base/sampler.py:35-199``): tokens int32, logprobs
bfloat16, top-k logprobs ``[B, Z]`` / ``[B, gamma + 1, Z]`` (or ``[sum L, Z]`` in the varlen
layout).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Final, Optional

import torch

from torch import Tensor


DEFAULT_TOP_LOGPROBS: Final[int] = 5

I32: torch.dtype = torch.int32
BF16: torch.dtype = torch.bfloat16


@dataclass(eq=False)
class TopTargets:

    # The top-k tokens with shape [ B, Z ] or [ B, gamma + 1, Z ].
    tokens: Tensor

    # Their log-probabilities, same shape.
    logprobs: Tensor

    @classmethod
    def empty_blocked(cls, batch_size: int, targets: int, timesteps: int = 1,
                      device=None) -> Optional["TopTargets"]:

        if targets > 0:

            shape = (batch_size, timesteps, targets) if timesteps > 1 else (batch_size, targets)

            return cls(tokens=torch.empty(shape, dtype=I32, device=device),
                       logprobs=torch.empty(shape, dtype=BF16, device=device))

        return None

    @classmethod
    def empty_varlen(cls, num_tokens: int, targets: int, device=None) -> Optional["TopTargets"]:

        if targets > 0:

            return cls(
                tokens=torch.empty(num_tokens, targets, dtype=I32, device=device),
                logprobs=torch.empty(num_tokens, targets, dtype=BF16, device=device),
            )

        return None


@dataclass(eq=False)
class LogProbabilities:

    # The selected tokens' log-probabilities, [ B, 1 ] or [ B, gamma + 1 ] (varlen: [ sum L ]).
    selected: Tensor

    # The top-k tokens and their log-probabilities.
    top_k: Optional[TopTargets] = None

    @classmethod
    def empty_blocked(cls, batch_size: int, timesteps: int = 1, top_k: int = 0,
                      device=None) -> "LogProbabilities":
        """`device` None: the current default device (the reference allocates under a device
        context; an explicit device avoids entering one on every call)."""

        selected = torch.empty(batch_size, timesteps, dtype=BF16, device=device)

        return cls(selected=selected, top_k=TopTargets.empty_blocked(batch_size, top_k, timesteps, device=device))

    @classmethod
    def empty_varlen(cls, num_tokens: int, top_k: int = 0, device=None) -> "LogProbabilities":

        selected = torch.empty(num_tokens, dtype=BF16, device=device)

        return cls(selected=selected, top_k=TopTargets.empty_varlen(num_tokens, top_k, device=device))


@dataclass(eq=False)
class Selection:

    # The selected next tokens, [ B, 1 ] int32.
    tokens: Tensor

    # The truncated distribution scattered over the target vocabulary, [ B, V_t ] bf16.
    probabilities: Optional[Tensor] = None

    # The selected tokens' log-probabilities.
    logprobs: Optional[LogProbabilities] = None

    @classmethod
    def from_buffers(
        cls,
        tokens: Tensor,
        probabilities: Optional[Tensor] = None,
        logprobs: bool = False,
        top_logprobs: int = 0,
    ) -> "Selection":

        buffer = None

        if logprobs:

            buffer = LogProbabilities.empty_blocked(batch_size=tokens.size(0), top_k=top_logprobs,
                                                    device=tokens.device)

        return cls(tokens=tokens, probabilities=probabilities, logprobs=buffer)

    @classmethod
    def empty(
        cls,
        batch_size: int,
        vocab_size: int,
        device: torch.device,
        probs: bool = False,
        logprobs: bool = False,
        top_logprobs: int = 0,
    ) -> "Selection":

        with torch.device(device):

            tokens = torch.empty((batch_size, 1), dtype=I32)
            probabilities = torch.empty((batch_size, vocab_size), dtype=BF16) if probs else None
            buffer = LogProbabilities.empty_blocked(batch_size, top_k=top_logprobs) if logprobs else None

            return cls(tokens=tokens, probabilities=probabilities, logprobs=buffer)


@dataclass(eq=False)
class Verification:

    # The drafted tokens with the correction / bonus token written at `offsets`, [ B, gamma + 1 ].
    tokens: Tensor

    # The number of accepted draft tokens, [ B, 1 ] int32.
    offsets: Tensor

    # The emitted tokens' log-probabilities.
    logprobs: Optional[LogProbabilities] = None

    @classmethod
    def from_tokens(
        cls,
        tokens: Tensor,
        batch_size: int,
        timesteps: int,
        logprobs: bool = False,
        varlen: bool = False,
        top_logprobs: int = 0,
    ) -> "Verification":

        buffer = None
        device = tokens.device
        offsets = tokens.new_empty(batch_size, 1, dtype=I32)

        if logprobs:

            if varlen:

                buffer = LogProbabilities.empty_varlen(tokens.size(0), top_k=top_logprobs, device=device)

            else:

                buffer = LogProbabilities.empty_blocked(batch_size, timesteps, top_k=top_logprobs, device=device)

        return cls(tokens=tokens, offsets=offsets, logprobs=buffer)
