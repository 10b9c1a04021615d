"""Tiling rung: dispatch resolution and in-flight buffer ownership (reference
``interface/base.py:45-276``).

``TwoStageTiling.factory`` resolves ``block_n`` from the dispatch table (or ``block_size``),
validates the configuration with the reference's ``ValueError`` conditions and allocates the
in-flight buffers: ``scratchpad [B * (gamma + 1), blocks * 128]`` uint32 and, for the verifier,
``values`` / ``indices [B * (gamma + 1), 128]``.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, Optional, Tuple, Union

import torch

from torch import Tensor

from sonic_sampler.base.sampler import DEFAULT_TOP_LOGPROBS
from sonic_sampler.interface.dispatch import (
    DispatchSummary,
    RuntimeConfig,
    TwoStageWarpConfig,
    VocabBucket,
)
from sonic_sampler.ops.base import MAX_K


FP32 = torch.float32
BF16 = torch.bfloat16
I32 = torch.int32
U32 = torch.uint32

# Tile widths the gfx950 kernels are compiled for.
SUPPORTED_BLOCK_N = (1024, 2048, 4096, 8192, 16384)


def cdiv(a: int, b: int) -> int:

    return -(-a // b)


@dataclass(eq=False)
class Vocabulary:

    # Columns of the logits.
    size: int

    # Vocabulary tiles.
    blocks: int

    @classmethod
    def resolve(cls, size: int, block_n: int) -> "Vocabulary":

        return cls(size=size, blocks=cdiv(size, block_n))

    def evolve(self, block_n: int) -> "Vocabulary":

        return Vocabulary(size=self.size, blocks=cdiv(self.size, block_n))


@dataclass(eq=True)
class TopKStrategy:

    """Tile-selection strategy selector (reference ``interface/base.py:63-118``).

    Accepted for API compatibility. The gfx950 kernels always use the exact LDS radix threshold
    select, which returns the same candidates as every reference strategy.
    """

    radix: bool = False
    sparse: bool = False
    scale: int = 4

    @classmethod
    def adaptive(cls, scale: int = 4) -> "TopKStrategy":

        return cls(radix=True, sparse=True, scale=scale)

    @classmethod
    def resolve(cls, config: RuntimeConfig) -> "TopKStrategy":

        if config.strategy == "radix":

            return cls(radix=True)

        if config.strategy == "adaptive":

            return cls.adaptive()

        return cls()

    @property
    def key(self) -> str:

        if self.radix:

            return "adaptive" if self.sparse else "radix"

        return "bitonic"

    @property
    def is_adaptive(self) -> bool:

        return self.radix and self.sparse

    @property
    def is_alternating(self) -> bool:

        return not self.radix

    @property
    def inverse(self) -> Optional[float]:

        return 1 / self.scale if self.is_adaptive else None


def resolve_dispatch(
    k: int,
    vocab_size: int,
    block_size: Optional[int],
    arch: Union[int, str, None],
    kind: Optional[str] = None,
) -> Tuple[Optional[VocabBucket], int]:
    """The vocabulary bucket of the table (of call kind `kind` where it has its own table with a
    bucket for `vocab_size`) and its smallest width, or no bucket and `block_size`."""

    if k > MAX_K:

        raise ValueError(f"maximum supported top-k value is {MAX_K}, got {k} instead")

    if k < 1 or k.bit_count() > 1:

        raise ValueError(f"top-k value must be a power of 2, got {k} instead")

    if block_size is None:

        if (dispatch := DispatchSummary.load(k=MAX_K, arch=arch)) is None:

            raise ValueError("unable to resolve dispatch summary for given top-k and architecture")

        if (bucket := dispatch.vocab.get(size=vocab_size)) is None:

            raise ValueError("unable to match tuning configuration for given vocabulary size")

        if kind is not None and (table := DispatchSummary.load(k=MAX_K, arch=arch, kind=kind)) is not None:

            if (own := table.vocab.get(size=vocab_size)) is not None:

                bucket = own

        return bucket, bucket.block_n

    if block_size not in SUPPORTED_BLOCK_N:

        raise ValueError(f"block_size must be one of {SUPPORTED_BLOCK_N}, got {block_size}")

    return None, block_size


def default_device(device=None) -> torch.device:

    if device is not None:

        return torch.device(device)

    current = torch.get_default_device()

    if current.type == "cpu" and torch.cuda.is_available():

        return torch.device(f"cuda:{torch.cuda.current_device()}")

    return current


@dataclass(eq=False, kw_only=True)
class TwoStageTiling:

    # Accepted for API compatibility (programmatic dependent launch has no gfx950 counterpart;
    # the stages are ordered launches on one stream).
    pdl: bool

    # Tile width.
    block_n: int

    # Vocabulary and tiles.
    vocabulary: Vocabulary

    # uint32 candidate buffer [rows, blocks * 128].
    scratchpad: Tensor

    # Tuned dispatch, when resolved from a table.
    dispatch: Optional[VocabBucket]

    # Tuned dispatch of further call kinds that share the buffers (`tuning(..., kind=)`).
    kind_dispatch: Dict[str, VocabBucket] = field(default_factory=dict)

    @classmethod
    def resolve(
        cls,
        vocab_size: int,
        k: int = MAX_K,
        top_logprobs: int = DEFAULT_TOP_LOGPROBS,
        block_size: Optional[int] = None,
        arch: Union[int, str, None] = None,
        ensure_multiblock: bool = True,
        kind: Optional[str] = None,
    ):

        dispatch, block_n = resolve_dispatch(k, vocab_size, block_size, arch, kind)
        vocabulary = Vocabulary.resolve(vocab_size, block_n)

        if ensure_multiblock and (blocks := vocabulary.blocks) <= 1:

            raise ValueError(f"total vocab blocks must be greater than 1, got {blocks} instead")

        if top_logprobs < 0 or top_logprobs > MAX_K:

            raise ValueError(f"top logprobs must be within the interval [0, {MAX_K}]")

        return dispatch, vocabulary, block_n

    @classmethod
    def factory(
        cls,
        vocab_size: int,
        batch_size: int = 32,
        lookahead: int = 0,
        k: int = MAX_K,
        top_logprobs: int = DEFAULT_TOP_LOGPROBS,
        block_size: Optional[int] = None,
        arch: Union[int, str, None] = None,
        enable_pdl: bool = True,
        ensure_multiblock: bool = True,
        unpacked_buffers: bool = True,
        values_dtype: torch.dtype = FP32,
        device=None,
        kinds: Tuple[Optional[str], ...] = (None,),
    ):
        """`kinds` names the call kinds that will use the buffers: the first one's table gives
        `dispatch`, the others' go to `kind_dispatch`, and the scratchpad holds the lists of the
        smallest width among them (None: the shared table)."""

        resolved = [cls.resolve(vocab_size=vocab_size, k=k, top_logprobs=top_logprobs, block_size=block_size,
                                arch=arch, ensure_multiblock=ensure_multiblock, kind=kind) for kind in kinds]
        dispatch = resolved[0][0]
        _, vocabulary, block_n = min(resolved, key=lambda r: r[2])
        extra = {kind: r[0] for kind, r in zip(kinds[1:], resolved[1:]) if kind is not None and r[0] is not None}

        target = default_device(device)
        total_rows = batch_size * (lookahead + 1)

        with torch.device(target):

            scratchpad = torch.empty(total_rows, vocabulary.blocks * k, dtype=I32).view(U32)

            values = indices = None

            if unpacked_buffers:

                values = torch.empty(total_rows, k, dtype=values_dtype)
                indices = torch.empty(total_rows, k, dtype=I32)

        instance = TwoStageTiling(
            pdl=enable_pdl,
            block_n=block_n,
            vocabulary=vocabulary,
            scratchpad=scratchpad,
            dispatch=dispatch,
            kind_dispatch=extra,
        )

        return instance, values, indices

    def tuning(
        self,
        size: int,
        strategy: Optional[TopKStrategy] = None,
        tuning: Optional[TwoStageWarpConfig] = None,
        kind: Optional[str] = None,
    ):
        """Warp config, strategy and block_n for a launch of `size` rows (reference ``:243-276``),
        from the table of call kind `kind` where the buffers were made for it. Without an explicit
        strategy or tuning the answer depends only on `size`, `kind` and the instance's tables, and
        is kept per instance (an eager call's host path looks it up once per row count)."""

        if strategy is None and tuning is None:

            cache = self.__dict__.setdefault("_tuning_cache", {})
            key = (size, kind, self.block_n)
            hit = cache.get(key)

            # an entry holds the tables it was computed from: replacing them invalidates it
            if hit is None or hit[0] is not self.dispatch or hit[1] is not self.kind_dispatch:

                hit = cache[key] = (self.dispatch, self.kind_dispatch, self._tuning(size, None, None, kind))

            return hit[2]

        return self._tuning(size, strategy, tuning, kind)

    def _tuning(self, size, strategy, tuning, kind):

        block_size = self.block_n
        k_strategy = strategy
        config = tuning
        dispatch = self.kind_dispatch.get(kind, self.dispatch) if kind is not None else self.dispatch

        if config is None and dispatch and (bucket := dispatch.batch.get(size=size)):

            if strategy and strategy.key in bucket.mapping:

                target = bucket.get(strategy.key)
                config, block_size = target.warp_config, target.block_n

            else:

                best = bucket.best
                config, block_size = best.warp_config, best.block_n
                k_strategy = k_strategy or TopKStrategy.resolve(best)

        # A vocabulary bucket spans many sizes, and a width tuned for its larger ones can leave a
        # smaller vocabulary in one tile, which the kernels do not take: the width the buffers
        # were made for (at least two tiles, checked at initialization) is used instead.
        if cdiv(self.vocabulary.size, block_size) < 2:

            block_size = self.block_n

        return config or TwoStageWarpConfig.default(), k_strategy or TopKStrategy(), block_size
