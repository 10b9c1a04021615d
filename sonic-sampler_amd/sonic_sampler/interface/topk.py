"""Standalone bounded top-k (reference ``interface/topk.py:39-161``).

``ss_topk`` makes two launches: a tile stage that writes the exact top-k of every (row, tile)
workgroup as a sorted candidate list, then a merge stage that takes the row's top-k from those
lists in descending order; for at least 48 rows of 16385-32768 columns at k <= 32 it makes one
launch instead, a 1024-thread workgroup per row. Ties go to the lowest column. bfloat16 and
float32 logits are accepted; values come back in the logits' dtype.

Returned ``values`` / ``indices`` are dense ``[..., k]`` views of the interface's buffers. (The
reference returns ``[rows, 128]`` views of buffers its kernel writes with row stride ``k``, which
mislays rows when ``k < 128``; the dense view is what that layout encodes.)
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional, Tuple

import torch

from torch import Tensor

from sonic_sampler import _native
from sonic_sampler.interface.base import TwoStageTiling, TopKStrategy, default_device
from sonic_sampler.interface.dispatch import TwoStageWarpConfig
from sonic_sampler.interface.functional.base import collapse_2d
from sonic_sampler.ops.base import MAX_K


BF16 = torch.bfloat16
FP32 = torch.float32
I32 = torch.int32

TOPK_ARGS = _native.Packer(_native.TopKArgs)


@dataclass(eq=False, kw_only=True)
class UnshardedBoundedTopK(TwoStageTiling):

    # The number of values to select.
    k: int

    # Values buffer [rows, 128] (bf16); written densely as [rows, k].
    values: Tensor

    # Indices buffer [rows, 128] (int32); written densely as [rows, k].
    indices: Tensor

    @classmethod
    def initialize(
        cls,
        vocab_size: int,
        block_size: Optional[int] = None,
        batch_size: int = 32,
        k: int = MAX_K,
        pdl: bool = True,
        arch=None,
        device=None,
    ) -> "UnshardedBoundedTopK":

        if k > MAX_K:

            raise ValueError(f"maximum supported top-k value is {MAX_K}, got {k} instead")

        if k < 1 or k.bit_count() > 1:

            raise ValueError(f"top-k value must be a power of 2, got {k} instead")

        factory, values, indices = cls.factory(
            vocab_size=vocab_size,
            batch_size=batch_size,
            k=MAX_K,
            block_size=block_size,
            arch=arch,
            enable_pdl=pdl,
            ensure_multiblock=True,
            unpacked_buffers=True,
            values_dtype=BF16,
            device=device,
            kinds=("topk",),
        )

        instance = cls(
            k=k,
            pdl=factory.pdl,
            block_n=factory.block_n,
            vocabulary=factory.vocabulary,
            scratchpad=factory.scratchpad,
            values=values,
            indices=indices,
            dispatch=factory.dispatch,
        )

        instance._wide = None

        return instance

    def clear(self) -> "UnshardedBoundedTopK":
        """Clears the buffers between correctness checks."""

        self.scratchpad.view(I32).zero_()
        self.values.fill_(-float("inf"))
        self.indices.fill_(-1)

        return self

    def _wide_buffers(self, rows: int) -> Tuple[Tensor, Tensor]:
        """64-bit candidate scratch and fp32 values for float32 logits (allocated once)."""

        if getattr(self, "_wide", None) is None:

            total = self.scratchpad.size(0)
            device = self.scratchpad.device

            self._wide = (
                torch.empty(total, self.vocabulary.blocks * MAX_K, dtype=torch.int64, device=device),
                torch.empty(total, MAX_K, dtype=FP32, device=device),
            )

        return self._wide

    def __call__(
        self,
        logits: Tensor,
        *,
        strategy: Optional[TopKStrategy] = None,
        tuning: Optional[TwoStageWarpConfig] = None,
    ) -> Tuple[Tensor, Tensor]:

        *batch_step, _ = logits.shape
        flat = collapse_2d(logits)
        n_rows = flat.size(0)

        if n_rows > self.scratchpad.size(0):

            raise ValueError(f"{n_rows} rows exceed the {self.scratchpad.size(0)} rows this "
                             "instance was initialized for")

        if flat.size(-1) != self.vocabulary.size:

            raise ValueError(f"expected {self.vocabulary.size} columns, got {flat.size(-1)}")

        if flat.stride(-1) != 1:

            raise ValueError("logits must be contiguous along the vocabulary")

        if flat.dtype not in (BF16, FP32):

            raise ValueError(f"logits must be bfloat16 or float32, got {flat.dtype}")

        _native.require_device(flat)

        _, _, block_n = self.tuning(n_rows, strategy, tuning)

        if flat.dtype == FP32:

            scratch, values = self._wide_buffers(n_rows)
            dtype = _native.SS_DTYPE_F32

        else:

            scratch, values = self.scratchpad, self.values
            dtype = _native.SS_DTYPE_BF16

        # ss_topk_args, field by field in declaration order (TOPK_ARGS.fields names them)
        packed = TOPK_ARGS.pack(
            flat.data_ptr(), flat.stride(0), dtype, n_rows, flat.size(-1), self.k, block_n, 0,
            scratch.data_ptr(), scratch.stride(0), values.data_ptr(), self.indices.data_ptr(),
            _native.stream_of(flat),
        )

        _native.check(_native.packed_entry("ss_topk")(packed), "ss_topk")

        k = self.k
        dense_values = values.view(-1)[: n_rows * k].view(n_rows, k)
        dense_indices = self.indices.view(-1)[: n_rows * k].view(n_rows, k)

        return dense_values.unflatten(0, batch_step), dense_indices.unflatten(0, batch_step)
