"""Argument resolution shared by the functional entry points (reference
``interface/functional/base.py:34-77``)."""

from __future__ import annotations

import random as _random
from typing import Optional, Tuple

import torch

from torch import Tensor

from sonic_sampler import _native
from sonic_sampler.interface.base import SUPPORTED_BLOCK_N
from sonic_sampler.ops.base import MAX_K

U32 = torch.uint32
I32 = torch.int32
BF16 = torch.bfloat16


def cdiv(a: int, b: int) -> int:

    return -(-a // b)


def validate_count_update(flag: bool, buffer: Optional[Tensor]) -> None:

    if flag and buffer is None:

        raise ValueError("`update_counts` is True but `decode_counts` is None")


def validate_block(block_n: int) -> None:

    if block_n not in SUPPORTED_BLOCK_N:

        raise ValueError(f"block_n must be one of {SUPPORTED_BLOCK_N}, got {block_n}")


def resolve_scratchpad(logits: Tensor, block_n: int, buffer: Optional[Tensor] = None):

    rows, cols = logits.shape if logits.ndim == 2 else logits.flatten(0, 1).shape
    vocab_blocks = cdiv(cols, block_n)

    if vocab_blocks <= 1:

        raise ValueError(f"total vocab blocks must be greater than 1, got {vocab_blocks} instead")

    scratchpad = buffer

    if scratchpad is None:

        scratchpad = logits.new_empty(rows, vocab_blocks * MAX_K, dtype=I32).view(U32)

    elif scratchpad.size(0) < rows or scratchpad.stride(-1) != 1 or scratchpad.stride(0) < vocab_blocks * MAX_K:

        raise ValueError("scratchpad too small for the given logits and block_n")

    return (rows, vocab_blocks), (rows,), scratchpad, vocab_blocks


def collapse_2d(value: Tensor) -> Tensor:

    return value.flatten(0, -2)


def unit_stride(name: str, tensor: Optional[Tensor]) -> None:

    if tensor is not None and tensor.dim() > 0 and tensor.stride(-1) != 1:

        raise ValueError(f"`{name}` must be contiguous along its last dimension")


def require_cover(name: str, tensor: Optional[Tensor], rows: int, cols: int, steps: int = 1) -> None:
    """A buffer the kernels address by slot: rows [0, rows), columns [0, cols) and, for a
    [slots, steps, cols] buffer, steps [0, steps). Its storage must hold the last such element: a
    strided view of a larger buffer passes (an engine's `draft_probs[:rows, t]`), while a buffer
    smaller than the slots it is indexed by raises here instead of being addressed past its end."""

    if tensor is None or rows <= 0 or cols <= 0:

        return

    last = tensor.storage_offset() + (rows - 1) * tensor.stride(0) + (cols - 1) * tensor.stride(-1)

    if tensor.dim() >= 3:

        last += (steps - 1) * tensor.stride(1)

    if last >= tensor.untyped_storage().nbytes() // tensor.element_size():

        raise ValueError(f"`{name}` does not cover the {rows} slots x {cols} columns it is indexed by "
                         f"(shape {tuple(tensor.shape)}, strides {tensor.stride()})")


def fresh_seed() -> int:
    """A seed drawn from torch's default CPU generator (fresh noise for a call without noise)."""

    return int(torch.randint(0, 2 ** 62, (1,), dtype=torch.int64).item())
