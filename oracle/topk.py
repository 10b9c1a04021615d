"""Bounded top-k as a stable descending sort -- TEST INFRASTRUCTURE ONLY.

Restates what ``UnshardedBoundedTopK.__call__`` (reference ``src/sonic_sampler/interface/topk.py:
98-161``) computes: per row, the k largest values and their indices, ties broken to the lowest
index (the packed key ``value << 16 | ~index`` of ``ops/encoding.py:63-91`` orders equal values by
increasing index). A stable descending sort is the textbook form of that order.
"""

from __future__ import annotations

from typing import Tuple

import torch

from torch import Tensor


def topk(logits: Tensor, k: int) -> Tuple[Tensor, Tensor]:
    """(values [rows, k] in the logits dtype, indices [rows, k] int32), ties to the lowest index.

    -0.0 and +0.0 compare equal (torch's sort), so their relative order is by index.
    """

    x = logits.detach().to("cpu")
    values, indices = x.sort(dim=-1, stable=True, descending=True)

    return values[..., :k].contiguous(), indices[..., :k].to(torch.int32).contiguous()
