"""Counter-based Gumbel noise (Philox4x32-10) as used in-register by the fused kernels.

The fused calls accept ``philox_seed`` / ``philox_offset`` instead of a noise plane; the noise of
(slot, timestep, token) is then ``bf16(log(bf16(-log(u))))`` with u drawn from Philox at counter
(token, slot, timestep, offset). These helpers write that noise (or the raw Philox words) out, e.g.
to feed it to a reference implementation or to the buffers of the noise-plane path.
"""

from __future__ import annotations

import torch

from sonic_sampler import _native


def materialize_gumbel(seed: int, offset: int, slots: int, timesteps: int, vocab: int,
                       device=None, out: torch.Tensor | None = None) -> torch.Tensor:
    """The [slots, timesteps, vocab] bf16 noise the kernels would draw in Philox mode."""

    if out is None:

        out = torch.empty(slots, timesteps, vocab, dtype=torch.bfloat16, device=device)

    _native.require_device(out)

    status = _native.load().ss_gumbel_materialize(
        seed & 0xFFFFFFFFFFFFFFFF, offset & 0xFFFFFFFF, slots, timesteps, vocab, out.data_ptr(),
        out.stride(0), out.stride(1), _native.stream_of(out),
    )
    _native.check(status, "ss_gumbel_materialize")

    return out


def philox_words(seed: int, offset: int, slots: int, timesteps: int, vocab: int, device=None) -> torch.Tensor:
    """The raw first Philox output word for every (slot, timestep, token), as int32 bits."""

    out = torch.empty(slots, timesteps, vocab, dtype=torch.int32, device=device)
    _native.require_device(out)

    status = _native.load().ss_philox_raw(seed & 0xFFFFFFFFFFFFFFFF, offset & 0xFFFFFFFF, slots,
                                          timesteps, vocab, out.data_ptr(), _native.stream_of(out))
    _native.check(status, "ss_philox_raw")

    return out
