"""Philox4x32-10 and the Gumbel noise transform in numpy -- TEST INFRASTRUCTURE ONLY.

Philox4x32-10 as published by Salmon, Moraes, Dror and Shaw ("Parallel random numbers: as easy as
1, 2, 3", SC'11) and in the Random123 library: ten rounds of
    (c0, c1, c2, c3) <- (hi(M1 c2) ^ c1 ^ k0, lo(M1 c2), hi(M0 c0) ^ c3 ^ k1, lo(M0 c0))
with M0 = 0xD2511F53, M1 = 0xCD9E8D57 and the key bumped by (0x9E3779B9, 0xBB67AE85) between
rounds. Pinned against the Random123 known-answer vectors in tests/test_oracle.py.

The noise the fused kernels draw for (slot s, timestep t, token v) uses counter (v, s, t, offset)
and key (seed & 0xffffffff, seed >> 32); the first output word x gives
    u = (2 * (x >> 9) + 1) / 2**24,   w = bf16(log(bf16(-log(u)))),
the reference's `exponential_(1.0).log_()` transform (src/sonic_sampler/core/buffer.py:118) applied
to a counter-based uniform.
"""

from __future__ import annotations

import numpy as np

M0 = np.uint64(0xD2511F53)
M1 = np.uint64(0xCD9E8D57)
W0 = np.uint32(0x9E3779B9)
W1 = np.uint32(0xBB67AE85)
MASK32 = np.uint64(0xFFFFFFFF)


def philox4x32_10(counter: np.ndarray, key: np.ndarray) -> np.ndarray:
    """counter: uint32 [..., 4]; key: uint32 [..., 2] (broadcastable). Returns uint32 [..., 4]."""

    c = [counter[..., i].astype(np.uint64) for i in range(4)]
    k0 = np.broadcast_to(key[..., 0], counter.shape[:-1]).astype(np.uint64)
    k1 = np.broadcast_to(key[..., 1], counter.shape[:-1]).astype(np.uint64)

    for _ in range(10):

        p0 = M0 * c[0]
        p1 = M1 * c[2]
        hi0, lo0 = p0 >> np.uint64(32), p0 & MASK32
        hi1, lo1 = p1 >> np.uint64(32), p1 & MASK32
        c = [
            (hi1 ^ c[1] ^ k0) & MASK32,
            lo1,
            (hi0 ^ c[3] ^ k1) & MASK32,
            lo0,
        ]
        k0 = (k0 + np.uint64(W0)) & MASK32
        k1 = (k1 + np.uint64(W1)) & MASK32

    return np.stack([x.astype(np.uint32) for x in c], axis=-1)


def noise_words(seed: int, offset: int, slots: int, steps: int, vocab: int) -> np.ndarray:
    """First Philox output word for every (slot, step, token): uint32 [slots, steps, vocab]."""

    s, t, v = np.meshgrid(np.arange(slots, dtype=np.uint32), np.arange(steps, dtype=np.uint32),
                          np.arange(vocab, dtype=np.uint32), indexing="ij")
    counter = np.stack([v, s, t, np.full_like(v, offset & 0xFFFFFFFF)], axis=-1)
    key = np.array([seed & 0xFFFFFFFF, (seed >> 32) & 0xFFFFFFFF], dtype=np.uint32)

    return philox4x32_10(counter, key)[..., 0]


def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest bfloat16 (ties to even), returned as float32."""

    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)) << np.uint64(16)

    return r.astype(np.uint32).view(np.float32)


def gumbel_from_words(words: np.ndarray) -> np.ndarray:
    """w = bf16(log(bf16(-log(u)))) as float32 (bf16-exact values)."""

    u = ((words >> np.uint32(9)).astype(np.float32) * np.float32(2) + np.float32(1)) * np.float32(2.0 ** -24)
    e = bf16_round(-np.log(u.astype(np.float32)))

    return bf16_round(np.log(e))
