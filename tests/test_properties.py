"""Property tests (hypothesis) of the oracle and of the CPU restatements of the device algorithms.

Each property holds for every input, not just for hand cases, and is stated independently of the
formula it checks: an ordering a plain Python sort defines, sets that only grow or shrink as a
parameter moves, a counter-based stream whose words do not depend on the shape of the draw, and the
row merge's result against the exact top-128 of the whole row. Examples are derandomized, so a run
is reproducible.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

from oracle import philox
from oracle import sampler as oracle
from oracle.topk import topk
from test_indexing import SS_K, row_merge, tile_lists
from test_oracle import tiny_state

BF16 = torch.bfloat16
SETTINGS = settings(max_examples=150, deadline=None, derandomize=True,
                    suppress_health_check=[HealthCheck.too_slow])

# values from a small pool, so that ties (and +-0, +-inf) are frequent
POOL = [-math.inf, -3.5, -1.0, -0.0, 0.0, 0.5, 1.0, 2.25, 7.0, math.inf]


@SETTINGS
@given(values=st.lists(st.sampled_from(POOL) | st.floats(-50, 50, width=32), min_size=2, max_size=300),
       log_k=st.integers(0, 7))
def test_topk_is_the_first_k_of_the_stable_descending_order(values, log_k):

    k = min(1 << log_k, len(values))
    x = torch.tensor([values], dtype=torch.float32)
    got_v, got_i = topk(x, k)
    order = sorted(range(len(values)), key=lambda c: (-values[c], c))[:k]

    assert got_i[0].tolist() == order
    assert got_v[0].tolist() == [values[c] for c in order]


def sorted_support(draw_values):
    """128 bf16 values in descending order (the merged top-128 a row stage truncates)."""

    v = torch.tensor(sorted(draw_values, reverse=True), dtype=torch.float32).to(BF16)

    return v[None]


def kept(values, ind, **params):

    st_ = tiny_state(**params)
    out, _ = oracle.truncate(values.clone(), ind, st_, 0)

    return torch.isfinite(out[0]).tolist()


support = st.lists(st.floats(-12, 12, width=32), min_size=SS_K, max_size=SS_K)


@SETTINGS
@given(values=support, k1=st.integers(1, SS_K), k2=st.integers(1, SS_K))
def test_top_k_keeps_a_prefix_that_grows_with_k(values, k1, k2):

    v = sorted_support(values)
    a = kept(v, oracle.TOP_K, top_k=torch.tensor([min(k1, k2)], dtype=torch.int32))
    b = kept(v, oracle.TOP_K, top_k=torch.tensor([max(k1, k2)], dtype=torch.int32))

    assert a == [True] * min(k1, k2) + [False] * (SS_K - min(k1, k2))
    assert all(y for x, y in zip(a, b) if x)


@SETTINGS
@given(values=support, p1=st.floats(0.01, 1.0), p2=st.floats(0.01, 1.0))
def test_top_p_keeps_a_prefix_from_position_0_that_grows_with_p(values, p1, p2):

    v = sorted_support(values)
    lo, hi = sorted((torch.tensor([p1]).to(BF16), torch.tensor([p2]).to(BF16)), key=float)
    a = kept(v, oracle.TOP_P, top_p=lo)
    b = kept(v, oracle.TOP_P, top_p=hi)

    for mask in (a, b):

        assert mask[0]
        assert mask == sorted(mask, reverse=True)   # True ... True False ... False

    assert all(y for x, y in zip(a, b) if x)


@SETTINGS
@given(values=support, m1=st.floats(0.0, 0.99), m2=st.floats(0.0, 0.99))
def test_min_p_keeps_a_prefix_from_position_0_that_shrinks_with_min_p(values, m1, m2):

    v = sorted_support(values)
    lo, hi = sorted((torch.tensor([m1]).to(BF16), torch.tensor([m2]).to(BF16)), key=float)
    a = kept(v, oracle.MIN_P, min_p=lo)
    b = kept(v, oracle.MIN_P, min_p=hi)

    for mask in (a, b):

        assert mask[0]
        assert mask == sorted(mask, reverse=True)

    assert all(x for x, y in zip(a, b) if y)


@SETTINGS
@given(seed=st.integers(0, 2**64 - 1), offset=st.integers(0, 2**32 - 1), slots=st.integers(1, 4),
       steps=st.integers(1, 3), vocab=st.integers(1, 40), extra=st.integers(1, 20))
def test_noise_words_do_not_depend_on_the_shape_of_the_draw(seed, offset, slots, steps, vocab, extra):
    """Counter-based: the word of (slot, step, token) is the same whatever else is drawn with it,
    and the Philox block of that counter is the same drawn alone."""

    small = philox.noise_words(seed, offset, slots, steps, vocab)
    large = philox.noise_words(seed, offset, slots + 1, steps + 1, vocab + extra)

    assert np.array_equal(small, large[:slots, :steps, :vocab])

    s, t, v = slots - 1, steps - 1, vocab - 1
    alone = philox.philox4x32_10(np.array([v, s, t, offset], dtype=np.uint32),
                                 np.array([seed & 0xFFFFFFFF, seed >> 32], dtype=np.uint32))
    assert alone[0] == small[s, t, v]


@SETTINGS
@given(x=st.floats(width=32, allow_nan=False))
def test_bf16_rounding_matches_torch_everywhere(x):

    want = torch.tensor([x], dtype=torch.float32).to(BF16).float().item()
    got = float(philox.bf16_round(np.array([x], dtype=np.float32))[0])

    assert got == want or (math.isinf(want) and got == want)


@pytest.mark.parametrize("block", [128])
@SETTINGS
@given(tiles=st.integers(2, 48), seed=st.integers(0, 2**32 - 1),
       pattern=st.sampled_from(["random", "ties", "hot", "equal-hot"]))
def test_row_merge_is_the_exact_top_128(block, tiles, seed, pattern):
    """The sampled merge, its exactness check, the refill and the radix bound, as the device runs
    them, return exactly the first 128 of the whole row by (value desc, column asc)."""

    rng = np.random.default_rng(seed)
    v = tiles * block - int(rng.integers(0, block // 2))
    values = rng.integers(0x7000, 0x9000, v) if pattern == "random" else rng.integers(0x8000, 0x8003, v)

    if pattern in ("hot", "equal-hot"):

        for t in rng.choice(v // block, size=int(rng.integers(1, min(20, v // block) + 1)), replace=False):

            n = int(rng.integers(1, block))
            cols = t * block + rng.choice(block, n, replace=False)
            values[cols] = 0x9000 if pattern == "equal-hot" else rng.integers(0x9000, 0x9010, n)

    got, _ = row_merge(tile_lists(values, block))
    exact = sorted(((int(k), j) for j, k in enumerate(values)), key=lambda e: (-e[0], e[1]))[:SS_K]
    exact += [(0, -1)] * (SS_K - len(exact))

    assert got == exact
