"""CPU emulations of the device kernels' shared-memory and scratch indexing (no GPU).

Each test restates one index computation of ``csrc/ss_sampling.h`` over every case the kernels can
meet and asserts that it stays inside the array it addresses, so a bound that only holds by
accident (or by a later pass overwriting the damage) fails here instead of on the device.
"""

from __future__ import annotations

import itertools

import numpy as np
import pytest

SS_K = 128
WAVE = 64
RUN = SS_K + 64   # TileSmem::run[wave] entries


def survivor_writes(popcounts):
    """Positions wave_survivors writes for the given per-position ballot popcounts (the lanes of
    a ballot write at cnt + mbcnt, i.e. cnt .. cnt + popcount - 1), and the final count."""

    cnt, written = 0, []

    for p in popcounts:

        if p and cnt <= SS_K:

            written.extend(range(cnt, cnt + p))

        cnt = min(cnt + p, SS_K + 1)

    return written, cnt


@pytest.mark.parametrize("E", [4, 8, 16, 32])
def test_wave_survivors_writes_stay_inside_the_run(E):

    rng = np.random.default_rng(E)
    cases = [[WAVE] * E, [0] * E, [1] * E, [63, 63, 63, 63] + [WAVE] * (E - 4)]
    cases += [list(rng.integers(0, WAVE + 1, E)) for _ in range(2000)]
    cases += [list(rng.choice([0, 1, 2, 40, 64], E)) for _ in range(2000)]

    for pops in cases:

        written, cnt = survivor_writes(pops)
        total = int(sum(pops))
        assert all(0 <= w < RUN for w in written), pops
        # an overflow (more than SS_K survivors) is still visible in the count
        assert (cnt > SS_K) == (total > SS_K)
        # without overflow every survivor was written exactly once, in order
        if total <= SS_K:

            assert written == list(range(total))


def test_wave_survivors_bound_is_tight_without_the_guard():
    """The unguarded form (writing while saturated at SS_K + 1) reaches index RUN."""

    cnt, worst = 0, 0

    for p in [WAVE, WAVE, 1, WAVE]:

        if p:

            worst = max(worst, cnt + p - 1)

        cnt = min(cnt + p, SS_K + 1)

    assert worst == RUN


def merge_prefix(tiles):

    return min(SS_K, (4 * SS_K) // tiles)


@pytest.mark.parametrize("tiles", list(range(2, 520)) + [1000, 4096, 65535])
def test_row_merge_slot_to_list_multiply_shift(tiles):
    """slot_list: (s * ceil(2^16 / kp)) >> 16 == s // kp for every sample slot s < tiles * kp."""

    kp = merge_prefix(tiles)

    if kp == 0:

        return

    kpm = (65536 + kp - 1) // kp
    s = np.arange(tiles * kp, dtype=np.int64)
    assert tiles * kp <= 4 * SS_K               # SampleSmem::col holds 4 * SS_K slots
    assert np.array_equal((s * kpm) >> 16, s // kp)


def merge_run(kp):

    return kp if 8 <= kp <= 64 and (kp & (kp - 1)) == 0 else 1


@pytest.mark.parametrize("tiles", list(range(2, 520)))
def test_row_merge_sample_reads_stay_inside_the_scratch_row(tiles):
    """load_samples: every (wave, lane, i) reads scr[list * SS_K + position] with position < kp,
    inside the row's tiles * SS_K candidates, and the slots of one call are distinct."""

    kp = merge_prefix(tiles)
    ns = tiles * kp
    run = merge_run(kp)
    seen = set()

    for wave, lane, i in itertools.product(range(4), range(WAVE), range(2)):

        if run > 1:

            lr = run.bit_length() - 1
            e = 2 * lane + i
            r, q = e >> lr, e & (run - 1)
            lst = wave * (SS_K >> lr) + r
            s = (lst << lr) + (run - 1 - q if r & 1 else q)

        else:

            s = 2 * (wave * WAVE + lane) + i
            lst = s // kp if kp else 0

        assert s < 4 * SS_K
        assert s not in seen
        seen.add(s)

        if s < ns:

            pos = s - lst * kp
            assert 0 <= pos < kp
            assert 0 <= lst * SS_K + pos < tiles * SS_K

    assert len(seen) == 4 * SS_K


def masked_survivors(keys16, T):
    """wave_survivors_masked for one wave: keys16[lane][j] (16-bit keys, E per lane) -> the run it
    writes (composites (key << 16) | (0xffff - column)), in write order, or None on overflow."""

    E = len(keys16[0])
    masks, counts = [], []

    for lane in range(WAVE):

        mask = 0

        for i in range(E // 2):

            lo, hi = keys16[lane][2 * i], keys16[lane][2 * i + 1]
            d = (min(max(lo - T, 0), 1)) | (min(max(hi - T, 0), 1) << 16)   # packed sat-sub, min 1
            mask |= d << i

        masks.append(mask & 0xffffffff)
        counts.append(bin(mask).count("1"))

    total = sum(counts)

    if total > SS_K:

        return None

    run = [None] * RUN
    pos = 0

    for lane in range(WAVE):

        mask, cb = masks[lane], 0xffff - 4 * lane

        while mask:

            b = (mask & -mask).bit_length() - 1
            mask &= mask - 1
            i, hi = b & 15, b >> 4
            key = keys16[lane][2 * i + hi]
            j = 2 * i + hi
            off = (j >> 2) * (256 * 4) + (j & 3)
            assert pos < RUN
            run[pos] = ((key << 16) | cb) - off
            pos += 1

    return run[:pos]


@pytest.mark.parametrize("E", [4, 8, 16, 32])
def test_masked_survivors_are_the_keys_above_the_threshold(E):

    rng = np.random.default_rng(100 + E)

    for trial in range(200):

        keys = rng.integers(0x7000, 0x9000, (WAVE, E)).tolist()
        T = int(np.sort(np.array(keys).ravel())[-rng.integers(1, 150)])
        run = masked_survivors(keys, T)
        expected = sorted(((k << 16) | (0xffff - ((j >> 2) * 1024 + 4 * lane + (j & 3))))
                          for lane in range(WAVE) for j, k in enumerate(keys[lane]) if k > T)

        if len(expected) > SS_K:

            assert run is None
            continue

        assert sorted(run) == expected
