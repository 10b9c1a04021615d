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


REFILL_LISTS = 16


def tile_lists(values, block):
    """Sorted candidate lists of the tile stage: per tile its top-128 (key, column) by (key desc,
    column asc), padded with absent entries (key 0)."""

    lists = []

    for t0 in range(0, len(values), block):

        entries = sorted(((int(k), t0 + j) for j, k in enumerate(values[t0:t0 + block])),
                         key=lambda e: (-e[0], e[1]))[:SS_K]
        lists.append(entries + [(0, -1)] * (SS_K - len(entries)))

    return lists


def row_merge(lists):
    """merge_row + merge_refill over the lists, restated step for step: returns the (key, column)
    top-128 and the path taken ("sampled", "refill" or "radix")."""

    tiles = len(lists)
    kp = merge_prefix(tiles)
    slot = lambda s: (s // kp, s % kp)  # noqa: E731

    def comp(key, g):

        return (key << 16) | (0xffff - g) if key else 0

    f = sorted((comp(lists[t][p][0], t * kp + p) for t in range(tiles) for p in range(kp)), reverse=True)
    f = (f + [0] * SS_K)[:SS_K]
    last = f[-1]
    llast = slot(0xffff - (last & 0xffff))[0] if last else tiles
    beats = 0

    if kp < SS_K:

        for t in range(tiles):

            kn = lists[t][kp][0]
            beats += bool(kn and (kn > last >> 16 or (kn == last >> 16 and t < llast)))

    if beats == 0:

        return [(c >> 16, lists[slot(0xffff - (c & 0xffff))[0]][slot(0xffff - (c & 0xffff))[1]][1] if c else -1)
                for c in f], "sampled"

    if beats > REFILL_LISTS or kp == 0:

        everything = sorted((e for lst in lists for e in lst if e[0]), key=lambda e: (-e[0], e[1]))[:SS_K]
        return everything + [(0, -1)] * (SS_K - len(everything)), "radix"

    def to_entry(c):

        if not c:

            return 0

        t, p = slot(0xffff - (c & 0xffff))
        return (c & 0xffff0000) | (0xffff - (t * SS_K + p))

    f = [to_entry(c) for c in f]

    for t0 in range(0, tiles, WAVE):

        cn = [comp(lists[t][kp][0], t * SS_K + kp) if t < tiles else 0 for t in range(t0, t0 + WAVE)]
        m = [lane for lane in range(WAVE) if cn[lane] > f[-1]]

        while m:

            lst = t0 + m[0]
            r = [comp(lists[lst][kp + 127 - e][0], lst * SS_K + kp + 127 - e) if e >= kp else 0
                 for e in range(SS_K)]
            merged = [max(a, b) for a, b in zip(f, r)]
            # the elementwise maximum must be bitonic (one descent, then one ascent at most)
            turns = sum(1 for i in range(1, SS_K - 1) if merged[i] < merged[i - 1] and merged[i] < merged[i + 1])
            assert turns <= 1
            f = sorted(merged, reverse=True)
            m = [lane for lane in m[1:] if cn[lane] > f[-1]]

    def column(c):

        if not c:

            return -1

        g = 0xffff - (c & 0xffff)
        return lists[g >> 7][g & 127][1]

    return [(c >> 16, column(c)) for c in f], "refill"


def refill_cases():

    rng = np.random.default_rng(7)
    block = 256  # small tiles keep the emulation fast; only the list structure matters

    for tiles in (2, 5, 32, 64, 100, 128, 256, 300, 512):

        v = tiles * block - (17 if tiles % 2 else 0)   # odd tile counts end in a partial tile
        yield f"random-{tiles}", rng.integers(0x7000, 0x9000, v)
        yield f"ties-{tiles}", rng.integers(0x8000, 0x8004, v)
        yield f"equal-{tiles}", np.full(v, 0x8100)
        spiked = rng.integers(0x7000, 0x8000, v)
        full = tiles - (1 if v % block else 0)
        hot = rng.choice(full, size=min(full, rng.integers(1, 24)), replace=False)
        for t in hot:

            spiked[t * block + rng.choice(block, 60, replace=False)] = rng.integers(0x9000, 0x9100, 60)

        yield f"spiked-{tiles}", spiked


@pytest.mark.parametrize("name,values", list(refill_cases()), ids=lambda x: x if isinstance(x, str) else "")
def test_row_merge_refill_is_exact(name, values):
    """The sampled merge, its exactness check and the refill give the exact top-128 by (value
    desc, column asc) on every path; the all-equal and spiked rows reach the refill and the radix
    bound."""

    lists = tile_lists(values, 256)
    got, path = row_merge(lists)
    exact = sorted(((int(k), j) for j, k in enumerate(values)), key=lambda e: (-e[0], e[1]))[:SS_K]
    exact += [(0, -1)] * (SS_K - len(exact))
    assert got == exact, (name, path)


def test_row_merge_refill_paths_are_reached():

    paths = {row_merge(tile_lists(values, 256))[1] for _, values in refill_cases()}
    assert paths == {"sampled", "refill", "radix"}


TOPK_REFILL_LISTS = 16


def topk_merge(values, block, k):
    """topk_merge_kernel restated step for step: the tiles' sorted top-k lists, the sampled merge
    (kp entries per list), the exactness check against the k-th merged composite, the whole-list
    refill with its element pairing, and the radix fallback. Returns ((key, column) top-k, path)."""

    tiles = -(-len(values) // block)
    lists = [sorted(((int(values[c]), c) for c in range(t * block, min(len(values), (t + 1) * block))),
                    key=lambda e: (-e[0], e[1]))[:k] for t in range(tiles)]
    comp = lambda e: (e[0] << 32) | (0xffffffff - e[1])  # noqa: E731
    ncand = tiles * k
    # k <= 64: 256 samples and a 64-wide top list; else 512 samples and 128
    slots, width = (256, 64) if k <= 64 else (512, SS_K)
    kp = k if ncand <= slots else (1 << ((slots // tiles).bit_length() - 1)) if tiles <= slots else 0
    if k <= 64 and kp == 0:

        slots, width = 512, SS_K
        kp = (1 << ((512 // tiles).bit_length() - 1)) if tiles <= 512 else 0

    exact = sorted((e for lst in lists for e in lst), key=lambda e: (-e[0], e[1]))[:k]

    if kp == 0:

        return exact, "radix"

    f = sorted((comp(lists[s // kp][s % kp]) for s in range(slots) if s // kp < tiles), reverse=True)
    f = (f + [0] * width)[:width]
    beats = sum(1 for t in range(tiles) if kp < k and comp(lists[t][kp]) > f[k - 1]) if kp < k else 0

    if beats > TOPK_REFILL_LISTS:

        return exact, "radix"

    for t0 in range(0, tiles if beats else 0, WAVE):

        nx = [comp(lists[t][kp]) if t < tiles else 0 for t in range(t0, t0 + WAVE)]
        m = [lane for lane in range(WAVE) if nx[lane] > f[k - 1]]

        while m:

            lst = lists[t0 + m[0]]
            r = [comp(lst[kp + width - 1 - e]) if e >= width - k + kp else 0 for e in range(width)]
            assert all(kp <= kp + width - 1 - e < k for e in range(width - k + kp, width))
            f = sorted((max(a, b) for a, b in zip(f, r)), reverse=True)
            m = [lane for lane in m[1:] if nx[lane] > f[k - 1]]

    got = [(c >> 32, 0xffffffff - (c & 0xffffffff)) for c in f[:k]]

    return got, ("refill" if beats else "sampled") if got == exact else "WRONG"


def topk_cases():

    rng = np.random.default_rng(11)

    for k, block, tiles in [(32, 256, 32), (32, 256, 16), (128, 256, 32), (128, 256, 5), (64, 256, 100),
                            (8, 256, 300), (128, 256, 512)]:

        v = tiles * block - 9
        yield k, f"random-{k}-{tiles}", rng.integers(0, 2 ** 31, v), block
        yield k, f"ties-{k}-{tiles}", rng.integers(1000, 1003, v), block
        spiked = rng.integers(0, 2 ** 30, v)
        for t in rng.choice(tiles - 1, size=min(tiles - 1, 6), replace=False):

            spiked[t * block + rng.choice(block, k, replace=False)] = rng.integers(2 ** 31, 2 ** 32, k)

        yield k, f"spiked-{k}-{tiles}", spiked, block


@pytest.mark.parametrize("k,name,values,block", list(topk_cases()),
                         ids=lambda x: x if isinstance(x, str) else "")
def test_topk_merge_is_exact(k, name, values, block):

    got, path = topk_merge(values, block, k)
    assert path != "WRONG", name


def test_topk_merge_paths_are_reached():

    paths = {topk_merge(values, block, k)[1] for k, _, values, block in topk_cases()}
    assert paths == {"sampled", "refill", "radix"}


@pytest.mark.parametrize("E", [4, 8, 16, 32, 128])
def test_topk_block_bound_shares(E):
    """topk_block_kernel's lower bound: wave w's share of k is ceil(k * n_w / V) for its n_w
    valid columns (chunk c gives it columns c * 1024 + 256 w .. + 255). The shares sum to at least
    k, a wave has a share iff it has columns, and a full block gives every wave k / 4."""

    block = 256 * E

    for k in (1, 2, 8, 32, 64, 128):

        for V in sorted({1, 2, 17, 255, 256, 257, 300, 1023, 1024, 1025, block // 2, block - 1, block} - {0}):

            if V > block:

                continue

            nw = [sum(min(max(V - (c * 1024 + 256 * w), 0), 256) for c in range(E // 4)) for w in range(4)]
            need = [(k * n + V - 1) // V if n else 0 for n in nw]
            assert sum(nw) == V
            assert sum(need) >= k
            assert all((n > 0) == (s > 0) for n, s in zip(nw, need))

            if V == block:

                assert need == [-(-k // 4)] * 4

    # the config-0 last tile at block 1024 (256 valid columns, all in wave 0) keeps a bound
    nw = [min(max(256 - 256 * w, 0), 256) for w in range(4)]
    assert [(32 * n + 255) // 256 if n else 0 for n in nw] == [32, 0, 0, 0]


def xcd_grouped(L, N):
    """ss_sampling.h xcd_grouped, restated."""

    q, r = N >> 3, N & 7
    x, local = L & 7, L >> 3
    return x * (q + 1) + local if x < r else r * (q + 1) + (x - r) * q + local


def test_xcd_grouped_is_a_bijection_with_contiguous_xcd_ranges():

    for N in list(range(1, 300)) + [1024, 1025, 2047, 4096, 65535]:

        v = [xcd_grouped(L, N) for L in range(N)]
        assert sorted(v) == list(range(N)), N

        for x in range(8):

            mine = sorted(v[L] for L in range(x, N, 8))
            assert mine == list(range(mine[0], mine[0] + len(mine))) if mine else True

    # config 4: 256 rows of 4 tiles; the 4 tiles of every row land on one XCD
    tiles = 4
    for L in range(1024):

        row = xcd_grouped(L, 1024) // tiles
        assert all(xcd_grouped(M, 1024) // tiles != row or M % 8 == L % 8 for M in range(L % 8, 1024, 1))


def packed_keys(u: int) -> int:
    """csrc/ss_sampling.h packed_keys on one 32-bit word (two bf16 halves), as 16-bit lane
    operations: m = arithmetic shift of each half by 15, t = u ^ (m | 0x80008000), t - m per half."""

    m = sum((0xffff if (u >> s) & 0x8000 else 0) << s for s in (0, 16))
    t = u ^ (m | 0x80008000)

    return sum(((((t >> s) & 0xffff) - ((m >> s) & 0xffff)) & 0xffff) << s for s in (0, 16))


def test_packed_keys_follow_the_order_of_the_values():
    """Keys of every non-NaN bf16 value sort as the values do, equal values (+0 and -0) share a
    key, and the two halves of a word are keyed independently (no carry between them)."""

    import torch

    bits = np.arange(0x10000, dtype=np.uint32)
    values = torch.from_numpy(bits.astype(np.int32).astype(np.int16)).view(torch.bfloat16).float().numpy()
    finite = ~np.isnan(values)
    keys = np.array([packed_keys(int(b)) & 0xffff for b in bits])
    v, k = values[finite], keys[finite]
    order = np.argsort(v, kind="stable")
    sv, sk = v[order], k[order]
    assert np.all(np.diff(sk) >= 0)
    assert np.all((np.diff(sk) == 0) == (np.diff(sv) == 0))
    assert packed_keys(0x80008000) == packed_keys(0x00000000) == 0x80008000
    assert (k > 0).all()

    rng = np.random.default_rng(7)

    for lo, hi in rng.integers(0, 0x10000, (2000, 2)).tolist():

        both = packed_keys(lo | (hi << 16))
        assert both & 0xffff == keys[lo] and both >> 16 == keys[hi]


# ------------------------------------------------------------------------------------------------
# Grammar staging with direct global-to-LDS loads (stage_grammar / stage_grammar_finish)
# ------------------------------------------------------------------------------------------------

STAGE_MAX_WORDS, BLOCK = 8192, 256


def stage_quads(vt):

    return (((vt + 31) >> 5) + 3) >> 2


def stage_region_quads(vt):

    quads = stage_quads(vt)
    blocks = (quads + 63) >> 6

    return blocks * 64 if blocks * 64 > quads else quads + 1


def emulate_staging(row_words, vt):
    """The workgroup memory stage_grammar + stage_grammar_finish leave for a grammar row: wave w of
    iteration i copies quads [256 i + 64 w, +64) when that block starts inside the row, lane l
    loading row quad q0 + l through the range-checked buffer (words past the row read 0) into
    region quad q0 + l; then the last word's bits past vt are cleared and, when the row ends on a
    block, the quad after it is zeroed. Returns the region (None: never written) and the set of
    written quads."""

    words = (vt + 31) >> 5
    quads = stage_quads(vt)
    region = [None] * (4 * stage_region_quads(vt))
    written = set()

    for i in range(STAGE_MAX_WORDS // 4 // BLOCK):

        for w in range(BLOCK // WAVE):

            q0 = i * BLOCK + w * WAVE

            if q0 >= quads:

                continue

            for lane in range(WAVE):

                q = q0 + lane
                written.add(q)

                for k in range(4):

                    word = 4 * q + k
                    region[word] = int(row_words[word]) if word < words else 0

    last = vt >> 5

    if vt & 31:

        owner = ((last >> 2) & (BLOCK - 1)) & ~63          # lane 0 of the wave holding that word
        assert (last >> 2) in written and (((last >> 2) % BLOCK) // WAVE) * WAVE == owner
        region[last] &= (1 << (vt & 31)) - 1

    if quads % 64 == 0:

        written.add(quads)
        region[4 * quads: 4 * quads + 4] = [0, 0, 0, 0]

    return region, written


@pytest.mark.parametrize("vt", [1, 31, 32, 33, 127, 128, 129, 4096, 4099, 8191, 8192, 32000, 32768,
                                65536 - 32, 65536 + 5, 131072 - 1, 200003, 262144 - 128, 262144])
def test_direct_grammar_staging_stays_in_its_region_and_reproduces_the_row(vt):

    rng = np.random.default_rng(vt)
    words = (vt + 31) >> 5
    row = rng.integers(0, 2 ** 32, size=words + 8, dtype=np.uint64)   # garbage past the row too
    region, written = emulate_staging(row, vt)
    quads = stage_quads(vt)
    # every written quad lies inside the allocated region
    assert max(written) < stage_region_quads(vt)
    # every quad a lookup can reach (word index clamped to 4 * quads) was written
    assert all(q in written for q in range(quads + 1))
    # bit v of the staged row is bit v of the grammar for v < vt, and clear for v >= vt up to the clamp
    for v in list(range(0, min(vt, 4096))) + list(range(max(0, vt - 4096), vt)):

        assert (region[v >> 5] >> (v & 31)) & 1 == (int(row[v >> 5]) >> (v & 31)) & 1

    for v in range(vt, min(128 * quads + 32, vt + 4096)):

        assert (region[min(v >> 5, 4 * quads)] >> (v & 31)) & 1 == 0


# ------------------------------------------------------------------------------------------------
# tile_stage's decisions (wave bounds, the floor at -inf, survivors, the exact cut's candidates)
# ------------------------------------------------------------------------------------------------

KEY_NEG_INF = 0x0080   # key of bf16 -inf; -NaN keys lie below it, absent elements are 0


def tile_stage_emulation(keys, E, valid):
    """The tile's candidate list as tile_stage builds it, restated step by step: `keys` is the
    tile's 256 * E keys by column (0 past `valid`). Returns the list's (key, column) entries in
    descending order and the path ("bounds", "fill" or "exact")."""

    block = len(keys)
    col = lambda t, j: (j >> 2) * 1024 + 4 * t + (j & 3)  # noqa: E731
    per_thread = [[int(keys[col(t, j)]) for j in range(E)] for t in range(256)]
    bounds = []

    for w in range(4):

        lanes = per_thread[64 * w: 64 * w + 64]
        m1 = [max(v) for v in lanes]
        m2 = [sorted(v)[-2] for v in lanes]
        bound = 0

        for b in range(15, 1, -1):

            c = bound | (1 << b)
            n = sum(x >= c for x in m1) + (0 if E >= 64 else sum(x >= c for x in m2))
            bound = c if n >= 32 else bound

        if bound <= KEY_NEG_INF and valid >= SS_K:

            bound = KEY_NEG_INF + 1

        bounds.append(bound)

    lo = min(bounds)
    t0 = lo - 1 if lo else 0
    cnt = [sum(k > t0 for v in per_thread[64 * w: 64 * w + 64] for k in v) for w in range(4)]
    floored = lo == KEY_NEG_INF + 1
    few = floored and sum(cnt) < SS_K
    everything = sorted(((int(k), c) for c, k in enumerate(keys)), key=lambda e: (-e[0], e[1]))
    lead = [c for c in range(256) if keys[c] == KEY_NEG_INF]   # wave 0's elements 0-3

    if few and len(lead) >= SS_K - sum(cnt):

        # wave 0 appends the first -inf keys of the first 256 columns to the merged survivors
        survivors = [e for e in everything if e[0] > t0]
        return survivors + [(KEY_NEG_INF, c) for c in lead[: SS_K - len(survivors)]], "fill"

    if max(cnt) > SS_K or few:

        # the candidates (lo, and -inf when floored) and the bisection all find the 128th key
        T = 0
        for b in range(15, -1, -1):

            c = T | (1 << b)
            T = c if sum(int(k) >= c for k in keys) >= SS_K else T

        above = [e for e in everything if e[0] > T]
        ties = [e for e in everything if e[0] == T][: SS_K - len(above)]
        return sorted(above + ties, key=lambda e: (-e[0], e[1])), "exact"

    survivors = [e for e in everything if e[0] > t0]
    return survivors[:SS_K], "bounds"


def tile_cases():

    rng = np.random.default_rng(11)

    for E in (16, 32, 64):

        block = 256 * E

        for valid in (block, block - 1, 1280 if E == 16 else block // 3, 200, 127, 100, 1):

            for admitted in (None, 3, 60, 127, 128, 200, 700):

                keys = rng.integers(0x6000, 0xA000, block)
                if admitted is not None:

                    keys[:] = KEY_NEG_INF
                    keys[rng.choice(valid, min(admitted, valid), replace=False)] = rng.integers(0x7000, 0x9000, min(admitted, valid))

                keys[valid:] = 0
                yield E, valid, admitted, keys

        # -NaN keys below -inf, and a wave with all of its admitted tokens
        keys = np.full(block, KEY_NEG_INF)
        keys[rng.choice(block, 50, replace=False)] = 0x40
        keys[: 64 * 4] = rng.integers(0x8000, 0x8100, 256)
        yield E, block, "nan", keys


@pytest.mark.parametrize("E,valid,admitted,keys", list(tile_cases()),
                         ids=lambda x: str(x) if not isinstance(x, np.ndarray) else "")
def test_tile_stage_keeps_the_exact_top_128(E, valid, admitted, keys):
    """With the bound floored above -inf, every path of the tile stage (bounds with enough
    survivors, the exact cut after too few or too many) yields the tile's exact first 128 by
    (key desc, column asc) among its valid columns; absent columns (key 0) never enter."""

    got, path = tile_stage_emulation(keys, E, valid)
    exact = sorted(((int(k), c) for c, k in enumerate(keys) if k > 0), key=lambda e: (-e[0], e[1]))[:SS_K]

    assert got == exact, (E, valid, admitted, path)


def test_tile_stage_paths():
    """Sparse admissions with full tiles take the bounds path when the tile holds 128 or more
    tokens and the wave-0 fill when it holds fewer; tiles of fewer than 128 valid columns never
    take the exact cut."""

    paths = {}

    for E, valid, admitted, keys in tile_cases():

        paths[(E, valid, admitted)] = tile_stage_emulation(keys, E, valid)[1]

    assert paths[(16, 4096, 200)] == "bounds" and paths[(16, 4096, 700)] == "bounds"
    assert paths[(16, 4096, 60)] == "fill" and paths[(64, 16384, 3)] == "fill"
    assert all(p == "bounds" for (E, valid, _), p in paths.items() if valid < SS_K)
