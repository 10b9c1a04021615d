"""GPU parity over a seeded sweep of tile shapes, grammar densities and value distributions.

Each case draws a tile width (2048-16384 columns), a tile count (rows of up to 80K columns, so that
the row merge runs from its whole-list regime at few tiles to its sampled one at 40) and a last
tile of a chosen width
(whole, or a few columns, or just under / at / over the 128 candidates a tile keeps), a grammar
(the random half-dense one, a few admitted tokens spread over the row, or a cluster of admitted
tokens inside one window) and a value distribution (spiked normal logits, a few distinct values so
that most keys tie, or one value everywhere). Every row runs every processor.

The bounded top-k sweep draws its own shapes (up to 128 tiles, k of 1-128, bf16 and fp32, and
row counts that take the one-workgroup-per-row launch) and compares values and indices bit for bit.

The multistep verifier's per-row top-128 ids are compared with the oracle's exactly: they are the
first 128 of the stable descending order of the processed row, so every path of the tile stage
(lower bounds, the floored bound of masked waves and its fill, the exact cut with its ties, tiles
of fewer than 128 valid columns) and of the row merge is checked to the index. The single-step
call on the same rows is checked by token, logprob and top-5 logprobs (whose -inf tail orders the
masked columns by index).
"""

from __future__ import annotations

import random

import pytest
import torch

from helpers import check_multistep, check_singular, expected_multistep_counts, run_verifier
from oracle import sampler as oracle
from test_gpu_paths import EVERY_PROCESSOR, autoregressive_case, random_host

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
BF16 = torch.bfloat16


def sweep_cases(count: int, seed: int):
    """(block, vocab, grammar, values, seed) of each case; a fixed list for a fixed seed."""

    rng = random.Random(seed)
    cases = []

    for n in range(count):

        block = rng.choice([2048, 4096, 8192, 16384])
        tiles = rng.randint(2, 81920 // block)
        last = rng.choice([block, 1, 3, 64, 127, 128, 129, 260, rng.randrange(1, block)])
        vocab = (tiles - 1) * block + last
        grammar = rng.choice(["random", "sparse", "cluster", "cluster"])
        values = rng.choice(["spiked", "spiked", "few", "flat"])
        cases.append((block, vocab, grammar, values, seed * 100 + n))

    return cases


CASES = sweep_cases(96, 7)


def sweep_logits(rows: int, vocab: int, values: str, seed: int) -> torch.Tensor:

    from bench import spiked_logits

    g = torch.Generator().manual_seed(seed)

    if values == "spiked":

        return spiked_logits(rows, vocab, seed)

    if values == "few":

        return (torch.randint(-2, 3, (rows, vocab), generator=g).float() * 0.75).to(BF16)

    return torch.full((rows, vocab), 0.5, dtype=BF16)


def set_grammar(host, vocab: int, kind: str, seed: int, d2t=None) -> None:
    """Replaces each (slot, timestep) grammar row of `host` unless `kind` is "random": "sparse"
    admits 1-300 of the `vocab` columns anywhere in the row, "cluster" 1-300 columns inside one
    window of at most 512 (so whole tiles admit nothing, and a tile's admitted tokens may sit in
    its first columns). With `d2t` the columns are draft columns and the bits set are their
    targets'."""

    if kind == "random":

        return

    g = torch.Generator().manual_seed(seed)
    slots, steps, words = host.grammar.shape
    bits = torch.zeros(slots * steps, words * 32, dtype=torch.bool)

    for r in range(slots * steps):

        allowed = int(torch.randint(1, 301, (1,), generator=g))

        if kind == "sparse":

            cols = torch.randperm(vocab, generator=g)[:allowed]

        else:

            width = min(vocab, max(allowed, int(torch.randint(allowed, 513, (1,), generator=g))))
            start = int(torch.randint(0, vocab - width + 1, (1,), generator=g))
            cols = start + torch.randperm(width, generator=g)[:allowed]

        bits[r, cols if d2t is None else d2t[cols].to(torch.int64)] = True

    packed = (bits.view(-1, words, 32).to(torch.int64) << torch.arange(32, dtype=torch.int64)).sum(-1)
    host.grammar.view(torch.int32).copy_((packed - ((packed >> 31) << 32)).to(torch.int32).view(slots, steps, words))


@pytest.mark.parametrize("block,vocab,grammar,values,seed", CASES)
def test_sweep_multistep_row_top128(block, vocab, grammar, values, seed):

    from bench import MultistepWorkload

    slots, batch, gamma = 4, 3, 2
    n = gamma + 1
    print(f"sweep multistep: block={block} V={vocab} grammar={grammar} values={values} seed={seed}", flush=True)
    g = torch.Generator().manual_seed(seed)
    host = random_host(slots, n, vocab, seed, EVERY_PROCESSOR, max_top_logprobs=4)
    set_grammar(host, vocab, grammar, seed + 1)
    logits = sweep_logits(batch * n, vocab, values, seed + 2)
    drafted = torch.randint(1, vocab, (batch * n,), generator=g).to(torch.int32)
    probabilities = torch.softmax(torch.randn(slots, gamma, vocab, generator=g) * 2, dim=-1).to(BF16)
    work = MultistepWorkload(logits=logits, drafted=drafted, buffers=host,
                             cu_seqlens=list(range(0, batch * n + 1, n)), lookahead=gamma, vocab=vocab,
                             max_top_logprobs=4, probabilities=probabilities)
    verification, buffers, verifier = run_verifier(work, update_counts=True, block_size=block)

    state = oracle.State.from_buffers(host)
    expected = oracle.multistep(logits, state, drafted, work.cu_seqlens, probabilities=probabilities,
                                logprobs=True, max_top_logprobs=4)
    indices = verifier.indices.cpu()

    for b, e in enumerate(expected):

        for i, idx in enumerate(e.row_indices):

            assert torch.equal(indices[work.cu_seqlens[b] + i], idx), (b, i)

    mismatched = check_multistep(verification, expected, work.cu_seqlens, logprobs=True, max_knife_fraction=0.34)
    counts = expected_multistep_counts(state.decode, expected, verification, work.cu_seqlens, mismatched)
    assert torch.equal(buffers.repetition.counts.decode.cpu(), counts)


@pytest.mark.parametrize("block,vocab,grammar,values,seed", CASES)
def test_sweep_autoregressive(block, vocab, grammar, values, seed):

    rows = 8
    print(f"sweep autoregressive: block={block} V={vocab} grammar={grammar} values={values} seed={seed}",
          flush=True)
    host = random_host(rows, 1, vocab, seed + 3, EVERY_PROCESSOR)
    set_grammar(host, vocab, grammar, seed + 4)
    logits = sweep_logits(rows, vocab, values, seed + 5).to(DEV)
    assert autoregressive_case(logits, host, block) >= rows - 2


@pytest.mark.parametrize("block,vocab,grammar,values,seed", CASES)
def test_sweep_drafting_d2t(block, vocab, grammar, values, seed):
    """Drafting through a random injective d2t into a larger target vocabulary, with slots, the
    drafted history and the probability scatter; the grammar (target vocabulary, staged in
    workgroup memory) admits draft columns as the case says."""

    from bench import to_device
    from sonic_sampler.interface import UnshardedFusedSingular

    slots, rows, gamma = 12, 8, 3
    g = torch.Generator().manual_seed(seed + 6)
    target_vocab = vocab + int(torch.randint(0, vocab + 1, (1,), generator=g))
    t = seed % (gamma + 1)
    print(f"sweep drafting: block={block} V_d={vocab} V_t={target_vocab} t={t} grammar={grammar} values={values} "
          f"seed={seed}", flush=True)
    host = random_host(slots, gamma + 1, target_vocab, seed + 7, EVERY_PROCESSOR)
    d2t = torch.randperm(target_vocab, generator=g)[:vocab].to(torch.int32)
    set_grammar(host, vocab, grammar, seed + 8, d2t=d2t)
    logits = sweep_logits(rows, vocab, values, seed + 9)
    slot_mapping = torch.randperm(slots, generator=g)[:rows].to(torch.int32)
    tokens = torch.randint(1, target_vocab, (rows, gamma + 1), generator=g).to(torch.int32)

    buffers = to_device(host, DEV)
    sampler = UnshardedFusedSingular.initialize(vocab_size=vocab, batch_size=rows, lookahead=gamma,
                                                block_size=block, max_top_logprobs=5, device=DEV)
    probs = torch.zeros(slots, target_vocab, dtype=BF16, device=DEV)
    dev_tokens = tokens.to(DEV)
    selection = sampler.drafting(logits.to(DEV), buffers, timestep=t, tokens=dev_tokens, probabilities=probs,
                                 slot_mapping=slot_mapping.to(DEV), d2t_mapping=d2t.to(DEV),
                                 target_vocab=target_vocab, in_place=True)
    torch.cuda.synchronize()

    state = oracle.State.from_buffers(host)
    expected = oracle.singular(logits, state, scope="draft", timestep=t, slot_mapping=slot_mapping.tolist(),
                               d2t=d2t, drafted=tokens, history=t, logprobs=False, probs=True,
                               max_top_logprobs=5)
    check_singular(selection, expected, logprobs=False, probabilities=probs, slot_mapping=slot_mapping)
    assert torch.equal(dev_tokens[:, t].cpu(), selection.tokens[:, 0].cpu())


def topk_cases(count: int, seed: int):
    """(block, vocab, rows, k, dtype, values, seed) of each bounded top-k case."""

    rng = random.Random(seed)
    cases = []

    for n in range(count):

        block = rng.choice([1024, 2048, 4096, 8192, 16384])
        tiles = rng.randint(2, min(128, 131072 // block))
        last = rng.choice([block, 1, 3, 64, 127, 128, 129, rng.randrange(1, block)])
        vocab = (tiles - 1) * block + last
        # 48 and 64 rows of 16385-32768 columns at k <= 32 take the one-workgroup-per-row launch
        rows = rng.choice([1, 5, 12, 48, 64]) if 16384 < vocab <= 32768 else rng.choice([1, 5, 12])
        k = 1 << rng.randint(0, 7)
        dtype = rng.choice(["bf16", "f32"])
        values = rng.choice(["spiked", "few", "flat", "cluster", "specials"])
        cases.append((block, vocab, rows, k, dtype, values, seed * 100 + n))

    return cases


TOPK_CASES = topk_cases(96, 11)


@pytest.mark.parametrize("block,vocab,rows,k,dtype,values,seed", TOPK_CASES)
def test_sweep_bounded_topk(block, vocab, rows, k, dtype, values, seed):
    """Bit-exact values and indices of `UnshardedBoundedTopK` against the stable-sort oracle.
    "cluster" raises 1-300 values inside one 512-column window (one tile holds the whole top-k, or
    two); "specials" mixes +-0 and +-inf into spiked rows."""

    from bench import spiked_logits
    from oracle.topk import topk as oracle_topk
    from sonic_sampler.interface import UnshardedBoundedTopK

    dt = torch.float32 if dtype == "f32" else BF16
    g = torch.Generator().manual_seed(seed)
    print(f"sweep top-k: block={block} V={vocab} rows={rows} k={k} {dtype} values={values} seed={seed}",
          flush=True)

    if values == "few":

        logits = torch.randint(-3, 4, (rows, vocab), generator=g).to(dt)

    elif values == "flat":

        logits = torch.full((rows, vocab), -1.25, dtype=dt)

    else:

        logits = spiked_logits(rows, vocab, seed, dtype=dt)

        for r in range(rows):

            if values == "cluster":

                n = int(torch.randint(1, 301, (1,), generator=g))
                start = int(torch.randint(0, max(1, vocab - 512), (1,), generator=g))
                cols = start + torch.randperm(min(512, vocab - start), generator=g)[:n]
                logits[r, cols] = (40.0 + torch.randint(0, 4, (len(cols),), generator=g).float()).to(dt)

            elif values == "specials":

                for v in (0.0, -0.0, float("inf"), float("-inf")):

                    cols = torch.randperm(vocab, generator=g)[:int(torch.randint(0, 40, (1,), generator=g))]
                    logits[r, cols] = v

    topk = UnshardedBoundedTopK.initialize(vocab_size=vocab, batch_size=rows, k=k, block_size=block, device=DEV)
    got_v, got_i = topk(logits.to(DEV))
    torch.cuda.synchronize()
    ev, ei = oracle_topk(logits, k)
    view = torch.int16 if dt == BF16 else torch.int32

    assert torch.equal(got_i.cpu(), ei), (got_i.cpu()[:2, :8], ei[:2, :8])
    assert torch.equal(got_v.cpu().view(view), ev.view(view))
