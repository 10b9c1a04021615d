"""Fused single-step sampling on the GPU vs the CPU oracle."""

import pytest
import torch

from helpers import check_singular, expected_singular_counts
from oracle import sampler as oracle

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def test_config1_autoregressive():

    from bench import c1_workload, to_device
    from sonic_sampler.interface import UnshardedFusedSingular

    work = c1_workload()
    batch, vocab = work.logits.shape
    print(f"config 1: B={batch} V={vocab}", flush=True)

    buffers = to_device(work.buffers, DEV)
    sampler = UnshardedFusedSingular.initialize(vocab_size=vocab, batch_size=batch, max_top_logprobs=5, device=DEV)
    selection = sampler.autoregressive(work.logits.to(DEV), buffers, update_counts=True, logprobs=True)
    torch.cuda.synchronize()

    state = oracle.State.from_buffers(work.buffers)
    expected = oracle.singular(work.logits, state, scope="target", logprobs=True, max_top_logprobs=5)
    mismatched, checked = check_singular(selection, expected, logprobs=True)
    print(f"knife-edge mismatches: {mismatched}, fully checked rows: {checked}", flush=True)
    assert checked >= batch - 4

    counts = expected_singular_counts(state.decode, expected, selection, mismatched)
    assert torch.equal(buffers.repetition.counts.decode.cpu(), counts)


def test_min_p_rounds_scores_to_bf16():
    """The kernel's min-p test compares bf16 scores with a bf16 threshold, as the reference's
    PyTorch path does (core/naive.py:316-326). Each row holds the logits (0, -1.203125, -4) at three
    columns in different tiles and -60 elsewhere, under min_p = bf16(0.3): in bf16 the second
    score (0.2275390625) equals the threshold bf16(0.30078125 * 0.7578125) and stays, while fp32
    scores would mask it (0.227712 < 0.228112). Noise of +10 on the first column makes the kept
    second column the selected token; a kernel with fp32 scores would select the first."""

    from sonic_sampler.core.buffer import SamplingBuffers
    from sonic_sampler.core.flags import Flags, ScopedIndicators
    from sonic_sampler.interface import UnshardedFusedSingular
    from bench import to_device

    rows, vocab = 8, 16384
    scoped = ScopedIndicators.from_params(
        size=rows, timesteps=1, multiplicative=[1.0] * rows, frequency=[0.0] * rows,
        presence=[0.0] * rows, biases=[{} for _ in range(rows)], temperature=[1.0] * rows,
        top_k=[128] * rows, top_p=[1.0] * rows, min_p=[0.3] * rows, top_logprobs=[0] * rows,
    )
    host = SamplingBuffers.default(size=rows, timesteps=1, vocab_size=vocab, device="cpu", noise=False)
    host.flags = Flags.from_scoped(scoped, device="cpu")
    host.min_p.fill_(0.3)
    assert float(host.min_p[0]) == 0.30078125
    host.weights.gumbel.target.zero_()
    logits = torch.full((rows, vocab), -60.0, dtype=torch.bfloat16)
    cols = [(1000 * r + 7, 5000 + 13 * r, 16000 + r) for r in range(rows)]

    for r, (c0, c1, c2) in enumerate(cols):

        logits[r, c0], logits[r, c1], logits[r, c2] = 0.0, -1.203125, -4.0
        host.weights.gumbel.target[r, 0, c0] = 10.0

    buffers = to_device(host, DEV)
    print("min-p at the bf16 rounding point", flush=True)
    sampler = UnshardedFusedSingular.initialize(vocab_size=vocab, batch_size=rows, block_size=2048, device=DEV)
    selection = sampler.autoregressive(logits.to(DEV), buffers, logprobs=True)
    torch.cuda.synchronize()

    assert [int(t) for t in selection.tokens[:, 0].cpu()] == [c1 for _, c1, _ in cols]
    state = oracle.State.from_buffers(host)
    expected = oracle.singular(logits, state, scope="target", logprobs=True)
    assert [e.token for e in expected] == [c1 for _, c1, _ in cols]
    check_singular(selection, expected, logprobs=True, max_knife_fraction=0.0)


def test_config1_philox_matches_materialized_noise():

    from bench import c1_workload, to_device
    from sonic_sampler.interface import UnshardedFusedSingular
    from sonic_sampler.noise import materialize_gumbel

    work = c1_workload()
    batch, vocab = work.logits.shape
    buffers = to_device(work.buffers, DEV)
    sampler = UnshardedFusedSingular.initialize(vocab_size=vocab, batch_size=batch, max_top_logprobs=5, device=DEV)
    logits = work.logits.to(DEV)

    print("config 1 with Philox noise", flush=True)
    a = sampler.autoregressive(logits, buffers, logprobs=True, philox_seed=77, philox_offset=3)
    noise = materialize_gumbel(77, 3, batch, 1, vocab, device=DEV)
    buffers.weights.gumbel.target.copy_(noise)
    b = sampler.autoregressive(logits, buffers, logprobs=True)
    torch.cuda.synchronize()

    assert torch.equal(a.tokens.cpu(), b.tokens.cpu())
    assert torch.equal(a.logprobs.selected.cpu(), b.logprobs.selected.cpu())

    state = oracle.State.from_buffers(work.buffers)
    expected = oracle.singular(work.logits, state, scope="target", noise=noise[:, 0].cpu(),
                               logprobs=True, max_top_logprobs=5)
    check_singular(a, expected, logprobs=True)


@pytest.mark.parametrize("seed", [0, 1, 2, 3])
def test_random_buffers_drafting_slots_d2t(seed):
    """Mixed random indicators, slot mapping, d2t, drafted history and probability scatter."""

    from sonic_sampler.core.buffer import SamplingBuffers
    from sonic_sampler.interface import UnshardedFusedSingular
    from bench import spiked_logits, to_device

    slots, rows, gamma, t = 12, 8, 3, 2
    draft_vocab, target_vocab = 4096, 8192
    g = torch.Generator().manual_seed(seed)

    host = SamplingBuffers.random(size=slots, timesteps=gamma + 1, vocab_size=target_vocab,
                                  device="cpu", seed=seed, max_top_logprobs=5)
    buffers = to_device(host, DEV)
    logits = spiked_logits(rows, draft_vocab, seed=100 + seed)
    slot_mapping = torch.randperm(slots, generator=g)[:rows].to(torch.int32)
    d2t = torch.randperm(target_vocab, generator=g)[:draft_vocab].to(torch.int32)
    tokens = torch.randint(1, target_vocab, (rows, gamma + 1), generator=g).to(torch.int32)
    print(f"random drafting seed={seed} indicators={[hex(int(v)) for v in host.flags.indicators.draft]}", flush=True)

    sampler = UnshardedFusedSingular.initialize(vocab_size=draft_vocab, batch_size=rows, lookahead=gamma,
                                                block_size=1024, max_top_logprobs=5, device=DEV)
    probs = torch.zeros(slots, target_vocab, dtype=torch.bfloat16, device=DEV)
    dev_tokens = tokens.to(DEV)
    selection = sampler.drafting(logits.to(DEV), buffers, timestep=t, tokens=dev_tokens, probabilities=probs,
                                 slot_mapping=slot_mapping.to(DEV), d2t_mapping=d2t.to(DEV),
                                 target_vocab=target_vocab, in_place=True)
    torch.cuda.synchronize()

    state = oracle.State.from_buffers(host)
    expected = oracle.singular(logits, state, scope="draft", timestep=t, slot_mapping=slot_mapping.tolist(),
                               d2t=d2t, drafted=tokens, history=t, logprobs=False,
                               probs=not host.flags.all_greedy, max_top_logprobs=5)
    check_singular(selection, expected, logprobs=False,
                   probabilities=probs if not host.flags.all_greedy else None, slot_mapping=slot_mapping)

    written = dev_tokens[:, t].cpu()
    assert torch.equal(written, selection.tokens[:, 0].cpu())


@pytest.mark.parametrize("seed", [10, 11, 12])
def test_random_buffers_autoregressive_logprobs(seed):

    from sonic_sampler.core.buffer import SamplingBuffers
    from sonic_sampler.interface import UnshardedFusedSingular
    from bench import spiked_logits, to_device

    rows, vocab = 16, 16384
    host = SamplingBuffers.random(size=rows, timesteps=1, vocab_size=vocab, device="cpu", seed=seed,
                                  max_top_logprobs=8)
    buffers = to_device(host, DEV)
    logits = spiked_logits(rows, vocab, seed=200 + seed)
    print(f"random autoregressive seed={seed}", flush=True)

    sampler = UnshardedFusedSingular.initialize(vocab_size=vocab, batch_size=rows, max_top_logprobs=8,
                                                block_size=2048, device=DEV)
    selection = sampler.autoregressive(logits.to(DEV), buffers, prefill=True, update_counts=True, logprobs=True)
    torch.cuda.synchronize()

    state = oracle.State.from_buffers(host)
    expected = oracle.singular(logits, state, scope="target", logprobs=True, max_top_logprobs=8)
    check_singular(selection, expected, logprobs=True)

    counts = oracle.apply_singular_counts(state.decode, expected, None, prefill=True)
    assert torch.equal(buffers.repetition.counts.decode.cpu(), counts)


def test_config4_drafting_full_size():

    from bench import c4_workload, to_device
    from sonic_sampler.interface import UnshardedFusedSingular

    work = c4_workload()
    rows = work.logits.size(0)
    slots = work.buffers.layout.rows
    print(f"config 4: rows={rows} slots={slots} V_d={work.vocab} V_t={work.target_vocab}", flush=True)

    buffers = to_device(work.buffers, DEV)
    sampler = UnshardedFusedSingular.initialize(vocab_size=work.vocab, batch_size=rows, lookahead=4,
                                                max_top_logprobs=5, device=DEV)
    probs = torch.zeros(slots, work.target_vocab, dtype=torch.bfloat16, device=DEV)
    tokens = work.tokens.to(DEV)
    selection = sampler.drafting(work.logits.to(DEV), buffers, timestep=work.timestep, tokens=tokens,
                                 probabilities=probs, slot_mapping=work.slot_mapping.to(DEV),
                                 d2t_mapping=work.d2t.to(DEV), target_vocab=work.target_vocab, in_place=True)
    torch.cuda.synchronize()

    state = oracle.State.from_buffers(work.buffers)
    expected = oracle.singular(work.logits, state, scope="draft", timestep=work.timestep,
                               slot_mapping=work.slot_mapping.tolist(), d2t=work.d2t, drafted=work.tokens,
                               history=work.timestep, probs=True, max_top_logprobs=5)
    check_singular(selection, expected, logprobs=False, probabilities=probs, slot_mapping=work.slot_mapping)

    # every selected token is grammar-admissible and in the d2t image
    image = set(work.d2t.tolist())
    assert all(int(t) in image for t in selection.tokens[:, 0].cpu())


@pytest.mark.parametrize("seed", [20, 21])
def test_concentrated_and_tied_rows(seed):
    """Rows that defeat the sampled merge (one tile holding most of the top-128) or the tile
    stage's lower bound (long runs of equal keys) take the exact radix paths; results must not
    change."""

    from sonic_sampler.core.buffer import SamplingBuffers
    from sonic_sampler.interface import UnshardedFusedSingular
    from bench import spiked_logits, to_device

    rows, vocab, block = 16, 65536, 2048
    g = torch.Generator().manual_seed(seed)
    logits = spiked_logits(rows, vocab, seed=300 + seed).float()
    for r in range(rows):
        kind = r % 4
        if kind == 0:    # 60 large values inside one tile
            tile = int(torch.randint(0, vocab // block, (1,), generator=g))
            cols = tile * block + torch.randperm(block, generator=g)[:60]
            logits[r, cols] = 25.0 + torch.rand(60, generator=g) * 5.0
        elif kind == 1:  # every logit equal
            logits[r] = 0.5
        elif kind == 2:  # a handful of distinct values
            logits[r] = torch.randint(-3, 4, (vocab,), generator=g).float()
    logits = logits.to(torch.bfloat16)
    host = SamplingBuffers.random(size=rows, timesteps=1, vocab_size=vocab, device="cpu", seed=seed,
                                  max_top_logprobs=8)
    buffers = to_device(host, DEV)
    print(f"concentrated / tied rows seed={seed}", flush=True)

    sampler = UnshardedFusedSingular.initialize(vocab_size=vocab, batch_size=rows, max_top_logprobs=8,
                                                block_size=block, device=DEV)
    selection = sampler.autoregressive(logits.to(DEV), buffers, logprobs=True)
    torch.cuda.synchronize()

    state = oracle.State.from_buffers(host)
    expected = oracle.singular(logits, state, scope="target", logprobs=True, max_top_logprobs=8)
    check_singular(selection, expected, logprobs=True)


def test_extreme_divisors_and_penalties():
    """Rows whose divisors fall outside the reciprocal fast path (a subnormal temperature, a
    subnormal repetition penalty on counted tokens, a temperature near the top of the bf16 range)
    and a huge frequency penalty: the IEEE chain runs on every element, +inf and tiny values tie
    in long runs, and the tokens must match the oracle. Top-k only and no logprobs, so no softmax
    ever sees an infinity."""

    from sonic_sampler.core.buffer import SamplingBuffers
    from sonic_sampler.core.flags import Flags, ScopedIndicators
    from sonic_sampler.interface import UnshardedFusedSingular
    from bench import spiked_logits, to_device

    rows, vocab = 16, 16384
    bf = lambda v: float(torch.tensor(v).to(torch.bfloat16))  # noqa: E731
    temperature = [bf(1e-39)] * 4 + [bf(0.8)] * 4 + [bf(3e38)] * 4 + [1.0] * 4
    multiplicative = [1.0] * 4 + [bf(1e-39)] * 4 + [1.0] * 8
    frequency = [0.0] * 12 + [bf(1e30)] * 4
    top_k = [50] * 4 + [20] * 4 + [128] * 4 + [64] * 4
    scoped = ScopedIndicators.from_params(
        size=rows, timesteps=1, multiplicative=multiplicative, frequency=frequency,
        presence=[0.0] * rows, biases=[{} for _ in range(rows)], temperature=temperature,
        top_k=top_k, top_p=[1.0] * rows, min_p=[0.0] * rows, top_logprobs=[0] * rows,
    )
    g = torch.Generator().manual_seed(5)
    host = SamplingBuffers.default(size=rows, timesteps=1, vocab_size=vocab, device="cpu", noise=False)
    host.flags = Flags.from_scoped(scoped, device="cpu")
    host.weights.gumbel.target.exponential_(1.0, generator=g).log_()
    host.temperature.copy_(torch.tensor(temperature).to(torch.bfloat16))
    host.top_k.copy_(torch.tensor(top_k, dtype=torch.int32))
    rep = host.repetition
    rep.multiplicative.copy_(torch.tensor(multiplicative).to(torch.bfloat16))
    rep.frequency.copy_(torch.tensor(frequency).to(torch.bfloat16))
    history = torch.randint(0, vocab, (rows, 256), generator=g)
    rep.counts.decode.zero_().scatter_add_(1, history, torch.ones_like(history, dtype=torch.int32))
    logits = spiked_logits(rows, vocab, seed=404)
    buffers = to_device(host, DEV)
    print("extreme divisors and penalties", flush=True)

    sampler = UnshardedFusedSingular.initialize(vocab_size=vocab, batch_size=rows, block_size=2048, device=DEV)
    selection = sampler.autoregressive(logits.to(DEV), buffers, logprobs=False)
    torch.cuda.synchronize()

    state = oracle.State.from_buffers(host)
    expected = oracle.singular(logits, state, scope="target", logprobs=False)
    tokens = selection.tokens[:, 0].cpu()
    assert [int(t) for t in tokens] == [e.token for e in expected]


def test_truncation_at_its_extremes():
    """Truncation parameters at their ends, with logprobs and the top logprobs: top-p keeping only
    the first candidate (p = 0.01) or nearly all, min-p at 0.99 (only values tied with the
    maximum survive) and at 0.5, top-k of 2, 3 and 127, and the three combined, at temperatures
    from 0.05 to 20 on tied and spiked rows."""

    from sonic_sampler.core.buffer import SamplingBuffers
    from sonic_sampler.core.flags import Flags, ScopedIndicators
    from sonic_sampler.interface import UnshardedFusedSingular
    from bench import spiked_logits, to_device

    rows, vocab = 16, 16384
    bf = lambda v: float(torch.tensor(v).to(torch.bfloat16))  # noqa: E731
    top_p = [bf(v) for v in (0.01, 0.99, 1.0, 1.0, 1.0, 1.0, 1.0, 1.0, 0.5, 0.01, 0.9, 1.0, 1.0, 0.3, 1.0, 0.05)]
    min_p = [bf(v) for v in (0.0, 0.0, 0.99, 0.5, 0.0, 0.0, 0.0, 0.0, 0.2, 0.99, 0.0, 0.05, 0.0, 0.0, 0.9, 0.0)]
    top_k = [128, 128, 128, 128, 2, 3, 127, 128, 3, 2, 50, 20, 128, 128, 128, 127]
    temperature = [bf(v) for v in (1.0, 0.05, 20.0, 1.0, 0.5, 3.0, 1.0, 0.05, 1.0, 20.0, 1.0, 0.7, 1.0, 2.0, 0.1, 1.0)]
    scoped = ScopedIndicators.from_params(
        size=rows, timesteps=1, multiplicative=[1.0] * rows, frequency=[0.0] * rows, presence=[0.0] * rows,
        biases=[{} for _ in range(rows)], temperature=temperature, top_k=top_k, top_p=top_p, min_p=min_p,
        top_logprobs=[5] * rows)
    g = torch.Generator().manual_seed(6)
    host = SamplingBuffers.default(size=rows, timesteps=1, vocab_size=vocab, device="cpu", noise=False)
    host.flags = Flags.from_scoped(scoped, device="cpu")
    host.weights.gumbel.target.exponential_(1.0, generator=g).log_()
    host.temperature.copy_(torch.tensor(temperature).to(torch.bfloat16))
    host.top_p.copy_(torch.tensor(top_p).to(torch.bfloat16))
    host.min_p.copy_(torch.tensor(min_p).to(torch.bfloat16))
    host.top_k.copy_(torch.tensor(top_k, dtype=torch.int32))
    host.top_logprobs.fill_(5)
    logits = spiked_logits(rows, vocab, seed=606)
    # tied rows: a few distinct values, so that truncation cuts through runs of equal candidates
    logits[1::4] = (torch.randint(-2, 3, (rows // 4, vocab), generator=g).float() * 2.0).to(torch.bfloat16)
    buffers = to_device(host, DEV)
    print("truncation at its extremes", flush=True)

    sampler = UnshardedFusedSingular.initialize(vocab_size=vocab, batch_size=rows, max_top_logprobs=5,
                                                block_size=2048, device=DEV)
    selection = sampler.autoregressive(logits.to(DEV), buffers, logprobs=True)
    torch.cuda.synchronize()

    state = oracle.State.from_buffers(host)
    expected = oracle.singular(logits, state, scope="target", logprobs=True, max_top_logprobs=5)
    _, checked = check_singular(selection, expected, logprobs=True, max_knife_fraction=0.1)
    assert checked >= rows - 1


def test_logit_bias_forcing_and_banning():
    """Logit bias at the ends of its use: +100 on one token forces it, -inf on each row's argmax
    (and its runner-up) bans them, alongside ordinary biases, with penalties and logprobs."""

    from sonic_sampler.interface import UnshardedFusedSingular
    from bench import spiked_logits, to_device

    from test_gpu_paths import EVERY_PROCESSOR, random_host

    rows, vocab = 12, 16384
    host = random_host(rows, 1, vocab, 8, EVERY_PROCESSOR)
    logits = spiked_logits(rows, vocab, seed=808)
    g = torch.Generator().manual_seed(8)
    bias = host.bias
    top2 = logits.float().topk(2, dim=-1).indices
    forced = torch.randint(0, vocab, (rows,), generator=g)

    for r in range(rows):

        if r % 3 == 0:

            bias[r, forced[r]] = 100.0

        elif r % 3 == 1:

            bias[r, top2[r]] = float("-inf")

    buffers = to_device(host, DEV)
    print("logit bias forcing and banning", flush=True)

    sampler = UnshardedFusedSingular.initialize(vocab_size=vocab, batch_size=rows, max_top_logprobs=5,
                                                block_size=4096, device=DEV)
    selection = sampler.autoregressive(logits.to(DEV), buffers, logprobs=True)
    torch.cuda.synchronize()

    state = oracle.State.from_buffers(host)
    expected = oracle.singular(logits, state, scope="target", logprobs=True, max_top_logprobs=5)
    check_singular(selection, expected, logprobs=True)
    tokens = selection.tokens[:, 0].cpu()

    for r in range(rows):

        if r % 3 == 1:

            assert int(tokens[r]) not in top2[r].tolist(), r


def test_merge_paths_at_128_tiles():
    """V = 131072 at block 1024: 128 candidate lists of which the row merge samples 4 entries
    each. Rows whose top-128 crowds into a few lists have those lists merged whole; rows with
    more crowded lists than the bound, or all-equal rows, take the radix merge. Every path must
    give the oracle's tokens and logprobs."""

    from helpers import merge_path_logits
    from sonic_sampler.core.buffer import SamplingBuffers
    from sonic_sampler.interface import UnshardedFusedSingular
    from bench import to_device

    rows, vocab, block = 20, 131072, 1024
    logits = merge_path_logits(rows, vocab, block, seed=61)
    host = SamplingBuffers.random(size=rows, timesteps=1, vocab_size=vocab, device="cpu", seed=62,
                                  max_top_logprobs=8)
    buffers = to_device(host, DEV)
    print(f"merge paths at 128 tiles: rows={rows}", flush=True)

    sampler = UnshardedFusedSingular.initialize(vocab_size=vocab, batch_size=rows, max_top_logprobs=8,
                                                block_size=block, device=DEV)
    selection = sampler.autoregressive(logits.to(DEV), buffers, logprobs=True)
    torch.cuda.synchronize()

    state = oracle.State.from_buffers(host)
    expected = oracle.singular(logits, state, scope="target", logprobs=True, max_top_logprobs=8)
    check_singular(selection, expected, logprobs=True)
