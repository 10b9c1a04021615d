"""Fused chain verification on the GPU vs the CPU oracle."""

import pytest
import torch

from helpers import check_multistep, expected_multistep_counts, run_verifier
from oracle import sampler as oracle

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def test_config2_greedy():

    from bench import c2_workload

    work = c2_workload()
    print(f"config 2: rows={work.logits.size(0)} V={work.vocab}", flush=True)
    verification, buffers, _ = run_verifier(work, update_counts=True)

    state = oracle.State.from_buffers(work.buffers)
    expected = oracle.multistep(work.logits, state, work.drafted, work.cu_seqlens, logprobs=True)
    check_multistep(verification, expected, work.cu_seqlens, logprobs=True, max_knife_fraction=0.0)

    counts = oracle.apply_multistep_counts(state.decode, expected, None)
    assert torch.equal(buffers.repetition.counts.decode.cpu(), counts)


def test_config3_stochastic_varlen():

    from bench import c3_workload

    work = c3_workload()
    print(f"config 3: rows={work.logits.size(0)} requests={len(work.cu_seqlens) - 1}", flush=True)
    verification, buffers, verifier = run_verifier(work, update_counts=True)

    state = oracle.State.from_buffers(work.buffers)
    expected = oracle.multistep(work.logits, state, work.drafted, work.cu_seqlens,
                                probabilities=work.probabilities, logprobs=True, max_top_logprobs=20)
    mismatched = check_multistep(verification, expected, work.cu_seqlens, logprobs=True)
    print(f"knife-edge mismatches: {mismatched}", flush=True)

    # the per-row top-128 ids are exact
    indices = verifier.indices.cpu()

    for b, e in enumerate(expected):

        for i, idx in enumerate(e.row_indices):

            assert torch.equal(indices[work.cu_seqlens[b] + i], idx), (b, i)

    counts = expected_multistep_counts(state.decode, expected, verification, work.cu_seqlens, mismatched)
    assert torch.equal(buffers.repetition.counts.decode.cpu(), counts)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_random_buffers_fixed_gamma_slots(seed):
    """Mixed random indicators (incl. 0x800, greedy, penalties, grammar) with slot mapping."""

    from bench import MultistepWorkload, spiked_logits, to_device
    from sonic_sampler.core.buffer import SamplingBuffers

    slots, batch, gamma, vocab = 10, 6, 3, 8192
    n = gamma + 1
    g = torch.Generator().manual_seed(seed)
    host = SamplingBuffers.random(size=slots, timesteps=n, vocab_size=vocab, device="cpu", seed=50 + seed,
                                  max_top_logprobs=4)
    logits = spiked_logits(batch * n, vocab, seed=300 + seed)
    slot_mapping = torch.randperm(slots, generator=g)[:batch].to(torch.int32)

    argmax = logits.float().argmax(-1)
    drafted = torch.where(torch.rand(batch * n, generator=g) < 0.6, argmax,
                          torch.randint(1, vocab, (batch * n,), generator=g)).to(torch.int32)
    probabilities = torch.softmax(torch.randn(slots, gamma, vocab, generator=g) * 2, dim=-1).to(torch.bfloat16)

    work = MultistepWorkload(logits=logits, drafted=drafted, buffers=host,
                             cu_seqlens=list(range(0, batch * n + 1, n)), lookahead=gamma, vocab=vocab,
                             max_top_logprobs=4, probabilities=probabilities)
    print(f"random multistep seed={seed} indicators={[hex(int(host.flags.indicators.target[int(s)])) for s in slot_mapping]}", flush=True)
    verification, buffers, _ = run_verifier(work, update_counts=True, block_size=1024,
                                            slot_mapping=slot_mapping.to(DEV))

    state = oracle.State.from_buffers(host)
    expected = oracle.multistep(logits, state, drafted, work.cu_seqlens, slot_mapping=slot_mapping.tolist(),
                                probabilities=probabilities, logprobs=True, max_top_logprobs=4)
    mismatched = check_multistep(verification, expected, work.cu_seqlens, logprobs=True, max_knife_fraction=0.34)

    counts = expected_multistep_counts(state.decode, expected, verification, work.cu_seqlens, mismatched,
                                       slot_mapping.tolist())
    assert torch.equal(buffers.repetition.counts.decode.cpu(), counts)


def test_all_accepted_emits_bonus_from_last_step():

    from bench import MultistepWorkload, spiked_logits
    from sonic_sampler.core.buffer import SamplingBuffers
    from sonic_sampler.core.flags import Flags, Indicator

    batch, gamma, vocab = 4, 3, 4096
    n = gamma + 1
    logits = spiked_logits(batch * n, vocab, seed=7)
    drafted = logits.float().argmax(-1).to(torch.int32)
    host = SamplingBuffers.default(size=batch, timesteps=n, vocab_size=vocab, device="cpu")
    host.flags = Flags.from_values(batch, n, Indicator.GREEDY, device="cpu")
    work = MultistepWorkload(logits=logits, drafted=drafted, buffers=host,
                             cu_seqlens=list(range(0, batch * n + 1, n)), lookahead=gamma, vocab=vocab,
                             max_top_logprobs=0)
    verification, _, _ = run_verifier(work, block_size=1024, logprobs=False)
    assert verification.offsets.cpu().flatten().tolist() == [gamma] * batch
    assert torch.equal(verification.tokens.cpu().flatten(), drafted)


def test_requests_without_drafts():
    """Variable lookahead down to a request of one row (no drafts: only the bonus row, offset 0)
    beside longer ones, stochastic and greedy, with slots: tokens, offsets, logprobs and the
    per-row top-128 ids against the oracle."""

    from bench import MultistepWorkload, spiked_logits
    from sonic_sampler.core.flags import Flags, Indicator

    gamma, vocab, slots = 3, 8192, 6
    cu = [0, 1, 4, 5, 9, 10]
    batch, rows = len(cu) - 1, cu[-1]
    host = random_buffers(slots, gamma + 1, vocab, seed=71)
    every = Indicator(0x3BF) | Indicator.TOP_K_LOGPROBS
    greedy = (every & ~Indicator.stochastic()) | Indicator.GREEDY
    host.flags = Flags.from_values(slots, gamma + 1, [every, greedy, every, every, greedy, every], device="cpu")
    host.top_k.copy_(torch.tensor([128, 1, 128, 50, 1, 128], dtype=torch.int32))
    logits = spiked_logits(rows, vocab, seed=72)
    g = torch.Generator().manual_seed(73)
    drafted = torch.randint(1, vocab, (rows,), generator=g).to(torch.int32)
    slot_mapping = torch.tensor([4, 1, 0, 5, 2], dtype=torch.int32)
    probabilities = torch.softmax(torch.randn(slots, gamma, vocab, generator=g) * 2, dim=-1).to(torch.bfloat16)
    work = MultistepWorkload(logits=logits, drafted=drafted, buffers=host, cu_seqlens=cu, lookahead=gamma,
                             vocab=vocab, max_top_logprobs=4, probabilities=probabilities, varlen=True)
    print(f"requests without drafts: cu_seqlens={cu}", flush=True)
    verification, buffers, verifier = run_verifier(work, update_counts=True, block_size=1024,
                                                   slot_mapping=slot_mapping.to("cuda:0"))

    state = oracle.State.from_buffers(host)
    expected = oracle.multistep(logits, state, drafted, cu, slot_mapping=slot_mapping.tolist(),
                                probabilities=probabilities, logprobs=True, max_top_logprobs=4)
    mismatched = check_multistep(verification, expected, cu, logprobs=True, max_knife_fraction=0.2)
    offsets = verification.offsets.reshape(-1).tolist()

    for b in (0, 2, 4):

        assert offsets[b] == 0, b          # one-row requests emit their bonus row's token

    indices = verifier.indices.cpu()

    for b, e in enumerate(expected):

        for i, idx in enumerate(e.row_indices):

            assert torch.equal(indices[cu[b] + i], idx), (b, i)

    counts = expected_multistep_counts(state.decode, expected, verification, cu, mismatched,
                                       slot_mapping.tolist())
    assert torch.equal(buffers.repetition.counts.decode.cpu(), counts)


def random_buffers(slots, timesteps, vocab, seed):

    from sonic_sampler.core.buffer import SamplingBuffers

    return SamplingBuffers.random(size=slots, timesteps=timesteps, vocab_size=vocab, device="cpu", seed=seed,
                                  max_top_logprobs=4)


def test_maximum_lookahead():
    """gamma = 63, the most one wave per request verifies: 64 rows per request, every processor
    on (the penalties see up to 63 drafted tokens of history), a greedy request whose drafts are
    its argmaxes (the chain runs to the bonus row 63), one whose chain breaks at row 40 and a
    stochastic one; the per-row top-128 ids, the tokens, offsets and logprobs against the
    oracle."""

    from bench import MultistepWorkload, spiked_logits
    from sonic_sampler.core.buffer import SamplingBuffers
    from sonic_sampler.core.flags import Flags, Indicator

    batch, gamma, vocab = 3, 63, 8192
    n = gamma + 1
    host = SamplingBuffers.random(size=batch, timesteps=n, vocab_size=vocab, device="cpu", seed=63,
                                  max_top_logprobs=4)
    every = Indicator(0x3BF) | Indicator.TOP_K_LOGPROBS
    greedy = (every & ~Indicator.stochastic()) | Indicator.GREEDY
    host.flags = Flags.from_values(batch, n, [greedy, greedy, every], device="cpu")
    host.top_k.copy_(torch.tensor([1, 1, 128], dtype=torch.int32))
    logits = spiked_logits(batch * n, vocab, seed=64)
    g = torch.Generator().manual_seed(65)
    state = oracle.State.from_buffers(host)
    drafted = torch.randint(1, vocab, (batch * n,), generator=g).to(torch.int32)
    # the greedy requests' drafts are their rows' argmaxes after the processors, the drafts before
    # each row counting as its history (the oracle's processed rows); one chain broken at row 40
    for b in (0, 1):

        for i in range(n):

            x = oracle.process_row(logits[b * n + i], state, b, int(state.target[b]), state.grammar[b, i],
                                   [int(t) for t in drafted[b * n: b * n + i]], None)
            drafted[b * n + i] = int(x.argmax())

    drafted[1 * n + 40] = (drafted[1 * n + 40] + 1) % vocab
    probabilities = torch.softmax(torch.randn(batch, gamma, vocab, generator=g) * 2, dim=-1).to(torch.bfloat16)
    work = MultistepWorkload(logits=logits, drafted=drafted, buffers=host,
                             cu_seqlens=list(range(0, batch * n + 1, n)), lookahead=gamma, vocab=vocab,
                             max_top_logprobs=4, probabilities=probabilities)
    print("maximum lookahead: gamma=63", flush=True)
    verification, buffers, verifier = run_verifier(work, update_counts=True, block_size=2048)

    expected = oracle.multistep(logits, state, drafted, work.cu_seqlens, probabilities=probabilities,
                                logprobs=True, max_top_logprobs=4)
    mismatched = check_multistep(verification, expected, work.cu_seqlens, logprobs=True, max_knife_fraction=0.34)
    offsets = verification.offsets.reshape(-1).tolist()

    assert 0 not in mismatched and offsets[0] == gamma
    assert 1 not in mismatched and offsets[1] == 40
    indices = verifier.indices.cpu()

    for b, e in enumerate(expected):

        for i, idx in enumerate(e.row_indices):

            assert torch.equal(indices[b * n + i], idx), (b, i)

    counts = expected_multistep_counts(state.decode, expected, verification, work.cu_seqlens, mismatched)
    assert torch.equal(buffers.repetition.counts.decode.cpu(), counts)


def test_merge_paths_at_128_tiles():
    """Multistep rows at V = 131072, block 1024 (128 lists, 4 sampled per list) whose top-128
    crowds into a few lists, into more lists than the whole-list bound, or ties everywhere: the
    per-row top-128 ids and the verification must match the oracle."""

    from bench import MultistepWorkload
    from helpers import merge_path_logits
    from sonic_sampler.core.buffer import SamplingBuffers

    batch, gamma, vocab, block = 5, 3, 131072, 1024
    n = gamma + 1
    g = torch.Generator().manual_seed(63)
    host = SamplingBuffers.random(size=batch, timesteps=n, vocab_size=vocab, device="cpu", seed=64,
                                  max_top_logprobs=4)
    logits = merge_path_logits(batch * n, vocab, block, seed=65)
    argmax = logits.float().argmax(-1)
    drafted = torch.where(torch.rand(batch * n, generator=g) < 0.5, argmax,
                          torch.randint(1, vocab, (batch * n,), generator=g)).to(torch.int32)
    probabilities = torch.softmax(torch.randn(batch, gamma, vocab, generator=g) * 2, dim=-1).to(torch.bfloat16)
    work = MultistepWorkload(logits=logits, drafted=drafted, buffers=host,
                             cu_seqlens=list(range(0, batch * n + 1, n)), lookahead=gamma, vocab=vocab,
                             max_top_logprobs=4, probabilities=probabilities)
    print(f"multistep merge paths at 128 tiles: rows={batch * n}", flush=True)
    verification, _, verifier = run_verifier(work, update_counts=True, block_size=block)

    state = oracle.State.from_buffers(host)
    expected = oracle.multistep(logits, state, drafted, work.cu_seqlens, probabilities=probabilities,
                                logprobs=True, max_top_logprobs=4)
    check_multistep(verification, expected, work.cu_seqlens, logprobs=True, max_knife_fraction=0.34)

    indices = verifier.indices.cpu()

    for b, e in enumerate(expected):

        for i, idx in enumerate(e.row_indices):

            assert torch.equal(indices[work.cu_seqlens[b] + i], idx), (b, i)


@pytest.mark.parametrize("block", [4096, 16384])
def test_temperature_rows_at_the_cut(block):
    """Temperature-only rows whose scaled keys tie where the tile stage cuts its top-128:
    temperatures with inexact reciprocals (neighbouring logits share a scaled key, so the cut goes
    by column), tiny logits under a large temperature (scaled keys collide in long runs), rows of
    equal logits and rows of a few distinct values (the exact cut). The last tile is partial. The
    per-row top-128 ids must match the oracle exactly."""

    from bench import MultistepWorkload, spiked_logits
    from sonic_sampler.core.buffer import SamplingBuffers
    from sonic_sampler.core.flags import Flags, ScopedIndicators

    batch, gamma, vocab = 6, 3, 65432
    n = gamma + 1
    rows = batch * n
    g = torch.Generator().manual_seed(71)
    bf = lambda v: float(torch.tensor(v).to(torch.bfloat16))  # noqa: E731
    temperature = [bf(t) for t in (3.0, 1.7, 50.0, 0.3, 7.0, 1.3)]
    scoped = ScopedIndicators.from_params(
        size=batch, timesteps=n, multiplicative=[1.0] * batch, frequency=[0.0] * batch,
        presence=[0.0] * batch, biases=[{} for _ in range(batch)], temperature=temperature,
        top_k=[128] * batch, top_p=[1.0] * batch, min_p=[0.0] * batch, top_logprobs=[4] * batch,
    )
    host = SamplingBuffers.default(size=batch, timesteps=n, vocab_size=vocab, device="cpu", noise=False)
    host.flags = Flags.from_scoped(scoped, device="cpu")
    host.weights.gumbel.target.exponential_(1.0, generator=g).log_()
    host.temperature.copy_(torch.tensor(temperature).to(torch.bfloat16))
    logits = spiked_logits(rows, vocab, seed=72).float()

    for r in range(rows):

        kind = r % 4

        if kind == 1:
            logits[r] = torch.randn(vocab, generator=g) * 1e-37
        elif kind == 2:
            logits[r] = 0.75
        elif kind == 3:
            logits[r] = torch.randint(-3, 4, (vocab,), generator=g).float() * 0.3

    logits = logits.to(torch.bfloat16)
    drafted = torch.randint(1, vocab, (rows,), generator=g, dtype=torch.int32)
    work = MultistepWorkload(logits=logits, drafted=drafted, buffers=host,
                             cu_seqlens=list(range(0, rows + 1, n)), lookahead=gamma, vocab=vocab,
                             max_top_logprobs=4, probabilities=None)
    print(f"temperature rows at the cut: block={block}", flush=True)
    verification, _, verifier = run_verifier(work, block_size=block)

    state = oracle.State.from_buffers(host)
    expected = oracle.multistep(logits, state, drafted, work.cu_seqlens, logprobs=True, max_top_logprobs=4)
    check_multistep(verification, expected, work.cu_seqlens, logprobs=True, max_knife_fraction=0.34)

    indices = verifier.indices.cpu()

    for b, e in enumerate(expected):

        for i, idx in enumerate(e.row_indices):

            assert torch.equal(indices[work.cu_seqlens[b] + i], idx), (b, i, temperature[b])


def test_config2_all_greedy_hint():
    """Config 2 with the all_greedy hint (no row launch: the request stage takes every row's argmax
    from the tiles' maxima) gives the oracle's verification and the same values / indices columns
    as the call without it."""

    from bench import c2_workload

    work = c2_workload()
    print("config 2 with the all_greedy hint", flush=True)
    plain, _, verifier = run_verifier(work)
    plain_indices = verifier.indices[:, 0].clone()
    hinted, buffers, verifier2 = run_verifier(work, all_greedy=True, update_counts=True)

    state = oracle.State.from_buffers(work.buffers)
    expected = oracle.multistep(work.logits, state, work.drafted, work.cu_seqlens, logprobs=True)
    check_multistep(hinted, expected, work.cu_seqlens, logprobs=True, max_knife_fraction=0.0)
    counts = oracle.apply_multistep_counts(state.decode, expected, None)
    assert torch.equal(buffers.repetition.counts.decode.cpu(), counts)
    assert torch.equal(hinted.tokens.cpu(), plain.tokens.cpu())
    assert torch.equal(hinted.offsets.cpu(), plain.offsets.cpu())
    assert torch.equal(verifier2.indices[:, 0].cpu(), plain_indices.cpu())
    assert torch.all(verifier2.values[:, 0].cpu() == 0)


def test_wrong_all_greedy_hint_marks_the_request():
    """A request whose indicator is not greedy under the all_greedy hint is not served and says
    so (offsets -1); the greedy requests of the same call still match the oracle."""

    from bench import MultistepWorkload, spiked_logits
    from sonic_sampler.core.buffer import SamplingBuffers
    from sonic_sampler.core.flags import Flags, Indicator

    batch, gamma, vocab = 6, 3, 16384
    n = gamma + 1
    logits = spiked_logits(batch * n, vocab, seed=17)
    g = torch.Generator().manual_seed(17)
    argmax = logits.float().argmax(-1)
    drafted = torch.where(torch.rand(batch * n, generator=g) < 0.7, argmax,
                          torch.randint(1, vocab, (batch * n,), generator=g)).to(torch.int32)
    host = SamplingBuffers.default(size=batch, timesteps=n, vocab_size=vocab, device="cpu")
    indicators = [Indicator.GREEDY] * batch
    indicators[2] = Indicator.TEMPERATURE        # the hint is wrong for request 2
    host.flags = Flags.from_values(batch, n, indicators, device="cpu")
    host.top_k.copy_(torch.tensor([1, 1, 128, 1, 1, 1], dtype=torch.int32))
    work = MultistepWorkload(logits=logits, drafted=drafted, buffers=host,
                             cu_seqlens=list(range(0, batch * n + 1, n)), lookahead=gamma, vocab=vocab,
                             max_top_logprobs=5)
    print("wrong all_greedy hint for request 2", flush=True)
    verification, _, _ = run_verifier(work, all_greedy=True, block_size=1024)

    offsets = verification.offsets.reshape(-1).cpu().tolist()
    assert offsets[2] == -1
    state = oracle.State.from_buffers(host)
    expected = oracle.multistep(logits, state, drafted, work.cu_seqlens, logprobs=True)
    tokens = verification.tokens.reshape(-1).cpu()

    for b in (0, 1, 3, 4, 5):

        assert offsets[b] == expected[b].offset, b
        m = work.cu_seqlens[b]
        assert [int(t) for t in tokens[m: m + offsets[b] + 1]] == expected[b].tokens, b
        assert torch.equal(tokens[m + offsets[b] + 1: m + n], drafted[m + offsets[b] + 1: m + n]), b

    # the request that is not served keeps its drafts
    assert torch.equal(tokens[2 * n: 3 * n], drafted[2 * n: 3 * n])


@pytest.mark.parametrize("in_place", [False, True])
def test_token_buffer_written_whole(in_place):
    """The verifier writes every row of the token buffer: each request's drafts with its emitted
    token at its offset, and the drafts of the rows outside every request (cu_seqlens starting
    above row 0 and ending before the last row), in a new buffer and in place over the drafts."""

    from bench import spiked_logits, to_device
    from sonic_sampler.core.buffer import SamplingBuffers
    from sonic_sampler.interface import UnshardedFusedMultistep

    gamma, vocab, rows = 3, 8192, 21
    cu = [2, 6, 8, 12, 16]            # four requests over rows 2..15; rows 0-1 and 16-20 are outside
    batch = len(cu) - 1
    logits = spiked_logits(rows, vocab, seed=23)
    g = torch.Generator().manual_seed(23)
    drafted = torch.randint(1, vocab, (rows,), generator=g).to(torch.int32)
    host = SamplingBuffers.random(size=batch, timesteps=gamma + 1, vocab_size=vocab, device="cpu", seed=23,
                                  max_top_logprobs=5)
    buffers = to_device(host, "cuda:0")
    # buffers for 6 requests of gamma + 1 rows: room for the 21 rows
    verifier = UnshardedFusedMultistep.initialize(vocab_size=vocab, lookahead=gamma, batch_size=6,
                                                  block_size=1024, max_top_logprobs=5, device="cuda:0")
    tokens = drafted.to("cuda:0")
    print(f"token buffer written whole, in_place={in_place}", flush=True)
    verification = verifier(logits.to("cuda:0"), tokens, buffers, logprobs=True, in_place=in_place,
                            cu_seqlens=torch.tensor(cu, dtype=torch.int32, device="cuda:0"))
    torch.cuda.synchronize()

    out = verification.tokens.cpu()
    offsets = verification.offsets.reshape(-1).cpu().tolist()
    assert (verification.tokens.data_ptr() == tokens.data_ptr()) == in_place
    assert torch.equal(out[:cu[0]], drafted[:cu[0]]) and torch.equal(out[cu[-1]:], drafted[cu[-1]:])

    state = oracle.State.from_buffers(host)
    shifted = [c - cu[0] for c in cu]
    expected = oracle.multistep(logits[cu[0]:cu[-1]], state, drafted[cu[0]:cu[-1]], shifted, logprobs=True)

    for b, e in enumerate(expected):

        m, end = cu[b], cu[b + 1]

        if e.knife:

            continue

        assert offsets[b] == e.offset, b
        assert [int(t) for t in out[m: m + offsets[b] + 1]] == e.tokens, b
        assert torch.equal(out[m + offsets[b] + 1: end], drafted[m + offsets[b] + 1: end]), b


def test_graph_replay_config2_all_greedy_hint():
    """Config 2 with the all_greedy hint captured in a hipGraph (tile and request launches only)
    and replayed over new logits, drafts and decode counts copied into the captured tensors: every
    replay equals the eager call, and the first ones the oracle."""

    from bench import c2_workload, to_device
    from sonic_sampler.interface import UnshardedFusedMultistep

    sets = [c2_workload(seed=1002 + 10 * k) for k in range(3)]
    base = sets[0]
    batch, n = len(base.cu_seqlens) - 1, base.lookahead + 1
    buffers = to_device(base.buffers, DEV)
    logits = base.logits.view(batch, n, -1).to(DEV)
    drafted = base.drafted.view(batch, n).to(DEV)
    decode = buffers.repetition.counts.decode
    verifier = UnshardedFusedMultistep.initialize(vocab_size=base.vocab, lookahead=base.lookahead,
                                                  batch_size=batch, max_top_logprobs=base.max_top_logprobs,
                                                  device=DEV)

    def load(k):

        logits.copy_(sets[k].logits.view(batch, n, -1))
        drafted.copy_(sets[k].drafted.view(batch, n))
        decode.copy_(sets[k].buffers.repetition.counts.decode)

    def call():

        return verifier(logits, drafted, buffers, update_counts=True, logprobs=True, all_greedy=True)

    def outputs(v):

        return [v.offsets.clone(), v.tokens.clone(), decode.clone()]

    eager = []

    for k in range(3):

        load(k)
        eager.append(outputs(call()))

    torch.cuda.synchronize()
    print("config 2 with the all_greedy hint, eager outputs for 3 input sets; capturing", flush=True)
    load(0)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())

    with torch.cuda.stream(side):

        call()

    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()

    with torch.cuda.graph(graph):

        captured = call()

    for rnd, k in enumerate([1, 2, 0, 2, 1]):

        load(k)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        print(f"replay {rnd}: input set {k}", flush=True)
        got = outputs(captured)

        for a, b in zip(got, eager[k]):

            assert torch.equal(a, b), f"replay {rnd} of input set {k} differs from the eager call"

        if rnd < 3:

            work = sets[k]
            state = oracle.State.from_buffers(work.buffers)
            expected = oracle.multistep(work.logits, state, work.drafted, work.cu_seqlens, logprobs=True)
            check_multistep(captured, expected, work.cu_seqlens, logprobs=True, max_knife_fraction=0.0)
            counts = oracle.apply_multistep_counts(state.decode, expected, None)
            assert torch.equal(got[-1].cpu(), counts)
