"""The reference's engine integration loops, end to end on device buffers.

Slot-based pre-allocation (reference docs/slot-based.md:33-315, capture :351-378): requests are
admitted into 256 of 512 slots with ``allocate`` on a copy stream (prompt histograms, penalties,
bias maps through the pinned relay, sampling parameters, grammar bitmasks, per-request generators),
then each iteration drafts gamma tokens through a d2t table into a larger target vocabulary under
per-timestep grammar masks (``drafting(..., in_place=True)`` writing ``tokens[:, t]`` and the draft
distribution into the strided view ``draft_probs[:rows, t]`` of one ``[slots, gamma, V_t]``
buffer, ``step_grammar`` between timesteps), verifies the chain against the target logits on the
same token and probability buffers with ``update_counts``, and advances the noise with
``step_weights`` (the ``ss_indexed_copy`` staging plus fresh draws). Every stage of every iteration
is checked against the CPU oracle composed from the device state it read. A second set of buffers,
admitted identically, runs the same iterations from one hipGraph capturing the gamma drafting
calls and the verifier (grammar and weight upkeep stay outside, as the guide prescribes), with the
slot mapping and logits copied in place; every replay must equal the eager iteration bit for bit.

Just-in-time batching (docs/just-in-time.md:35-287): a blank template is repopulated in batch
order before every iteration with ``update`` (counts, carried-over draft noise as
``target_gumbel``, parameters, prefill predicates), the loop runs on ``buffers[:rows]`` without a
slot mapping, and the draft noise and decode counts are read back into the requests.

The vocabularies are smaller than configuration 4's (8192 draft ids into 32768 target ids) so
that the oracle checks every row of three iterations within the test's time limit.
"""

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from helpers import check_multistep, check_singular, expected_multistep_counts
from oracle import sampler as oracle

pytestmark = pytest.mark.gpu

DEV = "cuda:0"

SLOTS, ROWS, GAMMA = 512, 256, 4
DRAFT_VOCAB, TARGET_VOCAB = 8192, 32768
TOP_Z = 5
ITERATIONS = 3
WORDS = TARGET_VOCAB // 32


# ------------------------------------------------------------------------------------------------
# Requests and their inputs (host side, seeded)
# ------------------------------------------------------------------------------------------------

def make_requests(count, seed, slots=None):
    """Requests of four kinds: 0 greedy; 1 stochastic verification of a greedy drafter (bit
    0x800), top-k and top logprobs; 2 stochastic both ways with penalties and min-p; 3 stochastic
    both ways under a grammar, with a bias map and top-p."""

    g = torch.Generator().manual_seed(seed)
    chosen = slots if slots is not None else list(range(count))
    requests = []

    for j, slot in enumerate(chosen):

        kind = j % 4
        prompt = torch.randint(0, TARGET_VOCAB, (int(torch.randint(4, 64, (1,), generator=g)),), generator=g)
        bias = None

        if kind in (1, 3):

            ids = torch.randperm(TARGET_VOCAB, generator=g)[:8].tolist()
            bias = {t: float(v) for t, v in zip(ids, (torch.rand(8, generator=g) * 6 - 3).tolist())}

        requests.append(SimpleNamespace(
            slot=slot, kind=kind, prompt=prompt,
            multiplicative=[1.0, 1.0, 1.2, 1.1][kind], frequency=[0.0, 0.0, 0.3, 0.0][kind],
            presence=[0.0, 0.0, 0.0, 0.5][kind], bias=bias,
            temperature=[1.0, 0.8, 1.3, 0.7][kind], top_k=[1, 50, 20, 128][kind],
            top_p=[1.0, 1.0, 1.0, 0.95][kind], min_p=[0.0, 0.0, 0.05, 0.0][kind],
            top_logprobs=[0, 3, 5, 2][kind], greedy_draft=kind == 1, grammar=kind == 3,
            seed=100000 * seed + j,
        ))

    return requests


def bitmask(request, iteration, timestep):
    """The request's grammar words at (iteration, timestep): each target id allowed with
    probability 0.3, as pinned int32 host words, or None without a grammar."""

    if not request.grammar:

        return None

    rng = np.random.default_rng([request.seed, iteration, timestep])
    bits = rng.random(TARGET_VOCAB) < 0.3
    words = np.packbits(bits.reshape(WORDS, 32), axis=1, bitorder="little").view("<u4").reshape(WORDS)

    words = torch.from_numpy(words.view(np.int32).copy())

    return words.pin_memory() if torch.cuda.is_available() else words


def generators(requests):
    """One persistent device generator per request, seeded from the request (as an engine seeds
    each request's generator once)."""

    return {r.slot: torch.Generator(DEV).manual_seed(r.seed) for r in requests}


def admit(buffers, requests, rngs, stream):
    """Slot-based admission of `requests` on `stream`; the compute stream waits for its event."""

    event = buffers.allocate(
        encodings=[r.prompt for r in requests], multiplicative=[r.multiplicative for r in requests],
        frequency=[r.frequency for r in requests], presence=[r.presence for r in requests],
        biases=[r.bias for r in requests], temperature=[r.temperature for r in requests],
        top_k=[r.top_k for r in requests], top_p=[r.top_p for r in requests],
        min_p=[r.min_p for r in requests], top_logprobs=[r.top_logprobs for r in requests],
        positions=[r.slot for r in requests], greedy_drafts=[r.greedy_draft for r in requests],
        bitmasks=[bitmask(r, 0, 0) for r in requests], generator=[rngs[r.slot] for r in requests],
        stream=stream)
    assert event is not None
    torch.cuda.current_stream().wait_event(event)


def draft_logits(iteration, timestep, rows):

    from bench import spiked_logits

    return spiked_logits(rows, DRAFT_VOCAB, seed=5000 + 10 * iteration + timestep)


def target_logits(iteration, drafted):
    """Target logits whose row (b, i) puts a dominant spike on the drafted token with probability
    0.7, so that chains stop at every position and some run to the bonus token."""

    from bench import spiked_logits

    rows = drafted.size(0)
    g = torch.Generator().manual_seed(6000 + iteration)
    x = spiked_logits(rows * (GAMMA + 1), TARGET_VOCAB, seed=6100 + iteration).float().view(rows, GAMMA + 1, -1)
    hit = torch.rand(rows, GAMMA, generator=g) < 0.7

    for b in range(rows):

        for i in range(GAMMA):

            if hit[b, i]:

                x[b, i, int(drafted[b, i])] += 25.0

    return x.to(torch.bfloat16)


# ------------------------------------------------------------------------------------------------
# Slot-based pre-allocation
# ------------------------------------------------------------------------------------------------

class SlotEngine:
    """One set of slot buffers with the engine's own token, probability and slot-mapping buffers."""

    def __init__(self, requests, copy_stream):

        from sonic_sampler.core.buffer import TINY, SamplingBuffers
        from sonic_sampler.interface import UnshardedFusedMultistep, UnshardedFusedSingular

        self.buffers = SamplingBuffers.default(size=SLOTS, timesteps=GAMMA + 1, vocab_size=TARGET_VOCAB,
                                               device=DEV, noise=False)
        # the same initial noise in every engine: admission redraws only what prefill needs
        w = self.buffers.weights
        g = torch.Generator(DEV).manual_seed(77)
        w.gumbel.target.exponential_(1.0, generator=g).log_()
        w.gumbel.draft.exponential_(1.0, generator=g).log_()
        w.uniform.uniform_(TINY, 1.0, generator=g)
        self.rngs = generators(requests)
        admit(self.buffers, requests, self.rngs, copy_stream)
        self.sampler = UnshardedFusedSingular.initialize(vocab_size=DRAFT_VOCAB, batch_size=ROWS,
                                                         lookahead=GAMMA, max_top_logprobs=TOP_Z, device=DEV)
        self.verifier = UnshardedFusedMultistep.initialize(vocab_size=TARGET_VOCAB, lookahead=GAMMA,
                                                           batch_size=ROWS, max_top_logprobs=TOP_Z, device=DEV)
        self.tokens = torch.zeros(ROWS, GAMMA + 1, dtype=torch.int32, device=DEV)
        self.draft_probs = torch.zeros(SLOTS, GAMMA, TARGET_VOCAB, dtype=torch.bfloat16, device=DEV)
        self.slot_mapping = torch.zeros(ROWS, dtype=torch.int32, device=DEV)
        self.draft_inputs = torch.zeros(GAMMA, ROWS, DRAFT_VOCAB, dtype=torch.bfloat16, device=DEV)
        self.target_inputs = torch.zeros(ROWS, GAMMA + 1, TARGET_VOCAB, dtype=torch.bfloat16, device=DEV)

    def draft(self, t, d2t):

        return self.sampler.drafting(self.draft_inputs[t], self.buffers, timestep=t, tokens=self.tokens[:ROWS],
                                     probabilities=self.draft_probs[:ROWS, t], slot_mapping=self.slot_mapping,
                                     d2t_mapping=d2t, target_vocab=TARGET_VOCAB, in_place=True)

    def verify(self):

        return self.verifier(self.target_inputs, self.tokens[:ROWS], self.buffers,
                             probabilities=self.draft_probs[:ROWS], slot_mapping=self.slot_mapping,
                             update_counts=True, logprobs=True, in_place=True)

    def step_grammar(self, order, iteration, timestep):

        self.buffers.step_grammar(bitmasks=[bitmask(r, iteration, timestep) for r in order],
                                  positions=[r.slot for r in order], timestep=timestep)

    def step_weights(self, order):

        self.buffers.step_weights(positions=[r.slot for r in order], indices=self.slot_mapping,
                                  generator=[self.rngs[r.slot] for r in order])


def check_admission(buffers, requests):
    """allocate's transfers landed: context histograms, zeroed decode counts, penalties, bias
    rows rebuilt from the maps (PinnedRelay.update_bias, then transfer), sampling parameters,
    indicator words and the step-0 grammar words."""

    bf = lambda v: float(torch.tensor(v).to(torch.bfloat16))  # noqa: E731
    rep = buffers.repetition
    context, decode, bias = rep.counts.context.cpu(), rep.counts.decode.cpu(), buffers.bias.cpu()
    grammar = buffers.grammar.view(torch.int32).cpu()
    packed = buffers.flags.packed.cpu().to(torch.int32)
    scalars = {name: getattr(buffers, name).float().cpu() for name in ("temperature", "top_p", "min_p")}
    ints = {name: getattr(buffers, name).cpu() for name in ("top_k", "top_logprobs")}
    pens = {name: getattr(rep, name).float().cpu() for name in ("multiplicative", "frequency", "presence")}

    for r in requests:

        s = r.slot
        hist = torch.bincount(r.prompt, minlength=TARGET_VOCAB).to(torch.int32)
        assert torch.equal(context[s], hist), s
        assert int(decode[s].abs().sum()) == 0, s
        if r.bias:

            # the row is rebuilt from the map: cleared, then the entries (rows admitted without a
            # map carry whatever the relay held, which no kernel reads with the bias bit off)
            row = torch.zeros(TARGET_VOCAB, dtype=torch.bfloat16)
            row[torch.tensor(list(r.bias))] = torch.tensor(list(r.bias.values())).to(torch.bfloat16)
            assert torch.equal(bias[s], row), s
            assert int(buffers.flags.indicators.target[s]) & 0x10

        for name in ("temperature", "top_p", "min_p"):

            assert float(scalars[name][s]) == bf(getattr(r, name)), (s, name)

        assert int(ints["top_k"][s]) == r.top_k and int(ints["top_logprobs"][s]) == r.top_logprobs

        for name in ("multiplicative", "frequency", "presence"):

            assert float(pens[name][s]) == bf(getattr(r, name)), (s, name)

        indicators = buffers.flags.indicators
        assert packed[s].tolist() == [int(indicators.target[s]), int(indicators.draft[s])], s
        assert bool(int(indicators.target[s]) & 0x40) == (r.top_k == 1)
        assert bool(int(indicators.target[s]) & 0x800) == r.greedy_draft
        mask = bitmask(r, 0, 0)
        expected = mask if mask is not None else torch.full((WORDS,), -1, dtype=torch.int32)
        assert torch.equal(grammar[s, 0], expected), s


def check_iteration(engine, state, order, iteration, d2t, drafted, targets, verification):
    """Each drafting step, the verification and the decode counts against the oracle composed from
    the state the kernels read (`state`: the buffers before drafting, with the grammar words as
    step_grammar left them)."""

    slots = [r.slot for r in order]
    probs = engine.draft_probs.cpu()

    for t in range(GAMMA):

        expected = oracle.singular(draft_logits(iteration, t, ROWS), state, scope="draft", timestep=t,
                                   slot_mapping=slots, d2t=d2t, drafted=drafted, history=t, probs=True,
                                   max_top_logprobs=TOP_Z)
        step = SimpleNamespace(tokens=drafted[:, t:t + 1], logprobs=None)
        mismatched, _ = check_singular(step, expected, logprobs=False, probabilities=probs[:, t],
                                       slot_mapping=slots)
        print(f"iteration {iteration} draft step {t}: knife-edge mismatches {mismatched}", flush=True)

    # greedy drafters leave their probability rows untouched (zero)
    for r in order:

        if r.greedy_draft or r.top_k == 1:

            assert int(probs[r.slot].float().abs().sum()) == 0, r.slot

    cu = list(range(0, ROWS * (GAMMA + 1) + 1, GAMMA + 1))
    expected = oracle.multistep(targets.view(-1, TARGET_VOCAB), state, drafted.reshape(-1), cu,
                                slot_mapping=slots, probabilities=probs, logprobs=True, max_top_logprobs=TOP_Z)
    mismatched = check_multistep(verification, expected, cu, logprobs=True)
    offsets = [int(o) for o in verification.offsets.reshape(-1).cpu()]
    print(f"iteration {iteration} verification: knife-edge mismatches {mismatched}, "
          f"offsets histogram {np.bincount(offsets, minlength=GAMMA + 1).tolist()}", flush=True)

    counts = expected_multistep_counts(state.decode, expected, verification, cu, mismatched, slots)
    assert torch.equal(engine.buffers.repetition.counts.decode.cpu(), counts)

    return offsets


def snapshot(buffers):
    """The members step_weights may change."""

    w = buffers.weights

    return [w.gumbel.target.clone(), w.gumbel.draft.clone(), w.uniform.clone()]


def check_step_weights(before, after, order):
    """step_weights staged the drafter's noise into the verifier's for stochastic drafters,
    redrew the noise of the batch's stochastic requests, and left every other slot alone.
    Compared per slot on the device."""

    target0, draft0, uniform0 = before
    target1, draft1, uniform1 = after
    same = lambda a, b: (a == b).flatten(1).all(1).cpu().tolist()  # noqa: E731
    kept_target, kept_draft, kept_uniform = same(target1, target0), same(draft1, draft0), same(uniform1, uniform0)
    staged = same(target1, draft0)
    batch = {r.slot: r for r in order}

    for s in range(SLOTS):

        r = batch.get(s)

        if r is None or r.top_k == 1:

            assert kept_target[s] and kept_draft[s] and kept_uniform[s], s

        elif r.greedy_draft:

            assert not kept_target[s] and kept_draft[s] and not kept_uniform[s], s   # target redrawn

        else:

            assert staged[s] and not kept_draft[s] and not kept_uniform[s], s       # staged, redrawn


def test_slot_based_speculative_loop_eager_and_captured():

    g = torch.Generator().manual_seed(11)
    slots = torch.randperm(SLOTS, generator=g)[:ROWS].tolist()
    requests = make_requests(ROWS, seed=1, slots=slots)
    d2t = torch.randperm(TARGET_VOCAB, generator=g)[:DRAFT_VOCAB].to(torch.int32)
    d2t_dev = d2t.to(DEV)
    copy_stream = torch.cuda.Stream()

    print(f"admitting {ROWS} requests into {SLOTS} slots (eager and graph buffer sets)", flush=True)
    eager = SlotEngine(requests, copy_stream)
    graphed = SlotEngine(requests, copy_stream)
    torch.cuda.synchronize()
    check_admission(eager.buffers, requests)
    assert torch.equal(eager.buffers.weights.gumbel.target.cpu(), graphed.buffers.weights.gumbel.target.cpu())

    graph = None
    captured = None
    accepted_any = rejected_any = False

    for it in range(ITERATIONS):

        order = [requests[j] for j in ([*range(ROWS)] if it == 0 else torch.randperm(ROWS, generator=g).tolist())]
        mapping = torch.tensor([r.slot for r in order], dtype=torch.int32)
        print(f"iteration {it}: eager drafting", flush=True)

        # ---- eager iteration -------------------------------------------------------------------
        eager.slot_mapping.copy_(mapping)

        if it > 0:

            eager.step_grammar(order, it, 0)

        for t in range(GAMMA):

            eager.draft_inputs[t].copy_(draft_logits(it, t, ROWS))

        state = oracle.State.from_buffers(eager.buffers)
        eager.draft_probs.zero_()

        for t in range(GAMMA):

            eager.draft(t, d2t_dev)
            eager.step_grammar(order, it, t + 1)

        drafted = eager.tokens.cpu()
        targets = target_logits(it, drafted)
        eager.target_inputs.copy_(targets)
        verification = eager.verify()
        torch.cuda.synchronize()
        state.grammar = eager.buffers.grammar.view(torch.int32).cpu()
        offsets = check_iteration(eager, state, order, it, d2t, drafted, targets, verification)
        accepted_any |= any(o > 0 for o in offsets)
        rejected_any |= any(o < GAMMA for o in offsets)
        eager_out = [eager.tokens.clone(), verification.offsets.clone(), verification.logprobs.selected.clone(),
                     eager.buffers.repetition.counts.decode.clone(), eager.draft_probs.clone()]

        # ---- the same iteration from one captured graph ----------------------------------------
        graphed.slot_mapping.copy_(mapping)
        graphed.draft_inputs.copy_(eager.draft_inputs)
        graphed.target_inputs.copy_(eager.target_inputs)

        for t in range(GAMMA + 1):

            if t > 0 or it > 0:

                graphed.step_grammar(order, it, t)

        torch.cuda.synchronize()

        if graph is None:

            print("capturing gamma drafting calls and the verifier in one graph", flush=True)
            graph = torch.cuda.CUDAGraph()

            with torch.cuda.graph(graph):

                graphed.draft_probs.zero_()

                for t in range(GAMMA):

                    graphed.draft(t, d2t_dev)

                captured = graphed.verify()

        print(f"iteration {it}: graph replay", flush=True)
        graph.replay()
        torch.cuda.synchronize()
        # logprobs are defined on each request's emitted span (positions 0..offset) only
        emitted = torch.arange(GAMMA + 1, device=DEV)[None] <= verification.offsets.view(-1, 1)
        eager_out[2] = eager_out[2][emitted]
        graph_out = [graphed.tokens, captured.offsets, captured.logprobs.selected[emitted],
                     graphed.buffers.repetition.counts.decode, graphed.draft_probs]

        for name, a, b in zip(("tokens", "offsets", "logprobs", "decode counts", "draft probabilities"),
                              eager_out, graph_out):

            assert torch.equal(a, b), f"iteration {it}: graph replay {name} differ from the eager loop"

        # ---- weight upkeep, outside the graph --------------------------------------------------
        before = snapshot(eager.buffers)
        eager.step_weights(order)
        graphed.step_weights(order)
        torch.cuda.synchronize()
        after = snapshot(eager.buffers)
        check_step_weights(before, after, order)

        for a, b in zip(after, snapshot(graphed.buffers)):

            assert torch.equal(a, b), f"iteration {it}: step_weights differs between the buffer sets"

    assert accepted_any and rejected_any


# ------------------------------------------------------------------------------------------------
# Just-in-time batching
# ------------------------------------------------------------------------------------------------

JIT_CAPACITY, JIT_VOCAB_DRAFT = 64, 8192


def test_just_in_time_loop_with_carried_state():
    """Three iterations over changing batches (requests leave, join with prefill, and change
    order): the template is repopulated with ``update`` on a copy stream, the loop runs on
    ``buffers[:rows]`` without a slot mapping, and each request's draft noise and decode counts are
    read back and carried into the next iteration (``target_gumbel`` for stochastic drafters)."""

    from sonic_sampler.core.buffer import SamplingBuffers
    from sonic_sampler.interface import UnshardedFusedMultistep, UnshardedFusedSingular

    pool = make_requests(48, seed=2)
    g = torch.Generator().manual_seed(12)
    d2t = torch.randperm(TARGET_VOCAB, generator=g)[:JIT_VOCAB_DRAFT].to(torch.int32)
    d2t_dev = d2t.to(DEV)

    for r in pool:

        r.context = torch.bincount(r.prompt, minlength=TARGET_VOCAB).to(torch.int32).to(DEV)
        r.decode = torch.zeros(TARGET_VOCAB, dtype=torch.int32, device=DEV)
        r.draft_weights = None
        r.started = False
        r.generator = torch.Generator(DEV).manual_seed(r.seed)

    template = SamplingBuffers.default(size=JIT_CAPACITY, timesteps=GAMMA + 1, vocab_size=TARGET_VOCAB, device=DEV)
    tokens = torch.zeros(JIT_CAPACITY, GAMMA + 1, dtype=torch.int32, device=DEV)
    draft_probs = torch.zeros(JIT_CAPACITY, GAMMA, TARGET_VOCAB, dtype=torch.bfloat16, device=DEV)
    copy_stream = torch.cuda.Stream()
    batches = [list(range(0, 40)), list(range(8, 48))[::-1], [5, 9, 41, 47, 2, 30, 31, 17, 12, 44, 3, 22]]

    for it, members in enumerate(batches):

        batch = [pool[j] for j in members]
        rows = len(batch)
        sampler = UnshardedFusedSingular.initialize(vocab_size=JIT_VOCAB_DRAFT, batch_size=rows, lookahead=GAMMA,
                                                    max_top_logprobs=TOP_Z, device=DEV)
        verifier = UnshardedFusedMultistep.initialize(vocab_size=TARGET_VOCAB, lookahead=GAMMA, batch_size=rows,
                                                      max_top_logprobs=TOP_Z, device=DEV)
        active = template[:rows]
        carried = [r.draft_weights if (r.started and not r.greedy_draft and r.top_k != 1) else None for r in batch]
        prefill = [not r.started for r in batch]
        print(f"jit iteration {it}: {rows} rows, {sum(prefill)} joining", flush=True)
        copy_stream.wait_stream(torch.cuda.current_stream())
        event = active.update(
            counts=[(r.context, r.decode) for r in batch], target_gumbel=carried,
            multiplicative=[r.multiplicative for r in batch], frequency=[r.frequency for r in batch],
            presence=[r.presence for r in batch], biases=[r.bias for r in batch],
            temperature=[r.temperature for r in batch], top_k=[r.top_k for r in batch],
            top_p=[r.top_p for r in batch], min_p=[r.min_p for r in batch],
            top_logprobs=[r.top_logprobs for r in batch], prefill=prefill,
            greedy_drafts=[r.greedy_draft for r in batch], bitmasks=[bitmask(r, it, 0) for r in batch],
            generator=[r.generator for r in batch], stream=copy_stream)
        torch.cuda.current_stream().wait_event(event)
        torch.cuda.synchronize()

        # the carried draft noise became the verifier's noise of its row
        for i, noise in enumerate(carried):

            if noise is not None:

                assert torch.equal(active.weights.gumbel.target[i], noise), (it, i)

        state = oracle.State.from_buffers(active)
        draft_probs.zero_()
        inputs = []

        for t in range(GAMMA):

            x = draft_logits(it, t, rows)[:, :JIT_VOCAB_DRAFT].contiguous()
            inputs.append(x)
            sampler.drafting(x.to(DEV), active, timestep=t, tokens=tokens[:rows], probabilities=draft_probs[:rows, t],
                             d2t_mapping=d2t_dev, target_vocab=TARGET_VOCAB, in_place=True)
            active.step_grammar(bitmasks=[bitmask(r, it, t + 1) for r in batch], timestep=t + 1)

        drafted = tokens[:rows].cpu()
        targets = target_logits(it, drafted)
        verification = verifier(targets.to(DEV), tokens[:rows], active, probabilities=draft_probs[:rows],
                                update_counts=True, logprobs=True, in_place=True)
        torch.cuda.synchronize()
        state.grammar = active.grammar.view(torch.int32).cpu()
        probs = draft_probs[:rows].cpu()

        for t in range(GAMMA):

            expected = oracle.singular(inputs[t], state, scope="draft", timestep=t, d2t=d2t, drafted=drafted,
                                       history=t, probs=True, max_top_logprobs=TOP_Z)
            check_singular(SimpleNamespace(tokens=drafted[:, t:t + 1], logprobs=None), expected, logprobs=False,
                           probabilities=probs[:, t])

        cu = list(range(0, rows * (GAMMA + 1) + 1, GAMMA + 1))
        expected = oracle.multistep(targets.view(-1, TARGET_VOCAB), state, drafted.reshape(-1), cu,
                                    probabilities=probs, logprobs=True, max_top_logprobs=TOP_Z)
        mismatched = check_multistep(verification, expected, cu, logprobs=True)
        counts = expected_multistep_counts(state.decode, expected, verification, cu, mismatched)
        assert torch.equal(active.repetition.counts.decode.cpu(), counts)

        # read back what the next iteration needs (one clone each, then row views)
        weights = active.weights.gumbel.draft.clone()
        decode = active.repetition.counts.decode.clone()

        for r, noise, dec in zip(batch, weights.unbind(), decode.unbind()):

            r.draft_weights = noise
            r.decode = dec
            r.started = True


class JitEngine:
    """A just-in-time template with its engine-owned buffers and the per-request state carried
    between iterations (context and decode counts, drafter noise, generator)."""

    def __init__(self, pool, rows, d2t):

        from sonic_sampler.core.buffer import TINY, SamplingBuffers
        from sonic_sampler.interface import UnshardedFusedMultistep, UnshardedFusedSingular

        self.template = SamplingBuffers.default(size=JIT_CAPACITY, timesteps=GAMMA + 1,
                                                vocab_size=TARGET_VOCAB, device=DEV, noise=False)
        # the same initial noise in every template: prefill redraws only the planes it needs
        w = self.template.weights
        g = torch.Generator(DEV).manual_seed(78)
        w.gumbel.target.exponential_(1.0, generator=g).log_()
        w.gumbel.draft.exponential_(1.0, generator=g).log_()
        w.uniform.uniform_(TINY, 1.0, generator=g)
        self.template.prepopulate(schedule=[rows])
        self.active = self.template[:rows]
        assert self.template[:rows] is self.active          # the cached slice a graph can bind to
        self.rows, self.d2t = rows, d2t
        self.sampler = UnshardedFusedSingular.initialize(vocab_size=JIT_VOCAB_DRAFT, batch_size=rows,
                                                         lookahead=GAMMA, max_top_logprobs=TOP_Z, device=DEV)
        self.verifier = UnshardedFusedMultistep.initialize(vocab_size=TARGET_VOCAB, lookahead=GAMMA,
                                                           batch_size=rows, max_top_logprobs=TOP_Z, device=DEV)
        self.tokens = torch.zeros(rows, GAMMA + 1, dtype=torch.int32, device=DEV)
        self.draft_probs = torch.zeros(rows, GAMMA, TARGET_VOCAB, dtype=torch.bfloat16, device=DEV)
        self.draft_inputs = torch.zeros(GAMMA, rows, JIT_VOCAB_DRAFT, dtype=torch.bfloat16, device=DEV)
        self.target_inputs = torch.zeros(rows, GAMMA + 1, TARGET_VOCAB, dtype=torch.bfloat16, device=DEV)
        self.state = {}

        for j, r in enumerate(pool):

            self.state[j] = SimpleNamespace(
                context=torch.bincount(r.prompt, minlength=TARGET_VOCAB).to(torch.int32).to(DEV),
                decode=torch.zeros(TARGET_VOCAB, dtype=torch.int32, device=DEV), draft_weights=None,
                started=False, generator=torch.Generator(DEV).manual_seed(r.seed))

    def populate(self, pool, members, iteration, copy_stream):

        batch = [pool[j] for j in members]
        st = [self.state[j] for j in members]
        carried = [s.draft_weights if (s.started and not r.greedy_draft and r.top_k != 1) else None
                   for r, s in zip(batch, st)]
        copy_stream.wait_stream(torch.cuda.current_stream())
        event = self.active.update(
            counts=[(s.context, s.decode) for s in st], target_gumbel=carried,
            multiplicative=[r.multiplicative for r in batch], frequency=[r.frequency for r in batch],
            presence=[r.presence for r in batch], biases=[r.bias for r in batch],
            temperature=[r.temperature for r in batch], top_k=[r.top_k for r in batch],
            top_p=[r.top_p for r in batch], min_p=[r.min_p for r in batch],
            top_logprobs=[r.top_logprobs for r in batch], prefill=[not s.started for s in st],
            greedy_drafts=[r.greedy_draft for r in batch], bitmasks=[bitmask(r, iteration, 0) for r in batch],
            generator=[s.generator for s in st], stream=copy_stream)
        torch.cuda.current_stream().wait_event(event)

    def draft(self, t):

        return self.sampler.drafting(self.draft_inputs[t], self.active, timestep=t, tokens=self.tokens,
                                     probabilities=self.draft_probs[:, t], d2t_mapping=self.d2t,
                                     target_vocab=TARGET_VOCAB, in_place=True)

    def verify(self):

        return self.verifier(self.target_inputs, self.tokens, self.active, probabilities=self.draft_probs,
                             update_counts=True, logprobs=True, in_place=True)

    def step_grammar(self, pool, members, iteration, timestep):

        self.active.step_grammar(bitmasks=[bitmask(pool[j], iteration, timestep) for j in members],
                                 timestep=timestep)

    def read_back(self, members):

        weights = self.active.weights.gumbel.draft.clone()
        decode = self.active.repetition.counts.decode.clone()

        for j, noise, dec in zip(members, weights.unbind(), decode.unbind()):

            s = self.state[j]
            s.draft_weights, s.decode, s.started = noise, dec, True


def test_just_in_time_loop_captured_in_a_graph():
    """The just-in-time loop at one batch size captured once (reference docs/just-in-time.md:
    289-330): the template's prefix slice is prepopulated, the gamma drafting calls and the
    verifier are captured against that fixed `buffers[:rows]` slice, and each iteration replays the
    graph after `update` has repopulated the slice and `step_grammar` has written the timesteps'
    masks (both outside the graph). A second template fed the same requests runs every iteration
    eagerly; replay and eager iteration must agree bit for bit, read-back state included, over
    three iterations whose batches differ in membership, order and prefill."""

    pool = make_requests(48, seed=3)
    rows = 32
    g = torch.Generator().manual_seed(13)
    d2t = torch.randperm(TARGET_VOCAB, generator=g)[:JIT_VOCAB_DRAFT].to(torch.int32).to(DEV)
    copy_stream = torch.cuda.Stream()
    eager, graphed = JitEngine(pool, rows, d2t), JitEngine(pool, rows, d2t)
    batches = [list(range(0, 32)), list(range(16, 48))[::-1], torch.randperm(48, generator=g)[:32].tolist()]
    graph = captured = None

    for it, members in enumerate(batches):

        print(f"jit capture iteration {it}: {sum(not eager.state[j].started for j in members)} joining", flush=True)

        for eng in (eager, graphed):

            eng.populate(pool, members, it, copy_stream)

            for t in range(GAMMA):

                eng.draft_inputs[t].copy_(draft_logits(it, t, rows)[:, :JIT_VOCAB_DRAFT])

        # eager iteration
        eager.draft_probs.zero_()

        for t in range(GAMMA):

            eager.draft(t)
            eager.step_grammar(pool, members, it, t + 1)

        targets = target_logits(it, eager.tokens.cpu())
        eager.target_inputs.copy_(targets)
        graphed.target_inputs.copy_(targets)
        verification = eager.verify()

        # graph iteration: the masks of timesteps 1..gamma go in before the replay
        for t in range(1, GAMMA + 1):

            graphed.step_grammar(pool, members, it, t)

        torch.cuda.synchronize()

        if graph is None:

            graph = torch.cuda.CUDAGraph()

            with torch.cuda.graph(graph):

                graphed.draft_probs.zero_()

                for t in range(GAMMA):

                    graphed.draft(t)

                captured = graphed.verify()

        graph.replay()
        torch.cuda.synchronize()
        emitted = torch.arange(GAMMA + 1, device=DEV)[None] <= verification.offsets.view(-1, 1)
        pairs = [("tokens", eager.tokens, graphed.tokens), ("offsets", verification.offsets, captured.offsets),
                 ("logprobs", verification.logprobs.selected[emitted], captured.logprobs.selected[emitted]),
                 ("decode counts", eager.active.repetition.counts.decode, graphed.active.repetition.counts.decode),
                 ("draft probabilities", eager.draft_probs, graphed.draft_probs),
                 ("verifier noise", eager.active.weights.gumbel.target, graphed.active.weights.gumbel.target)]

        for name, a, b in pairs:

            assert torch.equal(a, b), f"iteration {it}: graph replay {name} differ from the eager loop"

        eager.read_back(members)
        graphed.read_back(members)
