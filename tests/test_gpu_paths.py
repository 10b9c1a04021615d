"""GPU parity on the kernel paths the configuration tests do not reach.

* per-element (scalar) loads: vocabularies that are not multiples of 4, logits whose rows start 2
  bytes off an 8-byte boundary or whose row stride is not a multiple of 4, and d2t gathers over a
  draft vocabulary that is not a multiple of 4;
* the 8192-column tile, whose processor chain runs in two 4096-column halves, on rows with every
  processor on and a partial last tile ending in either half;
* outputs under hipGraph replay: one captured single-step call and one captured verification,
  replayed over three input sets copied into the captured tensors (logits, slot mapping,
  indicators, parameters, counts, noise), each replay checked against an eager call on the same
  inputs and against the oracle (the reference's contract that results hold across capture,
  docs/slot-based.md:351-378).
"""

import pytest
import torch

from helpers import (check_multistep, check_singular, expected_multistep_counts, expected_singular_counts,
                     load_into, run_verifier)
from oracle import sampler as oracle

pytestmark = pytest.mark.gpu

DEV = "cuda:0"

# grammar, repetition / frequency / presence penalties, bias, temperature, top-k, top-p, min-p
EVERY_PROCESSOR = 0x3BF


def random_host(slots, timesteps, vocab, seed, indicator=None, max_top_logprobs=5):

    from sonic_sampler.core.buffer import SamplingBuffers
    from sonic_sampler.core.flags import Indicator

    return SamplingBuffers.random(size=slots, timesteps=timesteps, vocab_size=vocab, device="cpu",
                                  seed=seed, max_top_logprobs=max_top_logprobs,
                                  indicators=None if indicator is None else Indicator(indicator))


def autoregressive_case(logits, host, block, *, prefill=False, slot_mapping=None):
    """One autoregressive call with logprobs and count updates, checked against the oracle."""

    from bench import to_device
    from sonic_sampler.interface import UnshardedFusedSingular

    rows, vocab = logits.shape
    buffers = to_device(host, DEV)
    sampler = UnshardedFusedSingular.initialize(vocab_size=vocab, batch_size=rows, max_top_logprobs=5,
                                                block_size=block, device=DEV)
    dev_slots = None if slot_mapping is None else slot_mapping.to(DEV)
    selection = sampler.autoregressive(logits, buffers, prefill=prefill, update_counts=True, logprobs=True,
                                       slot_mapping=dev_slots)
    torch.cuda.synchronize()

    state = oracle.State.from_buffers(host)
    slots = None if slot_mapping is None else slot_mapping.tolist()
    expected = oracle.singular(logits.cpu().contiguous(), state, scope="target", slot_mapping=slots,
                               logprobs=True, max_top_logprobs=5)
    mismatched, checked = check_singular(selection, expected, logprobs=True)

    counts = expected_singular_counts(state.decode, expected, selection, mismatched, slots, prefill=prefill)
    assert torch.equal(buffers.repetition.counts.decode.cpu(), counts)

    return checked


# ------------------------------------------------------------------------------------------------
# Per-element loads
# ------------------------------------------------------------------------------------------------

@pytest.mark.parametrize("indicator,seed", [(EVERY_PROCESSOR, 31), (None, 32)])
def test_scalar_path_vocabulary_not_a_multiple_of_4(indicator, seed):

    from bench import spiked_logits

    rows, vocab = 16, 50257
    print(f"scalar path: V={vocab} indicator={indicator} seed={seed}", flush=True)
    host = random_host(rows, 1, vocab, seed, indicator)
    logits = spiked_logits(rows, vocab, seed=500 + seed).to(DEV)
    assert autoregressive_case(logits, host, 2048) >= rows - 2


@pytest.mark.parametrize("layout", ["offset_2_bytes", "stride_not_multiple_of_4"])
def test_scalar_path_unaligned_logit_rows(layout):

    from bench import spiked_logits

    rows, vocab = 8, 16384
    print(f"scalar path: logits {layout}", flush=True)
    host = random_host(rows, 1, vocab, 33, EVERY_PROCESSOR)
    wide = spiked_logits(rows, vocab + 2, seed=533).to(DEV)
    # a view 2 bytes into every row (stride V + 2), or rows of stride V + 2 starting aligned
    logits = wide[:, 1:vocab + 1] if layout == "offset_2_bytes" else wide[:, :vocab]
    assert logits.stride(0) % 4 != 0 or logits.data_ptr() % 8 != 0
    assert autoregressive_case(logits, host, 2048) >= rows - 1


@pytest.mark.parametrize("seed", [40, 41])
def test_scalar_path_d2t_draft_vocabulary_not_a_multiple_of_4(seed):

    from bench import spiked_logits, to_device
    from sonic_sampler.interface import UnshardedFusedSingular

    slots, rows, gamma, t = 12, 8, 3, 2
    draft_vocab, target_vocab = 4099, 8192
    g = torch.Generator().manual_seed(seed)
    host = random_host(slots, gamma + 1, target_vocab, seed)
    buffers = to_device(host, DEV)
    logits = spiked_logits(rows, draft_vocab, seed=600 + seed)
    slot_mapping = torch.randperm(slots, generator=g)[:rows].to(torch.int32)
    d2t = torch.randperm(target_vocab, generator=g)[:draft_vocab].to(torch.int32)
    tokens = torch.randint(1, target_vocab, (rows, gamma + 1), generator=g).to(torch.int32)
    print(f"d2t scalar path seed={seed} indicators={[hex(int(v)) for v in host.flags.indicators.draft]}", flush=True)

    sampler = UnshardedFusedSingular.initialize(vocab_size=draft_vocab, batch_size=rows, lookahead=gamma,
                                                block_size=1024, max_top_logprobs=5, device=DEV)
    probs = torch.zeros(slots, target_vocab, dtype=torch.bfloat16, device=DEV)
    selection = sampler.drafting(logits.to(DEV), buffers, timestep=t, tokens=tokens.to(DEV),
                                 probabilities=probs, slot_mapping=slot_mapping.to(DEV),
                                 d2t_mapping=d2t.to(DEV), target_vocab=target_vocab, in_place=True)
    torch.cuda.synchronize()

    state = oracle.State.from_buffers(host)
    stochastic = not host.flags.all_greedy
    expected = oracle.singular(logits, state, scope="draft", timestep=t, slot_mapping=slot_mapping.tolist(),
                               d2t=d2t, drafted=tokens, history=t, probs=stochastic, max_top_logprobs=5)
    check_singular(selection, expected, logprobs=False, probabilities=probs if stochastic else None,
                   slot_mapping=slot_mapping)


def test_more_than_512_tiles():
    """586 tiles of 1024 columns (V = 600,000): the row merge samples nothing (512 / tiles < 1)
    and every row takes the radix merge over all 75,008 candidates, with every processor on."""

    from bench import spiked_logits

    rows, vocab = 4, 600_000
    print(f"more than 512 tiles: V={vocab}", flush=True)
    host = random_host(rows, 1, vocab, 512, EVERY_PROCESSOR)
    logits = spiked_logits(rows, vocab, seed=513).to(DEV)
    assert autoregressive_case(logits, host, 1024) >= rows - 1


def test_drafting_with_the_longest_history():
    """Drafting at timestep 64 (the longest history a wave stages) with every processor on: the
    penalties count the 64 drafted tokens of each row's history, through d2t and slots."""

    from bench import spiked_logits, to_device
    from sonic_sampler.interface import UnshardedFusedSingular

    slots, rows, gamma, t = 10, 8, 64, 64
    draft_vocab, target_vocab = 8192, 12288
    g = torch.Generator().manual_seed(64)
    host = random_host(slots, gamma + 1, target_vocab, 64, EVERY_PROCESSOR)
    buffers = to_device(host, DEV)
    logits = spiked_logits(rows, draft_vocab, seed=640)
    slot_mapping = torch.randperm(slots, generator=g)[:rows].to(torch.int32)
    d2t = torch.randperm(target_vocab, generator=g)[:draft_vocab].to(torch.int32)
    # histories drawn from the drafter's targets, so that they hit the rows' candidates often
    tokens = d2t[torch.randint(0, 256, (rows, gamma + 1), generator=g)].to(torch.int32)
    print("drafting at timestep 64", flush=True)

    sampler = UnshardedFusedSingular.initialize(vocab_size=draft_vocab, batch_size=rows, lookahead=gamma,
                                                block_size=2048, max_top_logprobs=5, device=DEV)
    probs = torch.zeros(slots, target_vocab, dtype=torch.bfloat16, device=DEV)
    selection = sampler.drafting(logits.to(DEV), buffers, timestep=t, tokens=tokens.to(DEV), probabilities=probs,
                                 slot_mapping=slot_mapping.to(DEV), d2t_mapping=d2t.to(DEV),
                                 target_vocab=target_vocab, in_place=True)
    torch.cuda.synchronize()

    state = oracle.State.from_buffers(host)
    expected = oracle.singular(logits, state, scope="draft", timestep=t, slot_mapping=slot_mapping.tolist(),
                               d2t=d2t, drafted=tokens, history=t, probs=True, max_top_logprobs=5)
    check_singular(selection, expected, logprobs=False, probabilities=probs, slot_mapping=slot_mapping)


@pytest.mark.parametrize("seed,draft_vocab,target_vocab,block", [(44, 6144, 8197, 2048), (45, 6144, 8197, 2048),
                                                                (46, 40000, 131075, 16384),
                                                                (47, 40000, 300007, 16384),
                                                                (48, 40000, 300007, 8192)])
def test_staged_grammar_target_vocabulary_not_a_multiple_of_32(seed, draft_vocab, target_vocab, block):
    """Drafting through d2t into a 8197-token target vocabulary (its last grammar word holds 5
    tokens) with every processor on: the tile kernel stages each row's 257 grammar words in
    workgroup memory, clears the bits past the vocabulary and reads a zero quad for clamped
    columns. Half the rows allow every token, including garbage bits past the vocabulary; d2t
    reaches the last target ids. A 300007-token target exceeds what the kernel stages (8192 words):
    its gathers read the grammar words from global memory (in four passes at 16384 columns)."""

    from bench import spiked_logits, to_device
    from sonic_sampler.interface import UnshardedFusedSingular

    slots, rows, gamma, t = 10, 8, 3, 1
    g = torch.Generator().manual_seed(seed)
    host = random_host(slots, gamma + 1, target_vocab, seed, indicator=EVERY_PROCESSOR)
    host.grammar.view(torch.int32)[::2] = -1
    logits = spiked_logits(rows, draft_vocab, seed=610 + seed)
    slot_mapping = torch.randperm(slots, generator=g)[:rows].to(torch.int32)
    d2t = torch.cat([torch.arange(target_vocab - 64, target_vocab),
                     torch.randperm(target_vocab - 64, generator=g)[:draft_vocab - 64]])
    d2t = d2t[torch.randperm(draft_vocab, generator=g)].to(torch.int32)
    tokens = torch.randint(1, target_vocab, (rows, gamma + 1), generator=g).to(torch.int32)
    buffers = to_device(host, DEV)
    print(f"staged grammar V_t={target_vocab} seed={seed}", flush=True)

    sampler = UnshardedFusedSingular.initialize(vocab_size=draft_vocab, batch_size=rows, lookahead=gamma,
                                                block_size=block, max_top_logprobs=5, device=DEV)
    probs = torch.zeros(slots, target_vocab, dtype=torch.bfloat16, device=DEV)
    selection = sampler.drafting(logits.to(DEV), buffers, timestep=t, tokens=tokens.to(DEV),
                                 probabilities=probs, slot_mapping=slot_mapping.to(DEV),
                                 d2t_mapping=d2t.to(DEV), target_vocab=target_vocab, in_place=True)
    torch.cuda.synchronize()

    state = oracle.State.from_buffers(host)
    expected = oracle.singular(logits, state, scope="draft", timestep=t, slot_mapping=slot_mapping.tolist(),
                               d2t=d2t, drafted=tokens, history=t, probs=True, max_top_logprobs=5)
    check_singular(selection, expected, logprobs=False, probabilities=probs, slot_mapping=slot_mapping)


@pytest.mark.parametrize("seed", [50, 51])
def test_scalar_path_multistep(seed):

    from bench import MultistepWorkload, spiked_logits

    slots, batch, gamma, vocab = 10, 6, 3, 50257
    n = gamma + 1
    g = torch.Generator().manual_seed(seed)
    host = random_host(slots, n, vocab, 70 + seed, max_top_logprobs=4)
    logits = spiked_logits(batch * n, vocab, seed=700 + seed)
    slot_mapping = torch.randperm(slots, generator=g)[:batch].to(torch.int32)
    argmax = logits.float().argmax(-1)
    drafted = torch.where(torch.rand(batch * n, generator=g) < 0.6, argmax,
                          torch.randint(1, vocab, (batch * n,), generator=g)).to(torch.int32)
    probabilities = torch.softmax(torch.randn(slots, gamma, vocab, generator=g) * 2, dim=-1).to(torch.bfloat16)
    work = MultistepWorkload(logits=logits, drafted=drafted, buffers=host,
                             cu_seqlens=list(range(0, batch * n + 1, n)), lookahead=gamma, vocab=vocab,
                             max_top_logprobs=4, probabilities=probabilities)
    print(f"multistep scalar path seed={seed}", flush=True)
    verification, buffers, _ = run_verifier(work, update_counts=True, block_size=2048,
                                            slot_mapping=slot_mapping.to(DEV))

    state = oracle.State.from_buffers(host)
    expected = oracle.multistep(logits, state, drafted, work.cu_seqlens, slot_mapping=slot_mapping.tolist(),
                                probabilities=probabilities, logprobs=True, max_top_logprobs=4)
    mismatched = check_multistep(verification, expected, work.cu_seqlens, logprobs=True, max_knife_fraction=0.34)

    counts = expected_multistep_counts(state.decode, expected, verification, work.cu_seqlens, mismatched,
                                       slot_mapping.tolist())
    assert torch.equal(buffers.repetition.counts.decode.cpu(), counts)


# ------------------------------------------------------------------------------------------------
# 8192-column tiles with every processor on (the chain in two halves)
# ------------------------------------------------------------------------------------------------

# the last tile holds 2048 columns (ends inside the first half) or 6144 (inside the second)
SPLIT_VOCABS = [3 * 8192 + 2048, 3 * 8192 + 6144]


@pytest.mark.parametrize("vocab", SPLIT_VOCABS)
def test_8192_tiles_autoregressive_every_processor(vocab):

    from bench import spiked_logits

    rows = 12
    print(f"8192 tiles, autoregressive: V={vocab}", flush=True)
    host = random_host(rows, 1, vocab, vocab % 97, EVERY_PROCESSOR)
    logits = spiked_logits(rows, vocab, seed=vocab).to(DEV)
    assert autoregressive_case(logits, host, 8192) >= rows - 1


@pytest.mark.parametrize("vocab,indicator", [(65536, EVERY_PROCESSOR), (57344 + 4100, EVERY_PROCESSOR),
                                             (131072, None), (40000, 0x400)])
def test_16384_tiles_autoregressive(vocab, indicator):
    """16384-column tiles (64 elements per thread): the processor chain in four 4096-column passes,
    survivor masks over 32 key pairs, the exact cut's tie scan in two groups; partial last tiles."""

    from bench import spiked_logits

    rows = 12
    print(f"16384 tiles, autoregressive: V={vocab} indicator={indicator}", flush=True)
    host = random_host(rows, 1, vocab, vocab % 91, indicator)
    logits = spiked_logits(rows, vocab, seed=vocab + 5).to(DEV)
    assert autoregressive_case(logits, host, 16384) >= rows - 1


@pytest.mark.parametrize("vocab", SPLIT_VOCABS)
def test_8192_tiles_drafting_history(vocab):
    """Drafting without d2t: the first t drafted columns extend the decode history."""

    from bench import spiked_logits, to_device
    from sonic_sampler.interface import UnshardedFusedSingular

    slots, rows, gamma, t = 10, 8, 4, 3
    g = torch.Generator().manual_seed(vocab)
    host = random_host(slots, gamma + 1, vocab, vocab % 89, EVERY_PROCESSOR)
    buffers = to_device(host, DEV)
    logits = spiked_logits(rows, vocab, seed=vocab + 1)
    slot_mapping = torch.randperm(slots, generator=g)[:rows].to(torch.int32)
    # half the history hits the row's own spikes, so the penalties change the top of the row
    spikes = logits.float().argsort(-1, descending=True)[:, :gamma + 1].to(torch.int32)
    tokens = torch.where(torch.rand(rows, gamma + 1, generator=g) < 0.5, spikes,
                         torch.randint(0, vocab, (rows, gamma + 1), generator=g).to(torch.int32))
    print(f"8192 tiles, drafting with history: V={vocab}", flush=True)

    sampler = UnshardedFusedSingular.initialize(vocab_size=vocab, batch_size=rows, lookahead=gamma,
                                                block_size=8192, max_top_logprobs=5, device=DEV)
    probs = torch.zeros(slots, vocab, dtype=torch.bfloat16, device=DEV)
    selection = sampler.drafting(logits.to(DEV), buffers, timestep=t, tokens=tokens.to(DEV),
                                 probabilities=probs, slot_mapping=slot_mapping.to(DEV))
    torch.cuda.synchronize()

    state = oracle.State.from_buffers(host)
    expected = oracle.singular(logits, state, scope="draft", timestep=t, slot_mapping=slot_mapping.tolist(),
                               drafted=tokens, history=t, probs=True, max_top_logprobs=5)
    check_singular(selection, expected, logprobs=False, probabilities=probs, slot_mapping=slot_mapping)


@pytest.mark.parametrize("vocab,block", [(v, 8192) for v in SPLIT_VOCABS] + [(65536, 16384), (40004, 16384)])
def test_8192_tiles_multistep_every_processor(vocab, block):

    from bench import MultistepWorkload, spiked_logits

    slots, batch, gamma = 8, 4, 3
    n = gamma + 1
    g = torch.Generator().manual_seed(vocab + 2)
    host = random_host(slots, n, vocab, vocab % 83, EVERY_PROCESSOR, max_top_logprobs=4)
    logits = spiked_logits(batch * n, vocab, seed=vocab + 3)
    slot_mapping = torch.randperm(slots, generator=g)[:batch].to(torch.int32)
    argmax = logits.float().argmax(-1)
    drafted = torch.where(torch.rand(batch * n, generator=g) < 0.6, argmax,
                          torch.randint(1, vocab, (batch * n,), generator=g)).to(torch.int32)
    probabilities = torch.softmax(torch.randn(slots, gamma, vocab, generator=g) * 2, dim=-1).to(torch.bfloat16)
    work = MultistepWorkload(logits=logits, drafted=drafted, buffers=host,
                             cu_seqlens=list(range(0, batch * n + 1, n)), lookahead=gamma, vocab=vocab,
                             max_top_logprobs=4, probabilities=probabilities)
    print(f"{block} tiles, multistep: V={vocab}", flush=True)
    verification, buffers, _ = run_verifier(work, update_counts=True, block_size=block,
                                            slot_mapping=slot_mapping.to(DEV))

    state = oracle.State.from_buffers(host)
    expected = oracle.multistep(logits, state, drafted, work.cu_seqlens, slot_mapping=slot_mapping.tolist(),
                                probabilities=probabilities, logprobs=True, max_top_logprobs=4)
    mismatched = check_multistep(verification, expected, work.cu_seqlens, logprobs=True, max_knife_fraction=0.25)

    counts = expected_multistep_counts(state.decode, expected, verification, work.cu_seqlens, mismatched,
                                       slot_mapping.tolist())
    assert torch.equal(buffers.repetition.counts.decode.cpu(), counts)


# ------------------------------------------------------------------------------------------------
# Sparse grammars: fewer admitted tokens than a tile's 128 candidates, so every tile's top-128 ends
# in ties at the -inf of the masked tokens and every tile takes the exact cut
# ------------------------------------------------------------------------------------------------

def sparse_grammar(host, vocab, allowed, seed):
    """Each (slot, timestep) grammar row of `host` admits `allowed` random tokens."""

    g = torch.Generator().manual_seed(seed)
    slots, steps, words = host.grammar.shape
    bits = torch.zeros(slots * steps, words * 32, dtype=torch.bool)

    for r in range(slots * steps):

        bits[r, torch.randperm(vocab, generator=g)[:allowed]] = True

    packed = (bits.view(-1, words, 32).to(torch.int64) << torch.arange(32, dtype=torch.int64)).sum(-1)
    host.grammar.view(torch.int32).copy_((packed - ((packed >> 31) << 32)).to(torch.int32).view(slots, steps, words))


@pytest.mark.parametrize("allowed,block", [(40, 4096), (3, 4096), (40, 16384), (3, 2048)])
def test_sparse_grammar_autoregressive(allowed, block):
    """Config-1 rows with every processor on and a grammar admitting 40 or 3 tokens: the sampled
    token is admitted, and with 3 admitted the top-5 logprobs end in -inf entries at the lowest
    masked columns, which only an exact tie rule at the cut gets right."""

    from bench import spiked_logits

    rows, vocab = 24, 128256
    print(f"sparse grammar, autoregressive: allowed={allowed} block={block}", flush=True)
    host = random_host(rows, 1, vocab, 60 + allowed, EVERY_PROCESSOR)
    sparse_grammar(host, vocab, allowed, seed=61 + allowed)
    logits = spiked_logits(rows, vocab, seed=62 + allowed).to(DEV)
    assert autoregressive_case(logits, host, block) >= rows - 1


@pytest.mark.parametrize("allowed", [40, 3])
def test_sparse_grammar_multistep(allowed):

    from bench import MultistepWorkload, spiked_logits

    slots, batch, gamma, vocab = 8, 4, 3, 128256
    n = gamma + 1
    g = torch.Generator().manual_seed(allowed)
    host = random_host(slots, n, vocab, 70 + allowed, EVERY_PROCESSOR, max_top_logprobs=4)
    sparse_grammar(host, vocab, allowed, seed=71 + allowed)
    logits = spiked_logits(batch * n, vocab, seed=72 + allowed)
    drafted = torch.randint(1, vocab, (batch * n,), generator=g).to(torch.int32)
    probabilities = torch.softmax(torch.randn(slots, gamma, vocab, generator=g) * 2, dim=-1).to(torch.bfloat16)
    work = MultistepWorkload(logits=logits, drafted=drafted, buffers=host,
                             cu_seqlens=list(range(0, batch * n + 1, n)), lookahead=gamma, vocab=vocab,
                             max_top_logprobs=4, probabilities=probabilities)
    print(f"sparse grammar, multistep: allowed={allowed}", flush=True)
    verification, buffers, verifier = run_verifier(work, update_counts=True, block_size=16384)

    state = oracle.State.from_buffers(host)
    expected = oracle.multistep(logits, state, drafted, work.cu_seqlens, probabilities=probabilities,
                                logprobs=True, max_top_logprobs=4)
    mismatched = check_multistep(verification, expected, work.cu_seqlens, logprobs=True, max_knife_fraction=0.25)
    indices = verifier.indices.cpu()

    for b, e in enumerate(expected):

        for i, idx in enumerate(e.row_indices):

            assert torch.equal(indices[work.cu_seqlens[b] + i], idx), (b, i)

    counts = expected_multistep_counts(state.decode, expected, verification, work.cu_seqlens, mismatched)
    assert torch.equal(buffers.repetition.counts.decode.cpu(), counts)


# ------------------------------------------------------------------------------------------------
# hipGraph replay
# ------------------------------------------------------------------------------------------------

def singular_outputs(selection):

    lp = selection.logprobs
    return [t.clone() for t in (selection.tokens, lp.selected, lp.top_k.tokens, lp.top_k.logprobs)]


def test_eager_calls_run_on_the_current_stream():
    """A call made under a side stream launches on it: the logits are written on that stream
    behind a GPU sleep, so a launch on any other stream would read the zeros they replace."""

    from bench import spiked_logits, to_device
    from sonic_sampler.interface import UnshardedFusedSingular

    rows, vocab = 8, 16384
    host = random_host(rows, 1, vocab, 81, EVERY_PROCESSOR)
    logits = spiked_logits(rows, vocab, seed=82)
    sampler = UnshardedFusedSingular.initialize(vocab_size=vocab, batch_size=rows, max_top_logprobs=5,
                                                block_size=4096, device=DEV)
    buffers = to_device(host, DEV)
    source = logits.to(DEV)
    target = torch.zeros_like(source)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    print("eager call under a side stream", flush=True)

    with torch.cuda.stream(side):

        torch.cuda._sleep(20_000_000)
        target.copy_(source)
        selection = sampler.autoregressive(target, buffers, logprobs=True)

    side.synchronize()
    expected = oracle.singular(logits, oracle.State.from_buffers(host), scope="target", logprobs=True,
                               max_top_logprobs=5)
    check_singular(selection, expected, logprobs=True)


def test_graph_replay_autoregressive_config1():

    from bench import c1_workload, to_device
    from sonic_sampler.interface import UnshardedFusedSingular

    sets = []

    for k in range(3):

        work = c1_workload(seed=1001 + 10 * k)
        slots = torch.randperm(64, generator=torch.Generator().manual_seed(k)).to(torch.int32)
        sets.append((work, slots))

    batch, vocab = sets[0][0].logits.shape
    buffers = to_device(sets[0][0].buffers, DEV)
    logits = sets[0][0].logits.to(DEV)
    slot_mapping = sets[0][1].to(DEV)
    sampler = UnshardedFusedSingular.initialize(vocab_size=vocab, batch_size=batch, max_top_logprobs=5, device=DEV)

    def load(k):

        work, slots = sets[k]
        load_into(buffers, work.buffers)
        logits.copy_(work.logits)
        slot_mapping.copy_(slots)

    def call():

        return sampler.autoregressive(logits, buffers, update_counts=True, logprobs=True,
                                      slot_mapping=slot_mapping)

    eager = []

    for k in range(3):

        load(k)
        eager.append(singular_outputs(call()) + [buffers.repetition.counts.decode.clone()])

    torch.cuda.synchronize()
    print("config 1 eager outputs for 3 input sets; capturing", flush=True)

    load(0)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())

    with torch.cuda.stream(side):

        call()                                   # warm-up on the capture stream's side

    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()

    with torch.cuda.graph(graph):

        captured = call()

    for rnd, k in enumerate([1, 0, 2, 1, 2, 0]):

        load(k)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = singular_outputs(captured) + [buffers.repetition.counts.decode.clone()]
        print(f"replay {rnd}: input set {k}", flush=True)

        for a, b in zip(got, eager[k]):

            assert torch.equal(a, b), f"replay {rnd} of input set {k} differs from the eager call"

        if rnd < 3:

            work, slots = sets[k]
            state = oracle.State.from_buffers(work.buffers)
            expected = oracle.singular(work.logits, state, scope="target", slot_mapping=slots.tolist(),
                                       logprobs=True, max_top_logprobs=5)
            mismatched, _ = check_singular(captured, expected, logprobs=True)

            counts = expected_singular_counts(state.decode, expected, captured, mismatched, slots.tolist())
            assert torch.equal(got[-1].cpu(), counts)


def test_graph_replay_drafting_config4():
    """Config 4 (drafting through d2t into a 262144-token target vocabulary, staged grammar)
    captured in a hipGraph and replayed over new logits, buffers, drafts, slots and d2t copied
    into the captured tensors: every replay equals the eager call, and the first ones the
    oracle."""

    from bench import c4_workload, to_device
    from sonic_sampler.interface import UnshardedFusedSingular

    sets = [c4_workload(seed=1004 + 10 * k) for k in range(3)]
    base = sets[0]
    rows, slots = base.logits.size(0), base.buffers.layout.rows
    buffers = to_device(base.buffers, DEV)
    logits = base.logits.to(DEV)
    tokens = base.tokens.to(DEV)
    slot_mapping = base.slot_mapping.to(DEV)
    d2t = base.d2t.to(DEV)
    probs = torch.zeros(slots, base.target_vocab, dtype=torch.bfloat16, device=DEV)
    sampler = UnshardedFusedSingular.initialize(vocab_size=base.vocab, batch_size=rows, lookahead=4,
                                                max_top_logprobs=5, device=DEV)

    def load(k):

        work = sets[k]
        load_into(buffers, work.buffers)
        logits.copy_(work.logits)
        tokens.copy_(work.tokens)
        slot_mapping.copy_(work.slot_mapping)
        d2t.copy_(work.d2t)
        probs.zero_()

    def call():

        return sampler.drafting(logits, buffers, timestep=base.timestep, tokens=tokens, probabilities=probs,
                                slot_mapping=slot_mapping, d2t_mapping=d2t, target_vocab=base.target_vocab,
                                in_place=True)

    eager = []

    for k in range(3):

        load(k)
        selection = call()
        eager.append([selection.tokens.clone(), probs.clone()])

    torch.cuda.synchronize()
    print("config 4 eager outputs for 3 input sets; capturing", flush=True)
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
        got = [captured.tokens.clone(), probs.clone()]

        for a, b in zip(got, eager[k]):

            assert torch.equal(a, b), f"replay {rnd} of input set {k} differs from the eager call"

        if rnd < 3:

            work = sets[k]
            state = oracle.State.from_buffers(work.buffers)
            expected = oracle.singular(work.logits, state, scope="draft", timestep=work.timestep,
                                       slot_mapping=work.slot_mapping.tolist(), d2t=work.d2t,
                                       drafted=work.tokens, history=work.timestep, probs=True,
                                       max_top_logprobs=5)
            check_singular(captured, expected, logprobs=False, probabilities=probs,
                           slot_mapping=work.slot_mapping)


def test_graph_replay_verifier_config3():

    from bench import c3_workload, to_device
    from sonic_sampler.interface import UnshardedFusedMultistep

    base = c3_workload()
    lengths = [base.cu_seqlens[b + 1] - base.cu_seqlens[b] for b in range(len(base.cu_seqlens) - 1)]
    sets = [(base, torch.arange(64, dtype=torch.int32))]

    for k in (1, 2):

        work = c3_workload(seed=1003 + 10 * k, lengths=lengths)
        sets.append((work, torch.randperm(64, generator=torch.Generator().manual_seed(k)).to(torch.int32)))

    batch = len(lengths)
    buffers = to_device(base.buffers, DEV)
    logits = base.logits.to(DEV)
    drafted = base.drafted.to(DEV)
    probs = base.probabilities.to(DEV)
    slot_mapping = sets[0][1].to(DEV)
    cu = torch.tensor(base.cu_seqlens, dtype=torch.int32, device=DEV)
    verifier = UnshardedFusedMultistep.initialize(vocab_size=base.vocab, lookahead=base.lookahead,
                                                  batch_size=batch, max_top_logprobs=20, device=DEV)

    def load(k):

        work, slots = sets[k]
        load_into(buffers, work.buffers)
        logits.copy_(work.logits)
        drafted.copy_(work.drafted)
        # request b reads the draft distribution of its slot
        probs.copy_(work.probabilities[torch.argsort(slots.long())])
        slot_mapping.copy_(slots)

    def call():

        return verifier(logits, drafted, buffers, probabilities=probs, update_counts=True, logprobs=True,
                        cu_seqlens=cu, slot_mapping=slot_mapping)

    starts = torch.tensor(base.cu_seqlens[:-1], dtype=torch.int64)
    request = torch.repeat_interleave(torch.arange(batch), torch.tensor(lengths))
    position = torch.arange(base.cu_seqlens[-1]) - starts[request]

    def outputs(v):
        """What the call defines: offsets, and tokens / logprobs / top logprobs of the emitted
        positions (rows past a request's offset are not written, as in the reference)."""

        offsets = v.offsets.reshape(-1).cpu()
        emitted = (position <= offsets[request]).to(DEV)
        top = v.logprobs.top_k
        return [v.offsets.clone(), v.tokens.reshape(-1)[emitted], v.logprobs.selected.reshape(-1)[emitted],
                top.tokens.reshape(-1, 20)[emitted], top.logprobs.reshape(-1, 20)[emitted],
                buffers.repetition.counts.decode.clone()]

    eager = []

    for k in range(3):

        load(k)
        eager.append(outputs(call()))

    torch.cuda.synchronize()
    print("config 3 eager outputs for 3 input sets; capturing", flush=True)

    load(0)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())

    with torch.cuda.stream(side):

        call()

    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()

    with torch.cuda.graph(graph):

        captured = call()

    for rnd, k in enumerate([2, 0, 1, 2, 1, 0]):

        load(k)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = outputs(captured)
        print(f"replay {rnd}: input set {k}", flush=True)

        for a, b in zip(got, eager[k]):

            assert torch.equal(a, b), f"replay {rnd} of input set {k} differs from the eager call"

        if rnd < 3:

            work, slots = sets[k]
            state = oracle.State.from_buffers(work.buffers)
            q = work.probabilities[torch.argsort(slots.long())]
            expected = oracle.multistep(work.logits, state, work.drafted, work.cu_seqlens,
                                        slot_mapping=slots.tolist(), probabilities=q, logprobs=True,
                                        max_top_logprobs=20)
            check_multistep(captured, expected, work.cu_seqlens, logprobs=True)


# ------------------------------------------------------------------------------------------------
# The two kernel layouts of the single-step path (tile grid + row merge, one workgroup per row)
# ------------------------------------------------------------------------------------------------

def layout_outputs(selection, probs, buffers, host, rows):
    """Outputs both layouts must produce identically: tokens, logprobs, the written top
    logprobs, the probability buffer and the decode counts."""

    out = [selection.tokens.cpu(), buffers.repetition.counts.decode.cpu()]

    if probs is not None:

        out.append(probs.cpu())

    if selection.logprobs is not None:

        out.append(selection.logprobs.selected.cpu())
        top = selection.logprobs.top_k

        if top is not None:

            written = torch.zeros(top.tokens.shape, dtype=torch.bool)

            for r in range(rows):

                ind = int(host.flags.indicators.target[r])

                if ind & 0x400 and not ind & 0x40:

                    written[r, :min(int(host.top_logprobs[r]), top.tokens.size(1))] = True

            out += [top.tokens.cpu()[written], top.logprobs.cpu()[written]]

    return out


@pytest.mark.parametrize("vocab,block,indicator,seed", [
    (16384, 2048, EVERY_PROCESSOR, 61), (32000, 4096, None, 62), (8191, 1024, None, 63),
    (30720, 8192, EVERY_PROCESSOR, 64)])
def test_layouts_agree_autoregressive(vocab, block, indicator, seed):

    from bench import spiked_logits, to_device
    from sonic_sampler.interface import UnshardedFusedSingular

    rows = 24
    host = random_host(rows, 1, vocab, seed, indicator)
    logits = spiked_logits(rows, vocab, seed=800 + seed).to(DEV)
    sampler = UnshardedFusedSingular.initialize(vocab_size=vocab, batch_size=rows, max_top_logprobs=5,
                                                block_size=block, device=DEV)
    results = {}

    for layout in ("tiles", "rowwise"):

        print(f"autoregressive V={vocab} block={block} layout={layout}", flush=True)
        buffers = to_device(host, DEV)
        selection = sampler.autoregressive(logits, buffers, update_counts=True, logprobs=True,
                                           kernel_layout=layout)
        torch.cuda.synchronize()
        results[layout] = layout_outputs(selection, None, buffers, host, rows)

        if layout == "rowwise":

            state = oracle.State.from_buffers(host)
            expected = oracle.singular(logits.cpu(), state, scope="target", logprobs=True, max_top_logprobs=5)
            check_singular(selection, expected, logprobs=True)

    for a, b in zip(results["tiles"], results["rowwise"]):

        assert torch.equal(a, b)


@pytest.mark.parametrize("block", [4096, 8192])
def test_layouts_agree_drafting_d2t_grammar(block):
    """Config-4 shape at 64 rows: d2t into a 262144-token target vocabulary with a 5% grammar
    mask; the rowwise layout stages each row's 32 KB of grammar words in workgroup memory."""

    from bench import c4_workload, to_device
    from sonic_sampler.interface import UnshardedFusedSingular

    work = c4_workload(rows=64, slots=128)
    rows = work.logits.size(0)
    slots = work.buffers.layout.rows
    sampler = UnshardedFusedSingular.initialize(vocab_size=work.vocab, batch_size=rows, lookahead=4,
                                                block_size=block, max_top_logprobs=5, device=DEV)
    results = {}

    for layout in ("tiles", "rowwise"):

        print(f"drafting d2t+grammar block={block} layout={layout}", flush=True)
        buffers = to_device(work.buffers, DEV)
        probs = torch.zeros(slots, work.target_vocab, dtype=torch.bfloat16, device=DEV)
        tokens = work.tokens.to(DEV)
        selection = sampler.drafting(work.logits.to(DEV), buffers, timestep=work.timestep, tokens=tokens,
                                     probabilities=probs, slot_mapping=work.slot_mapping.to(DEV),
                                     d2t_mapping=work.d2t.to(DEV), target_vocab=work.target_vocab,
                                     in_place=True, kernel_layout=layout)
        torch.cuda.synchronize()
        results[layout] = [selection.tokens.cpu(), probs.cpu(), tokens.cpu()]

        if layout == "rowwise":

            state = oracle.State.from_buffers(work.buffers)
            expected = oracle.singular(work.logits, state, scope="draft", timestep=work.timestep,
                                       slot_mapping=work.slot_mapping.tolist(), d2t=work.d2t,
                                       drafted=work.tokens, history=work.timestep, probs=True,
                                       max_top_logprobs=5)
            check_singular(selection, expected, logprobs=False, probabilities=probs,
                           slot_mapping=work.slot_mapping)

    for a, b in zip(results["tiles"], results["rowwise"]):

        assert torch.equal(a, b)


def test_concurrent_calls_from_two_threads_on_two_streams():
    """Two host threads, each with its own sampler instances, buffers and stream, call the decode
    step and the verifier alternately: every result equals the same call made alone. The library's
    host code keeps no per-call state outside the caller's buffers, and a ctypes call releases the
    interpreter lock, so the two threads' launches interleave."""

    import threading
    from types import SimpleNamespace

    from bench import spiked_logits, to_device
    from sonic_sampler.interface import UnshardedFusedMultistep, UnshardedFusedSingular

    rows, vocab, gamma, calls = 8, 16384, 2, 12
    n, batch = gamma + 1, rows // 2

    def make(seed):

        g = torch.Generator().manual_seed(seed)

        return SimpleNamespace(
            host=random_host(rows, n, vocab, seed, EVERY_PROCESSOR, max_top_logprobs=4),
            singular=UnshardedFusedSingular.initialize(vocab_size=vocab, batch_size=rows, max_top_logprobs=4,
                                                       block_size=4096, device=DEV),
            verifier=UnshardedFusedMultistep.initialize(vocab_size=vocab, lookahead=gamma, batch_size=batch,
                                                        max_top_logprobs=4, block_size=4096, device=DEV),
            logits=[spiked_logits(rows, vocab, seed=seed * 100 + i).to(DEV) for i in range(3)],
            target=[spiked_logits(batch * n, vocab, seed=seed * 100 + 50 + i).view(batch, n, vocab).to(DEV)
                    for i in range(3)],
            drafted=torch.randint(1, vocab, (batch, n), generator=g).to(torch.int32).to(DEV),
            probs=torch.softmax(torch.randn(batch, gamma, vocab, generator=g), dim=-1).to(torch.bfloat16).to(DEV),
            stream=torch.cuda.Stream())

    def run(ctx, out):

        with torch.cuda.stream(ctx.stream):

            buffers = to_device(ctx.host, DEV)

            for i in range(calls):

                if i % 2 == 0:

                    sel = ctx.singular.autoregressive(ctx.logits[i % 3], buffers, logprobs=True, philox_seed=7,
                                                      philox_offset=i)
                    out.append([t.clone() for t in (sel.tokens, sel.logprobs.selected)])

                else:

                    ver = ctx.verifier(ctx.target[i % 3], ctx.drafted, buffers, probabilities=ctx.probs,
                                       logprobs=True, philox_seed=9, philox_offset=i)
                    # logprobs are written for the emitted span only (positions up to the offset)
                    span = torch.arange(n, device=DEV)[None] <= ver.offsets
                    lp = torch.where(span, ver.logprobs.selected.float(), 0.0)
                    out.append([ver.tokens.clone(), ver.offsets.clone(), lp])

        ctx.stream.synchronize()

    contexts = [make(91), make(92)]
    torch.cuda.synchronize()
    alone = []

    for ctx in contexts:

        out = []
        run(ctx, out)
        alone.append(out)

    together = [[], []]
    print("two threads, two streams", flush=True)
    threads = [threading.Thread(target=run, args=(ctx, together[j])) for j, ctx in enumerate(contexts)]

    for t in threads:

        t.start()

    for t in threads:

        t.join()

    for j in range(2):

        assert len(together[j]) == calls

        for i in range(calls):

            for a, b in zip(alone[j][i], together[j][i]):

                assert torch.equal(a.cpu(), b.cpu()), (j, i)
