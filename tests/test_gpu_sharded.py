"""Sharded-vocabulary sampling, the part one GPU can show (reference
interface/functional/singular.py:80-83,129-133, ops/prologue.py:293,382, ops/topk/unpack.py:127-247,
greedy ops/singular.py:32-68): a row's vocabulary is split into W column shards; every shard runs
the tile stage on its own columns into its slice of a [W, tiles, 128] scratchpad row (the slices an
engine would all-gather), then one row stage merges all W slices and selects. The result must equal
the unsharded call bit for bit, and the oracle.
"""

import pytest
import torch

from helpers import check_singular
from oracle import sampler as oracle

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def buffer_kwargs(buffers, scope, step, d2t=None, drafted=None, timestep=None):

    rep = buffers.repetition
    return dict(
        indicators=getattr(buffers.flags, scope), grammar=buffers.grammar[:, step],
        context_counts=rep.counts.context, decode_counts=rep.counts.decode,
        repetition_penalties=rep.multiplicative, frequency_penalties=rep.frequency,
        presence_penalties=rep.presence, logit_bias=buffers.bias, temperature=buffers.temperature,
        top_k=buffers.top_k, top_p=buffers.top_p, min_p=buffers.min_p,
        top_k_logprobs=buffers.top_logprobs,
        gumbel_noise=getattr(buffers.weights.gumbel, scope)[:, step], d2t_mapping=d2t,
        drafted_tokens=drafted, timestep=timestep,
    )


def outputs(selection, buffers, probs=None):

    out = [selection.tokens.cpu(), buffers.repetition.counts.decode.cpu()]

    if selection.logprobs is not None:

        out.append(selection.logprobs.selected.cpu())

    if probs is not None:

        out.append(probs.cpu())

    return out


def run_sharded(logits, buffers, world, block_n, target_vocab, **kw):
    """W tile stages into one scratchpad, then the row stage; returns the selection."""

    from sonic_sampler.interface.functional import fused_singular

    rows, vocab = logits.shape
    shard = vocab // world
    tiles = -(-shard // block_n)
    scratch = torch.empty(rows, world * tiles * 128, dtype=torch.int32, device=DEV).view(torch.uint32)
    selection = None

    for rank in range(world):

        local = logits[:, rank * shard:(rank + 1) * shard]
        fused_singular(local, world_size=world, local_rank=rank, shard_size=shard, target_vocab=target_vocab,
                       block_n=block_n, scratchpad=scratch, stage="tiles", **kw)

    # the row stage reads only the scratchpad; any shard's logits give the local width
    selection = fused_singular(logits[:, :shard], world_size=world, local_rank=0, shard_size=shard,
                               target_vocab=target_vocab, block_n=block_n, scratchpad=scratch, stage="rows", **kw)
    torch.cuda.synchronize()

    return selection


def test_config1_split_into_8_shards():

    from bench import c1_workload, to_device
    from sonic_sampler.interface.functional import fused_singular

    work = c1_workload()
    rows, vocab = work.logits.shape
    world = 8
    print(f"config 1 in {world} shards of {vocab // world} columns", flush=True)
    logits = work.logits.to(DEV)
    common = dict(max_top_logprobs=5, update_counts=True, return_logprobs=True)

    whole = to_device(work.buffers, DEV)
    expected = fused_singular(logits, block_n=4096, **common, **buffer_kwargs(whole, "target", 0))
    torch.cuda.synchronize()

    parts = to_device(work.buffers, DEV)
    got = run_sharded(logits, parts, world, 4096, vocab, **common, **buffer_kwargs(parts, "target", 0))

    for a, b in zip(outputs(got, parts), outputs(expected, whole)):

        assert torch.equal(a, b)

    top_a, top_b = got.logprobs.top_k, expected.logprobs.top_k
    assert torch.equal(top_a.tokens.cpu(), top_b.tokens.cpu())
    assert torch.equal(top_a.logprobs.cpu(), top_b.logprobs.cpu())

    state = oracle.State.from_buffers(work.buffers)
    ref = oracle.singular(work.logits, state, scope="target", logprobs=True, max_top_logprobs=5)
    check_singular(got, ref, logprobs=True)


@pytest.mark.parametrize("seed", [70, 71])
def test_unaligned_shards_mixed_rows(seed):
    """4 shards of 4099 columns: shard offsets that are not multiples of 32 take the per-element
    layout; random indicator mixes include greedy rows (the greedy merge of all shards' maxima)."""

    from bench import spiked_logits, to_device
    from sonic_sampler.core.buffer import SamplingBuffers
    from sonic_sampler.interface.functional import fused_singular

    rows, world, shard = 16, 4, 4099
    vocab = world * shard
    host = SamplingBuffers.random(size=rows, timesteps=1, vocab_size=vocab, device="cpu", seed=seed,
                                  max_top_logprobs=5)
    logits = spiked_logits(rows, vocab, seed=seed + 1).to(DEV)
    print(f"4 shards of {shard} columns, seed {seed}", flush=True)
    common = dict(max_top_logprobs=5, update_counts=True, return_logprobs=True)

    whole = to_device(host, DEV)
    expected = fused_singular(logits, block_n=2048, **common, **buffer_kwargs(whole, "target", 0))
    parts = to_device(host, DEV)
    got = run_sharded(logits, parts, world, 2048, vocab, **common, **buffer_kwargs(parts, "target", 0))

    for a, b in zip(outputs(got, parts), outputs(expected, whole)):

        assert torch.equal(a, b)

    state = oracle.State.from_buffers(host)
    ref = oracle.singular(logits.cpu(), state, scope="target", logprobs=True, max_top_logprobs=5)
    check_singular(got, ref, logprobs=True)


def test_sharded_drafting_with_d2t_and_grammar():
    """A draft vocabulary of 4 x 2048 columns mapped through d2t into a 65536-token target
    vocabulary with a grammar mask and drafted history: shard w's columns are draft ids
    w * 2048 + c, remapped through d2t before every side-plane lookup."""

    from bench import spiked_logits, to_device
    from sonic_sampler.core.buffer import SamplingBuffers
    from sonic_sampler.interface.functional import fused_singular

    rows, world, shard, target, gamma, t = 12, 4, 2048, 65536, 3, 2
    draft = world * shard
    g = torch.Generator().manual_seed(5)
    host = SamplingBuffers.random(size=rows, timesteps=gamma + 1, vocab_size=target, device="cpu", seed=5,
                                  max_top_logprobs=5)
    d2t = torch.randperm(target, generator=g)[:draft].to(torch.int32)
    tokens = torch.randint(1, target, (rows, gamma + 1), generator=g).to(torch.int32)
    logits = spiked_logits(rows, draft, seed=6).to(DEV)
    print(f"sharded drafting: {world} shards of {shard} draft columns -> {target}", flush=True)

    results = []

    for sharded in (False, True):

        buffers = to_device(host, DEV)
        probs = torch.zeros(rows, target, dtype=torch.bfloat16, device=DEV)
        kw = dict(max_top_logprobs=5, lookahead=gamma, return_probabilities=True, draft_probabilities=probs,
                  **buffer_kwargs(buffers, "draft", t, d2t=d2t.to(DEV), drafted=tokens.to(DEV), timestep=t))

        if sharded:

            sel = run_sharded(logits, buffers, world, 1024, target, **kw)

        else:

            sel = fused_singular(logits, block_n=1024, target_vocab=target, **kw)
            torch.cuda.synchronize()

        results.append(outputs(sel, buffers, probs))

    for a, b in zip(*results):

        assert torch.equal(a, b)

    state = oracle.State.from_buffers(host)
    ref = oracle.singular(logits.cpu(), state, scope="draft", timestep=t, d2t=d2t, drafted=tokens, history=t,
                          probs=True, max_top_logprobs=5)
    assert [int(x) for x in results[1][0][:, 0]] == [r.token for r in ref] or any(r.knife for r in ref)
