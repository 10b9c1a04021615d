"""ss_fused_singular_noalloc (static device scratch) against ss_fused_singular (caller scratchpad).

Both entry points are called through the C-ABI on identical inputs; every output must be
bit-identical. The no-allocation calls run twice in a row, the second on a smaller input (fewer
rows and tiles), so a stale candidate list left in the shared static array by the first call would
show. A call larger than the static array must be refused with SS_ERR_SCRATCH_LIMIT.
"""

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def build_case(rows, vocab, seed):

    from bench import spiked_logits
    from sonic_sampler.core.buffer import SamplingBuffers

    host = SamplingBuffers.random(size=rows, timesteps=1, vocab_size=vocab, device="cpu", seed=seed,
                                  max_top_logprobs=5)
    return host, spiked_logits(rows, vocab, seed=900 + seed)


def run(host, logits, block, static_scratch):
    """One autoregressive call with logprobs, top-5 and count updates on fresh device buffers."""

    from bench import to_device
    from sonic_sampler.interface.functional import fused_singular

    buffers = to_device(host, DEV)
    rep = buffers.repetition
    selection = fused_singular(
        logits=logits.to(DEV), indicators=buffers.flags.target, max_top_logprobs=5, update_counts=True,
        return_logprobs=True, block_n=block, grammar=buffers.grammar[:, 0],
        context_counts=rep.counts.context, decode_counts=rep.counts.decode,
        repetition_penalties=rep.multiplicative, frequency_penalties=rep.frequency,
        presence_penalties=rep.presence, logit_bias=buffers.bias, temperature=buffers.temperature,
        top_k=buffers.top_k, top_p=buffers.top_p, min_p=buffers.min_p,
        top_k_logprobs=buffers.top_logprobs, gumbel_noise=buffers.weights.gumbel.target[:, 0],
        static_scratch=static_scratch,
    )
    torch.cuda.synchronize()
    lp = selection.logprobs
    # top logprobs are written up to the row's limit only (per-row count, bit 0x400, non-greedy)
    written = torch.zeros(lp.top_k.tokens.shape, dtype=torch.bool)

    for r, ind in enumerate(host.flags.indicators.target[:logits.size(0)]):

        if int(ind) & 0x400 and not int(ind) & 0x40:

            written[r, :min(int(host.top_logprobs[r]), 5)] = True

    return [selection.tokens.cpu(), lp.selected.cpu(), lp.top_k.tokens.cpu()[written],
            lp.top_k.logprobs.cpu()[written], rep.counts.decode.cpu()]


def test_noalloc_matches_scratchpad_entry_point_on_consecutive_calls():

    # the second call is smaller: fewer rows and fewer tiles per row
    cases = [(48, 65536, 4096, 11), (12, 20480, 2048, 12)]
    expected = []

    for rows, vocab, block, seed in cases:

        host, logits = build_case(rows, vocab, seed)
        print(f"scratchpad entry point: rows={rows} V={vocab} block={block}", flush=True)
        expected.append(run(host, logits, block, static_scratch=False))

    for (rows, vocab, block, seed), want in zip(cases, expected):

        host, logits = build_case(rows, vocab, seed)
        print(f"static-scratch entry point: rows={rows} V={vocab} block={block}", flush=True)
        got = run(host, logits, block, static_scratch=True)

        for name, a, b in zip(("tokens", "logprobs", "top tokens", "top logprobs", "decode counts"), got, want):

            assert torch.equal(a, b), f"{name} differ at rows={rows} V={vocab}"


def test_noalloc_refuses_calls_beyond_the_static_scratch():

    from sonic_sampler import _native

    lib = _native.load()
    tiles = 32
    rows = _native.STATIC_SCRATCH_BYTES // (tiles * 128 * 4) + 1
    args = _native.SingularArgs(rows=rows, vocab_size=tiles * 4096, block_n=4096)
    print(f"oversize static-scratch call: rows={rows} tiles={tiles} (checked before any launch)", flush=True)
    assert lib.ss_fused_singular_noalloc(ctypes.byref(args)) == _native.SS_ERR_SCRATCH_LIMIT
    assert b"static scratch" in lib.ss_status_string(_native.SS_ERR_SCRATCH_LIMIT)
